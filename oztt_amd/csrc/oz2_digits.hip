// A18 (split): Scheme II residues split into digit planes for the digit formats (FP8 route).
//
// Semantics (reference ozaki2/kernels/modslice_digit.cpp:142-243 with sparse_fix.h:48-78, host side
// split.hpp:157-279): per element the symmetric residue r = A' mod m_s (the same binary32 procedure
// as the INT8 residues, oz2_residue.hpp; m up to 2401) is split into digits that the e4m3 format
// holds exactly:
//   rounded (square m = q^2, and non-square "wide" moduli): h = Rnd(r * qinv), l = r - q*h;
//   sparse square (q odd): the rounded digits, then an odd digit with |.| >= 17 is moved by q
//     (l -= sgn(l) q with h += sgn(l); then h -= sgn(h) q), so both are in {|x| <= 16} or even <= 32;
//   Karatsuba (radix q = 16): h = Rnd((r + sgn(r)(q/2 - 1/2)) * qinv), l = r - q*h, s = h + l,
//     sgn(r) read from the sign bit;
//   one digit (m <= 33, |r| <= 16; split.hpp:202-205, modslice_digit.cpp:76-79): the residue itself.
// Planes per modulus in this order: l, h (and s for Karatsuba), or r alone; the moduli follow each
// other.
// Every step is one binary32 operation as in the reference (no contraction), so the digits equal
// the reference's bit for bit; they are integers of magnitude <= 32.
//
// Encoding: e4m3 (OCP, the format of the gfx950 FP8 matrix instructions; every digit is exact in
// it), converted with the hardware instruction, or int8.
//
// MI355X design: the blocked splitter of oz_tf32.hpp (one wave per 1 KB OZ_BLOCK block, coalesced
// FP64 reads, one contiguous 1 KB store per plane), with the generator running the planes itself:
// modulus by modulus, the residues of the wave's elements, their digits, then the modulus's 2 or 3
// planes, converted to e4m3 two digits per instruction. A and B can be split in one launch
// (oz2_split_digits_pair).
#pragma clang fp contract(off)

#include "oz2_residue.hpp"
#include "oz_internal.hpp"

namespace {

constexpr int XM_ROUND = 0, XM_KAR = 1, XM_SPARSE = 2, XM_ONE = 3;

__host__ __device__ constexpr int planes_of(int xm) { return xm == XM_KAR ? 3 : (xm == XM_ONE ? 1 : 2); }

struct DigitConsts {
    SplitConsts k;
    int S;
    float q[OZ2_MAXS], qinv[OZ2_MAXS];
    int xmode[OZ2_MAXS];
};

// Four digits (exact small integers) as the stored bytes: e4m3 codes, two per conversion
// instruction, or int8.
template <bool E4M3>
__device__ __forceinline__ uint32_t digit_bytes(float a, float b, float c, float d) {
    if constexpr (E4M3) {
        const int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
        return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    } else {
        return pack4((int)a, (int)b, (int)c, (int)d);
    }
}

// Runs the planes modulus by modulus (kDrivesPlanes): the residue of every element, its digits,
// then the modulus's 2 or 3 planes. The split mode is uniform per modulus, so its branches are
// scalar; within a mode the digits are computed without branches (the sparse rule as selects; its
// operations on small integers are exact, so integer arithmetic gives the reference's values).
template <int ND, bool E4M3>
struct DigitGen {
    static constexpr bool kDrivesPlanes = true;
    DigitConsts k;
    int S;
    struct State {
        float dig[ND];
    };
    __device__ __forceinline__ void load(State& st, double x, int32_t dl) const { make_digits<ND>(x, dl, st.dig); }
    template <class EMIT>
    __device__ __forceinline__ void run(State* st, EMIT&& emit) const {
        int p = 0;
        for (int s = 0; s < S; s++) {
            const int xm = k.xmode[s];
            const float q = k.q[s], qinv = k.qinv[s];
            float l[16], h[16], t[16];
            if (xm == XM_ONE) {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 16; e++) l[e] = residue_f<ND>(st[e].dig, k.k, s);
#pragma unroll
                for (int c = 0; c < 4; c++)
                    w[c] = digit_bytes<E4M3>(l[4 * c], l[4 * c + 1], l[4 * c + 2], l[4 * c + 3]);
                emit(p, w);
                p += 1;
                continue;
            }
            if (xm == XM_KAR) {
                const float half = q * 0.5f - 0.5f;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float r = residue_f<ND>(st[e].dig, k.k, s);
                    const float tt = __builtin_signbit(r) ? -half : half;  // sgn(r) (q/2 - 1/2)
                    h[e] = __builtin_rintf((r + tt) * qinv);
                    l[e] = r - h[e] * q;
                    t[e] = h[e] + l[e];
                }
            } else {
                const int qi = (int)q;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float r = residue_f<ND>(st[e].dig, k.k, s);
                    h[e] = __builtin_rintf(r * qinv);
                    l[e] = r - h[e] * q;
                }
                if (xm == XM_SPARSE) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        // an odd digit of magnitude >= 17 moves by q, l first (carrying into h), then h
                        int li = (int)l[e], hi = (int)h[e];
                        const int sl = li < 0 ? -1 : 1;
                        const bool fl = (li > 16 || li < -16) && (li & 1);
                        li = fl ? li - sl * qi : li;
                        hi = fl ? hi + sl : hi;
                        const bool fh = (hi > 16 || hi < -16) && (hi & 1);
                        hi = fh ? (hi < 0 ? hi + qi : hi - qi) : hi;
                        l[e] = (float)li;
                        h[e] = (float)hi;
                    }
                }
            }
            uint32_t w[4];
#pragma unroll
            for (int c = 0; c < 4; c++) w[c] = digit_bytes<E4M3>(l[4 * c], l[4 * c + 1], l[4 * c + 2], l[4 * c + 3]);
            emit(p, w);
#pragma unroll
            for (int c = 0; c < 4; c++) w[c] = digit_bytes<E4M3>(h[4 * c], h[4 * c + 1], h[4 * c + 2], h[4 * c + 3]);
            emit(p + 1, w);
            if (xm == XM_KAR) {
#pragma unroll
                for (int c = 0; c < 4; c++)
                    w[c] = digit_bytes<E4M3>(t[4 * c], t[4 * c + 1], t[4 * c + 2], t[4 * c + 3]);
                emit(p + 2, w);
                p += 3;
            } else {
                p += 2;
            }
        }
    }
};

template <int ND, bool E4M3>
int launch_digits(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                  const DigitConsts& k, int nplanes, uint8_t* planes, int layout, int prow, int pld, long long pstride) {
    const int kblocks = pld / 64;
    const long long nblocks = (long long)(prow / 16) * kblocks;
    const unsigned grid = oz::ceil_div(nblocks, 4);
    const DigitGen<ND, E4M3> gen{k, k.S};
    if (layout == 2)
        hipLaunchKernelGGL((split_block_kernel<DigitGen<ND, E4M3>, false>), dim3(grid), dim3(256), 0, dev->stream, X,
                           rows, cols, ld, mode, delta, gen, nplanes, reinterpret_cast<uint4*>(planes), kblocks,
                           nblocks, pstride / 16);
    else
        hipLaunchKernelGGL((split_block_kernel<DigitGen<ND, E4M3>, true>), dim3(grid), dim3(256), 0, dev->stream, X,
                           rows, cols, ld, mode, delta, gen, nplanes, reinterpret_cast<uint4*>(planes), kblocks,
                           nblocks, pstride / 16);
    return oz::launch_check(dev, "split_block_kernel");
}

template <int ND>
int launch_digits_enc(oz_dev* dev, bool e4m3, const double* X, int rows, int cols, int ld, int mode,
                      const int32_t* delta, const DigitConsts& k, int nplanes, uint8_t* planes, int layout, int prow,
                      int pld, long long pstride) {
    return e4m3 ? launch_digits<ND, true>(dev, X, rows, cols, ld, mode, delta, k, nplanes, planes, layout, prow, pld,
                                          pstride)
                : launch_digits<ND, false>(dev, X, rows, cols, ld, mode, delta, k, nplanes, planes, layout, prow, pld,
                                           pstride);
}

// Kernel constants of a digit descriptor, and its plane count; a message on failure.
const char* digit_consts(const oz2_digit_dev* dd, DigitConsts& k, int& np) {
    if (!dd || dd->mo.S < 1 || dd->mo.S > OZ2_MAXS || dd->mo.nd < 3 || dd->mo.nd > 5 || dd->encoding < 0 ||
        dd->encoding > 1)
        return "invalid digit descriptor";
    k = DigitConsts{};
    k.S = dd->mo.S;
    np = 0;
    for (int s = 0; s < dd->mo.S; s++) {
        const float m = dd->mo.m[s], q = dd->q[s];
        const int xm = dd->xmode[s];
        if (!(m >= 2.0f && m <= 2401.0f) || xm < XM_ROUND || xm > XM_ONE ||
            (xm == XM_ONE ? !(m <= 33.0f) : !(q >= 2.0f && q <= 64.0f)))
            return "a modulus, radix or split mode is not supported";
        k.k.m[s] = m;
        k.k.rinv[s] = dd->mo.rinv[s];
        for (int j = 0; j < 4; j++) k.k.c[j][s] = dd->mo.c[j][s];
        k.q[s] = q;
        k.qinv[s] = dd->qinv[s];
        k.xmode[s] = xm;
        np += planes_of(xm);
        if (np > OZ2_MAXPLANES) return "more digit planes than OZ2_MAXPLANES";
    }
    return nullptr;
}

template <int ND, bool E4M3>
int launch_digits_pair(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA, const double* B, int N,
                       int ldb, const int32_t* dB, const DigitConsts& k, int nplanes, uint8_t* pA, uint8_t* pB, int Mg,
                       int Ng, int Kg) {
    const int kblocks = Kg / 64;
    const long long nbA = (long long)(Mg / 16) * kblocks, nbB = (long long)(Ng / 16) * kblocks;
    const long long sA = (long long)Mg * Kg / 16, sB = (long long)Ng * Kg / 16;
    const long long grid = (nbA + 3) / 4 + (nbB + 3) / 4;
    if (grid > 0x7FFFFFFFll) return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits_pair: grid too large");
    const DigitGen<ND, E4M3> gen{k, k.S};
    hipLaunchKernelGGL((split_pair_kernel<DigitGen<ND, E4M3>>), dim3((unsigned)grid), dim3(256), 0, dev->stream, A, M,
                       K, lda, dA, reinterpret_cast<uint4*>(pA), nbA, sA, B, N, ldb, dB, reinterpret_cast<uint4*>(pB),
                       nbB, sB, kblocks, gen, nplanes);
    return oz::launch_check(dev, "split_pair_kernel<DigitGen>");
}

}  // namespace

extern "C" int oz2_digit_planes(const oz2_digit_dev* dd) {
    if (!dd || dd->mo.S < 1 || dd->mo.S > OZ2_MAXS) return -1;
    int n = 0;
    for (int s = 0; s < dd->mo.S; s++) n += planes_of(dd->xmode[s]);
    return n;
}

extern "C" int oz2_split_digits(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode,
                                const int32_t* delta, const oz2_digit_dev* dd, uint8_t* planes, int layout, int prow,
                                int pld, long long plane_stride) {
    if (int st = oz::use(dev)) return st;
    DigitConsts k;
    int np = 0;
    if (const char* e = digit_consts(dd, k, np)) return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits: %s", e);
    if (!X || !delta || !planes || rows <= 0 || cols <= 0 || ld < cols || (mode != 0 && mode != 1) ||
        (layout != 2 && layout != 3))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits: invalid arguments");
    const bool tran = layout == 3;
    const int need_rows = tran ? cols : rows, need_ld = tran ? rows : cols;
    if (prow < need_rows || pld < need_ld || pld % 64 != 0 || prow % 16 != 0 || plane_stride % 1024 != 0 ||
        plane_stride < (long long)prow * pld || ((uintptr_t)planes & 15u))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits: plane geometry %dx%d (stride %lld) does not fit", prow, pld,
                        plane_stride);
    const bool e4m3 = dd->encoding == 1;
    switch (dd->mo.nd) {
    case 3: return launch_digits_enc<3>(dev, e4m3, X, rows, cols, ld, mode, delta, k, np, planes, layout, prow, pld, plane_stride);
    case 4: return launch_digits_enc<4>(dev, e4m3, X, rows, cols, ld, mode, delta, k, np, planes, layout, prow, pld, plane_stride);
    default: return launch_digits_enc<5>(dev, e4m3, X, rows, cols, ld, mode, delta, k, np, planes, layout, prow, pld, plane_stride);
    }
}

extern "C" int oz2_split_digits_pair(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA,
                                     const double* B, int N, int ldb, const int32_t* dB, const oz2_digit_dev* dd,
                                     uint8_t* planesA, uint8_t* planesB, int Mg, int Ng, int Kg) {
    if (int st = oz::use(dev)) return st;
    DigitConsts k;
    int np = 0;
    if (const char* e = digit_consts(dd, k, np)) return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits_pair: %s", e);
    if (!A || !B || !dA || !dB || !planesA || !planesB || M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < N)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits_pair: invalid arguments");
    if (Mg < M || Ng < N || Kg < K || Mg % 16 || Ng % 16 || Kg % 64 || ((uintptr_t)planesA & 15u) ||
        ((uintptr_t)planesB & 15u))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits_pair: plane geometry %dx%d / %dx%d does not fit", Mg, Kg, Ng,
                        Kg);
    const bool e4m3 = dd->encoding == 1;
    switch (dd->mo.nd * 2 + (e4m3 ? 1 : 0)) {
    case 7: return launch_digits_pair<3, true>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, np, planesA, planesB, Mg, Ng, Kg);
    case 6: return launch_digits_pair<3, false>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, np, planesA, planesB, Mg, Ng, Kg);
    case 9: return launch_digits_pair<4, true>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, np, planesA, planesB, Mg, Ng, Kg);
    case 8: return launch_digits_pair<4, false>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, np, planesA, planesB, Mg, Ng, Kg);
    case 11: return launch_digits_pair<5, true>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, np, planesA, planesB, Mg, Ng, Kg);
    default: return launch_digits_pair<5, false>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, np, planesA, planesB, Mg, Ng, Kg);
    }
}

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
//     sgn(r) read from the sign bit.
// Planes per modulus in this order: l, h (and s for Karatsuba); the moduli follow each other.
// Every step is one binary32 operation as in the reference (no contraction), so the digits equal
// the reference's bit for bit; they are integers of magnitude <= 32.
//
// Encoding: e4m3 (OCP, the format of the gfx950 FP8 matrix instructions; every digit is exact in
// it), converted with the hardware instruction, or int8.
//
// MI355X design: the blocked splitter of oz_tf32.hpp (one wave per 1 KB OZ_BLOCK block, coalesced
// FP64 reads, one contiguous 1 KB store per plane). The generator computes a modulus's residue and
// all its digits when the first of its planes is requested and serves the others from the element
// state.
#pragma clang fp contract(off)

#include "oz2_residue.hpp"
#include "oz_internal.hpp"

namespace {

constexpr int XM_ROUND = 0, XM_KAR = 1, XM_SPARSE = 2;

struct DigitConsts {
    SplitConsts k;
    float q[OZ2_MAXS], qinv[OZ2_MAXS];
    int xmode[OZ2_MAXS];
    unsigned char pmod[OZ2_MAXPLANES], pdig[OZ2_MAXPLANES];  // plane -> modulus, digit position
};

// The digits of residue r (d[0] = l, d[1] = h, d[2] = s).
__device__ __forceinline__ void split_residue(float r, int xm, float q, float qinv, float* d) {
    if (xm == XM_KAR) {
        const float sgn = __builtin_signbit(r) ? -1.0f : 1.0f;
        const float t = sgn * (q * 0.5f - 0.5f);
        const float h = __builtin_rintf((r + t) * qinv);
        const float l = r - h * q;
        d[0] = l;
        d[1] = h;
        d[2] = h + l;
        return;
    }
    float h = __builtin_rintf(r * qinv);
    float l = r - h * q;
    if (xm == XM_SPARSE) {
        const int li = (int)l;
        if ((li > 16 || li < -16) && (li & 1)) {
            if (li < 0) {
                l = l + q;
                h = h - 1.0f;
            } else {
                l = l - q;
                h = h + 1.0f;
            }
        }
        const int hi = (int)h;
        if ((hi > 16 || hi < -16) && (hi & 1)) h = hi < 0 ? h + q : h - q;
    }
    d[0] = l;
    d[1] = h;
    d[2] = 0.0f;
}

template <int ND, bool E4M3>
struct DigitGen {
    DigitConsts k;
    struct State {
        float dig[ND];
        float d[3];
    };
    __device__ __forceinline__ void load(State& st, double x, int32_t dl) const { make_digits<ND>(x, dl, st.dig); }
    __device__ __forceinline__ int plane(State& st, int p) const {
        const int s = k.pmod[p], j = k.pdig[p];
        if (j == 0) split_residue(residue_f<ND>(st.dig, k.k, s), k.xmode[s], k.q[s], k.qinv[s], st.d);
        const float v = j == 0 ? st.d[0] : (j == 1 ? st.d[1] : st.d[2]);
        if constexpr (E4M3)
            return __builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xFF;
        else
            return (int)v;
    }
    OZ_PLANES_FROM_PLANE
};

template <int ND, bool E4M3>
int launch_digits(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                  const DigitConsts& k, int nplanes, uint8_t* planes, int layout, int prow, int pld, long long pstride) {
    const int kblocks = pld / 64;
    const long long nblocks = (long long)(prow / 16) * kblocks;
    const unsigned grid = oz::ceil_div(nblocks, 4);
    const DigitGen<ND, E4M3> gen{k};
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

}  // namespace

extern "C" int oz2_digit_planes(const oz2_digit_dev* dd) {
    if (!dd || dd->mo.S < 1 || dd->mo.S > OZ2_MAXS) return -1;
    int n = 0;
    for (int s = 0; s < dd->mo.S; s++) n += dd->xmode[s] == XM_KAR ? 3 : 2;
    return n;
}

extern "C" int oz2_split_digits(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode,
                                const int32_t* delta, const oz2_digit_dev* dd, uint8_t* planes, int layout, int prow,
                                int pld, long long plane_stride) {
    if (int st = oz::use(dev)) return st;
    if (!dd || dd->mo.S < 1 || dd->mo.S > OZ2_MAXS || dd->mo.nd < 3 || dd->mo.nd > 5 || dd->encoding < 0 ||
        dd->encoding > 1)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits: invalid digit descriptor");
    DigitConsts k{};
    int np = 0;
    for (int s = 0; s < dd->mo.S; s++) {
        const float m = dd->mo.m[s], q = dd->q[s];
        const int xm = dd->xmode[s];
        if (!(m >= 2.0f && m <= 2401.0f) || xm < XM_ROUND || xm > XM_SPARSE || !(q >= 2.0f && q <= 64.0f))
            return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits: modulus %g (radix %g, mode %d) not supported",
                            (double)m, (double)q, xm);
        k.k.m[s] = m;
        k.k.rinv[s] = dd->mo.rinv[s];
        for (int j = 0; j < 4; j++) k.k.c[j][s] = dd->mo.c[j][s];
        k.q[s] = q;
        k.qinv[s] = dd->qinv[s];
        k.xmode[s] = xm;
        for (int j = 0; j < (xm == XM_KAR ? 3 : 2); j++, np++) {
            if (np >= OZ2_MAXPLANES) return oz::fail(dev, OZ_ERR_ARG, "oz2_split_digits: more than %d planes", OZ2_MAXPLANES);
            k.pmod[np] = (unsigned char)s;
            k.pdig[np] = (unsigned char)j;
        }
    }
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

// A6-A8: Scheme II splitting of FP64 operands into int8 residue planes.
//
// Semantics (reference f64_tf.h:141-172 split_f64, slice_tf_core.h:67-76 tf_load_f64, digits.h:80-112
// oz2_make_digits, digits.h:165-179 oz2_residue, modslice_int8.cpp:60-95). The residues must equal
// the reference's bit for bit, and the reference defines them through a sequence of binary32
// operations: round-to-nearest-even, no fused multiply-add, denormal inputs and outputs flushed to
// zero. This file is compiled with -ffp-contract=off (no implicit contraction) and
// -fgpu-flush-denormals-to-zero (the kernels run with FP32 denormals flushed, the hardware
// equivalent of that rule). The signs of zeros may differ from the reference's model (its products
// with a zero factor are +0); a zero's sign never changes a digit or residue value.
//
// Per element x with exponent delta d:
//   1. x*2^d -> triple-float (hi, mid, lo) with integer operations on the FP64 words (exact);
//   2. nd digits: digit = rint(hi); hi -= digit; between digits the triple is multiplied by 2^20
//      and renormalized with two TwoSums and a FastTwoSum (only hi is ever rounded, so A' can be a
//      neighbour of the nearest integer; the reference documents |A'-X| <= 1);
//   3. per modulus: r = MR(d0 + MR(d1)*c0 + MR(d2)*c1) (nd = 3; 4/5 digits reduce in between),
//      MR(v) = v - rint(v*rinv)*m. Every product and sum there is an exact integer below 2^24
//      except the rounded v*rinv, so writing MR as rint + fma gives the same value.
//
// MI355X design. Layouts 2/3 (the GEMM's OZ_BLOCK tiles, the production path) run the blocked
// splitter of oz_tf32.hpp: one wave per 1 KB block, one contiguous 1 KB store per plane. Layouts 0/1
// (plain row-major planes): one thread per 4 elements along the contiguous dimension of the plane,
// so every store is a 32-bit word; layout 1 is transposed through LDS. The kernels are bound by
// their VALU work (about 12 operations per element and modulus), not by HBM.
#pragma clang fp contract(off)

#include "oz2_residue.hpp"

namespace {

// Layout 0: planes[s][r][c], thread = 4 consecutive c of one row r; grid covers prow x pld.
template <int ND>
__global__ void __launch_bounds__(256) split_row_kernel(const double* __restrict__ X, int rows, int cols, int ld,
                                                        int mode, const int32_t* __restrict__ delta, SplitConsts k,
                                                        int S, uint32_t* __restrict__ planes, int prow, int pq,
                                                        long long pstride_words) {
    const long long q = (long long)blockIdx.x * 256 + threadIdx.x;  // word index within a plane
    if (q >= (long long)prow * pq) return;
    const int r = (int)(q / pq);
    const int c0 = (int)(q % pq) * 4;
    float dig[4][ND];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int c = c0 + e;
        if (r < rows && c < cols) {
            const int32_t d = mode == 0 ? delta[r] : delta[c];
            make_digits<ND>(X[(size_t)r * ld + c], d, dig[e]);
        } else {
#pragma unroll
            for (int j = 0; j < ND; j++) dig[e][j] = 0.0f;
        }
    }
    uint32_t* out = planes + q;
    for (int s = 0; s < S; s++)
        out[(long long)s * pstride_words] =
            pack4(residue<ND>(dig[0], k, s), residue<ND>(dig[1], k, s), residue<ND>(dig[2], k, s), residue<ND>(dig[3], k, s));
}

// Layout 1: planes[s][c][r] (transposed), tile of 64 columns x 64 rows per workgroup. Thread
// (cc = t%64, g = t/64) computes the 16 elements rows g*16..g*16+15 of column cc; the words go
// through LDS so that the stores are 64-byte row segments.
template <int ND>
__global__ void __launch_bounds__(256) split_tran_kernel(const double* __restrict__ X, int rows, int cols, int ld,
                                                         int mode, const int32_t* __restrict__ delta, SplitConsts k,
                                                         int S, uint32_t* __restrict__ planes, int pld_words,
                                                         long long pstride_words) {
    __shared__ uint32_t tile[64][17];  // [column][row word], padded against bank conflicts
    const int t = threadIdx.x;
    const int cc = t & 63, g = t >> 6;
    const int c = blockIdx.x * 64 + cc;  // column of X = row of the plane
    const int rbase = blockIdx.y * 64 + g * 16;
    float dig[16][ND];
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int r = rbase + e;
        if (r < rows && c < cols) {
            const int32_t d = mode == 0 ? delta[r] : delta[c];
            make_digits<ND>(X[(size_t)r * ld + c], d, dig[e]);
        } else {
#pragma unroll
            for (int j = 0; j < ND; j++) dig[e][j] = 0.0f;
        }
    }
    // store phase mapping: thread -> plane row blockIdx.x*64 + t/4, words (t%4)*4 .. +4
    const int orow = blockIdx.x * 64 + (t >> 2);
    const int ow = blockIdx.y * 16 + (t & 3) * 4;
    for (int s = 0; s < S; s++) {
#pragma unroll
        for (int w = 0; w < 4; w++)
            tile[cc][g * 4 + w] = pack4(residue<ND>(dig[4 * w], k, s), residue<ND>(dig[4 * w + 1], k, s),
                                        residue<ND>(dig[4 * w + 2], k, s), residue<ND>(dig[4 * w + 3], k, s));
        __syncthreads();
        uint32_t* out = planes + (long long)s * pstride_words + (long long)orow * pld_words + ow;
        const uint4 v = make_uint4(tile[t >> 2][(t & 3) * 4], tile[t >> 2][(t & 3) * 4 + 1], tile[t >> 2][(t & 3) * 4 + 2],
                                   tile[t >> 2][(t & 3) * 4 + 3]);
        *reinterpret_cast<uint4*>(out) = v;
        __syncthreads();
    }
}

// Layouts 2/3 (OZ_BLOCK tiles): split_block_kernel of oz_tf32.hpp with this generator: the state of
// an element is A' in balanced base-256 bytes and its residue modulo the even modulus, if the set
// has one (from the reference's sequence on the digits); plane s is the residue modulo m_s. The
// generator runs the planes itself: the even modulus, the odd moduli below 17 (byte dot products and
// one FP32 reduction, oz2_residue.hpp), then the odd moduli from 17 up four at a time, with their dot
// products on the matrix cores and the integer remainder step on the VALU.
//
// Matrix-core dot products for nd = 3 (8 balanced bytes per element; v_mfma_i32_16x16x64_i8, operand
// layout as in oz_gemm.hip: lane l holds row l%16 of the first operand and column l%16 of the second,
// K bytes 16(l/16)..+15 of each; output register r of lane l is row 4(l/16) + r, column l%16). The
// second operand of lane l is the bytes of two of its own elements, e in its low 8 bytes and e' in its
// high 8. Row i = 4g + r of the first operand holds, in K chunk g only, the byte weights w_p of modulus
// p = r%2 of a pair of moduli (symmetric residues of 256^j) over the half h = r/2 of the chunk, and zero
// elsewhere. So D[4g + r][j] = dinit_p + w_p . (half h of the second operand of lane 16g + j), and
// output register r of lane l is the dot product of lane l's element (e for r < 2, e' above) with
// modulus p: every lane gets the four sums of its own two elements and two moduli, 8 MFMAs per pair of
// moduli for its 16 elements in place of 2 v_dot4 per element and modulus. The sums are exact
// integers, the same as the v_dot4 chain's. For nd = 4 and 5 (12 and 16 bytes) the v_dot4 chain stays.
typedef int v4i_t __attribute__((ext_vector_type(4)));

template <int ND>
struct ResidueGen {
    static constexpr bool kDrivesPlanes = true;
    static constexpr int W = balanced_words<ND>();
    SplitConsts k;
    struct State {
        uint32_t a[W];
        int even;
    };
    __device__ __forceinline__ void load(State& st, double x, int32_t d) const {
        float dig[ND];
        make_digits<ND>(x, d, dig);
        balanced_bytes<ND>(dig, st.a);
        st.even = k.even >= 0 ? residue<ND>(dig, k, k.even) : 0;
    }
    // x = r + (m-1)/2 in the low byte: adding 128 - (m-1)/2 keeps every byte in [1, 255] (no carry
    // into the next one), and xor 0x80 then subtracts 128 from each (two's complement bytes)
    template <class EMIT>
    __device__ __forceinline__ void emit_odd(EMIT& emit, int s, const uint32_t* pk) const {
        const uint32_t badd = k.badd[s];
        uint32_t w[4];
#pragma unroll
        for (int c = 0; c < 4; c++) w[c] = (pk[c] + badd) ^ 0x80808080u;
        emit(s, w);
    }
    template <class EMIT>
    __device__ __forceinline__ void run(State* st, EMIT&& emit) const {
        uint32_t w[4];
        if (k.even >= 0) {
#pragma unroll
            for (int c = 0; c < 4; c++) w[c] = pack4(st[4 * c].even, st[4 * c + 1].even, st[4 * c + 2].even, st[4 * c + 3].even);
            emit(k.even, w);
        }
        for (int i = 0; i < k.nsmall; i++) {
            const int s = k.small[i];
            int v[16];
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = (int)residue_odd<W>(st[e].a, k.w[s], k.m[s], k.rinv[s]);
#pragma unroll
            for (int c = 0; c < 4; c++) w[c] = pack4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
            emit(s, w);
        }
        if constexpr (W == 2) {
            const int lane = threadIdx.x & 63, r = lane & 3;
            const bool on = (lane >> 4) == ((lane & 15) >> 2);
            for (int g = 0; g < k.npair; g++) {
                const int s0 = __builtin_amdgcn_readfirstlane(k.pair[g][0]);
                const int s1 = __builtin_amdgcn_readfirstlane(k.pair[g][1]);
                const uint32_t w00 = __builtin_amdgcn_readfirstlane(k.w[s0][0]), w01 = __builtin_amdgcn_readfirstlane(k.w[s0][1]);
                const uint32_t w10 = __builtin_amdgcn_readfirstlane(k.w[s1][0]), w11 = __builtin_amdgcn_readfirstlane(k.w[s1][1]);
                const uint32_t lo = (r & 1) ? w10 : w00, hi = (r & 1) ? w11 : w01;
                const bool h = (r >> 1) != 0;
                const v4i_t wa = {on && !h ? (int)lo : 0, on && !h ? (int)hi : 0, on && h ? (int)lo : 0, on && h ? (int)hi : 0};
                const int d0 = k.dinit[s0], d1 = k.dinit[s1];
                const v4i_t c0 = {d0, d1, d0, d1};
                const uint32_t mg0 = k.magic[s0], mg1 = k.magic[s1];
                const int mn0 = k.mneg[s0], mn1 = k.mneg[s1];
                uint32_t pk0[4], pk1[4];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    int x0[4], x1[4];
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const State& ea = st[4 * c + 2 * t];
                        const State& eb = st[4 * c + 2 * t + 1];
                        const v4i_t b = {(int)ea.a[0], (int)ea.a[1], (int)eb.a[0], (int)eb.a[1]};
                        const v4i_t u = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, b, c0, 0, 0, 0);
                        x0[2 * t] = reduce_odd_int<W>(u[0], mg0, mn0);
                        x1[2 * t] = reduce_odd_int<W>(u[1], mg1, mn1);
                        x0[2 * t + 1] = reduce_odd_int<W>(u[2], mg0, mn0);
                        x1[2 * t + 1] = reduce_odd_int<W>(u[3], mg1, mn1);
                    }
                    pk0[c] = pack4(x0[0], x0[1], x0[2], x0[3]);
                    pk1[c] = pack4(x1[0], x1[1], x1[2], x1[3]);
                }
                emit_odd(emit, s0, pk0);
                if (s1 != s0) emit_odd(emit, s1, pk1);
            }
        } else {
            for (int g = 0; g < k.npair; g++)
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const int s = k.pair[g][p];
                    if (p == 1 && s == k.pair[g][0]) break;
                    uint32_t a[16][W];
#pragma unroll
                    for (int e = 0; e < 16; e++)
#pragma unroll
                        for (int i = 0; i < W; i++) a[e][i] = st[e].a[i];
                    int v[16];
                    residues_odd_int<W>(a, k.w[s], k.dinit[s], k.magic[s], k.mneg[s], v);
                    uint32_t pk[4];
#pragma unroll
                    for (int c = 0; c < 4; c++) pk[c] = pack4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
                    emit_odd(emit, s, pk);
                }
        }
    }
};

// The reference's sequence for every modulus (sets with more than one even modulus, which a
// pairwise coprime plan never has): the state is the nd digits.
template <int ND>
struct ResidueChainGen {
    SplitConsts k;
    struct State {
        float dig[ND];
    };
    __device__ __forceinline__ void load(State& st, double x, int32_t d) const { make_digits<ND>(x, d, st.dig); }
    __device__ __forceinline__ int plane(State& st, int s) const { return residue<ND>(st.dig, k, s); }
    OZ_PLANES_FROM_PLANE
};

template <int ND>
__global__ void digits_kernel(const double* __restrict__ X, int rows, int cols, int ld, int mode,
                              const int32_t* __restrict__ delta, float* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i % cols);
    float dig[ND];
    make_digits<ND>(X[(size_t)r * ld + c], mode == 0 ? delta[r] : delta[c], dig);
#pragma unroll
    for (int j = 0; j < ND; j++) out[i * ND + j] = dig[j];
}

int check_moduli(oz_dev* dev, const oz2_moduli_dev* mo) {
    if (!mo || mo->S < 1 || mo->S > OZ2_MAXS || mo->nd < 3 || mo->nd > 5)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_int8: invalid moduli descriptor");
    for (int s = 0; s < mo->S; s++)
        if (!(mo->m[s] >= 2.0f && mo->m[s] <= 255.0f))
            return oz::fail(dev, OZ_ERR_ARG, "oz2_split_int8: modulus %g outside the INT8 range", (double)mo->m[s]);
    return OZ_OK;
}

template <class GEN>
int launch_blocked(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                   const GEN& gen, int S, int8_t* planes, int layout, int pld, long long nblocks, long long pstride) {
    const int kblocks = pld / 64;
    const unsigned grid = oz::ceil_div(nblocks, 4);
    if (layout == 2)
        hipLaunchKernelGGL((split_block_kernel<GEN, false>), dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld,
                           mode, delta, gen, S, reinterpret_cast<uint4*>(planes), kblocks, nblocks, pstride / 16);
    else
        hipLaunchKernelGGL((split_block_kernel<GEN, true>), dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld,
                           mode, delta, gen, S, reinterpret_cast<uint4*>(planes), kblocks, nblocks, pstride / 16);
    return oz::launch_check(dev, "split_block_kernel");
}

template <int ND>
int launch_split(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                 const SplitConsts& k, int S, int8_t* planes, int layout, int prow, int pld, long long pstride,
                 bool one_even) {
    if (layout == 0) {
        const int pq = pld / 4;
        const long long words = (long long)prow * pq;
        hipLaunchKernelGGL(split_row_kernel<ND>, dim3(oz::ceil_div(words, 256)), dim3(256), 0, dev->stream, X, rows,
                           cols, ld, mode, delta, k, S, reinterpret_cast<uint32_t*>(planes), prow, pq, pstride / 4);
        return oz::launch_check(dev, "split_row_kernel");
    }
    if (layout >= 2) {
        const long long nblocks = (long long)(prow / 16) * (pld / 64);
        if (one_even)
            return launch_blocked(dev, X, rows, cols, ld, mode, delta, ResidueGen<ND>{k}, S, planes, layout, pld,
                                  nblocks, pstride);
        return launch_blocked(dev, X, rows, cols, ld, mode, delta, ResidueChainGen<ND>{k}, S, planes, layout, pld,
                              nblocks, pstride);
    }
    // transposed: plane rows = columns of X (prow of them, multiple of 64); plane bytes = rows of X
    hipLaunchKernelGGL(split_tran_kernel<ND>, dim3(prow / 64, pld / 64), dim3(256), 0, dev->stream, X, rows, cols, ld,
                       mode, delta, k, S, reinterpret_cast<uint32_t*>(planes), pld / 4, pstride / 4);
    return oz::launch_check(dev, "split_tran_kernel");
}

// Kernel constants of a moduli descriptor (oz2_residue.hpp); *evens counts the even moduli.
SplitConsts split_consts(const oz2_moduli_dev* mo, int* evens) {
    SplitConsts k{};
    k.even = -1;
    *evens = 0;
    for (int s = 0; s < mo->S; s++) {
        k.m[s] = mo->m[s];
        k.rinv[s] = mo->rinv[s];
        for (int j = 0; j < 4; j++) k.c[j][s] = mo->c[j][s];
        // symmetric residues of 256^j modulo m, four to a word (signed bytes)
        const int m = (int)mo->m[s];
        if (m % 2 == 1 && m >= 17) {
            const int U = mo->nd == 3 ? 18 : 19, sh = 24 - U, h = (m - 1) / 2;
            const long long half = 1ll << (U - 1);
            k.dinit[s] = (int)((half + m - 1) / m * m + h);
            k.magic[s] = (uint32_t)(((1ull << (32 - sh)) + m - 1) / m);
            k.badd[s] = (uint32_t)(128 - h) * 0x01010101u;
            k.mneg[s] = (1 << 24) - m;
        }
        if (m % 2 == 0) {
            k.even = s;
            (*evens)++;
        } else if (m < 17) {
            k.small[k.nsmall++] = s;
        } else if (k.npair && k.pair[k.npair - 1][1] < 0) {
            k.pair[k.npair - 1][1] = s;
        } else {
            k.pair[k.npair][0] = s;
            k.pair[k.npair++][1] = -1;
        }
        int p = 1;  // 256^j mod m
        for (int i = 0; i < 4; i++) {
            uint32_t word = 0;
            for (int j = 0; j < 4; j++) {
                const int sym = p > m / 2 ? p - m : p;
                word |= (uint32_t)(sym & 0xFF) << (8 * j);
                p = p * 256 % m;
            }
            k.w[s][i] = word;
        }
    }
    if (k.npair && k.pair[k.npair - 1][1] < 0)  // a last single modulus is paired with itself (stored once)
        k.pair[k.npair - 1][1] = k.pair[k.npair - 1][0];
    return k;
}

template <int ND>
int launch_pair(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA, const double* B, int N,
                int ldb, const int32_t* dB, const SplitConsts& k, int S, int8_t* pA, int8_t* pB, int Mg, int Ng,
                int Kg, bool one_even) {
    const int kblocks = Kg / 64;
    const long long nbA = (long long)(Mg / 16) * kblocks, nbB = (long long)(Ng / 16) * kblocks;
    const long long sA = (long long)Mg * Kg / 16, sB = (long long)Ng * Kg / 16;
    const long long grid = (nbA + 3) / 4 + (nbB + 3) / 4;
    if (grid > 0x7FFFFFFFll) return oz::fail(dev, OZ_ERR_ARG, "oz2_split_pair_int8: grid too large");
    auto* qA = reinterpret_cast<uint4*>(pA);
    auto* qB = reinterpret_cast<uint4*>(pB);
    if (one_even)
        hipLaunchKernelGGL((split_pair_kernel<ResidueGen<ND>>), dim3((unsigned)grid), dim3(256), 0, dev->stream, A, M,
                           K, lda, dA, qA, nbA, sA, B, N, ldb, dB, qB, nbB, sB, kblocks, ResidueGen<ND>{k}, S);
    else
        hipLaunchKernelGGL((split_pair_kernel<ResidueChainGen<ND>>), dim3((unsigned)grid), dim3(256), 0, dev->stream,
                           A, M, K, lda, dA, qA, nbA, sA, B, N, ldb, dB, qB, nbB, sB, kblocks, ResidueChainGen<ND>{k},
                           S);
    return oz::launch_check(dev, "split_pair_kernel");
}

}  // namespace

extern "C" int oz2_split_int8(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode,
                              const int32_t* delta, const oz2_moduli_dev* mo, int8_t* planes, int layout, int prow,
                              int pld, long long plane_stride) {
    if (int st = oz::use(dev)) return st;
    if (int st = check_moduli(dev, mo)) return st;
    if (!X || !delta || !planes || rows <= 0 || cols <= 0 || ld < cols || (mode != 0 && mode != 1) || layout < 0 ||
        layout > 3)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_int8: invalid arguments");
    // The plane must hold the operand: layouts 0/2 rows x cols, layouts 1/3 cols x rows.
    const bool tran = layout == 1 || layout == 3;
    const int need_rows = tran ? cols : rows, need_ld = tran ? rows : cols;
    const bool blocked = layout >= 2;
    if (prow < need_rows || pld < need_ld || pld % 64 != 0 || (layout == 1 && prow % 64 != 0) ||
        (blocked && (prow % 16 != 0 || plane_stride % 1024 != 0)) || plane_stride < (long long)prow * pld ||
        plane_stride % 16 != 0 || ((uintptr_t)planes & 15u))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_int8: plane geometry %dx%d (stride %lld) does not fit", prow, pld,
                        plane_stride);
    int evens = 0;
    const SplitConsts k = split_consts(mo, &evens);
    switch (mo->nd) {
    case 3:
        return launch_split<3>(dev, X, rows, cols, ld, mode, delta, k, mo->S, planes, layout, prow, pld, plane_stride,
                               evens <= 1);
    case 4:
        return launch_split<4>(dev, X, rows, cols, ld, mode, delta, k, mo->S, planes, layout, prow, pld, plane_stride,
                               evens <= 1);
    default:
        return launch_split<5>(dev, X, rows, cols, ld, mode, delta, k, mo->S, planes, layout, prow, pld, plane_stride,
                               evens <= 1);
    }
}

extern "C" int oz2_digits_f32(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode,
                              const int32_t* delta, int nd, float* digits) {
    if (int st = oz::use(dev)) return st;
    if (!X || !delta || !digits || rows <= 0 || cols <= 0 || ld < cols || nd < 3 || nd > 5 || (mode != 0 && mode != 1))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_digits_f32: invalid arguments");
    const unsigned grid = oz::ceil_div((long long)rows * cols, 256);
    if (nd == 3)
        hipLaunchKernelGGL(digits_kernel<3>, dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld, mode, delta, digits);
    else if (nd == 4)
        hipLaunchKernelGGL(digits_kernel<4>, dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld, mode, delta, digits);
    else
        hipLaunchKernelGGL(digits_kernel<5>, dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld, mode, delta, digits);
    return oz::launch_check(dev, "digits_kernel");
}

extern "C" int oz2_split_pair_int8(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA,
                                   const double* B, int N, int ldb, const int32_t* dB, const oz2_moduli_dev* mo,
                                   int8_t* planesA, int8_t* planesB, int Mg, int Ng, int Kg) {
    if (int st = oz::use(dev)) return st;
    if (int st = check_moduli(dev, mo)) return st;
    if (!A || !B || !dA || !dB || !planesA || !planesB || M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < N)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_pair_int8: invalid arguments");
    if (Mg < M || Ng < N || Kg < K || Mg % 16 || Ng % 16 || Kg % 64 || ((uintptr_t)planesA & 15u) ||
        ((uintptr_t)planesB & 15u))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_split_pair_int8: plane geometry %dx%d / %dx%d does not fit", Mg, Kg, Ng,
                        Kg);
    int evens = 0;
    const SplitConsts k = split_consts(mo, &evens);
    switch (mo->nd) {
    case 3: return launch_pair<3>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, mo->S, planesA, planesB, Mg, Ng, Kg, evens <= 1);
    case 4: return launch_pair<4>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, mo->S, planesA, planesB, Mg, Ng, Kg, evens <= 1);
    default: return launch_pair<5>(dev, A, M, K, lda, dA, B, N, ldb, dB, k, mo->S, planesA, planesB, Mg, Ng, Kg, evens <= 1);
    }
}

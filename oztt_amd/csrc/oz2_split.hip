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
// MI355X design: one thread per 4 elements along the contiguous dimension of the output plane, so
// every plane store is a 32-bit word and a wave writes 256 contiguous bytes. The B operand (layout
// 1) is transposed through LDS so that its planes are K-contiguous for the MFMA GEMM. The kernel
// is bound by its VALU work (about 12 operations per element and modulus), not by HBM.
#include "oz_internal.hpp"

#pragma clang fp contract(off)

namespace {

struct SplitConsts {
    float m[OZ2_MAXS];
    float rinv[OZ2_MAXS];
    float c[4][OZ2_MAXS];
};

// Step 1 (split_f64 + tf_load_f64).
__device__ __forceinline__ void load_triple(double x, int32_t d, float& hi, float& mid, float& lo) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(x);
    const uint32_t w1 = (uint32_t)(u >> 32), w0 = (uint32_t)u;
    const uint32_t sgn = w1 & 0x80000000u;
    const int32_t E = (int32_t)((w1 >> 20) & 0x7FFu);
    if (E == 0) {  // zero and subnormals
        hi = 0.0f;
        mid = 0.0f;
        lo = 0.0f;
        return;
    }
    uint32_t a = 0x400000u | ((w1 & 0x000FFFFFu) << 2) | (w0 >> 30);
    const uint32_t rem = w0 & 0x3FFFFFFFu;
    int32_t r = (int32_t)rem;
    if (rem >= 0x20000000u) {
        a += 1u;
        r = (int32_t)rem - 0x40000000;
    }
    const int32_t b = r >> 7;
    const uint32_t c = (uint32_t)r & 0x7Fu;
    const int32_t elsb = E - 1075 + d;
    const bool carry = (a == 0x800000u);
    const int32_t eh = carry ? elsb + 180 : elsb + 179;
    const uint32_t mh = carry ? 0u : ((a << 1) & 0x7FFFFFu);
    const int32_t es = elsb + 134;
    const uint32_t hb = (eh > 0 && eh < 255) ? (sgn | ((uint32_t)eh << 23) | mh) : 0u;
    const uint32_t sb = (es > 0 && es < 255) ? (sgn | ((uint32_t)es << 23)) : 0u;
    const uint32_t braw = 0x4B000000u | (((uint32_t)(b + 0x400000)) & 0x7FFFFFu);
    const uint32_t craw = 0x4B000000u | c;
    const float s = __uint_as_float(sb);
    hi = __uint_as_float(hb);
    mid = (__uint_as_float(braw) - 12582912.0f) * s;
    lo = ((__uint_as_float(craw) - 8388608.0f) * s) * 0.0078125f;
}

__device__ __forceinline__ void two_sum(float x, float y, float& s, float& e) {
    s = x + y;
    float bb = s - x;
    float aa = s - bb;
    aa = x - aa;
    bb = y - bb;
    e = aa + bb;
}

// Step 2: nd digits, top first.
template <int ND>
__device__ __forceinline__ void make_digits(double x, int32_t d, float* dig) {
    float hi, mid, lo;
    load_triple(x, d, hi, mid, lo);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        if (i > 0) {
            hi = hi * 1048576.0f;
            mid = mid * 1048576.0f;
            lo = lo * 1048576.0f;
            float s3, e4, s5, e6;
            two_sum(mid, lo, s3, e4);
            two_sum(hi, s3, s5, e6);
            hi = s5;
            mid = e6 + e4;  // FastTwoSum(e6, e4) -> (mid, lo)
            lo = e4 - (mid - e6);
        }
        const float t = __builtin_rintf(hi);
        hi = hi - t;
        dig[i] = t;
    }
}

__device__ __forceinline__ float mod_round(float v, float m, float rinv) {
    const float q = __builtin_rintf(v * rinv);
    return __builtin_fmaf(-q, m, v);  // exact: q*m and v - q*m are integers below 2^24
}

// Step 3 for one modulus.
template <int ND>
__device__ __forceinline__ int residue(const float* dig, const SplitConsts& k, int s) {
    const float m = k.m[s], ri = k.rinv[s];
    float acc = dig[ND - 1];
    acc = __builtin_fmaf(mod_round(dig[ND - 2], m, ri), k.c[0][s], acc);
    acc = __builtin_fmaf(mod_round(dig[ND - 3], m, ri), k.c[1][s], acc);
    if (ND >= 4) {
        acc = mod_round(acc, m, ri);
        if (ND >= 5) {
            acc = __builtin_fmaf(mod_round(dig[0], m, ri), k.c[3][s], acc);
            acc = mod_round(acc, m, ri);
        }
        acc = __builtin_fmaf(mod_round(dig[ND - 4], m, ri), k.c[2][s], acc);
    }
    return (int)mod_round(acc, m, ri);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)(d & 0xFF) << 24);
}

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

// Layouts 2/3 (OZ_BLOCK tiles): one wave per 1 KB block of 16 plane rows x 64 plane columns; the
// wave writes each plane's block with one contiguous 1 KB store (16 bytes per lane, lane l -> block
// bytes 16l..16l+15).
//   Layout 3 (TRAN, plane row = column of X): lane l computes plane row l/4, plane columns
//   16*(l%4)..+15 (= 16 consecutive rows of X in one column; a load instruction reads 4 runs of 16
//   consecutive doubles) and packs its 16 residues into its own stored chunk.
//   Layout 2: lane l computes plane column l of the 16 rows (each load instruction reads one
//   contiguous 512-byte row segment of X); the residues of a plane are transposed through a 1 KB
//   LDS image of the block (byte writes, then one 16-byte read per lane). The image is private to
//   the wave, whose LDS operations execute in order, so no barrier is needed.
__device__ __forceinline__ int block_swizzle(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

template <int ND, bool TRAN>
__global__ void __launch_bounds__(256) split_block_kernel(const double* __restrict__ X, int rows, int cols, int ld,
                                                          int mode, const int32_t* __restrict__ delta, SplitConsts k,
                                                          int S, uint4* __restrict__ planes, int kblocks,
                                                          long long nblocks, long long pstride_chunks) {
    const long long blk = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);  // block index within a plane
    if (blk >= nblocks) return;
    const int lane = threadIdx.x & 63;
    const int br = (int)(blk / kblocks), bk = (int)(blk % kblocks);
    float dig[16][ND];
    if constexpr (TRAN) {
        const int pr = br * 16 + (lane >> 2);       // plane row = column of X
        const int pc0 = bk * 64 + 16 * (lane & 3);  // first of this lane's 16 plane columns = rows of X
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int xr = pc0 + e, xc = pr;
            if (xr < rows && xc < cols) {
                const int32_t d = mode == 0 ? delta[xr] : delta[xc];
                make_digits<ND>(X[(size_t)xr * ld + xc], d, dig[e]);
            } else {
#pragma unroll
                for (int j = 0; j < ND; j++) dig[e][j] = 0.0f;
            }
        }
        const int rr = lane >> 2;
        uint4* out = planes + blk * 64 + rr * 4 + ((lane & 3) ^ block_swizzle(rr));
        for (int s = 0; s < S; s++) {
            uint4 v;
            v.x = pack4(residue<ND>(dig[0], k, s), residue<ND>(dig[1], k, s), residue<ND>(dig[2], k, s), residue<ND>(dig[3], k, s));
            v.y = pack4(residue<ND>(dig[4], k, s), residue<ND>(dig[5], k, s), residue<ND>(dig[6], k, s), residue<ND>(dig[7], k, s));
            v.z = pack4(residue<ND>(dig[8], k, s), residue<ND>(dig[9], k, s), residue<ND>(dig[10], k, s), residue<ND>(dig[11], k, s));
            v.w = pack4(residue<ND>(dig[12], k, s), residue<ND>(dig[13], k, s), residue<ND>(dig[14], k, s), residue<ND>(dig[15], k, s));
            out[(long long)s * pstride_chunks] = v;
        }
    } else {
        __shared__ __attribute__((aligned(16))) uint8_t image[4][1024];
        uint8_t* img = image[threadIdx.x >> 6];
        const int xc = bk * 64 + lane;  // plane column = column of X
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int xr = br * 16 + e;
            if (xr < rows && xc < cols) {
                const int32_t d = mode == 0 ? delta[xr] : delta[xc];
                make_digits<ND>(X[(size_t)xr * ld + xc], d, dig[e]);
            } else {
#pragma unroll
                for (int j = 0; j < ND; j++) dig[e][j] = 0.0f;
            }
        }
        // byte of (row e, column lane) inside the block image
        const int colpart = 16 * (lane >> 4), colbyte = lane & 15;
        uint4* out = planes + blk * 64 + lane;
        for (int s = 0; s < S; s++) {
#pragma unroll
            for (int e = 0; e < 16; e++)
                img[64 * e + (colpart ^ (16 * block_swizzle(e))) + colbyte] = (uint8_t)residue<ND>(dig[e], k, s);
            out[(long long)s * pstride_chunks] = *reinterpret_cast<const uint4*>(img + 16 * lane);
        }
    }
}

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

template <int ND>
int launch_split(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                 const SplitConsts& k, int S, int8_t* planes, int layout, int prow, int pld, long long pstride) {
    if (layout == 0) {
        const int pq = pld / 4;
        const long long words = (long long)prow * pq;
        hipLaunchKernelGGL(split_row_kernel<ND>, dim3(oz::ceil_div(words, 256)), dim3(256), 0, dev->stream, X, rows,
                           cols, ld, mode, delta, k, S, reinterpret_cast<uint32_t*>(planes), prow, pq, pstride / 4);
        return oz::launch_check(dev, "split_row_kernel");
    }
    if (layout >= 2) {
        const int kblocks = pld / 64;
        const long long nblocks = (long long)(prow / 16) * kblocks;
        const unsigned grid = oz::ceil_div(nblocks, 4);
        if (layout == 2)
            hipLaunchKernelGGL((split_block_kernel<ND, false>), dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld,
                               mode, delta, k, S, reinterpret_cast<uint4*>(planes), kblocks, nblocks, pstride / 16);
        else
            hipLaunchKernelGGL((split_block_kernel<ND, true>), dim3(grid), dim3(256), 0, dev->stream, X, rows, cols, ld,
                               mode, delta, k, S, reinterpret_cast<uint4*>(planes), kblocks, nblocks, pstride / 16);
        return oz::launch_check(dev, "split_block_kernel");
    }
    // transposed: plane rows = columns of X (prow of them, multiple of 64); plane bytes = rows of X
    hipLaunchKernelGGL(split_tran_kernel<ND>, dim3(prow / 64, pld / 64), dim3(256), 0, dev->stream, X, rows, cols, ld,
                       mode, delta, k, S, reinterpret_cast<uint32_t*>(planes), pld / 4, pstride / 4);
    return oz::launch_check(dev, "split_tran_kernel");
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
    SplitConsts k{};
    for (int s = 0; s < mo->S; s++) {
        k.m[s] = mo->m[s];
        k.rinv[s] = mo->rinv[s];
        for (int j = 0; j < 4; j++) k.c[j][s] = mo->c[j][s];
    }
    switch (mo->nd) {
    case 3: return launch_split<3>(dev, X, rows, cols, ld, mode, delta, k, mo->S, planes, layout, prow, pld, plane_stride);
    case 4: return launch_split<4>(dev, X, rows, cols, ld, mode, delta, k, mo->S, planes, layout, prow, pld, plane_stride);
    default: return launch_split<5>(dev, X, rows, cols, ld, mode, delta, k, mo->S, planes, layout, prow, pld, plane_stride);
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

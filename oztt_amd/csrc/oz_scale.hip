// A5: normalization exponents of the rows of A and the columns of B.
//
// Semantics (reference scale_f64_reader.cpp:106-197 with scale_bits.h:22-62 and expdelta.cpp:44-90):
// the largest |x| of a row/column, compared on FP64 bit patterns, is converted to BF16 (rounded
// down, up, or up with an extra step at an exact power of two), e = ceil(log2(bf16)) (0 for an
// all-zero row/column), delta = shift - e; maxima that are Inf/NaN, nonzero below 2^-126, or
// above the largest BF16 raise flag bits 4, 2, 1 and use e = 0.
//
// MI355X design. Each of the three BF16 roundings is a monotone map of |x|, so the BF16 of the
// maximum equals the maximum of the per-element BF16 values. The kernels therefore reduce a 32-bit
// key per element (the BF16 code; 1 for a nonzero value below 2^-126, 0 for zero, 0xFFFFFFFF for
// Inf/NaN) with plain 32-bit max operations: a row is one workgroup (coalesced along K), columns
// are 64-wide strips split over row chunks and combined with atomicMax into the output array
// itself, and a final pass turns keys into deltas and flags. HBM traffic is one read of X.
#include "oz_internal.hpp"

namespace {

constexpr uint32_t KEY_NAN = 0xFFFFFFFFu;  // Inf/NaN: dominates every other key
constexpr uint32_t KEY_TINY = 1u;          // nonzero maximum below 2^-126 (loses to any normal value)

// Key of |x| for the rounding mode (the BF16 code for normal in-range magnitudes; 0x7F80 above range).
template <int CEIL>
__device__ __forceinline__ uint32_t bf16_key(double x) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(x);
    const uint32_t h = (uint32_t)(u >> 32) & 0x7FFFFFFFu, l = (uint32_t)u;
    const int32_t E = (int32_t)(h >> 20);
    if (E == 0x7FF) return KEY_NAN;
    const int32_t e8 = E - 896;
    if (e8 <= 0) return (h | l) ? KEY_TINY : 0u;
    if (e8 >= 255) return 0x7F80u;
    uint32_t v = ((uint32_t)e8 << 7) | ((h >> 13) & 0x7Fu);
    const bool dropped = (h & 0x1FFFu) || l;
    if (CEIL == 1 && dropped) v += 1u;
    if (CEIL == 2 && (dropped || !(v & 0x7Fu))) v += 1u;
    return v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
    return v;
}

// One workgroup (256 threads) per row: key of the row maximum into out[row].
template <int CEIL>
__global__ void __launch_bounds__(256) row_key_kernel(const double* __restrict__ X, int cols, int ld,
                                                      uint32_t* __restrict__ out) {
    const double* row = X + (size_t)blockIdx.x * ld;
    uint32_t k = 0;
    for (int c = threadIdx.x; c < cols; c += 256) k = max(k, bf16_key<CEIL>(row[c]));
    k = wave_max(k);
    __shared__ uint32_t part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = max(max(part[0], part[1]), max(part[2], part[3]));
}

// Column strips: workgroup = 64 columns x 4 row phases over a chunk of `chunk` rows; the strip
// maximum is combined into out[col] (zeroed beforehand) with atomicMax.
template <int CEIL>
__global__ void __launch_bounds__(256) col_key_kernel(const double* __restrict__ X, int rows, int cols, int ld,
                                                      int chunk, uint32_t* __restrict__ out) {
    const int c = blockIdx.x * 64 + (threadIdx.x & 63);
    const int r0 = blockIdx.y * chunk;
    const int r1 = min(rows, r0 + chunk);
    uint32_t k = 0;
    if (c < cols)
        for (int r = r0 + (threadIdx.x >> 6); r < r1; r += 4) k = max(k, bf16_key<CEIL>(X[(size_t)r * ld + c]));
    __shared__ uint32_t part[256];
    part[threadIdx.x] = k;
    __syncthreads();
    if (threadIdx.x < 64 && c < cols) {
        const uint32_t m = max(max(part[threadIdx.x], part[threadIdx.x + 64]), max(part[threadIdx.x + 128], part[threadIdx.x + 192]));
        if (m) atomicMax(&out[c], m);
    }
}

// Keys -> delta = shift - ceil(log2(bf16)), flags (expdelta.cpp:73-80 and scale_bits.h:56-62).
__global__ void key_to_delta_kernel(uint32_t* __restrict__ io, int n, int shift, uint32_t* __restrict__ flags) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t bad = 0;
    if (i < n) {
        const uint32_t key = io[i];
        int32_t e = 0;
        if (key == KEY_NAN)
            bad = 4u;
        else if (key == KEY_TINY)
            bad = 2u;
        else if (key >= 0x7F80u)
            bad = 1u;
        else if (key != 0u) {
            const uint32_t E = (key >> 7) & 0xFFu, m = key & 0x7Fu;
            e = (int32_t)E - 127 + (m ? 1 : 0);
        }
        io[i] = (uint32_t)(shift - e);
    }
    const unsigned long long any = __ballot(bad != 0);
    if (any) {
        // OR the flags of the wave once (lanes with bad != 0 only)
        uint32_t v = bad;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v |= (uint32_t)__shfl_xor((int)v, off, 64);
        if ((threadIdx.x & 63) == 0) atomicOr(flags, v);
    }
}

__global__ void zero_u32_kernel(uint32_t* __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

template <int CEIL>
int launch_keys(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, uint32_t* keys) {
    if (mode == 0) {
        hipLaunchKernelGGL(row_key_kernel<CEIL>, dim3(rows), dim3(256), 0, dev->stream, X, cols, ld, keys);
        return oz::launch_check(dev, "row_key_kernel");
    }
    hipLaunchKernelGGL(zero_u32_kernel, dim3(oz::ceil_div(cols, 256)), dim3(256), 0, dev->stream, keys, cols);
    if (int st = oz::launch_check(dev, "zero_u32_kernel")) return st;
    // enough row chunks to give every CU several workgroups
    const int strips = (int)oz::ceil_div(cols, 64);
    int nchunk = std::max(1, std::min((rows + 63) / 64, 2048 / std::max(1, strips)));
    const int chunk = (rows + nchunk - 1) / nchunk;
    nchunk = (rows + chunk - 1) / chunk;
    hipLaunchKernelGGL(col_key_kernel<CEIL>, dim3(strips, nchunk), dim3(256), 0, dev->stream, X, rows, cols, ld,
                       chunk, keys);
    return oz::launch_check(dev, "col_key_kernel");
}

}  // namespace

extern "C" int oz_scale_f64(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, int ceil_mode,
                            int shift, int32_t* delta, uint32_t* flags) {
    if (int st = oz::use(dev)) return st;
    if (!X || !delta || !flags || rows <= 0 || cols <= 0 || ld < cols || (mode != 0 && mode != 1) || ceil_mode < 0 ||
        ceil_mode > 2)
        return oz::fail(dev, OZ_ERR_ARG, "oz_scale_f64: invalid arguments (rows=%d cols=%d ld=%d mode=%d ceil=%d)", rows,
                        cols, ld, mode, ceil_mode);
    uint32_t* keys = reinterpret_cast<uint32_t*>(delta);
    int st = ceil_mode == 0   ? launch_keys<0>(dev, X, rows, cols, ld, mode, keys)
             : ceil_mode == 1 ? launch_keys<1>(dev, X, rows, cols, ld, mode, keys)
                              : launch_keys<2>(dev, X, rows, cols, ld, mode, keys);
    if (st) return st;
    const int n = mode == 0 ? rows : cols;
    hipLaunchKernelGGL(key_to_delta_kernel, dim3(oz::ceil_div(n, 256)), dim3(256), 0, dev->stream, keys, n, shift, flags);
    return oz::launch_check(dev, "key_to_delta_kernel");
}

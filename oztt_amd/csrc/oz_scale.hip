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
// Branch-free: the in-range code is computed for every input, then the special cases replace it in
// increasing priority (above range, below range, Inf/NaN), so a wave never splits over its elements.
template <int CEIL>
__device__ __forceinline__ uint32_t bf16_key(double x) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(x);
    const uint32_t h = (uint32_t)(u >> 32) & 0x7FFFFFFFu, l = (uint32_t)u;
    const int32_t E = (int32_t)(h >> 20);
    const int32_t e8 = E - 896;
    uint32_t v = ((uint32_t)e8 << 7) | ((h >> 13) & 0x7Fu);
    const bool dropped = (h & 0x1FFFu) || l;
    if (CEIL == 1) v += dropped ? 1u : 0u;
    if (CEIL == 2) v += (dropped || !(v & 0x7Fu)) ? 1u : 0u;
    v = e8 >= 255 ? 0x7F80u : v;
    v = e8 <= 0 ? ((h | l) ? KEY_TINY : 0u) : v;
    return E == 0x7FF ? KEY_NAN : v;
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

// The delta and the flag bits of a maximum's key (the conversion of key_to_delta_kernel).
__device__ __forceinline__ int32_t key_delta(uint32_t key, int shift, uint32_t& bad) {
    int32_t e = 0;
    bad = 0;
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
    return shift - e;
}

// A's rows and B's columns in one launch of 1024-thread workgroups, deltas written directly:
//   workgroup j < ceil(N/W): columns Wj..Wj+W-1 of B over all of its K rows, thread t taking
//   column t % W and every P-th row from t / W (P = 1024/W phases). W = 32 (a wave reads two
//   256-byte row pieces per load; with 16 columns, 128-byte pieces, the strips read at 4.9 instead
//   of 5.7 TB/s at C3); for K <= 1024, W = 16, so that every thread's rows are one round of 16 loads
//   and there are twice as many strips (C1: 64 strips instead of 32 for 1024 columns);
//   workgroup ceil(N/W) + r: rows rR..rR+R-1 of A (R = 1 for K > 4096, more for shorter rows), each
//   thread a stride-(1024/R) run of its row's K values.
// The column strips read W K doubles each workgroup, the rows K: the long strips are dispatched
// first and the short rows fill in behind them, so no strip is left running alone at the end.
// The 16 waves' maxima meet in LDS; flags[0] (A) and flags[1] (B) collect the flag bits with atomicOr.
// Thread 0 and 1 of workgroup 0 zero clear[0..1] (when given): the flag slot of the next pass, so
// that a caller alternating between two slots needs no launch to clear them.
template <int CEIL, int W>
__global__ void __launch_bounds__(1024) scale_pair_kernel(const double* __restrict__ A, int M, int K, int lda,
                                                          const double* __restrict__ B, int N, int ldb, int shift,
                                                          int32_t* __restrict__ dA, int32_t* __restrict__ dB,
                                                          uint32_t* __restrict__ flags, uint32_t* __restrict__ clear,
                                                          int rows_per_wg) {
    static_assert(W == 16 || W == 32, "strip width");
    constexpr int P = 1024 / W;  // row phases of a strip
    __shared__ uint32_t part[1024];
    const int t = threadIdx.x;
    // the other flag slot, which no workgroup of this launch touches otherwise
    if (clear && blockIdx.x == 0 && t < 2) clear[t] = 0u;
    const int strips = (N + W - 1) / W;
    if ((int)blockIdx.x >= strips) {
        // R rows per workgroup (rows_per_wg: R = 8192 / K rounded down to a power of two, 1..16), so
        // that every thread has 8 loads in flight for K <= 8192: the 1024 / R threads of a row take a
        // stride-(1024 / R) run of its K values each, and its 16 / R waves meet in LDS.
        const int R = rows_per_wg, T = 1024 / R;
        const int q = t / T, tt = t - q * T;
        const int i = ((int)blockIdx.x - strips) * R + q;
        uint32_t k[4] = {0, 0, 0, 0};
        if (i < M) {
            const double* row = A + (size_t)i * lda;
            int c = tt;
            for (; c + 7 * T < K; c += 8 * T) {
                double v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = row[c + T * u];
#pragma unroll
                for (int u = 0; u < 8; u++) k[u & 3] = max(k[u & 3], bf16_key<CEIL>(v[u]));
            }
            for (; c < K; c += T) k[0] = max(k[0], bf16_key<CEIL>(row[c]));
        }
        const uint32_t kk = wave_max(max(max(k[0], k[1]), max(k[2], k[3])));
        if ((t & 63) == 0) part[t >> 6] = kk;
        __syncthreads();
        if (tt == 0 && i < M) {
            const int wpr = 16 / R;  // waves per row
            uint32_t m = 0;
            for (int w = 0; w < wpr; w++) m = max(m, part[q * wpr + w]);
            uint32_t bad;
            dA[i] = key_delta(m, shift, bad);
            if (bad) atomicOr(&flags[0], bad);
        }
    } else {
        const int col = (int)blockIdx.x * W + (t % W);
        const int ph = t / W;
        // 16 loads in flight per thread (16 P rows of the strip per round trip)
        uint32_t k[4] = {0, 0, 0, 0};
        if (col < N) {
            const double* p = B + col;
            int r = ph;
            for (; r + 15 * P < K; r += 16 * P) {
                double v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = p[(size_t)(r + P * u) * ldb];
#pragma unroll
                for (int u = 0; u < 16; u++) k[u & 3] = max(k[u & 3], bf16_key<CEIL>(v[u]));
            }
            for (; r + 3 * P < K; r += 4 * P) {
                double v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = p[(size_t)(r + P * u) * ldb];
#pragma unroll
                for (int u = 0; u < 4; u++) k[u] = max(k[u], bf16_key<CEIL>(v[u]));
            }
            for (; r < K; r += P) k[0] = max(k[0], bf16_key<CEIL>(p[(size_t)r * ldb]));
        }
        part[t] = max(max(k[0], k[1]), max(k[2], k[3]));  // part[W ph + c]
        __syncthreads();
        // P phases per column: 8 threads per column take P/8 phases each, then one thread 8 of those
        uint32_t m8 = 0;
        if (t < 8 * W) {
            const int c = t % W, q = t / W;
#pragma unroll
            for (int u = 0; u < P / 8; u++) m8 = max(m8, part[((P / 8) * q + u) * W + c]);
        }
        __syncthreads();
        if (t < 8 * W) part[t] = m8;  // part[W q + c]
        __syncthreads();
        if (t < W && (int)blockIdx.x * W + t < N) {
            uint32_t m = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) m = max(m, part[q * W + t]);
            uint32_t bad;
            dB[(int)blockIdx.x * W + t] = key_delta(m, shift, bad);
            if (bad) atomicOr(&flags[1], bad);
        }
    }
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

extern "C" int oz_scale_pair_f64(oz_dev* dev, const double* A, int M, int K, int lda, const double* B, int N, int ldb,
                                 int ceil_mode, int shift, int32_t* dA, int32_t* dB, uint32_t* flags,
                                 uint32_t* clear_flags) {
    if (int st = oz::use(dev)) return st;
    if (!A || !B || !dA || !dB || !flags || M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < N || ceil_mode < 0 ||
        ceil_mode > 2 || ((uintptr_t)flags & 3) || ((uintptr_t)clear_flags & 3) ||
        (clear_flags && clear_flags + 2 > flags && flags + 2 > clear_flags))
        return oz::fail(dev, OZ_ERR_ARG, "oz_scale_pair_f64: invalid arguments (M=%d N=%d K=%d lda=%d ldb=%d ceil=%d)",
                        M, N, K, lda, ldb, ceil_mode);
    int R = 1;  // rows of A per workgroup: 8 loads per thread for K <= 8192
    while (R < 16 && (long long)K * R * 2 <= 8192) R *= 2;
    const int W = K <= 1024 ? 16 : 32;  // columns of B per workgroup
    const long long blocks = ((long long)M + R - 1) / R + (N + W - 1) / W;
    if (blocks > 0x7FFFFFFFll) return oz::fail(dev, OZ_ERR_ARG, "oz_scale_pair_f64: grid too large");
    const dim3 grid((unsigned)blocks), block(1024);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, dev->stream, A, M, K, lda, B, N, ldb, shift, dA, dB, flags,
                           clear_flags, R);
    };
    if (W == 16)
        ceil_mode == 0 ? launch(scale_pair_kernel<0, 16>)
                       : (ceil_mode == 1 ? launch(scale_pair_kernel<1, 16>) : launch(scale_pair_kernel<2, 16>));
    else
        ceil_mode == 0 ? launch(scale_pair_kernel<0, 32>)
                       : (ceil_mode == 1 ? launch(scale_pair_kernel<1, 32>) : launch(scale_pair_kernel<2, 32>));
    return oz::launch_check(dev, "scale_pair_kernel");
}

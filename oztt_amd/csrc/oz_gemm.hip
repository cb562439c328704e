// A9: exact int8 x int8 -> int32 products on the CDNA4 matrix cores, batched over moduli.
//
// Semantics (reference bmm_int32_spill.cpp:265 as driven by ozaki2.cpp:333-350): for every modulus,
// C_s = A_s * B_s with exact int32 accumulation (the planner bounds |C_s| <= K*127^2 < 2^31,
// moduli.hpp:217-231). Integer MFMA accumulation is exact, so the result is independent of the
// summation order.
//
// MI355X design: both operands are K-contiguous int8 planes (A: M x K, Bt: N x K), zero-padded to
// the tile grid, so every global load is a 16-byte vector and every LDS fragment read feeds one
// v_mfma_i32_16x16x64_i8 directly (lane l holds row l%16, bytes 16*(l/16)..+15 of a 64-byte K
// slice for both operands; output lane l holds column l%16, rows 4*(l/16)..+3). A workgroup of 4
// waves computes a BM x BN tile; K advances in BK-byte steps through double-buffered LDS with the
// next step's global loads in flight during the current step's MFMAs. Workgroups are ordered
// moduli-major with the N tiles of one row band adjacent, so concurrently running workgroups
// share A rows in L2.
#include "oz_internal.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int BM, int BN, int BK, int WGM, int WGN>
struct GemmCfg {
    static constexpr int THREADS = 64 * WGM * WGN;
    static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
    static constexpr int FM = WM / 16, FN = WN / 16;    // 16x16 fragments per wave
    static constexpr int LDSROW = BK + 16;              // bytes per LDS row (padded)
    static constexpr int A_CHUNKS = BM * BK / 16;       // 16-byte chunks per stage
    static constexpr int B_CHUNKS = BN * BK / 16;
    static constexpr int A_PER_T = A_CHUNKS / THREADS;
    static constexpr int B_PER_T = B_CHUNKS / THREADS;
    static_assert(A_CHUNKS % THREADS == 0 && B_CHUNKS % THREADS == 0, "tile loads must divide evenly");
    static_assert(BK % 64 == 0, "K step is a multiple of the MFMA K (64)");
    static constexpr int LDS_BYTES = 2 * (BM + BN) * LDSROW;
};

template <int BM, int BN, int BK, int WGM, int WGN>
__global__ void __launch_bounds__(64 * WGM * WGN) gemm_i8_kernel(const int8_t* __restrict__ A,
                                                                  const int8_t* __restrict__ Bt,
                                                                  int32_t* __restrict__ C, int M, int N, int K, int lda,
                                                                  int ldb, int ldc, long long sA, long long sB,
                                                                  long long sC, int tiles_n, int tiles_per_batch) {
    using G = GemmCfg<BM, BN, BK, WGM, WGN>;
    __shared__ __attribute__((aligned(16))) int8_t lds[G::LDS_BYTES];
    constexpr int STAGE = (BM + BN) * G::LDSROW;  // bytes of one stage: A rows, then B rows

    const int tid = threadIdx.x;
    const int batch = blockIdx.x / tiles_per_batch;
    const int tile = blockIdx.x % tiles_per_batch;
    const int tm = tile / tiles_n, tn = tile % tiles_n;
    const int8_t* Ab = A + batch * sA + (long long)tm * BM * lda;
    const int8_t* Bb = Bt + batch * sB + (long long)tn * BN * ldb;

    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WGN, wn = wave % WGN;
    const int frow = lane & 15, fk = (lane >> 4) * 16;

    v4i acc[G::FM][G::FN];
#pragma unroll
    for (int i = 0; i < G::FM; i++)
#pragma unroll
        for (int j = 0; j < G::FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

    uint4 ra[G::A_PER_T], rb[G::B_PER_T];
    constexpr int CPR = BK / 16;  // 16-byte chunks per row of a stage
#define OZ_GEMM_GLOAD(k0)                                                                                   \
    do {                                                                                                    \
        _Pragma("unroll") for (int i = 0; i < G::A_PER_T; i++) {                                            \
            const int c = tid + i * G::THREADS;                                                             \
            ra[i] = *reinterpret_cast<const uint4*>(Ab + (long long)(c / CPR) * lda + (k0) + (c % CPR) * 16); \
        }                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < G::B_PER_T; i++) {                                            \
            const int c = tid + i * G::THREADS;                                                             \
            rb[i] = *reinterpret_cast<const uint4*>(Bb + (long long)(c / CPR) * ldb + (k0) + (c % CPR) * 16); \
        }                                                                                                   \
    } while (0)
#define OZ_GEMM_LSTORE(buf)                                                                              \
    do {                                                                                                 \
        int8_t* sa = lds + (buf) * STAGE;                                                                \
        int8_t* sb = sa + BM * G::LDSROW;                                                                \
        _Pragma("unroll") for (int i = 0; i < G::A_PER_T; i++) {                                         \
            const int c = tid + i * G::THREADS;                                                          \
            *reinterpret_cast<uint4*>(sa + (c / CPR) * G::LDSROW + (c % CPR) * 16) = ra[i];              \
        }                                                                                                \
        _Pragma("unroll") for (int i = 0; i < G::B_PER_T; i++) {                                         \
            const int c = tid + i * G::THREADS;                                                          \
            *reinterpret_cast<uint4*>(sb + (c / CPR) * G::LDSROW + (c % CPR) * 16) = rb[i];              \
        }                                                                                                \
    } while (0)

    const int nk = K / BK;
#define OZ_GEMM_COMPUTE(cur)                                                                                  \
    do {                                                                                                      \
        const int8_t* la = lds + (cur) * STAGE + (wm * G::WM + frow) * G::LDSROW + fk;                        \
        const int8_t* lb = lds + (cur) * STAGE + BM * G::LDSROW + (wn * G::WN + frow) * G::LDSROW + fk;       \
        _Pragma("unroll") for (int ks = 0; ks < BK; ks += 64) {                                               \
            v4i fa[G::FM], fb[G::FN];                                                                         \
            _Pragma("unroll") for (int i = 0; i < G::FM; i++) fa[i] =                                         \
                *reinterpret_cast<const v4i*>(la + i * 16 * G::LDSROW + ks);                                  \
            _Pragma("unroll") for (int j = 0; j < G::FN; j++) fb[j] =                                         \
                *reinterpret_cast<const v4i*>(lb + j * 16 * G::LDSROW + ks);                                  \
            _Pragma("unroll") for (int i = 0; i < G::FM; i++) _Pragma("unroll") for (int j = 0; j < G::FN; j++) \
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);          \
        }                                                                                                     \
    } while (0)
    OZ_GEMM_GLOAD(0);
    OZ_GEMM_LSTORE(0);
    __syncthreads();
    for (int kt = 0; kt + 1 < nk; kt++) {
        OZ_GEMM_GLOAD((kt + 1) * BK);
        OZ_GEMM_COMPUTE(kt & 1);
        OZ_GEMM_LSTORE((kt + 1) & 1);
        __syncthreads();
    }
    OZ_GEMM_COMPUTE((nk - 1) & 1);
#undef OZ_GEMM_COMPUTE
#undef OZ_GEMM_GLOAD
#undef OZ_GEMM_LSTORE

    int32_t* Cb = C + batch * sC + (long long)(tm * BM + wm * G::WM) * ldc + tn * BN + wn * G::WN;
#pragma unroll
    for (int i = 0; i < G::FM; i++)
#pragma unroll
        for (int j = 0; j < G::FN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                Cb[(long long)(i * 16 + (lane >> 4) * 4 + r) * ldc + j * 16 + (lane & 15)] = acc[i][j][r];
}

using Cfg128 = GemmCfg<128, 128, 128, 2, 2>;

}  // namespace

extern "C" int oz_gemm_i8(oz_dev* dev, const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N, int K, int batch,
                          int lda, int ldb, int ldc, long long strideA, long long strideB, long long strideC) {
    if (int st = oz::use(dev)) return st;
    constexpr int BM = 128, BN = 128, BK = 128;
    if (!A || !Bt || !C || M <= 0 || N <= 0 || K <= 0 || batch <= 0 || M % 256 || N % 256 || K % 128 || lda < K ||
        ldb < K || ldc < N || lda % 16 || ldb % 16 || ((uintptr_t)A & 15) || ((uintptr_t)Bt & 15))
        return oz::fail(dev, OZ_ERR_ARG, "oz_gemm_i8: unsupported shape M=%d N=%d K=%d lda=%d ldb=%d", M, N, K, lda, ldb);
    if (K % BK)
        return oz::fail(dev, OZ_ERR_ARG, "oz_gemm_i8: K=%d must be a multiple of %d", K, BK);
    const int tiles_n = N / BN, tiles_m = M / BM;
    const long long grid = (long long)tiles_m * tiles_n * batch;
    if (grid > 0x7FFFFFFFll) return oz::fail(dev, OZ_ERR_ARG, "oz_gemm_i8: grid too large");
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, BK, 2, 2>), dim3((unsigned)grid), dim3(Cfg128::THREADS), 0,
                       dev->stream, A, Bt, C, M, N, K, lda, ldb, ldc, strideA, strideB, strideC,
                       tiles_n, tiles_m * tiles_n);
    return oz::launch_check(dev, "gemm_i8_kernel");
}

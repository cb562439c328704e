// A9: exact int8 x int8 -> int32 products on the CDNA4 matrix cores, batched over moduli.
//
// Semantics (reference bmm_int32_spill.cpp:265 as driven by ozaki2.cpp:333-350): for every modulus,
// C_s = A_s * B_s with exact int32 accumulation (the planner bounds |C_s| <= K*127^2 < 2^31,
// moduli.hpp:217-231). Integer MFMA accumulation is exact, so the result does not depend on the
// summation order.
//
// MI355X design
//   - Operands are int8 planes in OZ_BLOCK tiles (written so by the splitter): 1 KB blocks of 16
//     rows x 64 K-bytes, the K/64 blocks of each 16-row band consecutive, zero-padded to the tile
//     grid, so no load is guarded. Inside a block, 16-byte chunk c of row r sits at chunk position
//     c ^ f(r), f(r) = ((r >> 1) ^ (r >> 2)) & 3.
//   - A workgroup of 4 waves (one per SIMD) computes a 256 x 256 tile; each wave owns 128 x 128
//     (4 x 4 blocks of v_mfma_i32_32x32x32_i8, 256 accumulator registers). A single wave keeps the
//     32x32x32 MFMA pipe close to full, unlike the 16x16x64 form (measured on MI355X). Lane l holds
//     row l%32 and the 16 K-bytes 16*(l/32).. of a 32-byte K slice of both operands; output register
//     q of lane l is row 8*(q/4) + 4*(l/32) + q%4, column l%32.
//   - K advances in 64-byte steps through a ring of NS LDS stages filled by direct global->LDS
//     loads (global_load_lds_dwordx4: lane l's 16 bytes land at the instruction's LDS base + 16*l),
//     NS-1 stages ahead of the MFMAs, with no register staging. One wave instruction copies one
//     whole 1 KB block, contiguous in HBM and in LDS, so a stage's 256 rows are 16 blocks per
//     operand and the swizzle comes with the data: the 64 lanes of each fragment read
//     (ds_read_b128, rows r..r+31, two chunk columns) spread evenly over the LDS banks.
//   - Workgroups are mapped to tiles XCD-aware (tile_of below).
#include "oz2_modular.hpp"
#include "oz_gemm_common.hpp"
#include "oz_internal.hpp"

namespace {

using namespace ozg;

// Output modes. PRODUCTS: C[b] = A[b] Bt[b]^T as int32. DIGITS: the same products reduced in the
// epilogue to the CRT digit for modulus b (oz2::crt_digit with dc.m/y/magic[b]), C as uint8. DIAG
// (scheme I): C[d] = sum_{i <= d} A[i] Bt[d-i]^T as int32 for the diagonals d < nbatch, the d+1
// slice pairs concatenated along K in one accumulation.
enum GemmMode { PRODUCTS = 0, DIGITS = 1, DIAG = 2 };

template <int MODE>
__global__ void __launch_bounds__(THREADS) gemm_i8_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ Bt,
                                                          void* __restrict__ C, int K, int ldc, long long sA,
                                                          long long sB, long long sC, int tiles_m, int tiles_n,
                                                          int nbatch, oz2::DigitConsts dc) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[NS * STAGE];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int batch, tm, tn;
    if constexpr (MODE == DIAG) {
        // Diagonal d has d+1 pairs: the heaviest go first (workgroups start in index order), and
        // within a diagonal the XCD-aware order applies.
        const int per = tiles_m * tiles_n, b = blockIdx.x / per;
        int unused;
        tile_of(blockIdx.x - b * per, tiles_m, tiles_n, 1, unused, tm, tn);
        batch = nbatch - 1 - b;
    } else {
        tile_of(blockIdx.x, tiles_m, tiles_n, nbatch, batch, tm, tn);
    }
    const int nk = K / BK;  // blocks per 16-row band
    const int nsteps = MODE == DIAG ? (batch + 1) * nk : nk;  // K steps of this tile
    const long long band = (long long)nk * 1024;  // bytes of one 16-row band
    // Lane l copies bytes 16l..16l+15 of each block; the tile's first band is 16*tm (A), 16*tn (B).
    const int8_t* Ab = A + (MODE == DIAG ? 0 : batch * sA) + (long long)tm * (BM / 16) * band + 16 * lane;
    const int8_t* Bb = Bt + (MODE == DIAG ? 0 : batch * sB) + (long long)tn * (BN / 16) * band + 16 * lane;
    // Byte offsets of K step u: block u of the bands, or for DIAG block u%nk of pair i = u/nk
    // (A plane i, B plane batch-i).
    auto step_off = [&](int u, long long& oa, long long& ob) {
        if constexpr (MODE == DIAG) {
            const int i = u / nk, kt = u - i * nk;
            oa = i * sA + (long long)kt * 1024;
            ob = (batch - i) * sB + (long long)kt * 1024;
        } else {
            oa = ob = (long long)u * 1024;
        }
    };

    // Loader: wave instruction j (= 4*i + wave) copies block (band j of the tile, K step kstep) to
    // bytes 1024j.. of the stage, i.e. rows 16j..16j+15 of the 256 x 64 stage, swizzle included.
#define OZ_GEMM_ISSUE(kstep, buf)                                                                                 \
    do {                                                                                                          \
        long long oa, ob;                                                                                         \
        step_off(kstep, oa, ob);                                                                                  \
        int8_t* sa = lds + (buf) * STAGE;                                                                         \
        _Pragma("unroll") for (int i = 0; i < LOADS_A; i++)                                                       \
            __builtin_amdgcn_global_load_lds(Ab + (4 * i + wave) * band + oa, (lds_void*)(sa + 1024 * (4 * i + wave)), \
                                             16, 0, 0);                                                           \
        _Pragma("unroll") for (int i = 0; i < LOADS_B; i++)                                                       \
            __builtin_amdgcn_global_load_lds(Bb + (4 * i + wave) * band + ob,                                     \
                                             (lds_void*)(sa + STAGE_A + 1024 * (4 * i + wave)), 16, 0, 0);        \
    } while (0)

    const int wm = wave >> 1, wn = wave & 1;
    int offA[2], offB[2];
    fragment_offsets(lane, wm, wn, offA, offB);

    v16i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0;

    // Pipeline. Loads run NS stages ahead: while stage kt is consumed, stages kt+1 .. kt+NS-1 are in
    // flight or landed. Fragments are double-buffered per 32-byte K substep (F, G: 8 fragments of
    // 4 registers each): substep (kt, 0) reads G = substep (kt, 1) while its MFMAs run on F;
    // substep (kt, 1) waits for stage kt+1, makes sure every wave has finished reading stage kt
    // (own LDS reads complete, then the barrier), refills that buffer with stage kt+NS, and reads
    // F = substep (kt+1, 0) while its MFMAs run on G. The tail re-loads the last valid stage
    // (clamped), so every step has the same number of loads in flight and the same wait count.
#pragma unroll
    for (int s = 0; s < NS; s++) OZ_GEMM_ISSUE(min(s, nsteps - 1), s);
    v4i fa[4], fb[4], ga[4], gb[4];
    wait_vmcnt<(LOADS_A + LOADS_B) * (NS - 1)>();  // stage 0
    stage_barrier();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        fa[i] = *reinterpret_cast<const v4i*>(lds + offA[0] + i * 32 * BK);
        fb[i] = *reinterpret_cast<const v4i*>(lds + offB[0] + i * 32 * BK);
    }
    // The issue order inside a step is fixed with sched_barrier fences (left alone, the compiler
    // sinks every fragment read to just before its first use, which stalls the MFMAs on LDS
    // latency): the 8 fragment reads of the other buffer, and after the barrier the 8 global->LDS
    // loads, go one per MFMA over the first 8 of the 16 MFMAs of each substep.
    for (int kt = 0; kt < nsteps; kt++) {
        const int8_t* cur = lds + (kt % NS) * STAGE;
        const int8_t* nxt = lds + ((kt + 1) % NS) * STAGE;
        // substep (kt, 0): MFMAs on F, reads of G = substep (kt, 1)
#pragma unroll
        for (int g = 0; g < 16; g++) {
            acc[g >> 2][g & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[g >> 2], fb[g & 3], acc[g >> 2][g & 3], 0, 0, 0);
            if (g < 4) ga[g] = *reinterpret_cast<const v4i*>(cur + offA[1] + g * 32 * BK);
            else if (g < 8) gb[g - 4] = *reinterpret_cast<const v4i*>(cur + offB[1] + (g - 4) * 32 * BK);
            __builtin_amdgcn_sched_barrier(0);
        }
        wait_vmcnt_lgkm0<(LOADS_A + LOADS_B) * (NS - 2)>();  // stage kt+1 landed; own reads of stage kt done
        stage_barrier();                                      // ... for every wave
        // substep (kt, 1): MFMAs on G, refill of stage kt's buffer, reads of F = substep (kt+1, 0)
        long long oa, ob;
        step_off(min(kt + NS, nsteps - 1), oa, ob);
        int8_t* sa = lds + (kt % NS) * STAGE;
#pragma unroll
        for (int g = 0; g < 16; g++) {
            acc[g >> 2][g & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ga[g >> 2], gb[g & 3], acc[g >> 2][g & 3], 0, 0, 0);
            if (g < 4) {
                __builtin_amdgcn_global_load_lds(Ab + (4 * g + wave) * band + oa, (lds_void*)(sa + 1024 * (4 * g + wave)),
                                                 16, 0, 0);
                fa[g] = *reinterpret_cast<const v4i*>(nxt + offA[0] + g * 32 * BK);
            } else if (g < 8) {
                const int i = g - 4;
                __builtin_amdgcn_global_load_lds(Bb + (4 * i + wave) * band + ob,
                                                 (lds_void*)(sa + STAGE_A + 1024 * (4 * i + wave)), 16, 0, 0);
                fb[i] = *reinterpret_cast<const v4i*>(nxt + offB[0] + i * 32 * BK);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#undef OZ_GEMM_ISSUE
    wait_vmcnt<0>();  // drain the clamped tail loads before the workgroup ends

    const long long c0 = batch * sC + (long long)(tm * BM + wm * 128) * ldc + tn * BN + wn * 128;
    if constexpr (MODE == DIGITS) {
        // Digits go through LDS (the stages are free once every wave has left the main loop) so
        // that each lane stores 16 contiguous bytes: the wave's 128 x 128 byte tile is written
        // with row stride 144 (rows r and r+4, written by the two lane halves, then fall on
        // different banks) and read back as 16-byte chunks, 8 per row.
        constexpr int TS = 144;
        static_assert(4 * 128 * TS <= NS * STAGE, "epilogue tiles fit in the stage ring");
        __syncthreads();
        uint8_t* tile = reinterpret_cast<uint8_t*>(lds) + wave * (128 * TS);
        const uint32_t m = dc.m[batch], y = dc.y[batch], mg = dc.magic[batch];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    tile[(32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3)) * TS + 32 * j + (lane & 31)] =
                        (uint8_t)oz2::crt_digit(acc[i][j][q], m, y, mg);
        uint8_t* Cb = static_cast<uint8_t*>(C) + c0;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int c = 64 * t + lane, r = c >> 3, x = 16 * (c & 7);
            *reinterpret_cast<uint4*>(Cb + (long long)r * ldc + x) = *reinterpret_cast<const uint4*>(tile + r * TS + x);
        }
    } else {
        int32_t* Cb = static_cast<int32_t*>(C) + c0;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    Cb[(long long)(32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3)) * ldc + 32 * j + (lane & 31)] =
                        acc[i][j][q];
    }
}

// Shape rules shared by both entry points; returns a message or nullptr.
const char* check_gemm(const int8_t* A, const int8_t* Bt, const void* C, int M, int N, int K, int batch, int ldc,
                       long long strideA, long long strideB, long long strideC) {
    if (!A || !Bt || !C || M <= 0 || N <= 0 || K <= 0 || batch <= 0 || M % BM || N % BN || K % BK || ldc < N ||
        ((uintptr_t)A & 15) || ((uintptr_t)Bt & 15) || strideA % 1024 || strideB % 1024 ||
        (batch > 1 && (strideA < (long long)M * K || strideB < (long long)N * K || strideC < (long long)M * ldc)))
        return "unsupported shape";
    if ((long long)(M / BM) * (N / BN) * batch > 0x7FFFFFFFll) return "grid too large";
    return nullptr;
}

template <int MODE>
int launch_gemm(oz_dev* dev, const int8_t* A, const int8_t* Bt, void* C, int M, int N, int K, int batch, int ldc,
                long long strideA, long long strideB, long long strideC, const oz2::DigitConsts& dc) {
    const int tiles_m = M / BM, tiles_n = N / BN;
    const unsigned grid = (unsigned)((long long)tiles_m * tiles_n * batch);
    hipLaunchKernelGGL(gemm_i8_kernel<MODE>, dim3(grid), dim3(THREADS), 0, dev->stream, A, Bt, C, K, ldc, strideA,
                       strideB, strideC, tiles_m, tiles_n, batch, dc);
    return oz::launch_check(dev, "gemm_i8_kernel");
}

}  // namespace

extern "C" int oz_gemm_i8(oz_dev* dev, const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N, int K, int batch,
                          int ldc, long long strideA, long long strideB, long long strideC) {
    if (int st = oz::use(dev)) return st;
    if (const char* e = check_gemm(A, Bt, C, M, N, K, batch, ldc, strideA, strideB, strideC))
        return oz::fail(dev, OZ_ERR_ARG, "oz_gemm_i8: %s (M=%d N=%d K=%d batch=%d)", e, M, N, K, batch);
    return launch_gemm<PRODUCTS>(dev, A, Bt, C, M, N, K, batch, ldc, strideA, strideB, strideC, oz2::DigitConsts{});
}

extern "C" int oz2_gemm_digits(oz_dev* dev, const int8_t* A, const int8_t* Bt, uint8_t* D, int M, int N, int K, int S,
                               int ldd, long long strideA, long long strideB, long long strideD,
                               const oz2_crt_dev* crt) {
    if (int st = oz::use(dev)) return st;
    if (const char* e = check_gemm(A, Bt, D, M, N, K, S, ldd, strideA, strideB, strideD))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_digits: %s (M=%d N=%d K=%d S=%d)", e, M, N, K, S);
    if (!crt || crt->S != S || S > OZ2_MAXS) return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_digits: S does not match crt");
    if (ldd % 16 || strideD % 16 || ((uintptr_t)D & 15))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_digits: D, ldd and strideD must be 16-byte aligned");
    oz2::DigitConsts dc{};
    for (int s = 0; s < S; s++) {
        const uint32_t m = crt->m[s];
        if (m < 2 || m > 255 || crt->y[s] >= m) return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_digits: bad modulus %u", m);
        dc.m[s] = m;
        dc.y[s] = crt->y[s];
        dc.magic[s] = (uint32_t)(0x100000000ull / m);
    }
    return launch_gemm<DIGITS>(dev, A, Bt, D, M, N, K, S, ldd, strideA, strideB, strideD, dc);
}

extern "C" int oz1_gemm_diag_i8(oz_dev* dev, const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N, int K,
                                int ndiag, int dmax, int ldc, long long strideA, long long strideB,
                                long long strideC) {
    if (int st = oz::use(dev)) return st;
    if (const char* e = check_gemm(A, Bt, C, M, N, K, ndiag, ldc, strideA, strideB, strideC))
        return oz::fail(dev, OZ_ERR_ARG, "oz1_gemm_diag_i8: %s (M=%d N=%d K=%d ndiag=%d)", e, M, N, K, ndiag);
    // one accumulation covers ndiag*K products of at most dmax^2: it must stay exact in int32
    if (dmax < 1 || dmax > 127 || (long long)ndiag * K * dmax * dmax > 0x7FFFFFFFll)
        return oz::fail(dev, OZ_ERR_ARG, "oz1_gemm_diag_i8: %d pairs of K=%d with digits up to %d can overflow int32",
                        ndiag, K, dmax);
    return launch_gemm<DIAG>(dev, A, Bt, C, M, N, K, ndiag, ldc, strideA, strideB, strideC, oz2::DigitConsts{});
}

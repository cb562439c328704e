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
//   - A workgroup of 4 waves (one per SIMD) computes a 256 x 256 tile; each wave owns 128 x 128 as
//     8 x 8 blocks of v_mfma_i32_16x16x64_i8 (256 accumulator registers). One MFMA operand is one
//     whole OZ_BLOCK: lane l holds row l%16 and K-bytes 16*(l/16)..+15 of both operands (A and B use
//     the same lane -> K map, so the sum runs over every K index once whatever order the matrix core
//     takes them in); output register q of lane l is row 4*(l/16) + q, column l%16. The 64 lanes of a
//     fragment read (ds_read_b128) cover one 1 KB block, so they fall on every LDS bank equally.
//     On MI355X the 16x16x64 form runs the same products at a higher clock under the power limit
//     than 32x32x32 (measured with random residues, which is what the matrix cores see).
//   - K advances in 64-byte steps through a ring of NS = 4 LDS stages (32 KB each) filled by direct
//     global->LDS loads (lds_copy_block: one wave instruction copies one block, contiguous in HBM and
//     in LDS, the swizzle included), NS-1 stages ahead of the MFMAs, with no register staging. The
//     load addresses are wave-uniform SGPR pairs plus one per-lane offset register.
//   - Each K step is one barrier and 64 MFMAs per wave; the 16 fragment reads of the next step (one
//     per 4 MFMAs) and the 8 loads that refill the ring (one per 8 MFMAs) are spread over them in a
//     fixed order (sched_barrier fences; left alone, the compiler bunches them).
//   - Workgroups are mapped to tiles so that all XCDs sweep the moduli in step (tile_of_lockstep):
//     the operands in flight then stay in the Infinity Cache, which keeps HBM traffic, and with it
//     power, down; the matrix cores are power-limited, so that raises their clock.
#include "oz2_modular.hpp"
#include "oz_gemm_common.hpp"
#include "oz_internal.hpp"

namespace {

using namespace ozg;

// Output modes. PRODUCTS: C[b] = A[b] Bt[b]^T as int32. DIGITS: the same products reduced in the
// epilogue to the CRT digit for modulus b ((C mod m_b) y_b mod m_b, from dc.m/y[b]; a digit 0 may be
// stored as m_b, oz2::mod_mul_f64), C as uint8. DIAG
// (scheme I): C[d] = sum_{i <= d} A[i] Bt[d-i]^T as int32 for the diagonals d < nbatch, the d+1
// slice pairs concatenated along K in one accumulation.
enum GemmMode { PRODUCTS = 0, DIGITS = 1, DIAG = 2 };

constexpr int LOADS = LOADS_A + LOADS_B;  // global->LDS loads per wave per K step

// The last tiles go to the XCDs that get there first. The hardware hands workgroups to the XCDs in
// turn (workgroup w to XCD w % 8) and each XCD runs its share at its own pace; the CUs of one XCD
// finish together, but the XCDs do not run at one speed (at C3 their last tiles ended up to 7% apart,
// a different XCD lagging on different runs), so with a fixed tile per workgroup the slowest XCD sets
// the launch time. So workgroup w < first runs item w of the lockstep tile sequence
// (tile_of_lockstep) as before, and the remaining items, the last sixteenth of every XCD's share
// (room enough for the speed differences seen; a pool tile mostly runs where its bands are not in
// L2, so a larger pool costs traffic; an eighth for Scheme I's diagonals), form a pool that the other workgroups take from in lockstep
// order, as they start; the grid holds 1/8 more workgroups than tiles, and a workgroup that finds
// the pool empty ends at once. Only the pool's workgroups pay for an atomic. The host sets `first`
// (launch_gemm; a launch of one wave has no pool). Pool counters (per device handle, zero between launches): q[0] the
// next item, q[1] the pool workgroups that have taken theirs; the last of them zeroes both.
struct TilePool {
    int* q;
    int first, total;
    // items of every XCD's share left to the pool: 1/frac of it
    __host__ static int first_of(int total, int frac) {
        const int per = total / 8;
        return 8 * (per - (per + frac - 1) / frac);
    }
    // thread 0 of a workgroup w >= first, once. The second atomic must not reach memory before the
    // first has: then, when the count reaches the number of pool workgroups, every one of them is done
    // with q[0], and the reset cannot be overtaken by a straggler's increment (which would leave q[0] = 1
    // and make the next launch on the handle skip a tile). Its operand is computed from the first one's
    // result (p >= 0, so the operand is 1), so it cannot be issued before that result has returned,
    // whatever the compiler schedules; no fence is needed (and an agent-scope release would write the
    // XCD's L2 back). The operand is made wave-uniform, so the compiler's atomic combining stays a
    // scalar multiply (a per-lane operand would make it loop over the lanes through M0).
    __device__ int take() const {
        const int p = atomicAdd(&q[0], 1);
        const int one = __builtin_amdgcn_readfirstlane(1 | (p >> 31));
        if (atomicAdd(&q[1], one) == (int)gridDim.x - first - 1) {
            atomicExch(&q[0], 0);
            atomicExch(&q[1], 0);
        }
        return first + p < total ? first + p : -1;
    }
};

template <int MODE, bool EVEN>
__global__ void __launch_bounds__(THREADS) gemm_i8_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ Bt,
                                                          void* __restrict__ C, int K, int ldc, long long sA,
                                                          long long sB, long long sC, int tiles_m, int tiles_n,
                                                          int nbatch, oz2::DigitConsts dc, int* __restrict__ queue,
                                                          int first) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[NS * STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int total = tiles_m * tiles_n * nbatch;
    int w = blockIdx.x;
    const TilePool pool{queue, first, total};
    if (w >= pool.first) {
        __shared__ int item;
        if (threadIdx.x == 0) item = pool.take();
        __syncthreads();
        w = __builtin_amdgcn_readfirstlane(item);
        if (w < 0) return;
    }
    int batch, tm, tn;
    // A launch of at most one tile per CU (no pool: first == total) runs in one wave, and each XCD
    // takes one contiguous range of the batch-major tile sequence (tile_of): whole moduli when a
    // modulus has at most a few tiles (C1: 16 tiles of 1024^2, two moduli per XCD), whose operand
    // bands then stay in that XCD's L2 (0.0594 against 0.0683 ms for the whole C1 pass). Larger
    // launches sweep the moduli in step over all XCDs (tile_of_lockstep), sharing each modulus's
    // operands through the Infinity Cache.
    if (first >= total)
        tile_of(w, tiles_m, tiles_n, nbatch, batch, tm, tn);
    else
        tile_of_lockstep(w, tiles_m, tiles_n, nbatch, batch, tm, tn);
    // Scheme I: diagonal d has d+1 pairs; the heaviest are dispatched first.
    if constexpr (MODE == DIAG) batch = nbatch - 1 - batch;
    // The map divides with VALU code; its results are wave-uniform, so they are moved to SGPRs
    // (left in VGPRs, every address derived from them is too, and the register allocator then
    // shuffles accumulators between AGPRs and VGPRs inside the main loop).
    batch = __builtin_amdgcn_readfirstlane(batch);
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    const int nk = K / BK;                                 // blocks per 16-row band
    const int nst = MODE == DIAG ? (batch + 1) * nk : nk;  // K steps of this tile
    const long long band = (long long)nk * 1024;           // bytes of one 16-row band
    const int8_t* Ab = A + (MODE == DIAG ? 0 : batch * sA) + (long long)tm * 16 * band;
    const int8_t* Bb = Bt + (MODE == DIAG ? 0 : batch * sB) + (long long)tn * 16 * band;
    const unsigned lane16 = 16u * lane;
    // DIAG: the K step being loaded is block lk of the bands of pair li (A plane li, B plane
    // batch-li), at byte offsets oA = li sA + 1024 lk and oB = (batch-li) sB + 1024 lk from the tile's
    // bands; lcount counts the steps loaded so far and stops at the last one (past the end the last
    // step is loaded again, so every step issues the same number of loads and the wait counts never
    // change). Running counters and offsets instead of st / nk and products: integer division runs
    // on the VALU, and all of this must stay on the SALU. The other modes load block
    // st = min(step, nst - 1) directly.
    int lk = 0, lcount = 0;
    long long oA = 0, oB = MODE == DIAG ? batch * sB : 0;
    auto next_stage = [&]() {  // branch-free: selects only
        if constexpr (MODE == DIAG) {
            const int adv = lcount < nst - 1;
            lcount += adv;
            lk += adv;
            oA += adv ? 1024 : 0;
            oB += adv ? 1024 : 0;
            const int wrap = lk == nk;
            lk = wrap ? 0 : lk;
            oA += wrap ? sA - band : 0;
            oB -= wrap ? sB + band : 0;
        }
    };
    // Load j (0..3) of this wave for A (issue) or B (issueB) of K step st: the block of band
    // q = 4*j + wave, rows 16q.. of the 256 x 64 stage, to byte 1024 q of the operand's half of
    // stage buffer buf. (The expressions are written with bnd = q & 15 and kb = q >> 4, kb being 0:
    // in this form the compiler keeps the address arithmetic in the loop on the SALU;
    // tests/test_gemm_asm.py checks the generated main loops.)
    auto issue = [&](int buf, int j, int st) {
        const int q = 4 * j + wave, bnd = q & 15, kb = q >> 4;
        long long go;
        if constexpr (MODE == DIAG)
            go = (long long)bnd * band + oA + (long long)kb * 1024;
        else
            go = (long long)bnd * band + (long long)(st + kb) * 1024;
        lds_copy_block(Ab + go, lds + buf * STAGE + (kb * 16 + bnd) * 1024, lane16);
    };
    auto issueB = [&](int buf, int j, int st) {
        const int q = 4 * j + wave, bnd = q & 15, kb = q >> 4;
        long long go;
        if constexpr (MODE == DIAG)
            go = (long long)bnd * band + oB + (long long)kb * 1024;
        else
            go = (long long)bnd * band + (long long)(st + kb) * 1024;
        lds_copy_block(Bb + go, lds + buf * STAGE + STAGE_A + (kb * 16 + bnd) * 1024, lane16);
    };
    const int wm = wave >> 1, wn = wave & 1;
    // Fragment reads: lane l takes the 16 bytes of row r = l%16, logical chunk c = l/16 of a block,
    // stored at byte 64 r + 16 (c ^ f(r)).
    const int r = lane & 15, c = lane >> 4;
    const int foff = 64 * r + 16 * (c ^ (((r >> 1) ^ (r >> 2)) & 3));
    v4i acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = v4i{0, 0, 0, 0};

    // Prologue: stages 0..NS-1 in flight, then the fragments of stage 0.
#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
        for (int j = 0; j < LOADS_A; j++) {
            issue(s, j, min(s, nst - 1));
            issueB(s, j, min(s, nst - 1));
        }
        next_stage();
    }
    v4i fa[8], fb[8], ga[8], gb[8];
    wait_vmcnt<LOADS * (NS - 1)>();
    stage_barrier();
    // fragment blk (0..7) of the wave's A rows (op 0) or B rows (op 1) in stage buffer buf
    auto rd = [&](int buf, int op, int blk) -> v4i {
        const int bnd = (op ? wn : wm) * 8 + blk;
        return *reinterpret_cast<const v4i*>(lds + buf * STAGE + op * STAGE_A + bnd * 1024 + foff);
    };
#pragma unroll
    for (int i = 0; i < 8; i++) {
        fa[i] = rd(0, 0, i);
        fb[i] = rd(0, 1, i);
    }

    // One K step: 64 MFMAs on (xa, xb); the 16 reads of (ya, yb) from stage buffer rbuf, one per 4
    // MFMAs in the order a0, b0..b7, a1..a7 (the first MFMAs of the next step need a0 and the b's);
    // the 8 loads of the next stage to load into buffer lbuf, one per 8 MFMAs.
    auto substep = [&](v4i* xa, v4i* xb, v4i* ya, v4i* yb, int rbuf, int lbuf, int lst) {
#pragma unroll
        for (int g = 0; g < 64; g++) {
            const int i = g >> 3, j = g & 7;
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], xb[j], acc[i][j], 0, 0, 0);
            if (g % 4 == 0) {
                const int t = g / 4;
                if (t == 0) ya[0] = rd(rbuf, 0, 0);
                else if (t <= 8) yb[t - 1] = rd(rbuf, 1, t - 1);
                else ya[t - 8] = rd(rbuf, 0, t - 8);
            }
            if (g % 8 == 6) {
                const int t = g / 8;
                if (t & 1) issueB(lbuf, t >> 1, lst);
                else issue(lbuf, t >> 1, lst);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // K step kt: wait until stage kt+1 has landed and this wave's reads of stage kt (into X) are
    // complete, then the barrier: every wave is done with stage kt's buffer, which is refilled with
    // stage kt+NS while the MFMAs run on X and Y reads stage kt+1. Two steps per trip (X and Y swap
    // roles). EVEN kernels (an even number of K steps in every tile: K/64 even) have no tail; the
    // others end an odd count with one more step.
    int kt = 0;
    auto trip = [&]() {
        wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
        stage_barrier();
        substep(fa, fb, ga, gb, (kt + 1) % NS, kt % NS, min(kt + NS, nst - 1));
        next_stage();
        wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
        stage_barrier();
        substep(ga, gb, fa, fb, (kt + 2) % NS, (kt + 1) % NS, min(kt + 1 + NS, nst - 1));
        next_stage();
        kt += 2;
    };
    // EVEN: K/64 is even and positive, so every tile has at least two steps; a loop that tests first
    // makes the compiler keep a path around it and zero the 256 accumulators twice on the way in.
    // (DIGITS only: in the other modes the bottom-tested loop moves accumulators inside the loop.)
    if constexpr (EVEN && MODE == DIGITS) {
        do trip();
        while (kt < nst);
    } else {
        for (; kt + 1 < nst; kt += 2) {
            wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
            stage_barrier();
            substep(fa, fb, ga, gb, (kt + 1) % NS, kt % NS, min(kt + NS, nst - 1));
            next_stage();
            wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
            stage_barrier();
            substep(ga, gb, fa, fb, (kt + 2) % NS, (kt + 1) % NS, min(kt + 1 + NS, nst - 1));
            next_stage();
        }
    }
    if constexpr (!EVEN) {
        if (kt < nst) {
            wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
            stage_barrier();
            substep(fa, fb, ga, gb, (kt + 1) % NS, kt % NS, min(kt + NS, nst - 1));
        }
    }
    wait_vmcnt<0>();  // drain the clamped tail loads before the workgroup ends

    const long long c0 = batch * sC + (long long)(tm * BM + wm * 128) * ldc + tn * BN + wn * 128;
    if constexpr (MODE == DIGITS) {
        // The int32 sums go through LDS and the digits are computed there, so the accumulators are
        // only ever stored (as in the int32 modes, which keeps them in AGPRs through the main loop;
        // VALU arithmetic on them makes the register allocator move them into VGPRs inside it).
        // Each wave owns 32 KB of the (now free) stage ring and writes its 128 x 128 sums in two
        // rounds of 64 rows, row-major with 16-int column groups swizzled by bits 2..3 of the row
        // (the four 16-lane groups of a write then cover all banks); every lane then reads 16
        // consecutive sums, reduces them to digits and stores them as one 16-byte chunk.
        __syncthreads();
        int32_t* tile = reinterpret_cast<int32_t*>(lds) + wave * (64 * 128);
        uint32_t m = 2, y = 0;
#pragma unroll
        for (int s = 0; s < OZ2_MAXS; s++)
            if (s == batch) {
                m = dc.m[s];
                y = dc.y[s];
            }
        uint8_t* Cb = static_cast<uint8_t*>(C) + c0;
        const double md = (double)m, yr = (double)y / md;
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int row = 16 * i + 4 * (lane >> 4) + q;  // (row >> 2) & 3 == lane >> 4
                        tile[row * 128 + ((16 * j) ^ (16 * (lane >> 4))) + (lane & 15)] = acc[4 * h + i][j][q];
                    }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int e = 64 * t + lane, row = e >> 3, cg = e & 7;
                const int* src = tile + row * 128 + ((16 * cg) ^ (16 * ((row >> 2) & 3)));
                int32_t c[16];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const v4i v = *reinterpret_cast<const v4i*>(src + 4 * k);
#pragma unroll
                    for (int q = 0; q < 4; q++) c[4 * k + q] = v[q];
                }
                uint32_t w[4];
                oz2::mod_mul_f64_x16(c, yr, md, w);
                // non-temporal: the digits (1.1 GB at C3) would only push the operand planes of the
                // modulus in progress out of the Infinity Cache
                typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]},
                                            reinterpret_cast<u32x4*>(Cb + (long long)(64 * h + row) * ldc + 16 * cg));
            }
        }
    } else {
        // non-temporal, as the digits: the int32 sums (C2: 512 MB) need not displace the operand planes
        int32_t* Cb = static_cast<int32_t*>(C) + c0;
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    __builtin_nontemporal_store(acc[i][j][q],
                                                &Cb[(long long)(16 * i + 4 * (lane >> 4) + q) * ldc + 16 * j + (lane & 15)]);
    }
}

// Shape rules shared by both entry points; returns a message or nullptr.
const char* check_gemm(const int8_t* A, const int8_t* Bt, const void* C, int M, int N, int K, int batch, int ldc,
                       long long strideA, long long strideB, long long strideC) {
    if (!A || !Bt || !C || M <= 0 || N <= 0 || K <= 0 || batch <= 0 || M % BM || N % BN || K % BK || ldc < N ||
        ((uintptr_t)A & 15) || ((uintptr_t)Bt & 15) || strideA % 1024 || strideB % 1024 ||
        (batch > 1 && (strideA < (long long)M * K || strideB < (long long)N * K || strideC < (long long)M * ldc)))
        return "unsupported shape";
    if ((long long)(M / BM) * (N / BN) * batch > (1ll << 30)) return "grid too large";
    return nullptr;
}

template <int MODE>
int launch_gemm(oz_dev* dev, const int8_t* A, const int8_t* Bt, void* C, int M, int N, int K, int batch, int ldc,
                long long strideA, long long strideB, long long strideC, const oz2::DigitConsts& dc) {
    const int tiles_m = M / BM, tiles_n = N / BN;
    const long long tiles = (long long)tiles_m * tiles_n * batch;
    // 1/8 more workgroups than tiles (at least one more per XCD): the XCDs that run ahead take more of
    // the pool's items, the others' spare workgroups find it empty (TilePool). The pool is the last
    // sixteenth of every XCD's share; Scheme I's diagonals differ up to p-fold in length and leave
    // the XCDs further apart, so theirs is an eighth (C2: 60.8 against 60.0 TFLOP/s). A launch of
    // at most one tile per CU runs in one wave with nothing to even out: no pool, no spare
    // workgroups (these would start only when the first tiles end, and lengthen the launch).
    const bool one_wave = dev->cus > 0 && tiles <= dev->cus;
    const int first = one_wave ? (int)tiles : TilePool::first_of((int)tiles, MODE == DIAG ? 8 : 16);
    const unsigned grid = one_wave ? (unsigned)tiles : (unsigned)(tiles + std::max<long long>(tiles / 8, 8));
    // K/64 even: every tile has an even number of K steps (DIAG: (d+1) K/64), no tail step
    if ((K / BK) % 2 == 0)
        oz::launch_product(dev, gemm_i8_kernel<MODE, true>, dim3(grid), dim3(THREADS), A, Bt, C, K, ldc, strideA,
                           strideB, strideC, tiles_m, tiles_n, batch, dc, dev->queue, first);
    else
        oz::launch_product(dev, gemm_i8_kernel<MODE, false>, dim3(grid), dim3(THREADS), A, Bt, C, K, ldc, strideA,
                           strideB, strideC, tiles_m, tiles_n, batch, dc, dev->queue, first);
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

// A18 (products + composition): the digit products of the FP8 route on the CDNA4 FP8 matrix cores.
//
// Semantics (reference ozaki2.cpp:228-285 run_digit_modulus and issue_digit_chunk, compose.cpp:115-153,
// split.hpp:541-661): output o of modulus s is the sum of npairs digit products over the full K,
// P_o = sum_t A_{a[t]} B_{b[t]}^T, which the reference obtains by concatenating the planes along K;
// every P_o is an exact integer of at most 2^24 in magnitude (the planner's concatenation bound), so
// FP32 accumulation is exact and the order of the sums does not matter. The reference then composes the residue
// D_s == sum_o c_o P_o (mod m_s) in FP32 (ModRound first, or a 2^12 split of P_o). Here the epilogue
// reduces P_o exactly: w_o = (c_o y_s mod m_s) * (P_o mod m_s) mod m_s, so that the terms of modulus
// s add up to D_s * y_s (mod m_s), the CRT digit of D_s; the reconstruction sums w_o * Q_s
// directly. The residue classes, and therefore the exact C', are the reference's.
//
// MI355X design: the pipeline of the int8 kernel (oz_gemm.hip): OZ_BLOCK operands copied straight
// into a 4-stage LDS ring by lds_copy_block (wave-uniform SGPR addresses), one barrier per 64-byte
// K step, 256 x 256 tile per workgroup and 128 x 128 per wave, tiles mapped so that the XCDs sweep
// the outputs in step (tile_of_lockstep), tile and output indices kept in SGPRs. The instruction
// is v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3): 4 x 4 of them per wave and K step, each taking a
// 32-row operand (two consecutive blocks) whose 64 K-bytes per row are the lane's two 16-byte
// chunks. Fragments are double-buffered across steps (X: this step, Y: the next, read while X's
// MFMAs run). The K steps of a tile run over its pairs one after another (the concatenation along
// K); the load side follows them with running offsets (no division on the way). The epilogue
// stages the sums through LDS and leaves as 16-byte row stores.
#include "oz2_modular.hpp"
#include "oz_gemm_common.hpp"
#include "oz_internal.hpp"

namespace {

using namespace ozg;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct GroupArgs {
    struct G {
        unsigned char a[4], b[4];
        uint32_t np_m;  // npairs << 16 | m
        uint32_t coef;
    } g[OZ2_MAXOUT];
};

constexpr int LOADS = LOADS_A + LOADS_B;  // global->LDS loads per wave per K step

__device__ __forceinline__ v16f mfma_f8(const v4i& alo, const v4i& ahi, const v4i& blo, const v4i& bhi,
                                        const v16f& c) {
    // format codes 0, 0: both operands e4m3; zero scale operands select the unscaled instruction
    const v8i a = __builtin_shufflevector(alo, ahi, 0, 1, 2, 3, 4, 5, 6, 7);
    const v8i b = __builtin_shufflevector(blo, bhi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// KIND 0: int32 sums P_o. KIND 1: uint16 CRT terms w_o. EVEN: K/64 is even, so every tile has an
// even number of K steps (npairs K/64) and the loop needs no tail step.
template <int KIND, bool EVEN>
__global__ void __launch_bounds__(THREADS) gemm_f8_groups_kernel(const uint8_t* __restrict__ A,
                                                                 const uint8_t* __restrict__ Bt, void* __restrict__ out,
                                                                 int K, int ldo, long long sA, long long sB,
                                                                 long long sO, int tiles_m, int tiles_n, int nout,
                                                                 GroupArgs ga) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int o, tm, tn;
    tile_of_lockstep(blockIdx.x, tiles_m, tiles_n, nout, o, tm, tn);
    // wave-uniform: kept in SGPRs (the map divides on the VALU), so the output's constants come in
    // by scalar loads and every load address below stays on the SALU
    o = __builtin_amdgcn_readfirstlane(o);
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    const GroupArgs::G g = ga.g[o];
    const int npairs = (int)(g.np_m >> 16);
    const int nk = K / BK;            // blocks per 16-row band
    const int nst = npairs * nk;      // K steps of this tile: the pairs' K ranges one after another
    const long long band = (long long)nk * 1024;
    const uint8_t* Ab = A + (long long)tm * 16 * band;
    const uint8_t* Bb = Bt + (long long)tn * 16 * band;
    const unsigned lane16 = 16u * lane;
    // The K step being loaded is block lk of pair li: A plane a[li] and B plane b[li], byte offsets
    // oA = a[li] sA + 1024 lk and oB = b[li] sB + 1024 lk from the tile's bands. The bases of the
    // pairs still to come wait in (nA1..nA3, nB1..nB3) and move up when a pair ends; lcount counts
    // the steps loaded and stops at the last one (past the end the last step is loaded again, so
    // every step issues the same loads and the wait counts never change). Selects only: no
    // division, no indexing, all on the SALU.
    long long oA = g.a[0] * sA, nA1 = g.a[1] * sA, nA2 = g.a[2] * sA, nA3 = g.a[3] * sA;
    long long oB = g.b[0] * sB, nB1 = g.b[1] * sB, nB2 = g.b[2] * sB, nB3 = g.b[3] * sB;
    int lk = 0, lcount = 0;
    auto next_stage = [&]() {
        const int adv = lcount < nst - 1;
        lcount += adv;
        lk += adv;
        oA += adv ? 1024 : 0;
        oB += adv ? 1024 : 0;
        const int wrap = lk == nk;
        lk = wrap ? 0 : lk;
        oA = wrap ? nA1 : oA;
        nA1 = wrap ? nA2 : nA1;
        nA2 = wrap ? nA3 : nA2;
        oB = wrap ? nB1 : oB;
        nB1 = wrap ? nB2 : nB1;
        nB2 = wrap ? nB3 : nB2;
    };
    // Load j (0..3) of this wave for A (issue) or B (issueB): the block of band q = 4 j + wave, rows
    // 16 q.. of the 256 x 64 stage, to byte 1024 q of the operand's half of stage buffer buf.
    auto issue = [&](int buf, int j) {
        const int q = 4 * j + wave, bnd = q & 15, kb = q >> 4;
        lds_copy_block(Ab + ((long long)bnd * band + oA + (long long)kb * 1024),
                       lds + buf * STAGE + (kb * 16 + bnd) * 1024, lane16);
    };
    auto issueB = [&](int buf, int j) {
        const int q = 4 * j + wave, bnd = q & 15, kb = q >> 4;
        lds_copy_block(Bb + ((long long)bnd * band + oB + (long long)kb * 1024),
                       lds + buf * STAGE + STAGE_A + (kb * 16 + bnd) * 1024, lane16);
    };
    const int wm = wave >> 1, wn = wave & 1;
    // Fragment reads: a 32 x 64 operand of the MFMA is two consecutive blocks; lane l takes row
    // fr = l%32 (byte 64 fr of the pair of blocks) and the logical chunks l/32 (lo) and 2 + l/32
    // (hi), stored at chunk positions c ^ f(fr); hi's position is lo's with bit 1 flipped.
    const int fr = lane & 31;
    const int foff = 64 * fr + 16 * ((lane >> 5) ^ (((fr >> 1) ^ (fr >> 2)) & 3));
    auto rd = [&](int buf, int op, int i, int h) -> v4i {
        const int base = buf * STAGE + op * STAGE_A + ((op ? wn : wm) * 128 + 32 * i) * BK;
        return *reinterpret_cast<const v4i*>(lds + base + (foff ^ (32 * h)));
    };
    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0.0f;

#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
        for (int j = 0; j < LOADS_A; j++) {
            issue(s, j);
            issueB(s, j);
        }
        next_stage();
    }
    v4i fal[4], fah[4], fbl[4], fbh[4], gal[4], gah[4], gbl[4], gbh[4];
    wait_vmcnt<LOADS * (NS - 1)>();
    stage_barrier();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        fal[i] = rd(0, 0, i, 0);
        fah[i] = rd(0, 0, i, 1);
        fbl[i] = rd(0, 1, i, 0);
        fbh[i] = rd(0, 1, i, 1);
    }

    // One K step: 16 MFMAs on X; at every even MFMA one fragment of Y (both halves) is read from
    // stage buffer rbuf, in the order a0, b0..b3, a1..a3 (what the next step's first MFMAs need);
    // at every odd one a load of the stage to come goes to buffer lbuf.
    auto substep = [&](v4i* xal, v4i* xah, v4i* xbl, v4i* xbh, v4i* yal, v4i* yah, v4i* ybl, v4i* ybh, int rbuf,
                       int lbuf) {
#pragma unroll
        for (int g2 = 0; g2 < 16; g2++) {
            const int i = g2 >> 2, j = g2 & 3;
            acc[i][j] = mfma_f8(xal[i], xah[i], xbl[j], xbh[j], acc[i][j]);
            const int t = g2 >> 1;
            if ((g2 & 1) == 0) {
                if (t == 0) {
                    yal[0] = rd(rbuf, 0, 0, 0);
                    yah[0] = rd(rbuf, 0, 0, 1);
                } else if (t <= 4) {
                    ybl[t - 1] = rd(rbuf, 1, t - 1, 0);
                    ybh[t - 1] = rd(rbuf, 1, t - 1, 1);
                } else {
                    yal[t - 4] = rd(rbuf, 0, t - 4, 0);
                    yah[t - 4] = rd(rbuf, 0, t - 4, 1);
                }
            } else {
                if (t & 1) issueB(lbuf, t >> 1);
                else issue(lbuf, t >> 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // K step kt: wait until stage kt+1 has landed and this wave's reads of stage kt (into X) are
    // complete, then the barrier: every wave is done with stage kt's buffer, which is refilled with
    // stage kt+NS while the MFMAs run on X and Y reads stage kt+1. Two steps per trip (X and Y swap).
    int kt = 0;
    for (; kt + 1 < nst; kt += 2) {
        wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
        stage_barrier();
        substep(fal, fah, fbl, fbh, gal, gah, gbl, gbh, (kt + 1) % NS, kt % NS);
        next_stage();
        wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
        stage_barrier();
        substep(gal, gah, gbl, gbh, fal, fah, fbl, fbh, (kt + 2) % NS, (kt + 1) % NS);
        next_stage();
    }
    if constexpr (!EVEN) {
        if (kt < nst) {
            wait_vmcnt_lgkm0<LOADS * (NS - 2)>();
            stage_barrier();
            substep(fal, fah, fbl, fbh, gal, gah, gbl, gbh, (kt + 1) % NS, kt % NS);
        }
    }
    wait_vmcnt<0>();  // drain the clamped tail loads before the ring is reused

    // Epilogue through LDS: the accumulators are only stored (arithmetic on them would make the
    // register allocator move them out of the AGPRs inside the main loop). Each wave owns 32 KB of
    // the free ring and writes its 128 x 128 sums in two rounds of 64 rows, row-major, the two
    // 32-column halves of a row swapped when bit 2 of the row is set (so the two 32-lane halves of
    // a write hit different banks). Every lane then reads 8 consecutive sums and stores them as
    // one 16-byte chunk (uint16 terms) or two (int32 sums).
    __syncthreads();
    float* tile = reinterpret_cast<float*>(lds) + wave * (64 * 128);
    const long long c0 = (long long)o * sO + (long long)(tm * BM + wm * 128) * ldo + tn * BN + wn * 128;
    const uint32_t mi = g.np_m & 0xFFFFu;
    const double md = (double)mi, cfr = (double)g.coef / md;
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int ii = 0; ii < 2; ii++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int row = 32 * ii + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);  // bit 2 = lane >> 5
                    tile[row * 128 + ((32 * j + (lane & 31)) ^ (32 * (lane >> 5)))] = acc[2 * h + ii][j][q];
                }
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int e = 64 * t + lane, row = e >> 4, cg = e & 15;
            const float* src = tile + row * 128 + ((8 * cg) ^ (32 * ((row >> 2) & 1)));
            const v4f v0 = *reinterpret_cast<const v4f*>(src), v1 = *reinterpret_cast<const v4f*>(src + 4);
            const long long at = c0 + (long long)(64 * h + row) * ldo + 8 * cg;
            if constexpr (KIND == 1) {
                // |P_o| < 2^24 and m <= 2401: |P_o| m < 2^36, within mod_mul_f64's range
                const float s[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                uint32_t w[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    w[k] = oz2::mod_mul_f64((double)s[2 * k], cfr, md) |
                           oz2::mod_mul_f64((double)s[2 * k + 1], cfr, md) << 16;
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + at) = uint4{w[0], w[1], w[2], w[3]};
            } else {
                int32_t* d = static_cast<int32_t*>(out) + at;
                *reinterpret_cast<v4i*>(d) = v4i{(int32_t)v0[0], (int32_t)v0[1], (int32_t)v0[2], (int32_t)v0[3]};
                *reinterpret_cast<v4i*>(d + 4) = v4i{(int32_t)v1[0], (int32_t)v1[1], (int32_t)v1[2], (int32_t)v1[3]};
            }
        }
    }
}

}  // namespace

extern "C" int oz2_gemm_groups_f8(oz_dev* dev, const uint8_t* A, const uint8_t* Bt, void* out, int M, int N, int K,
                                  const oz2_groups_dev* gd, int out_kind, int ldo, long long strideA, long long strideB,
                                  long long strideO) {
    if (int st = oz::use(dev)) return st;
    if (!A || !Bt || !out || !gd || M <= 0 || N <= 0 || K <= 0 || M % BM || N % BN || K % BK || ldo < N ||
        (out_kind != 0 && out_kind != 1) || gd->nout < 1 || gd->nout > OZ2_MAXOUT || gd->nplanes < 1 ||
        gd->nplanes > OZ2_MAXPLANES || ((uintptr_t)A & 15) || ((uintptr_t)Bt & 15) || strideA % 1024 ||
        strideB % 1024 || strideA < (long long)M * K || strideB < (long long)N * K ||
        (gd->nout > 1 && strideO < (long long)M * ldo))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_groups_f8: unsupported shape (M=%d N=%d K=%d nout=%d)", M, N, K,
                        gd ? gd->nout : 0);
    if (out_kind == 1 && (ldo % 8 || strideO % 8 || ((uintptr_t)out & 15)))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_groups_f8: uint16 terms need 16-byte aligned rows and planes");
    if (out_kind == 0 && (ldo % 4 || strideO % 4 || ((uintptr_t)out & 15)))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_groups_f8: int32 sums need 16-byte aligned rows and planes");
    if ((long long)(M / BM) * (N / BN) * gd->nout > 0x7FFFFFFFll)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_groups_f8: grid too large");
    GroupArgs ga{};
    for (int o = 0; o < gd->nout; o++) {
        const oz2_group_dev& g = gd->g[o];
        if (g.npairs < 1 || g.npairs > 4 || g.m < 2 || g.m > 2401 || g.coef >= g.m)
            return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_groups_f8: output %d malformed", o);
        for (int t = 0; t < g.npairs; t++) {
            if (g.a[t] >= gd->nplanes || g.b[t] >= gd->nplanes)
                return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_groups_f8: output %d names a plane beyond %d", o, gd->nplanes);
            ga.g[o].a[t] = g.a[t];
            ga.g[o].b[t] = g.b[t];
        }
        // FP32 accumulation is exact while every partial sum is an integer of at most 2^24 in magnitude,
        // which |P_o| <= bound <= 2^24 ensures; the epilogue reduces P_o in FP64 (the reference keeps
        // bound + m <= 2^24 for its FP32 composition, which this epilogue replaces)
        if (!(g.bound >= 0.0f) || (double)g.bound > 16777216.0)
            return oz::fail(dev, OZ_ERR_RANGE, "oz2_gemm_groups_f8: output %d can reach %g, beyond exact FP32", o,
                            (double)g.bound);
        ga.g[o].np_m = ((uint32_t)g.npairs << 16) | g.m;
        ga.g[o].coef = g.coef;
    }
    const int tiles_m = M / BM, tiles_n = N / BN;
    const unsigned grid = (unsigned)((long long)tiles_m * tiles_n * gd->nout);
    const int nout = gd->nout;
#define OZ_F8_LAUNCH(KIND, EVEN)                                                                                      \
    oz::launch_product(dev, gemm_f8_groups_kernel<KIND, EVEN>, dim3(grid), dim3(THREADS), A, Bt, out, K, ldo,     \
                       strideA, strideB, strideO, tiles_m, tiles_n, nout, ga)
    const bool even = (K / BK) % 2 == 0;
    if (out_kind == 1) {
        if (even) OZ_F8_LAUNCH(1, true);
        else OZ_F8_LAUNCH(1, false);
    } else {
        if (even) OZ_F8_LAUNCH(0, true);
        else OZ_F8_LAUNCH(0, false);
    }
#undef OZ_F8_LAUNCH
    return oz::launch_check(dev, "gemm_f8_groups_kernel");
}

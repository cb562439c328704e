// A18 (products + composition): the digit products of the FP8 route on the CDNA4 FP8 matrix cores.
//
// Semantics (reference ozaki2.cpp:228-285 run_digit_modulus and issue_digit_chunk, compose.cpp:115-153,
// split.hpp:541-661): output o of modulus s is the sum of npairs digit products over the full K,
// P_o = sum_t A_{a[t]} B_{b[t]}^T, which the reference obtains by concatenating the planes along K;
// every P_o is an exact integer below 2^24 (the planner's concatenation bound), so FP32 accumulation
// is exact and the order of the sums does not matter. The reference then composes the residue
// D_s == sum_o c_o P_o (mod m_s) in FP32 (ModRound first, or a 2^12 split of P_o). Here the epilogue
// reduces P_o exactly: w_o = (c_o y_s mod m_s) * (P_o mod m_s) mod m_s, so that the terms of modulus
// s add up to D_s * y_s (mod m_s), the CRT digit of D_s; the reconstruction sums w_o * Q_s
// directly. The residue classes, and therefore the exact C', are the reference's.
//
// MI355X design: the pipeline of the int8 kernel (oz_gemm.hip; OZ_BLOCK operands copied straight
// into a 4-stage LDS ring, XCD-aware tile map, 256 x 256 tile per workgroup, 128 x 128 per wave)
// with v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3): one instruction takes the whole 64-byte K step of
// a lane (the two 16-byte fragments the int8 kernel feeds to two instructions), so a stage is one
// substep of 16 MFMAs per wave. Fragments are double-buffered across stages (X: this stage, Y: the
// next, read while X's MFMAs run). A workgroup computes one output of one tile; the outputs with
// more pairs are dispatched first. The uint16 terms leave through LDS as 16-byte row stores.
#include "oz2_modular.hpp"
#include "oz_gemm_common.hpp"
#include "oz_internal.hpp"

namespace {

using namespace ozg;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct GroupArgs {
    struct G {
        unsigned char a[4], b[4];
        uint32_t np_m;  // npairs << 16 | m
        uint32_t coef, magic;
    } g[OZ2_MAXOUT];
};

constexpr int TS = 272;                     // epilogue row stride in bytes (128 uint16 + 16 bytes)
constexpr int EPI = 4 * 128 * TS;           // epilogue tiles of the 4 waves
constexpr int LDS_BYTES = EPI > NS * STAGE ? EPI : NS * STAGE;

__device__ __forceinline__ v8i frag(const uint8_t* p0, const uint8_t* p1) {
    const v4i lo = *reinterpret_cast<const v4i*>(p0), hi = *reinterpret_cast<const v4i*>(p1);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ v16f mfma_f8(const v8i& a, const v8i& b, const v16f& c) {
    // format codes 0, 0: both operands e4m3; zero scale operands select the unscaled instruction
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// KIND 0: int32 sums P_o. KIND 1: uint16 CRT terms w_o.
template <int KIND>
__global__ void __launch_bounds__(THREADS) gemm_f8_groups_kernel(const uint8_t* __restrict__ A,
                                                                 const uint8_t* __restrict__ Bt, void* __restrict__ out,
                                                                 int K, int ldo, long long sA, long long sB,
                                                                 long long sO, int tiles_m, int tiles_n, GroupArgs ga) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int per = tiles_m * tiles_n, o = blockIdx.x / per;
    int unused, tm, tn;
    tile_of(blockIdx.x - o * per, tiles_m, tiles_n, 1, unused, tm, tn);
    const int npairs = (int)(ga.g[o].np_m >> 16);
    const int nk = K / BK;
    const int nsteps = npairs * nk;
    const long long band = (long long)nk * 1024;
    const uint8_t* Ab = A + (long long)tm * (BM / 16) * band + 16 * lane;
    const uint8_t* Bb = Bt + (long long)tn * (BN / 16) * band + 16 * lane;
    auto step_off = [&](int u, long long& oa, long long& ob) {
        const int i = u / nk, kt = u - i * nk;
        oa = ga.g[o].a[i] * sA + (long long)kt * 1024;
        ob = ga.g[o].b[i] * sB + (long long)kt * 1024;
    };
    auto issue = [&](int kstep, int buf) {
        long long oa, ob;
        step_off(kstep, oa, ob);
        uint8_t* sa = lds + buf * STAGE;
#pragma unroll
        for (int i = 0; i < LOADS_A; i++)
            __builtin_amdgcn_global_load_lds(Ab + (4 * i + wave) * band + oa, (lds_void*)(sa + 1024 * (4 * i + wave)),
                                             16, 0, 0);
#pragma unroll
        for (int i = 0; i < LOADS_B; i++)
            __builtin_amdgcn_global_load_lds(Bb + (4 * i + wave) * band + ob,
                                             (lds_void*)(sa + STAGE_A + 1024 * (4 * i + wave)), 16, 0, 0);
    };

    const int wm = wave >> 1, wn = wave & 1;
    int offA[2], offB[2];
    fragment_offsets(lane, wm, wn, offA, offB);

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0.0f;

    // Loads run NS stages ahead (the tail re-loads the last valid stage, so the wait counts never
    // change). At the top of step kt the wave waits until stage kt+1 has landed and its own reads
    // of stage kt (into X) are complete, then the barrier: every wave is done with stage kt's
    // buffer, which is refilled with stage kt+NS while the MFMAs of X run, and Y reads stage kt+1.
#pragma unroll
    for (int s = 0; s < NS; s++) issue(min(s, nsteps - 1), s);
    v8i xa[4], xb[4], ya[4], yb[4];
    wait_vmcnt<(LOADS_A + LOADS_B) * (NS - 1)>();
    stage_barrier();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xa[i] = frag(lds + offA[0] + i * 32 * BK, lds + offA[1] + i * 32 * BK);
        xb[i] = frag(lds + offB[0] + i * 32 * BK, lds + offB[1] + i * 32 * BK);
    }

#define OZ_F8_STEP(XA, XB, YA, YB, KT)                                                                            \
    do {                                                                                                          \
        const int kt_ = (KT);                                                                                     \
        wait_vmcnt_lgkm0<(LOADS_A + LOADS_B) * (NS - 2)>();                                                       \
        stage_barrier();                                                                                          \
        const uint8_t* nxt = lds + ((kt_ + 1) % NS) * STAGE;                                                      \
        uint8_t* sa = lds + (kt_ % NS) * STAGE;                                                                   \
        long long oa, ob;                                                                                         \
        step_off(min(kt_ + NS, nsteps - 1), oa, ob);                                                              \
        _Pragma("unroll") for (int g = 0; g < 16; g++) {                                                          \
            acc[g >> 2][g & 3] = mfma_f8(XA[g >> 2], XB[g & 3], acc[g >> 2][g & 3]);                               \
            if (g < 4)                                                                                            \
                YA[g] = frag(nxt + offA[0] + g * 32 * BK, nxt + offA[1] + g * 32 * BK);                            \
            else if (g < 8)                                                                                       \
                YB[g - 4] = frag(nxt + offB[0] + (g - 4) * 32 * BK, nxt + offB[1] + (g - 4) * 32 * BK);            \
            else if (g < 12)                                                                                      \
                __builtin_amdgcn_global_load_lds(Ab + (4 * (g - 8) + wave) * band + oa,                            \
                                                 (lds_void*)(sa + 1024 * (4 * (g - 8) + wave)), 16, 0, 0);         \
            else                                                                                                  \
                __builtin_amdgcn_global_load_lds(Bb + (4 * (g - 12) + wave) * band + ob,                           \
                                                 (lds_void*)(sa + STAGE_A + 1024 * (4 * (g - 12) + wave)), 16, 0, \
                                                 0);                                                              \
            __builtin_amdgcn_sched_barrier(0);                                                                    \
        }                                                                                                         \
    } while (0)

    int kt = 0;
    for (; kt + 1 < nsteps; kt += 2) {
        OZ_F8_STEP(xa, xb, ya, yb, kt);
        OZ_F8_STEP(ya, yb, xa, xb, kt + 1);
    }
    if (kt < nsteps) OZ_F8_STEP(xa, xb, ya, yb, kt);
#undef OZ_F8_STEP
    wait_vmcnt<0>();  // drain the clamped tail loads before the workgroup ends

    const long long c0 = (long long)o * sO + (long long)(tm * BM + wm * 128) * ldo + tn * BN + wn * 128;
    if constexpr (KIND == 1) {
        __syncthreads();  // every wave has left the main loop: the ring is free
        uint8_t* tile = lds + wave * (128 * TS);
        const uint32_t m = ga.g[o].np_m & 0xFFFFu, coef = ga.g[o].coef, mg = ga.g[o].magic;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    *reinterpret_cast<uint16_t*>(tile + (32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3)) * TS +
                                                 2 * (32 * j + (lane & 31))) =
                        (uint16_t)oz2::crt_digit((int32_t)acc[i][j][q], m, coef, mg);
        uint16_t* Ob = static_cast<uint16_t*>(out) + c0;
#pragma unroll
        for (int t = 0; t < 32; t++) {  // 128 rows x 16 chunks of 16 bytes
            const int c = 64 * t + lane, r = c >> 4, x = 16 * (c & 15);
            *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(Ob + (long long)r * ldo) + x) =
                *reinterpret_cast<const uint4*>(tile + r * TS + x);
        }
    } else {
        int32_t* Ob = static_cast<int32_t*>(out) + c0;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    Ob[(long long)(32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3)) * ldo + 32 * j + (lane & 31)] =
                        (int32_t)acc[i][j][q];
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
        // FP32 accumulation is exact while |P_o| stays below 2^24 (the reference keeps bound + m <= 2^24)
        if (!(g.bound >= 0.0f) || (double)g.bound + g.m > 16777216.0)
            return oz::fail(dev, OZ_ERR_RANGE, "oz2_gemm_groups_f8: output %d can reach %g, beyond exact FP32", o,
                            (double)g.bound);
        ga.g[o].np_m = ((uint32_t)g.npairs << 16) | g.m;
        ga.g[o].coef = g.coef;
        ga.g[o].magic = (uint32_t)(0x100000000ull / g.m);
    }
    const int tiles_m = M / BM, tiles_n = N / BN;
    const unsigned grid = (unsigned)((long long)tiles_m * tiles_n * gd->nout);
    if (out_kind == 1)
        hipLaunchKernelGGL(gemm_f8_groups_kernel<1>, dim3(grid), dim3(THREADS), 0, dev->stream, A, Bt, out, K, ldo,
                           strideA, strideB, strideO, tiles_m, tiles_n, ga);
    else
        hipLaunchKernelGGL(gemm_f8_groups_kernel<0>, dim3(grid), dim3(THREADS), 0, dev->stream, A, Bt, out, K, ldo,
                           strideA, strideB, strideO, tiles_m, tiles_n, ga);
    return oz::launch_check(dev, "gemm_f8_groups_kernel");
}

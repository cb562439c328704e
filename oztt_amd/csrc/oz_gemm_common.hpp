// Shared pieces of the matrix-core product kernels (oz_gemm.hip: int8 x int8 -> int32;
// oz2_gemm_f8.hip: e4m3 x e4m3 -> fp32): the OZ_BLOCK operand stages, the XCD-aware tile map, the
// barrier and wait primitives of the direct global->LDS pipeline.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace ozg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// Workgroup -> (batch, tile row, tile column). Workgroups are dispatched round-robin over the 8
// XCDs (workgroup w runs on XCD w % 8), and each XCD has its own L2. The map gives every XCD one
// contiguous range of the logical tile sequence, and orders that sequence batch-major, then in
// groups of GROUP_M tile rows walked column by column, so the ~32 workgroups an XCD runs at a time
// cover a compact block of tiles and share their A rows and B columns in that L2. It is a
// bijection for any workgroup count.
constexpr int XCDS = 8, GROUP_M = 4;
__device__ __forceinline__ void tile_of(int w, int tiles_m, int tiles_n, int nbatch, int& batch, int& tm, int& tn) {
    const int total = tiles_m * tiles_n * nbatch;
    const int q = total / XCDS, r = total % XCDS;
    const int x = w % XCDS, j = w / XCDS;
    const int t = x * q + min(x, r) + j;  // logical index
    const int per_batch = tiles_m * tiles_n;
    batch = t / per_batch;
    const int u = t % per_batch;
    const int group = u / (GROUP_M * tiles_n);
    const int first_m = group * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int v = u % (GROUP_M * tiles_n);
    tm = first_m + v % gm;
    tn = v / gm;
}

// Workgroup -> (batch, tile row, tile column) with every XCD on the same batch at the same time.
// When the tile count P of a batch is a multiple of 8, batch b's tiles, in the grouped order of
// tile_of, are cut into 8 contiguous chunks of q = P/8 and XCD x takes chunk x: its j-th workgroup
// (w = 8j + x) gets tile j % q of its chunk of batch j / q. The XCDs then sweep the batches in
// step, so the operands in flight are those of one or two batches (at C3 size 2 x 64 MiB of int8
// planes per batch), which the 256 MB Infinity Cache holds; with tile_of's ranges the 8 XCDs would
// run 8 different batches and their L2 misses would go to HBM. Within a chunk the ~32 workgroups
// an XCD runs at a time still cover a compact GROUP_M x 8 block of tiles. Otherwise (P % 8 != 0)
// this is tile_of. A bijection for any workgroup count of P * nbatch.
__device__ __forceinline__ void tile_of_lockstep(int w, int tiles_m, int tiles_n, int nbatch, int& batch, int& tm,
                                                 int& tn) {
    const int P = tiles_m * tiles_n;
    if (P % XCDS) {
        tile_of(w, tiles_m, tiles_n, nbatch, batch, tm, tn);
        return;
    }
    const int q = P / XCDS, x = w % XCDS, j = w / XCDS;
    batch = j / q;
    const int u = x * q + (j - batch * q);
    const int group = u / (GROUP_M * tiles_n);
    const int first_m = group * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int v = u % (GROUP_M * tiles_n);
    tm = first_m + v % gm;
    tn = v / gm;
}

// Direct copy of one 1 KB block from global memory to LDS: lane l reads the 16 bytes at
// gbase + voff(l) and they land at LDS byte lbase + 16 l (global_load_lds_dwordx4). gbase and
// lbase are wave-uniform, so the address stays in SGPRs (one per-lane offset register serves every
// load). M0 carries the LDS base; the compiled kernels use M0 for nothing else, which
// tests/test_gemm_asm.py checks on the generated code. The load is counted by vmcnt like any
// other vector memory load; its consumers wait with wait_vmcnt.
__device__ __forceinline__ void lds_copy_block(const void* gbase, void* lbase, unsigned voff) {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const unsigned l = (unsigned)(uintptr_t)(lds_u8*)lbase;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(voff), "s"(gbase) : "memory");
}

// Workgroup barrier without the memory fences of __syncthreads(): those would wait for every
// outstanding load, including the direct-to-LDS loads of the stages still in flight. Each wave
// first waits (vmcnt) for its own loads of the stage about to be read, so after the barrier the
// whole stage is in LDS; the empty asm statements keep the compiler from moving LDS accesses
// across the barrier.
__device__ __forceinline__ void stage_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// s_waitcnt with vmcnt = N and the other counters left alone (gfx9 encoding of simm16: vmcnt
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// vmcnt = N and lgkmcnt = 0 (this wave's LDS reads complete).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

constexpr int BM = 256, BN = 256, BK = 64, NS = 4, THREADS = 256;
constexpr int STAGE_A = BM * BK, STAGE_B = BN * BK, STAGE = STAGE_A + STAGE_B;  // bytes
constexpr int LOADS_A = STAGE_A / 16 / THREADS, LOADS_B = STAGE_B / 16 / THREADS;  // per thread per stage
static_assert(LOADS_A == 4 && LOADS_B == 4, "each thread moves 4+4 chunks of 16 bytes per stage");


// Fragment offsets inside a stage for lane `lane` of wave (wm, wn): row r = lane%32 of each 32-row
// block, logical chunk c = 2*ks + lane/32 (ks = 0, 1: the two 32-byte K halves of the 64-byte step),
// stored at chunk position c ^ f(r) (f sees bits 1..3 of r only, so r%16 or r gives the same).
__device__ __forceinline__ void fragment_offsets(int lane, int wm, int wn, int* offA, int* offB) {
    const int frow = lane & 31;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const int pos = 16 * ((2 * ks + (lane >> 5)) ^ (((frow >> 1) ^ (frow >> 2)) & 3));
        offA[ks] = (wm * 128 + frow) * BK + pos;
        offB[ks] = STAGE_A + (wn * 128 + frow) * BK + pos;
    }
}

}  // namespace ozg

// The matrix cores' throughput ceiling on this GPU, as a yardstick for the product kernels'
// rooflines: each kernel issues one MFMA form back to back on operands held in registers (no
// memory traffic, no waits), with random operand bytes, for a 128 x 128 accumulator tile per wave
// (the product kernels' wave tile). Under load the MI355X runs at the clock its power limit
// allows, so this measures what the matrix cores deliver at that clock rather than the nominal
// peak. Prints one JSON line per form: {"form", "ms", "tops"}.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                                              \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::fprintf(stderr, "mfma_ceiling: %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                                     \
        }                                                                                     \
    } while (0)

constexpr int kWords = 1 << 20;  // operand words read once per thread (index masked into range)

__global__ void __launch_bounds__(256) f8_32x32x64(const int* __restrict__ src, float* __restrict__ dst, int iters) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    v8i a[4], b[4];
    for (int i = 0; i < 4; i++)
        for (int q = 0; q < 8; q++) {
            a[i][q] = src[(t * 64 + i * 8 + q) & (kWords - 1)];
            b[i][q] = src[(t * 64 + 32 + i * 8 + q) & (kWords - 1)];
        }
    v16f acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int g = 0; g < 16; g++)
            acc[g >> 2][g & 3] =
                __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[g >> 2], b[g & 3], acc[g >> 2][g & 3], 0, 0, 0, 0, 0, 0);
    }
    float s = 0;
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int q = 0; q < 16; q++) s += acc[i][j][q];
    dst[t] = s;
}

__global__ void __launch_bounds__(256) f8_16x16x128(const int* __restrict__ src, float* __restrict__ dst, int iters) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    v8i a[8], b[8];
    for (int i = 0; i < 8; i++)
        for (int q = 0; q < 8; q++) {
            a[i][q] = src[(t * 128 + i * 8 + q) & (kWords - 1)];
            b[i][q] = src[(t * 128 + 64 + i * 8 + q) & (kWords - 1)];
        }
    v4f acc[8][8];
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 8; j++) acc[i][j] = v4f{0, 0, 0, 0};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int g = 0; g < 64; g++)
            acc[g >> 3][g & 7] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[g >> 3], b[g & 7],
                                                                                 acc[g >> 3][g & 7], 0, 0, 0, 0, 0, 0);
    }
    float s = 0;
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 8; j++)
            for (int q = 0; q < 4; q++) s += acc[i][j][q];
    dst[t] = s;
}

__global__ void __launch_bounds__(256) i8_32x32x32(const int* __restrict__ src, float* __restrict__ dst, int iters) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    v4i a[4], b[4];
    for (int i = 0; i < 4; i++)
        for (int q = 0; q < 4; q++) {
            a[i][q] = src[(t * 32 + i * 4 + q) & (kWords - 1)];
            b[i][q] = src[(t * 32 + 16 + i * 4 + q) & (kWords - 1)];
        }
    v16i acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int g = 0; g < 16; g++)
            acc[g >> 2][g & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[g >> 2], b[g & 3], acc[g >> 2][g & 3], 0, 0, 0);
    }
    float s = 0;
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int q = 0; q < 16; q++) s += (float)acc[i][j][q];
    dst[t] = s;
}

__global__ void __launch_bounds__(256) i8_16x16x64(const int* __restrict__ src, float* __restrict__ dst, int iters) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    v4i a[8], b[8];
    for (int i = 0; i < 8; i++)
        for (int q = 0; q < 4; q++) {
            a[i][q] = src[(t * 64 + i * 4 + q) & (kWords - 1)];
            b[i][q] = src[(t * 64 + 32 + i * 4 + q) & (kWords - 1)];
        }
    v4i acc[8][8];
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 8; j++) acc[i][j] = v4i{0, 0, 0, 0};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int g = 0; g < 64; g++)
            acc[g >> 3][g & 7] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[g >> 3], b[g & 7], acc[g >> 3][g & 7], 0, 0, 0);
    }
    float s = 0;
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 8; j++)
            for (int q = 0; q < 4; q++) s += (float)acc[i][j][q];
    dst[t] = s;
}

// Random bytes that are finite e4m3 values (0x7F / 0xFF, NaN in e4m3, are moved by one).
__global__ void fill_random(int* p, int n, unsigned seed) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    unsigned x = (unsigned)i * 2654435761u ^ seed;
    x ^= x >> 13;
    x *= 0x5bd1e995u;
    x ^= x >> 15;
    unsigned r = 0;
    for (int k = 0; k < 4; k++) {
        unsigned b = (x >> (8 * k)) & 0xFFu;
        if ((b & 0x7Fu) == 0x7Fu) b ^= 1u;
        r |= b << (8 * k);
    }
    p[i] = (int)r;
}

}  // namespace

int main() {
    constexpr int grid = 2048, iters = 2000;  // 8 workgroups of 4 waves per CU, one wave per SIMD at a time
    int* src = nullptr;
    float* dst = nullptr;
    CHECK(hipMalloc(&src, sizeof(int) * kWords));
    CHECK(hipMalloc(&dst, sizeof(float) * 256 * grid));
    hipLaunchKernelGGL(fill_random, dim3(kWords / 256), dim3(256), 0, 0, src, kWords, 0x1234u);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    const double tile = 2.0 * 128 * 128;  // operations per unit of K of a wave's tile
    auto run = [&](const char* form, void (*k)(const int*, float*, int), double k_per_iter) {
        for (int w = 0; w < 2; w++) hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, 0, src, dst, iters);
        CHECK(hipGetLastError());
        CHECK(hipDeviceSynchronize());
        CHECK(hipEventRecord(e0, 0));
        hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, 0, src, dst, iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        const double ops = tile * k_per_iter * iters * grid * 4.0;
        std::printf("{\"form\": \"%s\", \"ms\": %.3f, \"tops\": %.1f}\n", form, ms, ops / (ms * 1e-3) / 1e12);
        std::fflush(stdout);
    };
    run("v_mfma_i32_16x16x64_i8", i8_16x16x64, 64);
    run("v_mfma_i32_32x32x32_i8", i8_32x32x32, 32);
    run("v_mfma_f32_32x32x64_f8f6f4", f8_32x32x64, 64);
    run("v_mfma_f32_16x16x128_f8f6f4", f8_16x16x128, 128);
    CHECK(hipFree(src));
    CHECK(hipFree(dst));
    return 0;
}

// Small-modulus arithmetic shared by the product epilogue and the CRT reconstruction of Scheme II.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "oz_hip.h"

namespace oz2 {

// x mod m for 0 <= x < 2^32 and m >= 2, with magic = floor(2^32 / m): q = mulhi(x, magic) is
// floor(x/m) or one less (x (2^32/m - magic) / 2^32 < 1), so one conditional subtraction finishes the
// remainder.
__device__ __forceinline__ uint32_t mod_small(uint32_t x, uint32_t m, uint32_t magic) {
    const uint32_t q = __umulhi(x, magic);
    uint32_t r = x - q * m;
    if (r >= m) r -= m;
    return r;
}

// CRT digit of an exact product c (|c| < 2^31): k = (c mod m) * y mod m in [0, m), y = (M/m)^-1 mod m.
__device__ __forceinline__ uint32_t crt_digit(int32_t c, uint32_t m, uint32_t y, uint32_t magic) {
    uint32_t r = mod_small(c < 0 ? (uint32_t)(-(int64_t)c) : (uint32_t)c, m, magic);
    if (c < 0 && r) r = m - r;
    return mod_small(r * y, m, magic);
}

// A representative of (c * y) mod m in [0, m] (m standing for 0) for integers c, y, m with
// 0 <= y < m and |c| m < 2^50, in four FP64-pipe operations counting the conversion of c
// (v_cvt_f64_i32, v_mul_f64, v_fract_f64, v_fma_f64); yr is y/m to within an ulp.
// t = RN(c yr) lies within |c| 2^-51 of c y/m, so its fractional part f (exact: v_fract_f64 is
// t - floor(t), clamped below 1) lies within delta = |c| 2^-51 of r/m modulo 1, r = (c y) mod m;
// f m is then within delta m < 1/2 of r, or of m when r = 0 and f fell just below 1. The FMA adds
// 2^52, where the spacing of doubles is 1, so its single rounding lands on 2^52 + r (or 2^52 + m),
// whose low 32 bits are r: no conversion back. Every consumer of these values reduces them modulo m
// (the CRT adds k Q_s, and m Q_s = M vanishes modulo M; the FP8 route's terms are summed modulo m),
// so m is as good as 0 and needs no fix-up.
__device__ __forceinline__ uint32_t mod_mul_f64(double c, double yr, double m) {
    const double v = __builtin_fma(__builtin_amdgcn_fract(c * yr), m, 0x1p52);
    return (uint32_t)__builtin_bit_cast(unsigned long long, v);
}

// mod_mul_f64 of 16 values at once, packed as bytes (values below 256: m <= 256) into 4 words, byte
// q of w[k] from c[4k + q]. In stages (all conversions, then all products, ...), so that no FP64
// operation waits on the one just before it: the product kernels run one wave per SIMD, with no
// other wave to cover the latency. Each word takes three byte permutes: the low bytes of d0, d1 and
// of d2, d3 side by side, then the two halves (written as shifts and ors, the compiler makes four
// operations of it).
__device__ __forceinline__ void mod_mul_f64_x16(const int32_t* c, double yr, double m, uint32_t* w) {
    double t[16];
#pragma unroll
    for (int e = 0; e < 16; e++) t[e] = (double)c[e];
#pragma unroll
    for (int e = 0; e < 16; e++) t[e] *= yr;
#pragma unroll
    for (int e = 0; e < 16; e++) t[e] = __builtin_amdgcn_fract(t[e]);
#pragma unroll
    for (int e = 0; e < 16; e++) t[e] = __builtin_fma(t[e], m, 0x1p52);
    uint32_t d[16];
#pragma unroll
    for (int e = 0; e < 16; e++) d[e] = (uint32_t)__builtin_bit_cast(unsigned long long, t[e]);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t lo = __builtin_amdgcn_perm(d[4 * k + 1], d[4 * k], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(d[4 * k + 3], d[4 * k + 2], 0x0c0c0400u);
        w[k] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
}

// Per-modulus constants of the digit epilogue (kernel argument).
struct DigitConsts {
    uint32_t m[OZ2_MAXS], y[OZ2_MAXS];
};

}  // namespace oz2

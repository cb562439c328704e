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

// (c * y) mod m in [0, m) for integers c, y with |c * y| < 2^40 and 2 <= m, in FP64 (one product,
// one floor, one FMA: the FP64 pipes run these at full rate, where the 32-bit integer multiplies of
// crt_digit run at a quarter). rinv = RN(1/m), mi = m as an integer. Exact: x = c*y is an integer
// below 2^53, so x is exact; RN(x * rinv) differs from x/m by less than |x/m| 2^-52 < 2^-12 / m. If
// x/m is not an integer it is at least 1/m away from one, so the floor is exact and the FMA (whose
// exact value, x - q m, is a small integer) gives the remainder; if x/m is an integer the floor is
// x/m or x/m - 1, giving 0 or m. So the FMA's result is an integer in [0, m]: it converts to uint32
// exactly, and min(r, r - m) in unsigned arithmetic maps m to 0 and keeps r < m (r - m wraps above
// it): two integer operations, with no compare, no condition register and no hazard wait. The same
// residue as crt_digit(c, m, y, .) for |c| < 2^31, y < m <= 255.
__device__ __forceinline__ uint32_t mod_mul_f64(double c, double y, double m, double rinv, uint32_t mi) {
    const double x = c * y;
    const uint32_t r = (uint32_t)__builtin_fma(-__builtin_floor(x * rinv), m, x);
    return min(r, r - mi);
}

// Per-modulus constants of the digit epilogue (kernel argument).
struct DigitConsts {
    uint32_t m[OZ2_MAXS], y[OZ2_MAXS];
};

}  // namespace oz2

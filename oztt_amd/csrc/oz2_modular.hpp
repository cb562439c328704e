// Small-modulus arithmetic shared by the product epilogue and the CRT reconstruction of Scheme II.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "oz_hip.h"

namespace oz2 {

// x mod m for 0 <= x < 2^32 and 2 <= m <= 255, with magic = floor(2^32 / m): q = mulhi(x, magic)
// is floor(x/m) or one less, so one conditional subtraction finishes the remainder.
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

// Per-modulus constants of the digit epilogue (kernel argument).
struct DigitConsts {
    uint32_t m[OZ2_MAXS], y[OZ2_MAXS], magic[OZ2_MAXS];
};

}  // namespace oz2

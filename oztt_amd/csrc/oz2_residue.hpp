// Scheme II residues of FP64 operands (steps 2-3 of the splitters in oz2_split.hip and
// oz2_digits.hip): the radix-2^20 digits of A' = x*2^delta and A' mod m, restating the reference's
// binary32 procedure (digits.h:80-112 oz2_make_digits, digits.h:165-179 oz2_residue). Files that
// include this header are compiled with -ffp-contract=off and -fgpu-flush-denormals-to-zero.
#pragma once
#pragma clang fp contract(off)

#include "oz_tf32.hpp"

namespace {

struct SplitConsts {
    float m[OZ2_MAXS];
    float rinv[OZ2_MAXS];
    float c[4][OZ2_MAXS];
};

// Step 2: nd digits, top first.
template <int ND>
__device__ __forceinline__ void make_digits(double x, int32_t d, float* dig) {
    float hi, mid, lo;
    load_triple(x, d, hi, mid, lo);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        if (i > 0) tf_mul_pow2(hi, mid, lo, 1048576.0f);  // tfMulP2 by 2^20
        const float t = __builtin_rintf(hi);
        hi = hi - t;
        dig[i] = t;
    }
}

__device__ __forceinline__ float mod_round(float v, float m, float rinv) {
    const float q = __builtin_rintf(v * rinv);
    return __builtin_fmaf(-q, m, v);  // exact: q*m and v - q*m are integers below 2^24
}

// Step 3 for one modulus: the symmetric residue (|r| <= floor(m/2) + 1) as an FP32 integer.
template <int ND>
__device__ __forceinline__ float residue_f(const float* dig, const SplitConsts& k, int s) {
    const float m = k.m[s], ri = k.rinv[s];
    float acc = dig[ND - 1];
    acc = __builtin_fmaf(mod_round(dig[ND - 2], m, ri), k.c[0][s], acc);
    acc = __builtin_fmaf(mod_round(dig[ND - 3], m, ri), k.c[1][s], acc);
    if (ND >= 4) {
        acc = mod_round(acc, m, ri);
        if (ND >= 5) {
            acc = __builtin_fmaf(mod_round(dig[0], m, ri), k.c[3][s], acc);
            acc = mod_round(acc, m, ri);
        }
        acc = __builtin_fmaf(mod_round(dig[ND - 4], m, ri), k.c[2][s], acc);
    }
    return mod_round(acc, m, ri);
}
template <int ND>
__device__ __forceinline__ int residue(const float* dig, const SplitConsts& k, int s) {
    return (int)residue_f<ND>(dig, k, s);
}

}  // namespace

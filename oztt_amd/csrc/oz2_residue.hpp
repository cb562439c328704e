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
    // INT8 moduli only (oz2_split_int8): byte j of w[s][i] is the symmetric residue of 2^(8 (4i + j))
    // modulo m_s, and `even` is the index of the even modulus of the set (pairwise coprime moduli
    // hold at most one), or -1.
    uint32_t w[OZ2_MAXS][4];
    int even;
    // odd moduli m >= 17 (residue_odd_int): the dot products start at dinit[s], a multiple of m plus
    // (m-1)/2 large enough to make the sum nonnegative; magic[s] = ceil(2^(32 - sh) / m) with
    // sh = 24 - U (below); badd[s] = (128 - (m-1)/2) in every byte. magic[s] = 0 selects the FP32
    // reduction (residue_odd) for smaller moduli.
    int dinit[OZ2_MAXS];
    uint32_t magic[OZ2_MAXS];
    uint32_t badd[OZ2_MAXS];
    int mneg[OZ2_MAXS];  // 2^24 - m
    // The plane lists of the blocked splitter (ResidueGen::run): the odd moduli from 17 up in pairs
    // for the matrix-core dot products (planes pair[g][0], pair[g][1]; a last single modulus is paired
    // with itself), and the odd moduli below 17 (small[0..nsmall)).
    int npair, nsmall;
    int pair[(OZ2_MAXS + 1) / 2][2];
    int small[OZ2_MAXS];
};

// Step 2: nd digits, top first.
template <int ND>
__device__ __forceinline__ void make_digits(double x, int32_t d, float* dig) {
    float hi, mid, lo;
    load_triple(x, d, hi, mid, lo);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        // tfMulP2 by 2^20, its TwoSums taken as FastTwoSums: the order they need holds on these chains
        // too (a digit leaves hi = 0 or a multiple of ulp(old hi) >= 2|mid|; see tf_mul_pow2_fast)
        if (i > 0) tf_mul_pow2_fast(hi, mid, lo, 1048576.0f);
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

namespace {

// ---- Exact residues of A' for odd INT8 moduli ----------------------------------------------
// For an odd modulus the reference's residue is the symmetric residue of A' itself: every step of
// its reduction (steps above) keeps the value congruent to A', and its last MR sees |v| < 2^22, so
// fl(v rinv) lies within |v/m| 2^-23 < 1/(2m) of v/m while v/m is at least 1/(2m) away from a
// half-integer (m odd): the rounding picks the nearest integer, and |r| <= (m-1)/2. Any exact
// computation of that residue therefore gives the reference's value. Here A' is written once per
// element in balanced base 256, A' = sum_j a_j 256^j with bytes a_j in [-128, 127], and per modulus
// v = sum_j a_j w_j with w_j the symmetric residue of 256^j (|w_j| <= 127) takes one signed 4-byte
// dot product per 32-bit word of the digits; |v| <= 16 * 128 * 127 < 2^18, so one FP32 reduction
// (exact: integers below 2^24, and the rounding argument above) gives the residue. An even modulus
// (at most one: the moduli are pairwise coprime) can meet an exact tie at +-m/2, where the reference's
// result depends on its intermediate values, so it keeps the reference's own sequence (residue_f).

// 32-bit words of the balanced base-256 digits of A' (|A'| < 2^(20 ND + 1)).
template <int ND>
constexpr int balanced_words() {
    return ND == 3 ? 2 : (ND == 4 ? 3 : 4);
}

// A' from its nd radix-2^20 digits (exact integers in FP32), then the balanced bytes: adding 0x80 at
// every byte position (with carries) makes every byte b_j = a_j + 128 nonnegative, and b_j ^ 0x80
// is a_j as a two's-complement byte.
template <int ND>
__device__ __forceinline__ void balanced_bytes(const float* dig, uint32_t* a) {
    if constexpr (ND == 3) {
        const long long x = ((long long)(int)dig[0] << 40) + ((long long)(int)dig[1] << 20) + (long long)(int)dig[2];
        const unsigned long long y = (unsigned long long)x + 0x8080808080808080ull;
        a[0] = (uint32_t)y ^ 0x80808080u;
        a[1] = (uint32_t)(y >> 32) ^ 0x80808080u;
    } else {
        __int128 x = 0;
#pragma unroll
        for (int j = 0; j < ND; j++) x = x * 1048576 + (int)dig[j];
        constexpr int W = balanced_words<ND>();
        unsigned __int128 bias = 0;
#pragma unroll
        for (int i = 0; i < W; i++) bias = (bias << 32) | 0x80808080u;
        const unsigned __int128 y = (unsigned __int128)x + bias;
#pragma unroll
        for (int i = 0; i < W; i++) a[i] = (uint32_t)(y >> (32 * i)) ^ 0x80808080u;
    }
}

// |sum_j a_j w_j| < 2^(U-1) for the balanced bytes of A': 2^17 with 8 bytes (nd = 3), 2^18 with up to 16.
template <int W>
constexpr int dot_bits() {
    return W == 2 ? 18 : 19;
}

// The same residue with integer operations only, for odd m >= 17: u = sum_j a_j w_j + dinit lies in
// [0, 2^U); q = floor(u (2^sh magic) / 2^32) with sh = 24 - U is exactly floor(u / m), because
// 2^sh magic exceeds 2^32 / m by less than 2^sh and u 2^sh < 2^24, so the excess adds less than
// 2^-8 < 1/m to u/m (checked exhaustively over the whole range for every odd 17 <= m <= 255). Then
// x = u - q m is in [0, m), and x - (m-1)/2 is the symmetric residue (dinit holds (m-1)/2 plus a
// multiple of m). Both products are 24-bit multiplies, which run at the full VALU rate. The values
// returned are x plus a multiple of 2^24 (their low bytes, the ones stored, are x's).
// The 16 elements of a lane at once, in stages (all dot products, then the quotients, then the
// remainders), so that no instruction waits on the one just before it. The first dot product of each
// element takes dinit from a scalar register (the three-operand form: no copy of dinit per element).
template <int W>
__device__ __forceinline__ void residues_odd_int(const uint32_t (*a)[W], const uint32_t* w, int dinit, uint32_t magic,
                                                 int mneg, int* x) {
    uint32_t wv[W];
#pragma unroll
    for (int i = 0; i < W; i++) wv[i] = __builtin_amdgcn_readfirstlane(w[i]);
    int u[16];
#pragma unroll
    for (int e = 0; e < 16; e++) {
        asm("v_dot4_i32_i8 %0, %1, %2, %3" : "=v"(u[e]) : "v"(a[e][0]), "v"(wv[0]), "s"(dinit));
#pragma unroll
        for (int i = 1; i < W; i++) u[e] = __builtin_amdgcn_sdot4((int)a[e][i], (int)wv[i], u[e], false);
    }
    constexpr int sh = 24 - dot_bits<W>();
    uint32_t q[16];
#pragma unroll
    for (int e = 0; e < 16; e++)
        q[e] = (uint32_t)(((unsigned long long)(((uint32_t)u[e] << sh) & 0xFFFFFFu) * (magic & 0xFFFFFFu)) >> 32);
    // u - q m modulo 2^24 as u + q (2^24 - m), one unsigned 24-bit multiply-add (mneg = 2^24 - m;
    // written out, since the compiler widens it to a 32-bit multiply); only the low byte is stored,
    // and it is that of u - q m
#pragma unroll
    for (int e = 0; e < 16; e++) asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(x[e]) : "v"(q[e]), "s"(mneg), "v"(u[e]));
}

// The remainder step of residues_odd_int for one sum u in [0, 2^U) (the dot products computed
// elsewhere, for example on the matrix cores).
template <int W>
__device__ __forceinline__ int reduce_odd_int(int u, uint32_t magic, int mneg) {
    constexpr int sh = 24 - dot_bits<W>();
    const uint32_t q = (uint32_t)(((unsigned long long)(((uint32_t)u << sh) & 0xFFFFFFu) * (magic & 0xFFFFFFu)) >> 32);
    int x;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(x) : "v"(q), "s"(mneg), "v"(u));
    return x;
}

// The symmetric residue of A' (balanced bytes a) modulo an odd m, as an FP32 integer.
template <int W>
__device__ __forceinline__ float residue_odd(const uint32_t* a, const uint32_t* w, float m, float rinv) {
    int v = __builtin_amdgcn_sdot4((int)a[0], (int)w[0], 0, false);
#pragma unroll
    for (int i = 1; i < W; i++) v = __builtin_amdgcn_sdot4((int)a[i], (int)w[i], v, false);
    const float vf = (float)v;
    return __builtin_fmaf(-__builtin_rintf(vf * rinv), m, vf);
}

}  // namespace

// A10-A11: CRT reconstruction of Scheme II to FP64.
//
// Semantics (reference recon_crt.cpp:293 + recon_writer.cpp:70, f64_tf.h:327-400): from the S exact
// products C_s (C' = C_s mod m_s) recover C' in (-M/2, M/2), M = prod m_s, and return
// C' * 2^(eA_i + eB_j - 2b) as FP64, with results below the normal range flushed to signed zero.
// The reference approximates C'/M as a triple-float fraction (one pass, absolute accuracy about
// 2^-67) or two passes (granularity 2^-124) and rounds ties away from zero. These kernels compute C'
// exactly and round once to nearest-even, so they are at least as accurate as either reference
// mode and serve both.
//
// Per element, with k_s = (C_s mod m_s) * y_s mod m_s and Q_s = M/m_s (host constants):
//   V = sum_s k_s Q_s  (<= S M),   t = the integer nearest V / M,   C' = V - t M,
// (the digits written by the product kernels may hold m_s for 0: that adds M to V, which t removes),
// with C' taken in (floor(M/2) - M, floor(M/2)].
//
// MI355X design: exact integer arithmetic in FP64 limbs. Q_s and M are given as L = nw limbs of
// 32 bits, each an exact double; every product k_s * limb (< 2^12 * 2^32) and every limb sum over at
// most 24 moduli stays below 2^53, so the accumulation is plain FP64 FMAs, exact and full rate on
// the VALU (the 32x32 -> 64-bit integer multiplies of a word-based accumulator are quarter rate).
// t comes from an FP64 estimate of V / M, whose error is below 2^-45; when the estimate lies within
// delta = 2^-28 + 2/M of a half-integer, C' is compared exactly with floor(M/2) and corrected by one
// M. Carries are then propagated (floor by 2^32, exact), the magnitude is taken, and its 32-bit
// words are rounded once to FP64. One thread computes 4 consecutive output elements of a row; the
// constants are kernel arguments (uniform, read with scalar loads).
#include <algorithm>
#include <cmath>

#include "oz2_modular.hpp"
#include "oz_internal.hpp"

namespace {

using oz2::mod_small;

// V = sum_k U_k 2^(64 k - OFF) >= 0 (64-bit words) -> V 2^e2 rounded to nearest-even, negated if
// neg; 0 when V = 0, signed zero below 2^-1022 (f64_tf.h:45-47), infinity above the FP64 range. The
// leading nonzero word and the one below it form a 128-bit window, everything under the window only
// matters as the sticky bit. Selects only, no branches.
template <int NU, int OFF>
__device__ __forceinline__ double words_to_double(const uint64_t* U, int e2, bool neg) {
    uint64_t first = U[0], second = 0, below = 0;
    int base = 0;
#pragma unroll
    for (int k = 1; k < NU; k++) {
        const bool nz = U[k] != 0;
        below = nz ? (below | second) : below;
        second = nz ? first : second;
        first = nz ? U[k] : first;
        base = nz ? 64 * k : base;
    }
    const int lz = __builtin_clzll(first | 1ull);  // 63 for first = 0 (then the result is 0 anyway)
    const uint64_t hi = lz ? (first << lz) | (second >> (64 - lz)) : first;
    const bool sticky = below != 0 || (second << lz) != 0;
    uint64_t mant = hi >> 11;
    const bool rb = (hi >> 10) & 1ull;
    const bool st = (hi & 0x3FFull) != 0 || sticky;
    mant += (rb && (st || (mant & 1ull))) ? 1ull : 0ull;
    const int carry = (int)(mant >> 53);
    mant >>= carry;
    const int exp_lead = base - OFF + 63 - lz + e2 + carry;  // exponent of the leading bit
    const uint64_t bits = ((uint64_t)(exp_lead + 1023) << 52) | (mant & 0x000FFFFFFFFFFFFFull);
    double r = __longlong_as_double((long long)bits);
    r = exp_lead > 1023 ? __builtin_huge_val() : r;
    r = exp_lead < -1022 ? 0.0 : r;
    r = neg ? -r : r;
    return first == 0 ? 0.0 : r;
}

// V = sum_l x_l 2^(32 l) >= 0 from normalized limbs (every x_l in [0, 2^32)) -> words_to_double; the
// limbs are read as 64-bit words, with a zero limb below x_0 when L is odd.
template <int L>
__device__ __forceinline__ double magnitude_to_double(const double* x, int e2, bool neg) {
    constexpr int NU = (L + 1) / 2, OFF = (L & 1) ? 32 : 0;  // V = sum_k U_k 2^(64 k - OFF)
    uint64_t U[NU];
#pragma unroll
    for (int k = 0; k < NU; k++) {
        const int lo = 2 * k - (L & 1);
        const uint64_t wl = lo >= 0 ? (uint64_t)(uint32_t)x[lo] : 0ull;
        U[k] = ((uint64_t)(uint32_t)x[lo + 1] << 32) | wl;
    }
    return words_to_double<NU, OFF>(U, e2, neg);
}

// Limb formats of the accumulator. Wide32: limbs of 32 bits holding their integers as they are
// (digits and terms up to 2^12). Byte40: limbs of 40 bits holding their integers times 2^-90 (the
// byte digits of the product kernels, which enter the FMAs as FP64 denormals, see crt_digits_kernel).
// carry: multiplier that maps a limb to its carry count; limb: a carry count in the limb's own
// scale; unit: a carry count in the next limb's scale.
struct Wide32 {
    static constexpr double carry = 0x1p-32, limb = 0x1p32, unit = 1.0;
};
struct Byte40 {
    static constexpr double carry = 0x1p50, limb = 0x1p-50, unit = 0x1p-90;
};

// Kernel constants: limbs of Q_s, M, floor(M/2), M - floor(M/2) (32-bit limbs as exact doubles).
struct CrtLimbs {
    using Format = Wide32;
    int S, shift, b;
    double radix;  // 2^32 (a kernel argument, so that it sits in a scalar register)
    double invM;   // 1/M rounded
    double delta;  // exact-path threshold: 2^-28 + 2/M
    double Q[OZ2_MAXS][8];
    double Mw[8], Mhalf[8], Mrest[8];
    uint32_t m[OZ2_MAXS], y[OZ2_MAXS], magic[OZ2_MAXS];
    // CRT terms of the digit formats: the terms of modulus s are tidx[s][0..tcount[s])
    unsigned char tcount[OZ2_MAXS], tidx[OZ2_MAXS][4];
};

// The same for the byte digits: 40-bit limbs, at most 5 (S M < 24 * 2^192 < 2^200).
constexpr int kMaxLimbs40 = 5;
struct CrtLimbs40 {
    using Format = Byte40;
    int S, shift, b;
    double radix;  // 2^40
    double invM;   // 2^90 / M rounded (the limbs hold V 2^-90)
    double delta;  // exact-path threshold: 2^-28 + 2/M
    double Q[OZ2_MAXS][kMaxLimbs40];  // limbs of Q_s times 2^984: a digit k enters as k 2^-1074
    double Mw[kMaxLimbs40], Mhalf[kMaxLimbs40], Mrest[kMaxLimbs40];  // limbs times 2^-90
    double pow40[kMaxLimbs40];  // 2^(40 l): the weights of the limbs (scalar registers, not literals)
};

// Carry propagation: limbs 0..L-2 into [0, 2^W), the top limb keeps the sign. Exact: every value is
// an integer (in the format's scale) below 2^53.
template <int L, class F>
__device__ __forceinline__ void normalize(double* x) {
#pragma unroll
    for (int l = 0; l + 1 < L; l++) {
        const double c = __builtin_floor(x[l] * F::carry);
        x[l] = __builtin_fma(-c, F::limb, x[l]);
        x[l + 1] = __builtin_fma(c, F::unit, x[l + 1]);
    }
}
// Sign of a normalized limb vector.
template <int L>
__device__ __forceinline__ int limb_sign(const double* x) {
    if (x[L - 1] != 0.0) return x[L - 1] > 0.0 ? 1 : -1;
    bool nz = false;
#pragma unroll
    for (int l = 0; l + 1 < L; l++) nz |= x[l] != 0.0;
    return nz ? 1 : 0;
}

// Half an ulp of a positive normal double (2^(e - 53) for s in [2^e, 2^(e+1))), from its exponent bits.
__device__ __forceinline__ double half_ulp(double s) {
    return __hiloint2double((__double2hiint(s) & 0x7FF00000) - (53 << 20), 0);
}

// Byte40 limbs (normalized, each an integer in [0, 2^40) times 2^-90) -> V 2^e2 rounded to nearest-even,
// negated if neg; 0 when V = 0, signed zero below 2^-1022 (f64_tf.h:45-47), infinity above the FP64
// range. A cascade of FP64 additions from the top limb down, s_j = RN(s_(j-1) + T_j) with T_j the j-th
// limb from the top at its weight, each stage's error e_j from FastTwoSum (|s| >= |T_j| or s = 0). At
// most one stage rounds: the terms below a rounding stage are worth less than half an ulp of it, so
// the later sums return it unchanged and their errors are their whole terms, each below the grid unit
// of the rounding stage, which is at most h = ulp(s)/2. s is therefore RN(V), except when the rounding
// stage's error was exactly +h (the tie went down to the even neighbour) and a nonzero term follows
// it: V is then above the midpoint and s moves one ulp up. Only the rounding stage can have e_j == h,
// so the fix is read off every stage's error against the final s's h. tests/test_crt_round.py checks
// this sequence against exact rational rounding.
template <int L>
__device__ __forceinline__ double magnitude40(const double* x, int e2, bool neg, const CrtLimbs40& a) {
    double T[L];
#pragma unroll
    for (int j = 0; j < L; j++) T[j] = x[L - 1 - j] * a.pow40[L - 1 - j];  // exact: powers of two
    double s = T[0], e[L];
#pragma unroll
    for (int j = 1; j < L; j++) {
        const double sn = s + T[j];
        e[j] = T[j] - (sn - s);
        s = sn;
    }
    const double h = half_ulp(s);
    bool fix = false, below = false;  // (bitwise: lane masks, no branches or selects)
#pragma unroll
    for (int j = L - 1; j >= 1; j--) {
        fix = fix | (below & (e[j] == h));
        below = below | (T[j] != 0.0);
    }
    const double r0 = fix ? __builtin_fma(2.0, h, s) : s;
    const int ex = ((__double2hiint(r0) >> 20) & 0x7FF) - 1023 + 90 + e2;  // exponent of the result
    double r = __builtin_ldexp(r0, 90 + e2);
    r = ex < -1022 ? 0.0 : r;
    r = neg ? -r : r;
    return r0 == 0.0 ? 0.0 : r;
}

template <int L>
__device__ __forceinline__ double magnitude(const double* x, int e2, bool neg, const CrtLimbs& a) {
    return magnitude_to_double<L>(x, e2, neg);
}
template <int L>
__device__ __forceinline__ double magnitude(const double* x, int e2, bool neg, const CrtLimbs40& a) {
    return magnitude40<L>(x, e2, neg, a);
}

// x = V (exact limbs, each below 2^53) -> C' * 2^e2 rounded to nearest-even (subnormal -> signed 0).
// C' = V - t M with t the nearest integer to an FP64 estimate of V/M. Its sign is that of q - t
// whenever |C'| is not tiny, so the limbs are multiplied by that sign before the carries are
// propagated, which leaves the magnitude in nonnegative limbs; a tiny C' of the other sign shows as
// a negative top limb and is negated once more (rare). An estimate near a half-integer is settled
// exactly against floor(M/2) (rare).
template <int L, class A>
__device__ __forceinline__ double crt_finish(double* x, const A& a, int e2) {
    using F = typename A::Format;
    double vd = x[L - 1];
#pragma unroll
    for (int l = L - 2; l >= 0; l--) vd = __builtin_fma(vd, a.radix, x[l]);  // (the radix from a register)
    const double q = vd * a.invM;
    const double t = __builtin_rint(q);
#pragma unroll
    for (int l = 0; l < L; l++) x[l] = __builtin_fma(-t, a.Mw[l], x[l]);  // |t M_l| <= 25 M_l: exact
    bool neg = q - t < 0.0;
    if (__builtin_fabs(q - t) > 0.5 - a.delta) {
        // the estimate may pick the wrong neighbour: compare C' with floor(M/2) exactly
        normalize<L, F>(x);
        double y[L];
#pragma unroll
        for (int l = 0; l < L; l++) y[l] = x[l] - a.Mhalf[l];
        normalize<L, F>(y);
        if (limb_sign<L>(y) > 0) {  // C' > floor(M/2)
#pragma unroll
            for (int l = 0; l < L; l++) x[l] -= a.Mw[l];
            normalize<L, F>(x);
        } else {
#pragma unroll
            for (int l = 0; l < L; l++) y[l] = x[l] + a.Mrest[l];
            normalize<L, F>(y);
            if (limb_sign<L>(y) <= 0) {  // C' <= floor(M/2) - M
#pragma unroll
                for (int l = 0; l < L; l++) x[l] += a.Mw[l];
                normalize<L, F>(x);
            }
        }
        neg = x[L - 1] < 0.0;
    }
    // |C'| in nonnegative limbs: flip every limb's sign bit by one mask (an xor per limb)
    const int sm = neg ? (int)0x80000000u : 0;
#pragma unroll
    for (int l = 0; l < L; l++) x[l] = __hiloint2double(__double2hiint(x[l]) ^ sm, __double2loint(x[l]));
    normalize<L, F>(x);
    if (x[L - 1] < 0.0) {  // |C'| so small that the estimate's sign was wrong
#pragma unroll
        for (int l = 0; l < L; l++) x[l] = -x[l];
        normalize<L, F>(x);
        neg = !neg;
    }
    return magnitude<L>(x, e2, neg, a);
}

// x += k * Q_s (k < 2^12)
template <int L>
__device__ __forceinline__ void limb_add(double* x, double k, const double* Q) {
#pragma unroll
    for (int l = 0; l < L; l++) x[l] = __builtin_fma(k, Q[l], x[l]);
}

// From the exact products C_s (int32): one thread per output element.
template <int L>
__global__ void __launch_bounds__(256) crt_kernel(const int32_t* __restrict__ C, int M, int N, int ldc, long long sC,
                                                  CrtLimbs a, const int32_t* __restrict__ dA,
                                                  const int32_t* __restrict__ dB, double* __restrict__ out, int ldo) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= N) return;
    const int32_t* c = C + (long long)i * ldc + j;
    double x[L];
#pragma unroll
    for (int l = 0; l < L; l++) x[l] = 0.0;
#pragma unroll
    for (int s = 0; s < OZ2_MAXS; s++)
        if (s < a.S) limb_add<L>(x, (double)oz2::crt_digit(c[(long long)s * sC], a.m[s], a.y[s], a.magic[s]), a.Q[s]);
    const int g = 2 * a.shift - (dA[i] + dB[j]);  // eA + eB
    out[(long long)i * ldo + j] = crt_finish<L>(x, a, g - 2 * a.b);
}

// From the CRT digits k_s (uint8, written by the product kernel, k_s <= m_s <= 255): one thread per 4
// consecutive output elements of a row, so that each plane read is one 32-bit word per thread.
// Limbs of 40 bits: every k_s Q_s,l < 2^48 and every sum over at most 24 moduli stays below 2^53, so
// 4 limbs cover the C3 plan (S M < 2^139) where 32-bit limbs need 5. A digit enters its FMAs as the
// FP64 denormal k 2^-1074 (its byte in the low word, zero above: one bit-field extract, no
// conversion), against limbs of Q_s stored times 2^984, so the accumulators hold V 2^-90 exactly
// (integers times 2^-90 below 2^-37: normal doubles).
template <int L>
__global__ void __launch_bounds__(256) crt_digits_kernel(const uint8_t* __restrict__ D, int M, int N, int ldd,
                                                         long long sD, CrtLimbs40 a, const int32_t* __restrict__ dA,
                                                         const int32_t* __restrict__ dB, double* __restrict__ out,
                                                         int ldo) {
    const int j0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    const int i = blockIdx.y;
    if (j0 >= N) return;
    const uint32_t* d = reinterpret_cast<const uint32_t*>(D + (long long)i * ldd + j0);
    const long long sw = sD / 4;
    // every plane's word is requested before the first is used (the planes past S read plane S-1
    // again, so that no load waits on a branch)
    uint32_t v[OZ2_MAXS];
#pragma unroll
    for (int s = 0; s < OZ2_MAXS; s++) v[s] = d[(long long)min(s, a.S - 1) * sw];
    double x[4][L];
#pragma unroll
    for (int e = 0; e < 4; e++)
#pragma unroll
        for (int l = 0; l < L; l++) x[e][l] = 0.0;
#pragma unroll
    for (int s = 0; s < OZ2_MAXS; s++)
        if (s < a.S) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const double k = __hiloint2double(0, (int)((v[s] >> (8 * e)) & 0xFFu));  // k 2^-1074
#pragma unroll
                for (int l = 0; l < L; l++) x[e][l] = __builtin_fma(k, a.Q[s][l], x[e][l]);
            }
        }
    const int gi = 2 * a.shift - dA[i] - 2 * a.b;
    double r[4];
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = j0 + e < N ? crt_finish<L>(x[e], a, gi - dB[j0 + e]) : 0.0;
    double* o = out + (long long)i * ldo + j0;
    if (j0 + 3 < N && !(reinterpret_cast<uintptr_t>(o) & 15)) {
        // non-temporal: C (512 MB at C3) is not read again by the pass (0.418 against 0.431 ms)
        typedef double f64x2 __attribute__((ext_vector_type(2)));
        __builtin_nontemporal_store(f64x2{r[0], r[1]}, reinterpret_cast<f64x2*>(o));
        __builtin_nontemporal_store(f64x2{r[2], r[3]}, reinterpret_cast<f64x2*>(o) + 1);
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (j0 + e < N) o[e] = r[e];
    }
}

// From the uint16 CRT terms w_o of the digit formats (oz2_gemm_groups_f8): the terms of modulus s
// add up to k_s modulo m_s (sum < 4 m_s, reduced), then as above. One thread per 4 consecutive
// output elements (one 8-byte load per term).
template <int L>
__global__ void __launch_bounds__(256) crt_terms_kernel(const uint16_t* __restrict__ W, int M, int N, int ldw,
                                                        long long sW, CrtLimbs a, const int32_t* __restrict__ dA,
                                                        const int32_t* __restrict__ dB, double* __restrict__ out,
                                                        int ldo) {
    const int j0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    const int i = blockIdx.y;
    if (j0 >= N) return;
    const uint2* w = reinterpret_cast<const uint2*>(W + (long long)i * ldw + j0);
    const long long sw = sW / 4;
    double x[4][L];
#pragma unroll
    for (int e = 0; e < 4; e++)
#pragma unroll
        for (int l = 0; l < L; l++) x[e][l] = 0.0;
#pragma unroll
    for (int s = 0; s < OZ2_MAXS; s++) {
        if (s < a.S) {
            uint32_t u[4] = {0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < 4; t++)
                if (t < a.tcount[s]) {
                    const uint2 v = w[(long long)a.tidx[s][t] * sw];
                    u[0] += v.x & 0xFFFFu;
                    u[1] += v.x >> 16;
                    u[2] += v.y & 0xFFFFu;
                    u[3] += v.y >> 16;
                }
#pragma unroll
            for (int e = 0; e < 4; e++) limb_add<L>(x[e], (double)mod_small(u[e], a.m[s], a.magic[s]), a.Q[s]);
        }
    }
    const int gi = 2 * a.shift - dA[i] - 2 * a.b;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (j0 + e < N) out[(long long)i * ldo + j0 + e] = crt_finish<L>(x[e], a, gi - dB[j0 + e]);
}

// Kernel constants of a CRT descriptor whose moduli are at most mmax.
int crt_limbs(oz_dev* dev, const char* name, const oz2_crt_dev* crt, uint32_t mmax, CrtLimbs& a) {
    a = CrtLimbs{};
    a.radix = 4294967296.0;
    a.S = crt->S;
    a.shift = crt->shift;
    a.b = crt->b;
    // M = prod m_s from the moduli (checked against the descriptor's words)
    uint32_t Mw[9] = {1, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int s = 0; s < crt->S; s++) {
        const uint32_t m = crt->m[s];
        if (m < 2 || m > mmax || crt->y[s] >= m) return oz::fail(dev, OZ_ERR_ARG, "%s: modulus out of range", name);
        a.m[s] = m;
        a.y[s] = crt->y[s];
        a.magic[s] = (uint32_t)(0x100000000ull / m);
        uint64_t carry = 0;
        for (int w = 0; w < 9; w++) {
            const uint64_t p = (uint64_t)Mw[w] * m + carry;
            Mw[w] = (uint32_t)p;
            carry = p >> 32;
        }
    }
    for (int w = 0; w < 8; w++)
        if (Mw[w] != crt->Mw[w]) return oz::fail(dev, OZ_ERR_ARG, "%s: Mprod is not the product of the moduli", name);
    if (Mw[8]) return oz::fail(dev, OZ_ERR_ARG, "%s: Mprod exceeds 256 bits", name);
    // S * M must fit the nw words of the accumulator
    {
        bool over = false;
        uint64_t carry = 0;
        for (int w = 0; w < 8; w++) {
            const uint64_t p = (uint64_t)Mw[w] * (uint64_t)crt->S + carry;
            over |= w >= crt->nw && (uint32_t)p != 0;
            carry = p >> 32;
        }
        if (over || carry) return oz::fail(dev, OZ_ERR_ARG, "%s: S*Mprod does not fit %d words", name, crt->nw);
    }
    uint32_t half[8], rest[8];
    uint32_t r = 0;
    for (int w = 7; w >= 0; w--) {
        const uint64_t cur = ((uint64_t)r << 32) | Mw[w];
        half[w] = (uint32_t)(cur >> 1);
        r = (uint32_t)(cur & 1u);
    }
    uint32_t borrow = 0;
    for (int w = 0; w < 8; w++) {
        const uint64_t d = (uint64_t)Mw[w] - half[w] - borrow;
        rest[w] = (uint32_t)d;
        borrow = (uint32_t)(d >> 63);
    }
    for (int w = 0; w < 8; w++) {
        a.Mw[w] = Mw[w];
        a.Mhalf[w] = half[w];
        a.Mrest[w] = rest[w];
    }
    for (int s = 0; s < crt->S; s++) {  // Q_s = M / m_s by long division
        uint64_t rem = 0;
        for (int w = 7; w >= 0; w--) {
            const uint64_t cur = (rem << 32) | Mw[w];
            a.Q[s][w] = (double)(uint32_t)(cur / crt->m[s]);
            rem = cur % crt->m[s];
        }
    }
    double Md = 0.0;
    for (int w = 7; w >= 0; w--) Md = Md * 4294967296.0 + (double)Mw[w];
    a.invM = 1.0 / Md;
    a.delta = 0x1p-28 + 2.0 / Md;
    return OZ_OK;
}

template <int L>
int launch_crt(oz_dev* dev, const void* C, int kind, int M, int N, int ldc, long long sC, const CrtLimbs& a,
               const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    if (kind == 2) {
        hipLaunchKernelGGL(crt_terms_kernel<L>, dim3(oz::ceil_div(N, 1024), M), dim3(256), 0, dev->stream,
                           static_cast<const uint16_t*>(C), M, N, ldc, sC, a, dA, dB, out, ldo);
        return oz::launch_check(dev, "crt_terms_kernel");
    }
    hipLaunchKernelGGL(crt_kernel<L>, dim3(oz::ceil_div(N, 256), M), dim3(256), 0, dev->stream,
                       static_cast<const int32_t*>(C), M, N, ldc, sC, a, dA, dB, out, ldo);
    return oz::launch_check(dev, "crt_kernel");
}

// Constants of the byte-digit kernel from those of the 32-bit limbs: the 40-bit limbs of Q_s, M,
// floor(M/2) and M - floor(M/2), scaled as CrtLimbs40 states, and the number of limbs that S M needs.
uint64_t limb40(const double* words, int l) {  // bits 40 l .. 40 l + 39 of 8 exact 32-bit words
    uint64_t r = 0;
    for (int b = 0; b < 40; b++) {
        const int q = 40 * l + b;
        if (q < 256 && (((uint64_t)words[q / 32] >> (q % 32)) & 1u)) r |= 1ull << b;
    }
    return r;
}
int crt_limbs40(const CrtLimbs& a, CrtLimbs40& b) {
    b = CrtLimbs40{};
    b.S = a.S;
    b.shift = a.shift;
    b.b = a.b;
    b.radix = 0x1p40;
    for (int l = 0; l < kMaxLimbs40; l++) b.pow40[l] = std::ldexp(1.0, 40 * l);
    b.invM = std::ldexp(a.invM, 90);
    b.delta = a.delta;
    // bit length of S M (S M < 2^200): the limbs needed
    uint32_t sm[9] = {};
    uint64_t carry = 0;
    for (int w = 0; w < 8; w++) {
        const uint64_t p = (uint64_t)(uint32_t)a.Mw[w] * (uint64_t)a.S + carry;
        sm[w] = (uint32_t)p;
        carry = p >> 32;
    }
    sm[8] = (uint32_t)carry;
    int bits = 0;
    for (int w = 8; w >= 0 && !bits; w--)
        if (sm[w]) bits = 32 * w + 32 - __builtin_clz(sm[w]);
    const int L = std::max(2, (bits + 39) / 40);
    for (int l = 0; l < kMaxLimbs40; l++) {
        for (int s = 0; s < a.S; s++) b.Q[s][l] = std::ldexp((double)limb40(a.Q[s], l), 984);
        b.Mw[l] = std::ldexp((double)limb40(a.Mw, l), -90);
        b.Mhalf[l] = std::ldexp((double)limb40(a.Mhalf, l), -90);
        b.Mrest[l] = std::ldexp((double)limb40(a.Mrest, l), -90);
    }
    return L;
}

template <int L>
int launch_crt_digits(oz_dev* dev, const uint8_t* D, int M, int N, int ldd, long long sD, const CrtLimbs40& a,
                      const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    hipLaunchKernelGGL(crt_digits_kernel<L>, dim3(oz::ceil_div(N, 1024), M), dim3(256), 0, dev->stream, D, M, N, ldd,
                       sD, a, dA, dB, out, ldo);
    return oz::launch_check(dev, "crt_digits_kernel");
}

// All entry points: C is int32 products (kind 0, element strides), uint8 digits (kind 1, byte
// strides) or uint16 terms (kind 2, element strides); rows go on the grid's y (at most 65535 per
// launch), so the launch is split in row chunks.
int crt_launch(oz_dev* dev, const void* C, int kind, int M, int N, int ldc, long long strideC, int nw,
               const CrtLimbs& a, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    const size_t esz = kind == 1 ? 1 : kind == 2 ? 2 : 4;
    if (kind == 1) {
        CrtLimbs40 b;
        const int L = crt_limbs40(a, b);
        for (int i0 = 0; i0 < M; i0 += 65535) {
            const int rows = std::min(65535, M - i0);
            const uint8_t* Di = static_cast<const uint8_t*>(C) + (size_t)i0 * ldc;
            double* oi = out + (long long)i0 * ldo;
            int st;
            switch (L) {
            case 2: st = launch_crt_digits<2>(dev, Di, rows, N, ldc, strideC, b, dA + i0, dB, oi, ldo); break;
            case 3: st = launch_crt_digits<3>(dev, Di, rows, N, ldc, strideC, b, dA + i0, dB, oi, ldo); break;
            case 4: st = launch_crt_digits<4>(dev, Di, rows, N, ldc, strideC, b, dA + i0, dB, oi, ldo); break;
            default: st = launch_crt_digits<5>(dev, Di, rows, N, ldc, strideC, b, dA + i0, dB, oi, ldo); break;
            }
            if (st) return st;
        }
        return OZ_OK;
    }
    for (int i0 = 0; i0 < M; i0 += 65535) {
        const int rows = std::min(65535, M - i0);
        const void* Ci = static_cast<const char*>(C) + (size_t)i0 * ldc * esz;
        double* oi = out + (long long)i0 * ldo;
        int st;
        switch (nw) {
        case 3: st = launch_crt<3>(dev, Ci, kind, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 4: st = launch_crt<4>(dev, Ci, kind, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 5: st = launch_crt<5>(dev, Ci, kind, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 6: st = launch_crt<6>(dev, Ci, kind, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 7: st = launch_crt<7>(dev, Ci, kind, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        default: st = launch_crt<8>(dev, Ci, kind, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        }
        if (st) return st;
    }
    return OZ_OK;
}

int crt_f64(oz_dev* dev, const char* name, const void* C, bool digits, int M, int N, int ldc, long long strideC,
            const oz2_crt_dev* crt, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    if (int st = oz::use(dev)) return st;
    if (!C || !crt || !dA || !dB || !out || M <= 0 || N <= 0 || ldc < N || ldo < N || crt->S < 1 ||
        crt->S > OZ2_MAXS || crt->nw < 3 || crt->nw > 8 || (digits && (ldc % 4 || strideC % 4 || ((uintptr_t)C & 3))))
        return oz::fail(dev, OZ_ERR_ARG, "%s: invalid arguments", name);
    CrtLimbs a;
    if (int st = crt_limbs(dev, name, crt, 255u, a)) return st;
    return crt_launch(dev, C, digits ? 1 : 0, M, N, ldc, strideC, crt->nw, a, dA, dB, out, ldo);
}

}  // namespace

extern "C" int oz2_crt_f64(oz_dev* dev, const int32_t* C, int M, int N, int ldc, long long strideC,
                           const oz2_crt_dev* crt, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    return crt_f64(dev, "oz2_crt_f64", C, false, M, N, ldc, strideC, crt, dA, dB, out, ldo);
}

extern "C" int oz2_crt_digits_f64(oz_dev* dev, const uint8_t* D, int M, int N, int ldd, long long strideD,
                                  const oz2_crt_dev* crt, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    return crt_f64(dev, "oz2_crt_digits_f64", D, true, M, N, ldd, strideD, crt, dA, dB, out, ldo);
}

extern "C" int oz2_crt_terms_f64(oz_dev* dev, const uint16_t* W, int M, int N, int ldw, long long strideW, int nterms,
                                 const unsigned char* term_modulus, const oz2_crt_dev* crt, const int32_t* dA,
                                 const int32_t* dB, double* out, int ldo) {
    const char* name = "oz2_crt_terms_f64";
    if (int st = oz::use(dev)) return st;
    if (!W || !term_modulus || !crt || !dA || !dB || !out || M <= 0 || N <= 0 || ldw < N || ldo < N || nterms < 1 ||
        nterms > OZ2_MAXOUT || crt->S < 1 || crt->S > OZ2_MAXS || crt->nw < 3 || crt->nw > 8 || ldw % 4 ||
        strideW % 4 || ((uintptr_t)W & 7) || (nterms > 1 && strideW < (long long)M * ldw))
        return oz::fail(dev, OZ_ERR_ARG, "%s: invalid arguments", name);
    CrtLimbs a;
    if (int st = crt_limbs(dev, name, crt, 2401u, a)) return st;
    for (int o = 0; o < nterms; o++) {
        const int s = term_modulus[o];
        if (s >= crt->S) return oz::fail(dev, OZ_ERR_ARG, "%s: term %d names modulus %d", name, o, s);
        if (a.tcount[s] == 4) return oz::fail(dev, OZ_ERR_ARG, "%s: more than 4 terms for modulus %d", name, s);
        a.tidx[s][a.tcount[s]++] = (unsigned char)o;
    }
    return crt_launch(dev, W, 2, M, N, ldw, strideW, crt->nw, a, dA, dB, out, ldo);
}

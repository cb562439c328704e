// oz_oracle — CPU restatement of the reference ozTTgemm numerics. TEST INFRASTRUCTURE ONLY.
// See oz_oracle.hpp for the rules of use and how each function is pinned.
//
// Build flags matter: -ffp-contract=off -fno-fast-math (the reference builds the same way,
// Makefile:51-53), x86-64 SSE arithmetic for float/double, 80-bit long double, libquadmath.
#include "oz_oracle.hpp"

#include <quadmath.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <random>
#include <vector>

namespace {

// ---------------------------------------------------------------------------------------------
// FP32 operation model of the reference's tile operations (experiments/src/checks/sfpu_tf_emu.hpp:66-88,
// the model the reference compared with its hardware): each add/sub/mul is one binary32 RNE
// operation, no FMA; denormal inputs and outputs become signed zero; a product with a zero factor
// is +0; Rnd is (|v|+2^23)-2^23 with the sign of v, +0 for a zero result.
// ---------------------------------------------------------------------------------------------
inline float flush(float x) { return (x != 0.0f && std::fabs(x) < FLT_MIN) ? std::copysign(0.0f, x) : x; }
inline float f_add(float a, float b) { return flush(flush(a) + flush(b)); }
inline float f_sub(float a, float b) { return flush(flush(a) - flush(b)); }
inline float f_mul(float a, float b) {
    a = flush(a);
    b = flush(b);
    if (a == 0.0f || b == 0.0f) return 0.0f;
    return flush(a * b);
}
inline float f_rnd(float v) {
    v = flush(v);
    const float a = std::fabs(v);
    if (!(a < 8388608.0f)) return v;
    const float t = (a + 8388608.0f) - 8388608.0f;
    return t == 0.0f ? 0.0f : std::copysign(t, v);
}
inline float bits_f(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint32_t f_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

// Error-free sums in the order of the reference procedures (sfpu_tf_proc.h:61-74).
inline void two_sum(float x, float y, float& s, float& e) {
    s = f_add(x, y);
    float bb = f_sub(s, x);
    float aa = f_sub(s, bb);
    aa = f_sub(x, aa);
    bb = f_sub(y, bb);
    e = f_add(aa, bb);
}
inline void fast_two_sum(float a, float b, float& s, float& t) {
    s = f_add(a, b);
    const float w = f_sub(s, a);
    t = f_sub(b, w);
}

// Triple-float times a power-of-two radix, renormalized (tfMulP2, sfpu_tf_proc.h:160-169).
inline void tf_mul_pow2(float& hi, float& mid, float& lo, float r) {
    hi = f_mul(hi, r);
    mid = f_mul(mid, r);
    lo = f_mul(lo, r);
    float s3, e4, s5, e6;
    two_sum(mid, lo, s3, e4);
    two_sum(hi, s3, s5, e6);
    hi = s5;
    fast_two_sum(e6, e4, mid, lo);
}

// ModRound: d - Rnd(d*rinv)*m (sfpu_tf_proc.h:316-319).
inline float mod_round(float d, float m, float rinv) {
    float s = f_mul(d, rinv);
    s = f_rnd(s);
    s = f_mul(s, m);
    return f_sub(d, s);
}

// split_f64 (f64_tf.h:141-172): FP64 x*2^d -> hi, braw, craw, s bit patterns, integer ops only.
void split_words(uint32_t w1, uint32_t w0, int32_t d, uint32_t& hi, uint32_t& braw, uint32_t& craw, uint32_t& s) {
    const uint32_t sgn = w1 & 0x80000000u;
    const int32_t E = (int32_t)((w1 >> 20) & 0x7FFu);
    if (E == 0) {
        hi = 0u;
        braw = 0x4B000000u;
        craw = 0x4B000000u;
        s = 0u;
        return;
    }
    // 53-bit significand -> 23-bit head (rounded to nearest on the dropped 30 bits), signed 23-bit
    // middle and 7-bit tail.
    uint32_t a = 0x400000u | ((w1 & 0x000FFFFFu) << 2) | (w0 >> 30);
    const uint32_t rem = w0 & 0x3FFFFFFFu;
    int32_t r = (int32_t)rem;
    if (rem >= 0x20000000u) {
        a += 1u;
        r = (int32_t)rem - 0x40000000;
    }
    const int32_t b = r >> 7;
    const uint32_t c = (uint32_t)r & 0x7Fu;
    const int32_t elsb = E - 1075 + d;
    int32_t eh;
    uint32_t mh;
    if (a == 0x800000u) {
        eh = elsb + 180;
        mh = 0u;
    } else {
        eh = elsb + 179;
        mh = (a << 1) & 0x7FFFFFu;
    }
    const int32_t es = elsb + 134;
    hi = (eh > 0 && eh < 255) ? (sgn | ((uint32_t)eh << 23) | mh) : 0u;
    s = (es > 0 && es < 255) ? (sgn | ((uint32_t)es << 23)) : 0u;
    braw = 0x4B000000u | (((uint32_t)(b + 0x400000)) & 0x7FFFFFu);
    craw = 0x4B000000u | c;
}

// tf_load_f64 (slice_tf_core.h:67-76): mid = (braw - 1.5*2^23)*s, lo = (craw - 2^23)*s*2^-7.
void load_triple(double x, int32_t d, float& hi, float& mid, float& lo) {
    uint64_t u;
    std::memcpy(&u, &x, 8);
    uint32_t h, br, cr, s;
    split_words((uint32_t)(u >> 32), (uint32_t)u, d, h, br, cr, s);
    const float sf = bits_f(s);
    hi = bits_f(h);
    mid = f_mul(f_add(bits_f(br), -12582912.0f), sf);
    lo = f_mul(f_mul(f_add(bits_f(cr), -8388608.0f), sf), 0.0078125f);
}

// oz2_make_digits (digits.h:80-112): nd digits, top first.
void make_digits(double x, int32_t d, int nd, float* dig) {
    float hi, mid, lo;
    load_triple(x, d, hi, mid, lo);
    for (int i = 0; i < nd; ++i) {
        if (i > 0) tf_mul_pow2(hi, mid, lo, 1048576.0f);
        const float t = f_rnd(hi);
        hi = f_sub(hi, t);
        dig[i] = t;
    }
}

// 2^e mod m for e >= 0 (moduli.hpp:688-692).
float pow2mod(int e, long mod) {
    long r = 1 % mod, base = 2 % mod;
    for (int i = 0; i < e; ++i) r = (r * base) % mod;
    return (float)r;
}

// oz2_residue (digits.h:165-179) on digits given top first (dig[0] = d_{nd-1}, ..., dig[nd-1] = d0).
float residue(const float* dig, int nd, float m, float rinv, const float* c) {
    const float d0 = dig[nd - 1], d1 = dig[nd - 2], d2 = dig[nd - 3];
    float acc = d0;
    float t = mod_round(d1, m, rinv);
    acc = f_add(acc, f_mul(t, c[0]));
    t = mod_round(d2, m, rinv);
    acc = f_add(acc, f_mul(t, c[1]));
    if (nd >= 4) {
        acc = mod_round(acc, m, rinv);
        if (nd >= 5) {
            t = mod_round(dig[0], m, rinv);  // d4
            acc = f_add(acc, f_mul(t, c[3]));
            acc = mod_round(acc, m, rinv);
        }
        t = mod_round(dig[nd - 4], m, rinv);  // d3
        acc = f_add(acc, f_mul(t, c[2]));
    }
    return mod_round(acc, m, rinv);
}

inline int32_t delta_of(const int32_t* delta, int mode, int r, int c) { return mode == 0 ? delta[r] : delta[c]; }

// ---------------------------------------------------------------------------------------------
// Reconstruction helpers of the reference (f64_tf.h:174-400)
// ---------------------------------------------------------------------------------------------
void dec32(uint32_t u, int32_t& e, int32_t& sig) {
    const int32_t ee = (int32_t)((u >> 23) & 0xFFu);
    if (ee == 0) {
        e = 0;
        sig = 0;
        return;
    }
    e = ee;
    const int32_t s = (int32_t)(0x800000u | (u & 0x7FFFFFu));
    sig = (u & 0x80000000u) ? -s : s;
}
uint64_t pack_f64(uint64_t A, uint32_t Whi, uint32_t Wlo, int32_t total, uint64_t sgn) {
    const unsigned __int128 p = (unsigned __int128)A * (((unsigned __int128)Whi << 32) | Wlo);
    const uint64_t hi = (uint64_t)(p >> 64);
    const int32_t n = (hi >> 63) ? 63 : 62;
    int32_t exp2 = n + 64 + total;
    uint64_t mant;
    bool up;
    if (n == 63) {
        mant = hi >> 11;
        up = (hi & 0x400ull) != 0;
    } else {
        mant = hi >> 10;
        up = (hi & 0x200ull) != 0;
    }
    if (up) {
        mant += 1ull;
        if (mant >> 53) {
            mant >>= 1;
            exp2 += 1;
        }
    }
    const int32_t ebias = exp2 + 1023;
    if (ebias <= 0) return sgn;
    if (ebias >= 2047) return sgn | 0x7FF0000000000000ull;
    return sgn | ((uint64_t)ebias << 52) | (mant & 0x000FFFFFFFFFFFFFull);
}
struct A128 {
    uint32_t w[4];
};
void a128_add(A128& a, int32_t k, uint32_t v) {
    for (; k < 4 && v; ++k) {
        const uint32_t o = a.w[k];
        a.w[k] = o + v;
        v = (a.w[k] < o);
    }
}
void a128_sub(A128& a, int32_t k, uint32_t v) {
    for (; k < 4 && v; ++k) {
        const uint32_t o = a.w[k];
        a.w[k] = o - v;
        v = (o < v);
    }
}
void a128_term(A128& a, int32_t sig, int32_t sh) {
    if (!sig || sh <= -24) return;
    const bool neg = sig < 0;
    const uint64_t m = (uint64_t)(neg ? -(int64_t)sig : (int64_t)sig);
    const uint64_t v = (sh < 0) ? (m >> (uint32_t)(-sh)) : (m << (sh & 31));
    const int32_t w = (sh < 0) ? 0 : (sh >> 5);
    if (!v) return;
    if (neg) {
        a128_sub(a, w, (uint32_t)v);
        a128_sub(a, w + 1, (uint32_t)(v >> 32));
    } else {
        a128_add(a, w, (uint32_t)v);
        a128_add(a, w + 1, (uint32_t)(v >> 32));
    }
}
void a128_add_limbs(A128& a, const float* limb, int nl) {
    for (int i = 0; i < nl; i++) {
        int32_t e, sig;
        dec32(f_bits(limb[i]), e, sig);
        a128_term(a, sig, e - 26);
    }
}
uint64_t a128_frac_to_f64(A128 a, int32_t g, uint32_t Whi, uint32_t Wlo, int32_t qw) {
    const uint32_t top = a.w[3];
    if (top + 0x08000000u >= 0x10000000u || top == 0xF8000000u) {
        if ((int32_t)top >= 0x08000000)
            a128_sub(a, 3, 0x10000000u);
        else if ((int32_t)top < -0x08000000 || (a.w[0] | a.w[1] | a.w[2]) == 0u)
            a128_add(a, 3, 0x10000000u);
    }
    const bool neg = (a.w[3] & 0x80000000u) != 0;
    if (neg) {
        for (int i = 0; i < 4; i++) a.w[i] = ~a.w[i];
        a128_add(a, 0, 1u);
    }
    if (!(a.w[0] | a.w[1] | a.w[2] | a.w[3])) return 0ull;
    int32_t wsh = 0;
    while (a.w[3 - wsh] == 0) wsh++;
    const int32_t lz = 32 * wsh + __builtin_clz(a.w[3 - wsh]);
    uint64_t A;
    if (lz <= 64) {
        const int32_t k = (64 - lz) >> 5, off = (64 - lz) & 31;
        A = (((uint64_t)a.w[k + 1] << 32) | a.w[k]) >> off;
        if (off) A |= (uint64_t)a.w[k + 2] << (64 - off);
    } else {
        A = (((uint64_t)a.w[1] << 32) | a.w[0]) << (lz - 64);
    }
    return pack_f64(A, Whi, Wlo, qw + g - lz - 60, neg ? 0x8000000000000000ull : 0ull);
}

// Number of trailing reciprocal fragments added with the cheap step (moduli.hpp:772-800).
uint32_t choose_small_tail(const float* rp, uint32_t nrp, const int* m, uint32_t s) {
    if (nrp > 8) return 0;
    float worst[8] = {0};
    float vmax = 0.f;
    for (uint32_t t = 0; t < nrp; t++) {
        for (uint32_t i = 0; i < s; i++) {
            const float v = std::fabs(rp[(size_t)i * nrp + t]) * (float)(m[i] / 2 + 1);
            if (v > worst[t]) worst[t] = v;
        }
        if (worst[t] > vmax) vmax = worst[t];
    }
    const float scale = vmax < 1.f ? vmax : 1.f;
    const float eps = (float)std::ldexp((double)scale, -30);
    uint32_t n = 0;
    for (uint32_t t = nrp; t-- > 0;) {
        if (worst[t] <= eps)
            n++;
        else
            break;
    }
    return n;
}

// Triple-float accumulator of the CRT pass (recon_crt.cpp kernel_main with recon_crt_proc.h).
struct CrtAcc {
    float hi = 0, mid = 0, lo = 0;
    // tfAddS<3> (sfpu_tf_proc.h:184-198)
    void add(float v) {
        float s0, e0;
        {
            const float t0 = f_add(hi, v);
            float t1 = f_sub(t0, hi);
            float t2 = f_sub(t0, t1);
            t2 = f_sub(hi, t2);
            t1 = f_sub(v, t1);
            e0 = f_add(t2, t1);
            s0 = t0;
        }
        hi = s0;
        const float t0 = f_add(mid, e0);
        float t2 = f_sub(t0, mid);
        float tm = f_sub(t0, t2);
        tm = f_sub(mid, tm);
        t2 = f_sub(e0, t2);
        t2 = f_add(tm, t2);
        mid = t0;
        lo = f_add(lo, t2);
    }
    // tfAddSmall<3> (sfpu_tf_proc.h:237-258)
    void add_small(float v) {
        const float t0 = f_add(mid, v);
        float t2 = f_sub(t0, mid);
        float t1 = f_sub(t0, t2);
        t1 = f_sub(mid, t1);
        t2 = f_sub(v, t2);
        t2 = f_add(t1, t2);
        mid = t0;
        lo = f_add(lo, t2);
    }
    // drop_integer (recon_crt_proc.h:56-60)
    void drop_integer() { hi = f_sub(hi, f_rnd(hi)); }
};

// decode_signmag_residue (recon_crt.cpp:219-249) on the value of C_i.
float decode_residue(int32_t C, float m, float rinv, float m16) {
    const uint32_t mag = C < 0 ? (uint32_t)(-(int64_t)C) : (uint32_t)C;
    const float sgn = C > 0 ? 1.0f : (C < 0 ? -1.0f : 0.0f);
    float chi = f_mul((float)(int32_t)(mag & 0x7FFF0000u), 1.52587890625e-05f);
    float keep = mod_round(chi, m, rinv);
    keep = f_mul(keep, m16);
    float t = mod_round((float)(int32_t)(mag & 0xFFFFu), m, rinv);
    t = f_add(t, keep);
    t = f_mul(t, sgn);
    return mod_round(t, m, rinv);
}

// One pass of the reference CRT for one element: three limbs of frac.
void crt_pass(const int32_t* C, size_t stride, size_t idx, const orc_crt_consts& k, const float* rp, int nrp,
              uint32_t nsmall, float* limbs) {
    CrtAcc acc;
    for (int i = 0; i < k.S; i++) {
        const float m = (float)k.m[i], rinv = k.rinv[i];
        const float r = decode_residue(C[(size_t)i * stride + idx], m, rinv, k.m16[i]);
        const float kk = mod_round(f_mul(r, (float)k.yi[i]), m, rinv);
        for (int t = 0; t < nrp; t++) {
            const float term = f_mul(kk, rp[i * nrp + t]);
            if ((uint32_t)t >= (uint32_t)nrp - nsmall)
                acc.add_small(term);
            else
                acc.add(term);
        }
        acc.drop_integer();
    }
    limbs[0] = acc.hi;
    limbs[1] = acc.mid;
    limbs[2] = acc.lo;
}

// ---------------------------------------------------------------------------------------------
// 256-bit unsigned integers for the exact CRT
// ---------------------------------------------------------------------------------------------
struct U256 {
    uint64_t w[4] = {0, 0, 0, 0};
};
void u256_mul_small(U256& x, uint64_t k) {
    unsigned __int128 carry = 0;
    for (int i = 0; i < 4; i++) {
        const unsigned __int128 p = (unsigned __int128)x.w[i] * k + carry;
        x.w[i] = (uint64_t)p;
        carry = p >> 64;
    }
}
void u256_add(U256& x, const U256& y) {
    unsigned __int128 c = 0;
    for (int i = 0; i < 4; i++) {
        const unsigned __int128 s = (unsigned __int128)x.w[i] + y.w[i] + c;
        x.w[i] = (uint64_t)s;
        c = s >> 64;
    }
}
void u256_sub(U256& x, const U256& y) {
    uint64_t borrow = 0;
    for (int i = 0; i < 4; i++) {
        const unsigned __int128 d = (unsigned __int128)x.w[i] - y.w[i] - borrow;
        x.w[i] = (uint64_t)d;
        borrow = (uint64_t)(d >> 64) ? 1 : 0;
    }
}
int u256_cmp(const U256& x, const U256& y) {
    for (int i = 3; i >= 0; i--)
        if (x.w[i] != y.w[i]) return x.w[i] < y.w[i] ? -1 : 1;
    return 0;
}
// x / small (exact division assumed or floor)
U256 u256_div_small(const U256& x, uint64_t d) {
    U256 q;
    unsigned __int128 r = 0;
    for (int i = 3; i >= 0; i--) {
        const unsigned __int128 cur = (r << 64) | x.w[i];
        q.w[i] = (uint64_t)(cur / d);
        r = cur % d;
    }
    return q;
}

// Signed 256-bit two's complement value times 2^e, rounded to FP64 nearest-even; below the
// normal range -> signed zero.
double u256_to_double(U256 v, int e) {
    const bool neg = (v.w[3] >> 63) != 0;
    if (neg) {
        for (int i = 0; i < 4; i++) v.w[i] = ~v.w[i];
        U256 one;
        one.w[0] = 1;
        u256_add(v, one);
    }
    int top = -1;
    for (int i = 3; i >= 0; i--)
        if (v.w[i]) {
            top = 64 * i + 63 - __builtin_clzll(v.w[i]);
            break;
        }
    if (top < 0) return neg ? -0.0 : 0.0;
    // value = v * 2^e; leading bit at position top -> exponent top + e
    auto bit = [&](int p) -> uint64_t { return p < 0 ? 0 : (v.w[p >> 6] >> (p & 63)) & 1ull; };
    uint64_t mant = 0;
    for (int p = top; p > top - 53; p--) mant = (mant << 1) | bit(p);
    const int lowest = top - 52;  // position of the last kept bit
    bool guard = lowest - 1 >= 0 ? bit(lowest - 1) : false;
    bool sticky = false;
    for (int p = lowest - 2; p >= 0; p--)
        if (bit(p)) {
            sticky = true;
            break;
        }
    int exp2 = top + e;  // value = mant * 2^(exp2 - 52)
    if (guard && (sticky || (mant & 1))) {
        mant += 1;
        if (mant >> 53) {
            mant >>= 1;
            exp2 += 1;
        }
    }
    if (exp2 < -1022) return neg ? -0.0 : 0.0;
    if (exp2 > 1023) return neg ? -HUGE_VAL : HUGE_VAL;
    const double r = std::ldexp((double)mant, exp2 - 52);
    return neg ? -r : r;
}

// Exact CRT of one element: C' = sum_i k_i (M/m_i) mod M with k_i = (r_i y_i) mod m_i, returned as
// the symmetric representative in (-M/2, M/2] (two's complement).
struct ExactCrt {
    int S;
    long m[24], y[24];
    U256 Mv, Q[24];
    ExactCrt(int S_, const int* mm) : S(S_) {
        Mv.w[0] = 1;
        for (int i = 0; i < S; i++) {
            m[i] = mm[i];
            u256_mul_small(Mv, (uint64_t)mm[i]);
        }
        for (int i = 0; i < S; i++) {
            Q[i] = u256_div_small(Mv, (uint64_t)m[i]);
            long P = 1;
            for (int j = 0; j < S; j++)
                if (j != i) P = (P * (m[j] % m[i])) % m[i];
            y[i] = 0;
            for (long t = 1; t < m[i]; t++)
                if ((P * t) % m[i] == 1) {
                    y[i] = t;
                    break;
                }
        }
    }
    U256 value(const int32_t* r) const {
        U256 acc;
        for (int i = 0; i < S; i++) {
            const long ri = ((long)r[i] % m[i] + m[i]) % m[i];
            U256 t = Q[i];
            u256_mul_small(t, (uint64_t)((ri * y[i]) % m[i]));
            u256_add(acc, t);
            while (u256_cmp(acc, Mv) >= 0) u256_sub(acc, Mv);
        }
        U256 twice = acc;
        u256_add(twice, acc);
        if (u256_cmp(twice, Mv) > 0) {
            U256 mma = Mv;
            u256_sub(mma, acc);
            U256 neg;
            u256_sub(neg, mma);
            acc = neg;
        }
        return acc;
    }
};

}  // namespace

// ---------------------------------------------------------------------------------------------
// Scheme I (ozaki1/kernels/slice_tf_body.h:86-131, recon_tf_i32in.cpp:116-157, f64_tf.h:253-300)
// ---------------------------------------------------------------------------------------------
// tfMulR: triple-float times a general radix with Dekker splitting by 4097 (sfpu_tf_proc.h:108-141);
// the register names follow the procedure so that the operation order can be checked line by line.
void tf_mul_r(float& hi, float& mid, float& lo, float r) {
    float acc_hi = hi, acc_mid = mid, acc_lo = lo, term, tmp0, tmp1, tmp2, keep;
    acc_lo = f_mul(acc_lo, r);
    tmp1 = f_mul(acc_mid, 4097.0f);
    tmp2 = f_sub(tmp1, acc_mid);
    tmp1 = f_sub(tmp1, tmp2);
    tmp2 = f_sub(acc_mid, tmp1);
    tmp1 = f_mul(tmp1, r);
    tmp2 = f_mul(tmp2, r);
    term = f_add(tmp1, tmp2);
    keep = f_sub(term, tmp1);
    tmp0 = f_sub(tmp2, keep);
    tmp1 = f_mul(acc_hi, 4097.0f);
    tmp2 = f_sub(tmp1, acc_hi);
    tmp1 = f_sub(tmp1, tmp2);
    tmp2 = f_sub(acc_hi, tmp1);
    tmp1 = f_mul(tmp1, r);
    tmp2 = f_mul(tmp2, r);
    acc_mid = f_add(tmp1, tmp2);
    keep = f_sub(acc_mid, tmp1);
    acc_hi = f_sub(tmp2, keep);
    tmp0 = f_add(tmp0, acc_lo);
    two_sum(term, tmp0, tmp1, tmp2);
    two_sum(acc_hi, tmp1, term, tmp0);
    two_sum(acc_mid, term, acc_hi, tmp1);
    tmp2 = f_add(tmp2, tmp0);
    fast_two_sum(tmp1, tmp2, acc_mid, acc_lo);
    hi = acc_hi;
    mid = acc_mid;
    lo = acc_lo;
}
// tfMulRadix: the power-of-two form when the radix has no significand bits (sfpu_tf.h:131-134).
inline void tf_mul_radix(float& hi, float& mid, float& lo, float r) {
    if ((f_bits(r) & 0x7FFFFFu) == 0u)
        tf_mul_pow2(hi, mid, lo, r);
    else
        tf_mul_r(hi, mid, lo, r);
}
// tfAddS<3> (sfpu_tf_proc.h:184-198) on a plain triple.
void tf_add_s(float& hi, float& mid, float& lo, float v) {
    float tmp0 = f_add(hi, v);
    float tmp1 = f_sub(tmp0, hi);
    float tmp2 = f_sub(tmp0, tmp1);
    tmp2 = f_sub(hi, tmp2);
    tmp1 = f_sub(v, tmp1);
    tmp1 = f_add(tmp2, tmp1);
    hi = tmp0;
    tmp0 = f_add(mid, tmp1);
    tmp2 = f_sub(tmp0, mid);
    float term = f_sub(tmp0, tmp2);
    term = f_sub(mid, term);
    tmp2 = f_sub(tmp1, tmp2);
    tmp2 = f_add(term, tmp2);
    mid = tmp0;
    lo = f_add(lo, tmp2);
}
// acc64_term and assemble_tf_f64 (f64_tf.h:214-300): three limbs -> FP64 times W 2^qw 2^g.
int64_t acc64_term(int32_t sig, int32_t sh) {
    if (!sig) return 0;
    if (sh >= 0) return (int64_t)((uint64_t)(int64_t)sig << sh);
    if (sh <= -32) return 0;
    const uint32_t n = (uint32_t)(-sh);
    const int32_t m = sig < 0 ? -sig : sig;
    const int64_t q = (int64_t)(m >> n);
    return sig < 0 ? -q : q;
}
uint64_t assemble_tf_f64(uint32_t hb, uint32_t mb, uint32_t lb, int32_t g, uint32_t Whi, uint32_t Wlo, int32_t qw) {
    int32_t eh, em, el, gh, gm, gl;
    dec32(hb, eh, gh);
    dec32(mb, em, gm);
    dec32(lb, el, gl);
    if (gh == 0 && gm == 0 && gl == 0) return 0ull;
    int32_t ebase = std::max(eh, std::max(em, el));
    const int64_t ch = acc64_term(gh, eh - ebase + 37), cm = acc64_term(gm, em - ebase + 37),
                  cl = acc64_term(gl, el - ebase + 37);
    int64_t acc = ch + cm + cl;
    if (acc == 0) {
        if (ch) eh = gh = 0;
        if (cm) em = gm = 0;
        if (cl) el = gl = 0;
        if (gh == 0 && gm == 0 && gl == 0) return 0ull;
        ebase = std::max(eh, std::max(em, el));
        acc = acc64_term(gh, eh - ebase + 37) + acc64_term(gm, em - ebase + 37) + acc64_term(gl, el - ebase + 37);
    }
    if (acc == 0) return 0ull;
    const uint64_t sgn = acc < 0 ? 0x8000000000000000ull : 0ull;
    uint64_t A = acc < 0 ? (uint64_t)(-acc) : (uint64_t)acc;
    const int32_t shA = __builtin_clzll(A);
    A <<= shA;
    return pack_f64(A, Whi, Wlo, qw + g + (ebase - 187) - shA, sgn);
}
// radix^-(L+2) as a 64-bit significand and exponent (ozaki1/plan.hpp:446-460, bits.hpp:35-40).
void oz1_scale_w(int radix, int L, uint32_t& Whi, uint32_t& Wlo, int32_t& qw) {
    long double w = 1.0L;
    for (int i = 0; i < L + 2; i++) w /= (long double)radix;
    int e;
    const long double f = frexpl(w, &e);
    const unsigned long long W = (unsigned long long)ldexpl(f, 64);
    Whi = (uint32_t)(W >> 32);
    Wlo = (uint32_t)W;
    qw = e - 64;
}

// A8 for any modulus up to 4096: the residues of A' as values of type T, planes[s][r][c].
template <class T>
static void residue_planes(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                           const int* m, T* planes) {
    std::vector<float> rinv(S), cw((size_t)S * 4);
    for (int s = 0; s < S; s++) {
        const __float128 q = (__float128)1 / (__float128)m[s];
        rinv[s] = (float)(double)q;
        for (int j = 0; j < 4; j++) cw[(size_t)s * 4 + j] = pow2mod(20 * (j + 1), m[s]);
    }
    const size_t plane = (size_t)rows * cols;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float dig[5];
        for (int c = 0; c < cols; c++) {
            make_digits(X[(size_t)r * ld + c], delta_of(delta, mode, r, c), nd, dig);
            for (int s = 0; s < S; s++) {
                const float v = residue(dig, nd, (float)m[s], rinv[s], &cw[(size_t)s * 4]);
                planes[(size_t)s * plane + (size_t)r * cols + c] = (T)(int)v;
            }
        }
    }
}

extern "C" {

uint64_t orc_hash_f64(const double* c, size_t n) {
    uint64_t h = 1469598103934665603ull;
    for (size_t z = 0; z < n; z++) {
        uint64_t u;
        std::memcpy(&u, &c[z], 8);
        for (int b = 0; b < 64; b += 8) {
            h ^= (u >> b) & 0xFFu;
            h *= 1099511628211ull;
        }
    }
    return h;
}

void orc_inputs(unsigned seed, double phi, size_t na, size_t nb, double* a, double* b) {
    std::mt19937 rng(seed);
    if (phi < 0) {
        std::uniform_real_distribution<double> u(-1, 1);
        for (size_t i = 0; i < na; i++) a[i] = u(rng);
        for (size_t i = 0; i < nb; i++) b[i] = u(rng);
        return;
    }
    std::uniform_real_distribution<double> u(0, 1);
    std::normal_distribution<double> normal(0, 1);
    auto value = [&] {
        const double v = u(rng);
        const double z = normal(rng);
        return (v - 0.5) * std::exp(phi * z);
    };
    for (size_t i = 0; i < na; i++) a[i] = value();
    for (size_t i = 0; i < nb; i++) b[i] = value();
}

void orc_scale(const double* X, int rows, int cols, int ld, int mode, int ceil_mode, int shift, int32_t* delta,
               uint32_t* flags) {
    const int nout = mode == 0 ? rows : cols;
    uint32_t bad = 0;
    for (int o = 0; o < nout; o++) {
        uint64_t mx = 0;  // max of the magnitude bit patterns (sign cleared)
        const int n = mode == 0 ? cols : rows;
        for (int t = 0; t < n; t++) {
            const double x = mode == 0 ? X[(size_t)o * ld + t] : X[(size_t)t * ld + o];
            uint64_t u;
            std::memcpy(&u, &x, 8);
            u &= 0x7FFFFFFFFFFFFFFFull;
            mx = std::max(mx, u);
        }
        const uint32_t h = (uint32_t)(mx >> 32), l = (uint32_t)mx;
        // oz_absf64_to_bf16<CEIL> (scale_bits.h:34-45)
        uint16_t v16;
        const int32_t E = (int32_t)((h >> 20) & 0x7FFu);
        if (E == 0x7FF)
            v16 = 0xFFC0u;
        else {
            const int32_t e8 = E - 896;
            if (e8 <= 0)
                v16 = (h | l) ? 0xFF80u : 0u;
            else if (e8 >= 255)
                v16 = 0x7F80u;
            else {
                uint32_t v = ((uint32_t)e8 << 7) | ((h >> 13) & 0x7Fu);
                if (ceil_mode == 1 && ((h & 0x1FFFu) || l)) v += 1u;
                if (ceil_mode == 2 && ((h & 0x1FFFu) || l || !(v & 0x7Fu))) v += 1u;
                v16 = (uint16_t)v;
            }
        }
        // oz_bf16_scale_exp (scale_bits.h:56-62)
        const uint32_t BE = (v16 >> 7) & 0xFFu, bm = v16 & 0x7Fu;
        int32_t e;
        if (BE == 0u)
            e = 0;
        else if (BE == 0xFFu) {
            e = 0;
            bad |= !(v16 & 0x8000u) ? 1u : bm ? 4u : 2u;
        } else
            e = (int32_t)BE - 127 + (bm ? 1 : 0);
        delta[o] = shift - e;
    }
    *flags |= bad;
}

void orc_split_f64(uint32_t w1, uint32_t w0, int32_t d, uint32_t* out4) {
    split_words(w1, w0, d, out4[0], out4[1], out4[2], out4[3]);
}

void orc_load_triple(double x, int32_t d, float* out3) { load_triple(x, d, out3[0], out3[1], out3[2]); }

void orc_oz2_digits(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd,
                    float* digits) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++)
            make_digits(X[(size_t)r * ld + c], delta_of(delta, mode, r, c), nd, digits + ((size_t)r * cols + c) * nd);
}

void orc_oz2_residues(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                      const int* m, int8_t* planes) {
    residue_planes(X, rows, cols, ld, mode, delta, nd, S, m, planes);
}

void orc_oz2_residues16(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                        const int* m, int16_t* planes) {
    residue_planes(X, rows, cols, ld, mode, delta, nd, S, m, planes);
}

// modslice_digit.cpp:195-218 + sparse_fix.h:53-73: the digits of residue r (d[0] = l, d[1] = h,
// d[2] = s), in the FP32 operation model. xmode 0 rounded, 1 Karatsuba, 2 sparse square.
static int split_residue(float r, int xmode, float q, float qinv, float* d) {
    if (xmode == 3) {  // one digit: the residue itself (split.hpp:202-205, modslice_digit.cpp:76-79)
        d[0] = r;
        return 1;
    }
    if (xmode == 1) {
        float sgn = std::signbit(r) ? 1.0f : 0.0f;          // Ltz
        sgn = f_add(f_mul(sgn, -2.0f), 1.0f);                // MulS -2, AddS 1
        const float t = f_mul(sgn, f_sub(f_mul(q, 0.5f), 0.5f));
        const float h = f_rnd(f_mul(f_add(r, t), qinv));
        const float l = f_sub(r, f_mul(h, q));
        d[0] = l;
        d[1] = h;
        d[2] = f_add(h, l);
        return 3;
    }
    float h = f_rnd(f_mul(r, qinv));
    float l = f_sub(r, f_mul(h, q));
    if (xmode == 2) {
        const float al = std::fabs(l);
        if (al > 16.5f && ((int)al & 1)) {
            if (l < 0.0f) {
                l = f_add(l, q);
                h = f_sub(h, 1.0f);
            } else {
                l = f_sub(l, q);
                h = f_add(h, 1.0f);
            }
        }
        const float ah = std::fabs(h);
        if (ah > 16.5f && ((int)ah & 1)) h = h < 0.0f ? f_add(h, q) : f_sub(h, q);
    }
    d[0] = l;
    d[1] = h;
    return 2;
}

void orc_oz2_digit_planes(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                          const int* m, const int* q, const int* xmode, int8_t* planes) {
    std::vector<float> rinv(S), cw((size_t)S * 4);
    std::vector<int> poff(S);
    int np = 0;
    for (int s = 0; s < S; s++) {
        const __float128 qq = (__float128)1 / (__float128)m[s];
        rinv[s] = (float)(double)qq;
        for (int j = 0; j < 4; j++) cw[(size_t)s * 4 + j] = pow2mod(20 * (j + 1), m[s]);
        poff[s] = np;
        np += xmode[s] == 1 ? 3 : (xmode[s] == 3 ? 1 : 2);
    }
    const size_t plane = (size_t)rows * cols;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float dig[5], d[3];
        for (int c = 0; c < cols; c++) {
            make_digits(X[(size_t)r * ld + c], delta_of(delta, mode, r, c), nd, dig);
            for (int s = 0; s < S; s++) {
                const float v = residue(dig, nd, (float)m[s], rinv[s], &cw[(size_t)s * 4]);
                const float qf = (float)q[s];
                const int n = split_residue(v, xmode[s], qf, 1.0f / qf, d);
                for (int j = 0; j < n; j++)
                    planes[(size_t)(poff[s] + j) * plane + (size_t)r * cols + c] = (int8_t)(int)d[j];
            }
        }
    }
}

float orc_modround(float d, float m, float rinv) { return mod_round(d, m, rinv); }

int64_t orc_gemm_i8(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K) {
    int64_t mx = 0;
#pragma omp parallel for schedule(static) reduction(max : mx)
    for (int i = 0; i < M; i++) {
        std::vector<int64_t> acc(N, 0);
        for (int k = 0; k < K; k++) {
            const int64_t a = A[(size_t)i * K + k];
            if (!a) continue;
            const int8_t* b = B + (size_t)k * N;
            for (int j = 0; j < N; j++) acc[j] += a * b[j];
        }
        for (int j = 0; j < N; j++) {
            mx = std::max(mx, acc[j] < 0 ? -acc[j] : acc[j]);
            C[(size_t)i * N + j] = (int32_t)acc[j];
        }
    }
    return mx;
}

void orc_crt_constants(int S, const int* m, int b, orc_crt_consts* k) {
    std::memset(k, 0, sizeof(*k));
    k->S = S;
    k->b = b;
    for (int i = 0; i < S; i++) k->m[i] = m[i];
    // y_i = (prod_{j != i} m_j)^-1 mod m_i (extended Euclid), moduli.hpp:619-625
    for (int i = 0; i < S; i++) {
        long P = 1, mi = m[i];
        for (int j = 0; j < S; j++)
            if (j != i) P = (P * (m[j] % mi)) % mi;
        long t = 0, nt = 1, r = mi, nr = P % mi;
        while (nr != 0) {
            const long q = r / nr;
            long tmp = t - q * nt;
            t = nt;
            nt = tmp;
            tmp = r - q * nr;
            r = nr;
            nr = tmp;
        }
        if (t < 0) t += mi;
        k->yi[i] = (int)t;
    }
    // KM = M * 2^-2b in long double (moduli.hpp:628-631); W and qw by frexpl (bits.hpp:35-40)
    long double Mld = 1.0L;
    for (int i = 0; i < S; i++) Mld *= (long double)m[i];
    const long double KMl = Mld * std::pow(2.0L, -2.0 * b);
    k->KM = (double)KMl;
    int e;
    const long double f = frexpl(KMl, &e);
    const unsigned long long W = (unsigned long long)ldexpl(f, 64);
    k->Whi = (uint32_t)(W >> 32);
    k->Wlo = (uint32_t)W;
    k->qw = e - 64;
    // 12-bit fragments of 1/m_i (moduli.hpp:654-686)
    const float SPL = 4097.0f;
    auto top12 = [&](__float128 v) {
        const float p = (float)(double)v;
        if (p == 0.0f) return 0.0f;
        const float c = (float)((double)SPL * (double)p);
        return (float)((double)c - (double)(float)((double)c - (double)p));
    };
    for (int i = 0; i < S; i++) {
        const __float128 r = (__float128)1 / (__float128)m[i];
        const __float128 gran = powq((__float128)2, -(__float128)64);
        const __float128 Rg = roundq(r / gran) * gran;
        __float128 v = Rg;
        for (int t = 0; t < 5; ++t) {
            k->rp1[i][t] = top12(v);
            v -= (__float128)k->rp1[i][t];
        }
        const __float128 sum1 = Rg - v;
        v = r - sum1;
        for (int t = 0; t < 3; ++t) {
            k->rp2[i][t] = (t + 1 < 3) ? top12(v) : (float)(double)v;
            v -= (__float128)k->rp2[i][t];
        }
        v = r;
        for (int t = 0; t < 5; ++t) {
            k->rp0[i][t] = (t + 1 < 5) ? top12(v) : (float)(double)v;
            v -= (__float128)k->rp0[i][t];
        }
        k->rinv[i] = (float)(double)r;
        for (int j = 0; j < 4; j++) k->c[j][i] = pow2mod(20 * (j + 1), m[i]);
        k->m16[i] = pow2mod(16, m[i]);
    }
    k->nsmall0 = choose_small_tail(&k->rp0[0][0], 5, k->m, (uint32_t)S);
    k->nsmall1 = choose_small_tail(&k->rp1[0][0], 5, k->m, (uint32_t)S);
    k->nsmall2 = choose_small_tail(&k->rp2[0][0], 3, k->m, (uint32_t)S);
}

void orc_oz2_crt_ref(const int32_t* C, int M, int N, int S, const int* m, int b, int nd, int two_pass,
                     const int32_t* dA, const int32_t* dB, double* out) {
    orc_crt_consts k;
    orc_crt_constants(S, m, b, &k);
    const int32_t shift = b - 20 * (nd - 1);
    const int32_t sh2 = 2 * shift;
    const size_t stride = (size_t)M * N;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        for (int j = 0; j < N; j++) {
            const size_t idx = (size_t)i * N + j;
            const int32_t gg = sh2 - (dA[i] + dB[j]);
            float limbs[3];
            uint64_t u;
            if (!two_pass) {
                crt_pass(C, stride, idx, k, &k.rp0[0][0], 5, k.nsmall0, limbs);
                A128 a{{0, 0, 0, 0}};
                a128_add_limbs(a, limbs, 3);
                u = a128_frac_to_f64(a, gg, k.Whi, k.Wlo, k.qw);
            } else {
                A128 a{{0, 0, 0, 0}};
                crt_pass(C, stride, idx, k, &k.rp1[0][0], 5, k.nsmall1, limbs);
                a128_add_limbs(a, limbs, 3);
                crt_pass(C, stride, idx, k, &k.rp2[0][0], 3, k.nsmall2, limbs);
                a128_add_limbs(a, limbs, 3);
                u = a128_frac_to_f64(a, gg, k.Whi, k.Wlo, k.qw);
            }
            std::memcpy(&out[idx], &u, 8);
        }
    }
}

void orc_oz2_crt_exact_int(const int32_t* r, int S, const int* m, uint64_t* out4) {
    ExactCrt x(S, m);
    const U256 v = x.value(r);
    for (int i = 0; i < 4; i++) out4[i] = v.w[i];
}

void orc_oz2_crt_exact(const int32_t* C, int M, int N, int S, const int* m, int b, int nd, const int32_t* dA,
                       const int32_t* dB, double* out) {
    const int32_t shift = b - 20 * (nd - 1);
    const size_t stride = (size_t)M * N;
    const ExactCrt x(S, m);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        int32_t r[24];
        for (int j = 0; j < N; j++) {
            const size_t idx = (size_t)i * N + j;
            for (int s = 0; s < S; s++) r[s] = C[(size_t)s * stride + idx];
            const U256 v = x.value(r);
            const int g = 2 * shift - (dA[i] + dB[j]);  // eA + eB
            out[idx] = u256_to_double(v, g - 2 * b);
        }
    }
}

void orc_gemm_quad_sample(const double* A, const double* B, int M, int N, int K, int nsample, const int* rows,
                          const int* cols, double* out) {
    (void)M;
#pragma omp parallel for schedule(dynamic)
    for (int t = 0; t < nsample; t++) {
        __float128 s = 0;
        const int i = rows[t], j = cols[t];
        for (int k = 0; k < K; k++) s += (__float128)A[(size_t)i * K + k] * (__float128)B[(size_t)k * N + j];
        out[t] = (double)s;
    }
}

// One block of rows [ib, i1) of the Dot2 GEMM, every column, in the reference's loop order (row
// blocks of 8, column blocks of 512, k outermost inside a block). The reference builds its
// evaluator with -O3 -march=native (Makefile:16, :132); this library travels to hosts other than
// the one it is built on, so the same code is compiled three times, for AVX-512, for AVX2 with FMA
// and for the baseline instruction set, and dot2_block picks by the CPU's features at run time
// (__builtin_cpu_supports, which tests features and so holds on any vendor's CPU). No choice
// changes a result: contraction stays off, the vectorized loop runs over independent columns, and
// the only FMA is the explicit one of TwoProduct (a library call on the baseline path).
__attribute__((always_inline)) static inline void dot2_block_body(const double* __restrict A,
                                                                  const double* __restrict B, int N, int K, int ib,
                                                                  int i1, double* __restrict Chi,
                                                                  double* __restrict Clo) {
    const int JB = 512;
    for (int j0 = 0; j0 < N; j0 += JB) {
        const int j1 = std::min(j0 + JB, N);
        for (int k = 0; k < K; ++k) {
            const double* __restrict Br = B + (size_t)k * N;
            for (int i = ib; i < i1; ++i) {
                const double a = A[(size_t)i * K + k];
                double* __restrict chi = Chi + (size_t)i * N;
                double* __restrict clo = Clo + (size_t)i * N;
                for (int j = j0; j < j1; ++j) {
                    const double bb = Br[j];
                    const double p = a * bb, e = std::fma(a, bb, -p);
                    const double c0 = chi[j];
                    const double s = c0 + p, z = s - c0;
                    clo[j] += (c0 - (s - z)) + (p - z) + e;
                    chi[j] = s;
                }
            }
        }
    }
}
__attribute__((target("avx512f,avx512dq,avx512vl,avx2,fma"))) static void dot2_block_avx512(
    const double* __restrict A, const double* __restrict B, int N, int K, int ib, int i1, double* __restrict Chi,
    double* __restrict Clo) {
    dot2_block_body(A, B, N, K, ib, i1, Chi, Clo);
}
__attribute__((target("avx2,fma"))) static void dot2_block_avx2(const double* __restrict A, const double* __restrict B,
                                                                 int N, int K, int ib, int i1, double* __restrict Chi,
                                                                 double* __restrict Clo) {
    dot2_block_body(A, B, N, K, ib, i1, Chi, Clo);
}
static void dot2_block_base(const double* __restrict A, const double* __restrict B, int N, int K, int ib, int i1,
                            double* __restrict Chi, double* __restrict Clo) {
    dot2_block_body(A, B, N, K, ib, i1, Chi, Clo);
}
static void dot2_block(const double* A, const double* B, int N, int K, int ib, int i1, double* Chi, double* Clo) {
    static const int level = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512dq") &&
                                     __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("fma")
                                 ? 2
                             : __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") ? 1
                                                                                              : 0;
    if (level == 2)
        dot2_block_avx512(A, B, N, K, ib, i1, Chi, Clo);
    else if (level == 1)
        dot2_block_avx2(A, B, N, K, ib, i1, Chi, Clo);
    else
        dot2_block_base(A, B, N, K, ib, i1, Chi, Clo);
}

void orc_dot2_gemm(const double* A, const double* B, int M, int N, int K, int r0, int r1, double* Chi, double* Clo) {
    (void)M;
    const int IB = 8;
    for (size_t z = (size_t)r0 * N; z < (size_t)r1 * N; z++) Chi[z] = Clo[z] = 0.0;
#pragma omp parallel for schedule(static)
    for (int ib = r0; ib < r1; ib += IB) dot2_block(A, B, N, K, ib, std::min(ib + IB, r1), Chi, Clo);
}

// Scheme I slicer (slice_tf_body.h:86-131 with the step of sfpu_tf_emu.hpp:193-198): p digits of
// x*2^delta in radix `radix`, digit bound dmax, planes[i][r][c] as int8.
void orc_oz1_slices(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int p, int radix,
                    int dmax, int8_t* planes) {
    const float r = (float)radix, dm = (float)dmax;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < cols; j++) {
            float hi, mid, lo;
            load_triple(X[(size_t)i * ld + j], delta_of(delta, mode, i, j), hi, mid, lo);
            for (int t = 0; t < p; t++) {
                tf_mul_radix(hi, mid, lo, r);
                float d = f_rnd(hi);
                if (d < -dm)
                    d = -dm;
                else if (d >= dm)
                    d = dm;
                hi = f_sub(hi, d);
                planes[((size_t)t * rows + i) * cols + j] = (int8_t)(int)d;
            }
        }
}

// tfMulR with each limb product and its error taken by one multiply and one FMA (TwoProduct), in the
// FP32 model: the form the GPU's slicer and reconstruction use where it gives tf_mul_r's result.
static void tf_mul_r_twoproduct(float& hi, float& mid, float& lo, float r) {
    auto f_fma = [](float a, float b, float c) { return flush(std::fmaf(flush(a), flush(b), flush(c))); };
    const float acc_lo = f_mul(lo, r);
    const float p1 = f_mul(mid, r);
    float tmp0 = f_fma(mid, r, -p1);
    const float p0 = f_mul(hi, r);
    const float f0 = f_fma(hi, r, -p0);
    tmp0 = f_add(tmp0, acc_lo);
    float sa, ea, sb, eb, r0, ec;
    two_sum(p1, tmp0, sa, ea);
    two_sum(f0, sa, sb, eb);
    two_sum(p0, sb, r0, ec);
    const float g = f_add(ea, eb);
    hi = r0;
    fast_two_sum(ec, g, mid, lo);
}

// The TwoProduct form with two of its TwoSums taken as FastTwoSums, the form the GPU's slicer uses: FastTwoSum(a, b) gives TwoSum's (sum, error) exactly when |a| >= |b| (or a = 0)
// and nothing overflows or is flushed. (p1, tmp0): tmp0 is the rounding error of mid*r plus lo*r, at
// most about one unit in the last place of p1; (p0, sb): sb collects the lower limbs' products, below
// one unit in the last place of p0. `violations` counts the calls where that order does not hold.
static void tf_mul_r_fast(float& hi, float& mid, float& lo, float r, int64_t& violations) {
    auto f_fma = [](float a, float b, float c) { return flush(std::fmaf(flush(a), flush(b), flush(c))); };
    const float acc_lo = f_mul(lo, r);
    const float p1 = f_mul(mid, r);
    float tmp0 = f_fma(mid, r, -p1);
    const float p0 = f_mul(hi, r);
    const float f0 = f_fma(hi, r, -p0);
    tmp0 = f_add(tmp0, acc_lo);
    float sa, ea, sb, eb, r0, ec;
    if (p1 != 0.0f && std::fabs(p1) < std::fabs(tmp0)) violations++;
    fast_two_sum(p1, tmp0, sa, ea);
    two_sum(f0, sa, sb, eb);
    if (p0 != 0.0f && std::fabs(p0) < std::fabs(sb)) violations++;
    fast_two_sum(p0, sb, r0, ec);
    const float g = f_add(ea, eb);
    hi = r0;
    fast_two_sum(ec, g, mid, lo);
}

// Equivalence check of tfMulR forms against Dekker's (tf_mul_r, the reference's) on n pseudo-random
// chains; form(hi, mid, lo, r, violations) is the other form. mode 0, the slicer: x*2^d of a random
// double, scaled near 1/2 or 50-100 binades below, then `planes` digits in radix r with bound dmax; a
// chain counts as covered when the GPU takes the TwoProduct form for it (x's last significand bit
// weighs at least 2^-126, or x is zero; and |hi| r <= dmax + 1/2, so that the state never grows), and
// as differing when any digit differs. mode 1, the reconstruction: Horner chains of up to `planes`
// diagonal sums (int32, added as the reference's high and low parts), all covered; differing when a
// triple differs. Returns the number of covered chains that differ; *covered receives the covered
// count and *violations the form's precondition failures on covered chains.
// tfMulP2 with both TwoSums taken as FastTwoSums, the form the GPU's slicer uses for a power-of-two
// radix: (mid, lo) with |lo| at most a unit in the last place of mid, and (hi, fl(mid + lo)) with
// |mid| <= |hi|/2 in every slicer state. `violations` counts the calls where that order does not hold.
static void tf_mul_pow2_fast(float& hi, float& mid, float& lo, float r, int64_t& violations) {
    hi = f_mul(hi, r);
    mid = f_mul(mid, r);
    lo = f_mul(lo, r);
    float s3, e4, s5, e6;
    if (mid != 0.0f && std::fabs(mid) < std::fabs(lo)) violations++;
    fast_two_sum(mid, lo, s3, e4);
    if (hi != 0.0f && std::fabs(hi) < std::fabs(s3)) violations++;
    fast_two_sum(hi, s3, s5, e6);
    hi = s5;
    fast_two_sum(e6, e4, mid, lo);
}

}  // extern "C"

template <class FORM, class REF>
static int64_t check_forms(FORM form, REF ref, int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                           int64_t* covered, int64_t* violations, bool all_chains = false) {
    const float r = (float)radix, dm = (float)dmax;
    int64_t bad = 0, cov = 0, viol = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad, cov, viol)
    for (int64_t it = 0; it < n; it++) {
        std::mt19937_64 g(seed * 0x9E3779B97F4A7C15ull + (uint64_t)it);
        bool same = true, covered_chain = true;
        int64_t v = 0;
        if (mode == 0) {
            uint64_t u = g();
            const int E = (int)(g() % 2047);
            u = (u & 0x800FFFFFFFFFFFFFull) | ((uint64_t)E << 52);
            double x;
            std::memcpy(&x, &u, 8);
            int k = (int)(g() % 9);
            if (g() % 2 == 0) k = 50 + (int)(g() % 51);
            const int32_t d = -2 - k - (E - 1023);
            float h1, m1, l1;
            load_triple(x, d, h1, m1, l1);
            float h2 = h1, m2 = m1, l2 = l1;
            covered_chain = all_chains || ((E == 0 || E - 1075 + d >= -126) && std::fabs(h1) * r <= dm + 0.5f);
            for (int t = 0; t < planes; t++) {
                ref(h1, m1, l1, r);
                form(h2, m2, l2, r, v);
                float a = f_rnd(h1), b = f_rnd(h2);
                a = a < -dm ? -dm : (a >= dm ? dm : a);
                b = b < -dm ? -dm : (b >= dm ? dm : b);
                same = same && a == b;
                h1 = f_sub(h1, a);
                h2 = f_sub(h2, b);
            }
        } else if (mode == 2) {
            // Scheme II digit chains (make_digits): the scaled element below 2^sh, digit = Rnd(hi) with
            // no clamp, then `planes` multiplications by the radix, each followed by a digit
            uint64_t u = g();
            const int E = (int)(g() % 2047);
            u = (u & 0x800FFFFFFFFFFFFFull) | ((uint64_t)E << 52);
            double x;
            std::memcpy(&x, &u, 8);
            const int sh = (int)(g() % 25);
            int k = (int)(g() % 9);
            if (g() % 2 == 0) k = 50 + (int)(g() % 51);
            const int32_t d = sh - 1 - k - (E - 1023);
            float h1, m1, l1;
            load_triple(x, d, h1, m1, l1);
            float h2 = h1, m2 = m1, l2 = l1;
            for (int t = 0; t <= planes; t++) {
                if (t > 0) {
                    ref(h1, m1, l1, r);
                    form(h2, m2, l2, r, v);
                }
                const float a = f_rnd(h1), b = f_rnd(h2);
                same = same && a == b;
                h1 = f_sub(h1, a);
                h2 = f_sub(h2, b);
            }
        } else {
            const int p = 1 + (int)(g() % (uint64_t)planes);
            float h1 = 0, m1 = 0, l1 = 0, h2 = 0, m2 = 0, l2 = 0;
            for (int dd = 0; dd < p; dd++) {
                if (dd) {
                    ref(h1, m1, l1, r);
                    form(h2, m2, l2, r, v);
                }
                int64_t w;
                switch (g() % 4) {
                case 0: w = (int64_t)(g() % 4294967295ull) - 2147483647; break;
                case 1: w = (g() & 1) ? 2147483647 : -2147483647; break;
                case 2: w = (int64_t)(g() % 200001) - 100000; break;
                default: w = 0;
                }
                const float vh = (float)(int32_t)((uint32_t)w & 0xFFFFFF00u), vl = (float)(int32_t)((uint32_t)w & 0xFFu);
                tf_add_s(h1, m1, l1, vh);
                tf_add_s(h1, m1, l1, vl);
                tf_add_s(h2, m2, l2, vh);
                tf_add_s(h2, m2, l2, vl);
            }
            same = f_bits(h1) == f_bits(h2) && f_bits(m1) == f_bits(m2) && f_bits(l1) == f_bits(l2);
        }
        if (covered_chain) {
            cov++;
            viol += v;
            if (!same) bad++;
        }
    }
    *covered = cov;
    if (violations) *violations = viol;
    return bad;
}

extern "C" {

// Dekker's form against the TwoProduct form (tf_mul_r_twoproduct).
int64_t orc_check_tf_mul_r_forms(int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                                 int64_t* covered) {
    auto form = [](float& h, float& m, float& l, float r, int64_t&) { tf_mul_r_twoproduct(h, m, l, r); };
    auto ref = [](float& h, float& m, float& l, float r) { tf_mul_r(h, m, l, r); };
    return check_forms(form, ref, mode, n, seed, radix, dmax, planes, covered, nullptr);
}

// Dekker's form against the TwoProduct form with FastTwoSums (tf_mul_r_fast); *violations counts its
// precondition failures.
int64_t orc_check_tf_mul_r_fast(int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                                int64_t* covered, int64_t* violations) {
    auto form = [](float& h, float& m, float& l, float r, int64_t& v) { tf_mul_r_fast(h, m, l, r, v); };
    auto ref = [](float& h, float& m, float& l, float r) { tf_mul_r(h, m, l, r); };
    return check_forms(form, ref, mode, n, seed, radix, dmax, planes, covered, violations);
}

// tfMulP2 (the reference's, for a power-of-two radix) against tf_mul_pow2_fast on every chain of the
// mode (*covered = n; mode 0: slicer chains, 1: reconstruction chains, 2: Scheme II digit chains,
// digits.h:80-112); *violations counts its precondition failures.
int64_t orc_check_tf_mul_pow2_fast(int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                                   int64_t* covered, int64_t* violations) {
    auto form = [](float& h, float& m, float& l, float r, int64_t& v) { tf_mul_pow2_fast(h, m, l, r, v); };
    auto ref = [](float& h, float& m, float& l, float r) { tf_mul_pow2(h, m, l, r); };
    return check_forms(form, ref, mode, n, seed, radix, dmax, planes, covered, violations, true);
}

// Diagonal partial products P_d = sum_{i<=d} A_i B_{d-i} (ozaki1/gemm.hpp:315, stages.hpp:157), exact in
// int64; A: p planes M x K, B: p planes K x N (row-major); P: ndiag planes M x N as int32. Returns the
// largest |P| seen.
int64_t orc_oz1_gemm_diag(const int8_t* A, const int8_t* B, int32_t* P, int M, int N, int K, int p, int ndiag) {
    int64_t big = 0;
#pragma omp parallel for schedule(static) reduction(max : big)
    for (int i = 0; i < M; i++) {
        std::vector<int64_t> row((size_t)N);
        for (int d = 0; d < ndiag; d++) {
            std::fill(row.begin(), row.end(), 0);
            for (int a = 0; a <= d && a < p; a++) {
                const int b = d - a;
                if (b >= p) continue;
                const int8_t* Ar = A + ((size_t)a * M + i) * K;
                const int8_t* Bp = B + (size_t)b * K * N;
                for (int k = 0; k < K; k++) {
                    const int64_t av = Ar[k];
                    if (!av) continue;
                    const int8_t* Br = Bp + (size_t)k * N;
                    for (int j = 0; j < N; j++) row[j] += av * Br[j];
                }
            }
            for (int j = 0; j < N; j++) {
                big = std::max<int64_t>(big, row[j] < 0 ? -row[j] : row[j]);
                P[((size_t)d * M + i) * N + j] = (int32_t)row[j];
            }
        }
    }
    return big;
}

// Horner reconstruction and FP64 assembly of scheme I (recon_tf_i32in.cpp:116-157 with decode :87-113,
// recon_f64_writer.cpp:148-160, assemble_tf_f64). P: ndiag int32 planes M x N. signmag = 1: the INT8
// partial products (magnitude split at bit 8, sign multiplied back); 0: two's-complement split
// (v & ~0xFF) + (v & 0xFF). The first nsingle diagonals are read with one conversion (two's complement
// only). out = (hi+mid+lo) * radix^-(L+2) * 2^-(dA+dB).
void orc_oz1_recon(const int32_t* P, int M, int N, int ndiag, int radix, int signmag, int nsingle, const int32_t* dA,
                   const int32_t* dB, double* out) {
    uint32_t Whi, Wlo;
    int32_t qw;
    oz1_scale_w(radix, ndiag - 1, Whi, Wlo, qw);
    const float r = (float)radix;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float hi = 0.0f, mid = 0.0f, lo = 0.0f;
            for (int d = 0; d < ndiag; d++) {
                if (d > 0) tf_mul_radix(hi, mid, lo, r);
                const int32_t v = P[((size_t)d * M + i) * N + j];
                if (d < nsingle) {
                    tf_add_s(hi, mid, lo, (float)v);
                    continue;
                }
                float vh, vl;
                if (signmag) {
                    const uint32_t mag = v < 0 ? (uint32_t)(-(int64_t)v) : (uint32_t)v;
                    const float sg = v > 0 ? 1.0f : (v < 0 ? -1.0f : 0.0f);
                    vh = f_mul((float)(int32_t)(mag & 0x7FFFFF00u), sg);
                    vl = f_mul((float)(int32_t)(mag & 0xFFu), sg);
                } else {
                    vh = (float)(int32_t)((uint32_t)v & 0xFFFFFF00u);
                    vl = (float)(int32_t)((uint32_t)v & 0xFFu);
                }
                tf_add_s(hi, mid, lo, vh);
                tf_add_s(hi, mid, lo, vl);
            }
            const uint64_t u = assemble_tf_f64(f_bits(hi), f_bits(mid), f_bits(lo), -(dA[i] + dB[j]), Whi, Wlo, qw);
            std::memcpy(&out[(size_t)i * N + j], &u, 8);
        }
}

void orc_oz1_recon_blocks(const int32_t* P, int M, int N, int ndiag, int nkb, int radix, const int32_t* dA,
                          const int32_t* dB, double* out) {
    uint32_t Whi, Wlo;
    int32_t qw;
    oz1_scale_w(radix, ndiag - 1, Whi, Wlo, qw);
    const float r = (float)radix;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float ph = 0.0f, pm = 0.0f, pl = 0.0f;  // limbs carried from the previous blocks
            for (int kb = 0; kb < nkb; kb++) {
                float hi = 0.0f, mid = 0.0f, lo = 0.0f;
                for (int d = 0; d < ndiag; d++) {
                    if (d > 0) tf_mul_radix(hi, mid, lo, r);
                    tf_add_s(hi, mid, lo, (float)P[(((size_t)kb * ndiag + d) * M + i) * N + j]);
                }
                if (kb > 0) {
                    tf_add_s(hi, mid, lo, pl);
                    tf_add_s(hi, mid, lo, pm);
                    tf_add_s(hi, mid, lo, ph);
                }
                ph = hi;
                pm = mid;
                pl = lo;
            }
            const uint64_t u = assemble_tf_f64(f_bits(ph), f_bits(pm), f_bits(pl), -(dA[i] + dB[j]), Whi, Wlo, qw);
            std::memcpy(&out[(size_t)i * N + j], &u, 8);
        }
}

void orc_oz1_scale_w(int radix, int L, uint32_t* Whi, uint32_t* Wlo, int32_t* qw) { oz1_scale_w(radix, L, *Whi, *Wlo, *qw); }

// Scheme I INT8 end to end (ozaki1.cpp run(): scale with nshift -1 and rounding up, p slices of
// radix 254, diagonal products, Horner reconstruction). A: M x K, B: K x N row-major, dimensions
// already padded. Returns the largest |P_d|.
int64_t orc_oz1_int8_gemm(const double* A, const double* B, int M, int N, int K, int p, double* out) {
    std::vector<int32_t> dA(M), dB(N);
    uint32_t fl = 0;
    orc_scale(A, M, K, K, 0, 1, -1, dA.data(), &fl);
    orc_scale(B, K, N, N, 1, 1, -1, dB.data(), &fl);
    std::vector<int8_t> sa((size_t)p * M * K), sb((size_t)p * K * N);
    orc_oz1_slices(A, M, K, K, 0, dA.data(), p, 254, 127, sa.data());
    orc_oz1_slices(B, K, N, N, 1, dB.data(), p, 254, 127, sb.data());
    std::vector<int32_t> P((size_t)p * M * N);
    const int64_t big = orc_oz1_gemm_diag(sa.data(), sb.data(), P.data(), M, N, K, p, p);
    orc_oz1_recon(P.data(), M, N, p, 254, 1, 0, dA.data(), dB.data(), out);
    return big;
}

}  // extern "C"

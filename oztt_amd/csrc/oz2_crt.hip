// A10-A11: CRT reconstruction of Scheme II to FP64.
//
// Semantics (reference recon_crt.cpp:293 + recon_writer.cpp:70, f64_tf.h:327-400): from the S exact
// products C_s (C' = C_s mod m_s) recover C' in (-M/2, M/2), M = prod m_s, and return
// C' * 2^(eA_i + eB_j - 2b) as FP64, with results below the normal range flushed to signed zero.
// The reference approximates C'/M as a triple-float fraction (one pass, absolute accuracy about
// 2^-67) or two passes (granularity 2^-124) and rounds ties away from zero. This kernel computes C'
// exactly and rounds once to nearest-even, so it is at least as accurate as either reference mode
// and serves both.
//
// Per element, with k_s = (C_s mod m_s) * y_s mod m_s and Q_s = M/m_s (host constants):
//   acc = sum_s k_s * Q_s   (nw 32-bit words, < S*M), C' = acc mod M, then the symmetric
//   representative; the residues use exact integer division by the small moduli.
// MI355X design: one thread per output element; the S planes are read coalesced (plane-major),
// the constants are kernel arguments (uniform, held in scalar registers), the multiword
// arithmetic is 32-bit multiply-add with carries.
#include "oz2_modular.hpp"
#include "oz_internal.hpp"

namespace {

using oz2::mod_small;

template <int NW>
__device__ __forceinline__ double to_double_scaled(const uint32_t* w, int e2) {
    // w: two's complement NW-word integer; returns w * 2^e2 rounded to nearest-even (subnormal -> 0)
    uint32_t v[NW];
    const bool neg = (w[NW - 1] >> 31) != 0;
    if (neg) {
        uint32_t c = 1;
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const uint64_t t = (uint64_t)(~w[i]) + c;
            v[i] = (uint32_t)t;
            c = (uint32_t)(t >> 32);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NW; i++) v[i] = w[i];
    }
    int top = -1;  // index of the highest nonzero word
#pragma unroll
    for (int i = 0; i < NW; i++)
        if (v[i]) top = i;
    if (top < 0) return neg ? -0.0 : 0.0;
    // gather the 96 bits below and including the leading bit: hi word, next, next
    const uint32_t w2 = v[top];
    const uint32_t w1 = top >= 1 ? v[top - 1] : 0u;
    const uint32_t w0 = top >= 2 ? v[top - 2] : 0u;
    bool sticky_low = false;
#pragma unroll
    for (int i = 0; i < NW; i++)
        if (i < top - 2 && v[i]) sticky_low = true;
    const int lz = __clz(w2);
    // normalize the 96-bit window so that the leading bit is bit 95
    uint64_t hi64 = ((uint64_t)w2 << 32) | w1;  // bits 95..32 of the window
    uint32_t lo32 = w0;
    if (lz) {
        hi64 = (hi64 << lz) | (lo32 >> (32 - lz));
        lo32 <<= lz;
    }
    // hi64 holds the leading 64 bits; keep 53, round on the remaining 11 bits + lo32 + lower words
    uint64_t mant = hi64 >> 11;
    const uint64_t rest = hi64 & 0x7FFull;
    const bool guard = (rest >> 10) & 1ull;
    const bool sticky = (rest & 0x3FFull) || lo32 || sticky_low;
    // value = mant * 2^(position of mant LSB) with the leading bit at 32*top + 31 - lz
    int exp_lead = 32 * top + 31 - lz + e2;  // exponent of the leading bit
    if (guard && (sticky || (mant & 1ull))) {
        mant += 1ull;
        if (mant >> 53) {
            mant >>= 1;
            exp_lead += 1;
        }
    }
    if (exp_lead < -1022) return neg ? -0.0 : 0.0;
    if (exp_lead > 1023) return neg ? -__builtin_huge_val() : __builtin_huge_val();
    const uint64_t bits = ((uint64_t)(exp_lead + 1023) << 52) | (mant & 0x000FFFFFFFFFFFFFull);
    const double r = __longlong_as_double((long long)bits);
    return neg ? -r : r;
}

struct CrtArgs {
    oz2_crt_dev k;
    uint32_t magic[OZ2_MAXS];  // floor(2^32/m)
    uint32_t Mhalf[8];         // floor(M/2)
    double invM;               // 1 / Mprod (quotient estimate)
    // Moduli in groups of consecutive moduli whose product mG stays below 2^32 (the digit kernel):
    // sum_{s in g} k_s Q_s = QG_g * sum_{s in g} k_s w_s with w_s = mG_g / m_s and QG_g = Mprod / mG_g.
    int G;
    unsigned char gid[OZ2_MAXS], glast[OZ2_MAXS];  // group of modulus s; s is its group's last
    uint32_t mG[OZ2_MAXS], w[OZ2_MAXS];
    uint32_t QG[OZ2_MAXS][8];
};

// acc = sum_s k_s Q_s (< S*M) -> the symmetric representative of acc mod M, scaled by 2^e2, as FP64.
template <int NW>
__device__ __forceinline__ double crt_finish(uint32_t* acc, const CrtArgs& a, int e2) {
    // q = floor(acc / M) from FP64 approximations (|error| <= 1), then acc -= q*M with one correction
    double ahi = 0.0;
#pragma unroll
    for (int w = NW - 1; w >= 0; w--) ahi = ahi * 4294967296.0 + (double)acc[w];
    uint32_t q = (uint32_t)__builtin_floor(ahi * a.invM);
    {
        uint32_t carry = 0, borrow = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const uint64_t p = (uint64_t)q * a.k.Mw[w] + carry;
            carry = (uint32_t)(p >> 32);
            const uint64_t d = (uint64_t)acc[w] - (uint32_t)p - borrow;
            acc[w] = (uint32_t)d;
            borrow = (uint32_t)(d >> 63);
        }
        if (borrow || carry) {  // q was one too large: add M back
            uint32_t c2 = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const uint64_t t = (uint64_t)acc[w] + a.k.Mw[w] + c2;
                acc[w] = (uint32_t)t;
                c2 = (uint32_t)(t >> 32);
            }
        }
    }
    // q was one too small: subtract M once more when acc >= M (compare from the top word)
    {
        int cmp = 0;
#pragma unroll
        for (int w = NW - 1; w >= 0; w--)
            if (cmp == 0 && acc[w] != a.k.Mw[w]) cmp = acc[w] > a.k.Mw[w] ? 1 : -1;
        if (cmp >= 0) {
            uint32_t borrow = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const uint64_t d = (uint64_t)acc[w] - a.k.Mw[w] - borrow;
                acc[w] = (uint32_t)d;
                borrow = (uint32_t)(d >> 63);
            }
        }
    }
    // symmetric representative: acc > floor(M/2) -> acc - M
    {
        int cmp = 0;
#pragma unroll
        for (int w = NW - 1; w >= 0; w--)
            if (cmp == 0 && acc[w] != a.Mhalf[w]) cmp = acc[w] > a.Mhalf[w] ? 1 : -1;
        if (cmp > 0) {
            uint32_t borrow = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const uint64_t d = (uint64_t)acc[w] - a.k.Mw[w] - borrow;
                acc[w] = (uint32_t)d;
                borrow = (uint32_t)(d >> 63);
            }
        }
    }
    return to_double_scaled<NW>(acc, e2);
}

// acc += k * Q_s (NW words)
template <int NW>
__device__ __forceinline__ void crt_add(uint32_t* acc, uint32_t k, const uint32_t* Q) {
    uint32_t carry = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        const uint64_t p = (uint64_t)k * Q[w] + acc[w] + carry;
        acc[w] = (uint32_t)p;
        carry = (uint32_t)(p >> 32);
    }
}

// From the exact products C_s (int32): one thread per output element.
template <int NW>
__global__ void __launch_bounds__(256) crt_kernel(const int32_t* __restrict__ C, int M, int N, int ldc, long long sC,
                                                  CrtArgs a, const int32_t* __restrict__ dA,
                                                  const int32_t* __restrict__ dB, double* __restrict__ out, int ldo) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= N) return;
    const int32_t* c = C + (long long)i * ldc + j;
    uint32_t acc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) acc[w] = 0;
    for (int s = 0; s < a.k.S; s++)
        crt_add<NW>(acc, oz2::crt_digit(c[(long long)s * sC], a.k.m[s], a.k.y[s], a.magic[s]), a.k.Q[s]);
    const int g = 2 * a.k.shift - (dA[i] + dB[j]);  // eA + eB
    out[(long long)i * ldo + j] = crt_finish<NW>(acc, a, g - 2 * a.k.b);
}

// From the CRT digits k_s (uint8, written by the product kernel): one thread per 4 consecutive
// output elements of a row, so that each plane read is one 32-bit word per thread.
template <int NW>
__global__ void __launch_bounds__(256) crt_digits_kernel(const uint8_t* __restrict__ D, int M, int N, int ldd,
                                                         long long sD, CrtArgs a, const int32_t* __restrict__ dA,
                                                         const int32_t* __restrict__ dB, double* __restrict__ out,
                                                         int ldo) {
    const int j0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    const int i = blockIdx.y;
    if (j0 >= N) return;
    const uint32_t* d = reinterpret_cast<const uint32_t*>(D + (long long)i * ldd + j0);
    const long long sw = sD / 4;
    uint32_t acc[4][NW];
#pragma unroll
    for (int e = 0; e < 4; e++)
#pragma unroll
        for (int w = 0; w < NW; w++) acc[e][w] = 0;
    // every plane's word is requested before the first is used (S loads in flight per thread)
    const int S = a.k.S;
    uint32_t v[OZ2_MAXS];
#pragma unroll
    for (int s = 0; s < OZ2_MAXS; s++) v[s] = s < S ? d[(long long)s * sw] : 0u;
    // per group g: u = sum_{s in g} k_s w_s < count * mG < 2^34, reduced mod mG (at most three
    // subtractions), then acc += u * QG_g
    uint64_t u[4] = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < OZ2_MAXS; s++) {
        if (s < S) {
            const uint32_t ws = a.w[s];
#pragma unroll
            for (int e = 0; e < 4; e++) u[e] += (uint64_t)(((v[s] >> (8 * e)) & 0xFFu) * ws);
            if (a.glast[s]) {
                const int g = a.gid[s];
                const uint64_t mg = a.mG[g];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint64_t x = u[e];
                    x = x >= mg ? x - mg : x;
                    x = x >= mg ? x - mg : x;
                    x = x >= mg ? x - mg : x;
                    crt_add<NW>(acc[e], (uint32_t)x, a.QG[g]);
                    u[e] = 0;
                }
            }
        }
    }
    const int gi = 2 * a.k.shift - dA[i] - 2 * a.k.b;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (j0 + e < N) out[(long long)i * ldo + j0 + e] = crt_finish<NW>(acc[e], a, gi - dB[j0 + e]);
}

// Plane -> modulus of the uint16 CRT terms (digit formats).
struct TermMap {
    unsigned char mod[OZ2_MAXOUT];
};

// From the uint16 CRT terms w_o of the digit formats (oz2_gemm_groups_f8): acc = sum_o w_o Q_{s(o)},
// which is congruent to sum_s k_s Q_s modulo M because the terms of modulus s add up to k_s modulo
// m_s and m_s Q_s = M. One thread per 4 consecutive output elements (one 8-byte load per term).
template <int NW>
__global__ void __launch_bounds__(256) crt_terms_kernel(const uint16_t* __restrict__ W, int M, int N, int ldw,
                                                        long long sW, int nterms, CrtArgs a, TermMap tmap,
                                                        const int32_t* __restrict__ dA, const int32_t* __restrict__ dB,
                                                        double* __restrict__ out, int ldo) {
    const int j0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    const int i = blockIdx.y;
    if (j0 >= N) return;
    const uint2* w = reinterpret_cast<const uint2*>(W + (long long)i * ldw + j0);
    const long long sw = sW / 4;
    uint32_t acc[4][NW];
#pragma unroll
    for (int e = 0; e < 4; e++)
#pragma unroll
        for (int q = 0; q < NW; q++) acc[e][q] = 0;
    // batches of 8 terms: the 8 loads are in flight together
    for (int o0 = 0; o0 < nterms; o0 += 8) {
        uint2 v[8];
#pragma unroll
        for (int t = 0; t < 8; t++) v[t] = o0 + t < nterms ? w[(long long)(o0 + t) * sw] : make_uint2(0u, 0u);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            if (o0 + t < nterms) {
                const uint32_t* Q = a.k.Q[tmap.mod[o0 + t]];
                crt_add<NW>(acc[0], v[t].x & 0xFFFFu, Q);
                crt_add<NW>(acc[1], v[t].x >> 16, Q);
                crt_add<NW>(acc[2], v[t].y & 0xFFFFu, Q);
                crt_add<NW>(acc[3], v[t].y >> 16, Q);
            }
        }
    }
    const int gi = 2 * a.k.shift - dA[i] - 2 * a.k.b;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (j0 + e < N) out[(long long)i * ldo + j0 + e] = crt_finish<NW>(acc[e], a, gi - dB[j0 + e]);
}

template <int NW>
int launch_terms(oz_dev* dev, const uint16_t* W, int M, int N, int ldw, long long sW, int nterms, const CrtArgs& a,
                 const TermMap& tmap, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    hipLaunchKernelGGL(crt_terms_kernel<NW>, dim3(oz::ceil_div(N, 1024), M), dim3(256), 0, dev->stream, W, M, N, ldw,
                       sW, nterms, a, tmap, dA, dB, out, ldo);
    return oz::launch_check(dev, "crt_terms_kernel");
}

template <int NW>
int launch_crt(oz_dev* dev, const void* C, bool digits, int M, int N, int ldc, long long sC, const CrtArgs& a,
               const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    if (digits) {
        hipLaunchKernelGGL(crt_digits_kernel<NW>, dim3(oz::ceil_div(N, 1024), M), dim3(256), 0, dev->stream,
                           static_cast<const uint8_t*>(C), M, N, ldc, sC, a, dA, dB, out, ldo);
        return oz::launch_check(dev, "crt_digits_kernel");
    }
    hipLaunchKernelGGL(crt_kernel<NW>, dim3(oz::ceil_div(N, 256), M), dim3(256), 0, dev->stream,
                       static_cast<const int32_t*>(C), M, N, ldc, sC, a, dA, dB, out, ldo);
    return oz::launch_check(dev, "crt_kernel");
}

// Kernel constants of a CRT descriptor whose moduli are at most mmax.
int crt_args(oz_dev* dev, const char* name, const oz2_crt_dev* crt, uint32_t mmax, CrtArgs& a) {
    a = CrtArgs{};
    a.k = *crt;
    for (int s = 0; s < crt->S; s++) {
        if (crt->m[s] < 2 || crt->m[s] > mmax) return oz::fail(dev, OZ_ERR_ARG, "%s: modulus out of range", name);
        a.magic[s] = (uint32_t)(0x100000000ull / crt->m[s]);
    }
    // floor(M/2)
    uint32_t r = 0;
    for (int w = 7; w >= 0; w--) {
        const uint64_t cur = ((uint64_t)r << 32) | crt->Mw[w];
        a.Mhalf[w] = (uint32_t)(cur >> 1);
        r = (uint32_t)(cur & 1u);
    }
    a.invM = 1.0 / crt->Mtop;
    // groups of consecutive moduli with product below 2^32; QG = Mprod / mG by long division
    a.G = 0;
    for (int s = 0; s < crt->S;) {
        uint64_t mg = 1;
        int n = 0;
        while (s + n < crt->S && mg * crt->m[s + n] < 0x100000000ull) mg *= crt->m[s + n++];
        const int g = a.G++;
        a.mG[g] = (uint32_t)mg;
        for (int t = 0; t < n; t++) {
            a.w[s + t] = (uint32_t)(mg / crt->m[s + t]);
            a.gid[s + t] = (unsigned char)g;
            a.glast[s + t] = t == n - 1;
        }
        uint64_t rem = 0;
        for (int w = 7; w >= 0; w--) {
            const uint64_t cur = (rem << 32) | crt->Mw[w];
            a.QG[g][w] = (uint32_t)(cur / mg);
            rem = cur % mg;
        }
        if (rem) return oz::fail(dev, OZ_ERR_ARG, "%s: Mprod is not the product of the moduli", name);
        s += n;
    }
    return OZ_OK;
}

// Both entry points: C is int32 products (element strides) or uint8 digits (byte strides).
int crt_f64(oz_dev* dev, const char* name, const void* C, bool digits, int M, int N, int ldc, long long strideC,
            const oz2_crt_dev* crt, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    if (int st = oz::use(dev)) return st;
    if (!C || !crt || !dA || !dB || !out || M <= 0 || N <= 0 || ldc < N || ldo < N || crt->S < 1 ||
        crt->S > OZ2_MAXS || crt->nw < 3 || crt->nw > 8 || crt->Mtop <= 0.0 ||
        (digits && (ldc % 4 || strideC % 4 || ((uintptr_t)C & 3))))
        return oz::fail(dev, OZ_ERR_ARG, "%s: invalid arguments", name);
    CrtArgs a{};
    if (int st = crt_args(dev, name, crt, 255u, a)) return st;
    const size_t esz = digits ? 1 : 4;
    // the grid puts rows on y (at most 65535 per launch): launch in row chunks
    for (int i0 = 0; i0 < M; i0 += 65535) {
        const int rows = std::min(65535, M - i0);
        const void* Ci = static_cast<const char*>(C) + (size_t)i0 * ldc * esz;
        double* oi = out + (long long)i0 * ldo;
        int st;
        switch (crt->nw) {
        case 3: st = launch_crt<3>(dev, Ci, digits, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 4: st = launch_crt<4>(dev, Ci, digits, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 5: st = launch_crt<5>(dev, Ci, digits, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 6: st = launch_crt<6>(dev, Ci, digits, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        case 7: st = launch_crt<7>(dev, Ci, digits, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        default: st = launch_crt<8>(dev, Ci, digits, rows, N, ldc, strideC, a, dA + i0, dB, oi, ldo); break;
        }
        if (st) return st;
    }
    return OZ_OK;
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
        nterms > OZ2_MAXOUT || crt->S < 1 || crt->S > OZ2_MAXS || crt->nw < 3 || crt->nw > 8 || crt->Mtop <= 0.0 ||
        ldw % 4 || strideW % 4 || ((uintptr_t)W & 7) || (nterms > 1 && strideW < (long long)M * ldw))
        return oz::fail(dev, OZ_ERR_ARG, "%s: invalid arguments", name);
    CrtArgs a;
    if (int st = crt_args(dev, name, crt, 2401u, a)) return st;
    TermMap tmap{};
    for (int o = 0; o < nterms; o++) {
        if (term_modulus[o] >= crt->S) return oz::fail(dev, OZ_ERR_ARG, "%s: term %d names modulus %d", name, o, term_modulus[o]);
        tmap.mod[o] = term_modulus[o];
    }
    for (int i0 = 0; i0 < M; i0 += 65535) {
        const int rows = std::min(65535, M - i0);
        const uint16_t* Wi = W + (size_t)i0 * ldw;
        double* oi = out + (long long)i0 * ldo;
        int st;
        switch (crt->nw) {
        case 3: st = launch_terms<3>(dev, Wi, rows, N, ldw, strideW, nterms, a, tmap, dA + i0, dB, oi, ldo); break;
        case 4: st = launch_terms<4>(dev, Wi, rows, N, ldw, strideW, nterms, a, tmap, dA + i0, dB, oi, ldo); break;
        case 5: st = launch_terms<5>(dev, Wi, rows, N, ldw, strideW, nterms, a, tmap, dA + i0, dB, oi, ldo); break;
        case 6: st = launch_terms<6>(dev, Wi, rows, N, ldw, strideW, nterms, a, tmap, dA + i0, dB, oi, ldo); break;
        case 7: st = launch_terms<7>(dev, Wi, rows, N, ldw, strideW, nterms, a, tmap, dA + i0, dB, oi, ldo); break;
        default: st = launch_terms<8>(dev, Wi, rows, N, ldw, strideW, nterms, a, tmap, dA + i0, dB, oi, ldo); break;
        }
        if (st) return st;
    }
    return OZ_OK;
}

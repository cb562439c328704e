// A17: Scheme I reconstruction: Horner sum of the diagonal partial products and FP64 assembly.
//
// Semantics (reference ozaki1/kernels/recon_tf_i32in.cpp:116-157 with the decode at :87-113,
// recon_f64_writer.cpp:148-160, common/kernels/f64_tf.h:174-300). Per output element, with the
// partial sums P_d (int32) of the diagonals d = 0..L:
//   S = (((P_0) * radix + P_1) * radix + ...) + P_L      in triple-float (tfMulR / tfMulP2, tfAddS),
// each P_d entering as two exact FP32 values: for the INT8 products (signmag = 1) the magnitude split
// at bit 8 with the sign multiplied back, for two's-complement sums (signmag = 0) (v & ~0xFF) and
// (v & 0xFF); the first nsingle diagonals (two's complement only, |P_d| <= 2^24) enter as one value.
// Then C = (hi + mid + lo) * radix^-(L+2) * 2^-(dA+dB): the limbs are gathered in a 64-bit window
// below the largest limb, multiplied by the 64-bit significand W of radix^-(L+2) and rounded to FP64
// (ties away from zero on the guard bit; subnormal results become signed zero). The result equals
// the reference's bit for bit; the FP32 operations follow the rules of oz_tf32.hpp.
//
// MI355X design: one thread per output element; the L+1 planes are read coalesced (plane-major);
// the Horner step is about 75 FP32 operations per diagonal, the assembly integer arithmetic.
#pragma clang fp contract(off)

#include <cmath>

#include "oz_tf32.hpp"

namespace {

__device__ __forceinline__ void dec32(uint32_t u, int32_t& e, int32_t& sig) {
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

// +-A * W * 2^total rounded to FP64 (A, W in [2^63, 2^64)); the guard bit decides, ties go away from
// zero; subnormals become signed zero, overflow infinity.
__device__ __forceinline__ uint64_t pack_f64(uint64_t A, uint64_t W, int32_t total, uint64_t sgn) {
    const uint64_t hi = __umul64hi(A, W);
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

// sig * 2^sh in a 64-bit window, truncated toward zero below it.
__device__ __forceinline__ int64_t acc64_term(int32_t sig, int32_t sh) {
    if (!sig) return 0;
    if (sh >= 0) return (int64_t)((uint64_t)(int64_t)sig << sh);
    if (sh <= -32) return 0;
    const uint32_t n = (uint32_t)(-sh);
    const int32_t m = sig < 0 ? -sig : sig;
    const int64_t q = (int64_t)(m >> n);
    return sig < 0 ? -q : q;
}

// The three limbs gathered 37 bits above the largest limb's exponent, then scaled and rounded; a
// window that cancels to zero is gathered again from the limbs that fell below it.
__device__ __forceinline__ uint64_t assemble_tf_f64(float fh, float fm, float fl, int32_t g, uint64_t W, int32_t qw) {
    int32_t eh, em, el, gh, gm, gl;
    dec32(__float_as_uint(fh), eh, gh);
    dec32(__float_as_uint(fm), em, gm);
    dec32(__float_as_uint(fl), el, gl);
    if (gh == 0 && gm == 0 && gl == 0) return 0ull;
    int32_t ebase = max(eh, max(em, el));
    const int64_t ch = acc64_term(gh, eh - ebase + 37), cm = acc64_term(gm, em - ebase + 37),
                  cl = acc64_term(gl, el - ebase + 37);
    int64_t acc = ch + cm + cl;
    if (acc == 0) {
        if (ch) eh = gh = 0;
        if (cm) em = gm = 0;
        if (cl) el = gl = 0;
        if (gh == 0 && gm == 0 && gl == 0) return 0ull;
        ebase = max(eh, max(em, el));
        acc = acc64_term(gh, eh - ebase + 37) + acc64_term(gm, em - ebase + 37) + acc64_term(gl, el - ebase + 37);
    }
    if (acc == 0) return 0ull;
    const uint64_t sgn = acc < 0 ? 0x8000000000000000ull : 0ull;
    uint64_t A = acc < 0 ? (uint64_t)(-acc) : (uint64_t)acc;
    const int32_t shA = __clzll((long long)A);
    A <<= shA;
    return pack_f64(A, W, qw + g + (ebase - 187) - shA, sgn);
}

template <bool POW2, bool FMA, bool SIGNMAG>
__global__ void __launch_bounds__(256) recon_kernel(const int32_t* __restrict__ P, int M, int N, int ldp, long long sP,
                                                    int ndiag, int nsingle, float radix, uint64_t W, int32_t qw,
                                                    const int32_t* __restrict__ dA, const int32_t* __restrict__ dB,
                                                    double* __restrict__ out, int ldo) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= N) return;
    const int32_t* p = P + (long long)i * ldp + j;
    float hi = 0.0f, mid = 0.0f, lo = 0.0f;
    // batches of 8 diagonals: the 8 loads are in flight together
    for (int d0 = 0; d0 < ndiag; d0 += 8) {
        int32_t vb[8];
#pragma unroll
        for (int t = 0; t < 8; t++) vb[t] = d0 + t < ndiag ? p[(long long)(d0 + t) * sP] : 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int d = d0 + t;
            if (d >= ndiag) break;
            if (d > 0) tf_mul_radix<POW2, FMA>(hi, mid, lo, radix);
            const int32_t v = vb[t];
            if (!SIGNMAG && d < nsingle) {
                tf_add_s(hi, mid, lo, (float)v);
                continue;
            }
            float vh, vl;
            if constexpr (SIGNMAG) {
                const uint32_t mag = v < 0 ? (uint32_t)(-(int64_t)v) : (uint32_t)v;
                const float sg = v > 0 ? 1.0f : (v < 0 ? -1.0f : 0.0f);
                vh = (float)(int32_t)(mag & 0x7FFFFF00u) * sg;
                vl = (float)(int32_t)(mag & 0xFFu) * sg;
            } else {
                vh = (float)(int32_t)((uint32_t)v & 0xFFFFFF00u);
                vl = (float)(int32_t)((uint32_t)v & 0xFFu);
            }
            tf_add_s(hi, mid, lo, vh);
            tf_add_s(hi, mid, lo, vl);
        }
    }
    const uint64_t u = assemble_tf_f64(hi, mid, lo, -(dA[i] + dB[j]), W, qw);
    // non-temporal: C is not read again by the pass
    __builtin_nontemporal_store(__longlong_as_double((long long)u), &out[(long long)i * ldo + j]);
}

// One K block of the reconstruction that runs block by block (reference recon_tf_f32in.cpp:54-89
// with recon_f64_writer.cpp; ozaki1/plan.hpp:104-109): the block's diagonal sums P_d, exact
// integers of at most 2^24 (the FP32 products of the reference), enter whole into the Horner
// evaluation; then, after the first block, the three limbs carried from the previous blocks are
// added (lo, then mid, then hi). Every block but the last stores the limbs; the last assembles C.
template <bool POW2, bool FMA, bool ACC, bool EMIT>
__global__ void __launch_bounds__(256) recon_block_kernel(const int32_t* __restrict__ P, int M, int N, int ldp,
                                                          long long sP, int ndiag, float radix, float* __restrict__ L,
                                                          long long sL, int ldl, uint64_t W, int32_t qw,
                                                          const int32_t* __restrict__ dA,
                                                          const int32_t* __restrict__ dB, double* __restrict__ out,
                                                          int ldo) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= N) return;
    const int32_t* p = P + (long long)i * ldp + j;
    float hi = 0.0f, mid = 0.0f, lo = 0.0f;
    for (int d0 = 0; d0 < ndiag; d0 += 8) {
        int32_t vb[8];
#pragma unroll
        for (int t = 0; t < 8; t++) vb[t] = d0 + t < ndiag ? p[(long long)(d0 + t) * sP] : 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int d = d0 + t;
            if (d >= ndiag) break;
            if (d > 0) tf_mul_radix<POW2, FMA>(hi, mid, lo, radix);
            tf_add_s(hi, mid, lo, (float)vb[t]);
        }
    }
    float* l = L + (long long)i * ldl + j;
    if constexpr (ACC) {
        const float ph = l[0], pm = l[sL], pl = l[2 * sL];
        tf_add_s(hi, mid, lo, pl);
        tf_add_s(hi, mid, lo, pm);
        tf_add_s(hi, mid, lo, ph);
    }
    if constexpr (EMIT) {
        l[0] = hi;
        l[sL] = mid;
        l[2 * sL] = lo;
    } else {
        const uint64_t u = assemble_tf_f64(hi, mid, lo, -(dA[i] + dB[j]), W, qw);
        out[(long long)i * ldo + j] = __longlong_as_double((long long)u);
    }
}

template <bool POW2, bool FMA, bool ACC, bool EMIT>
int launch_block(oz_dev* dev, const int32_t* P, int M, int N, int ldp, long long sP, const oz1_recon_dev* r, float* L,
                 long long sL, int ldl, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    const uint64_t W = ((uint64_t)r->Whi << 32) | r->Wlo;
    for (int i0 = 0; i0 < M; i0 += 65535) {
        const int rows = min(65535, M - i0);
        hipLaunchKernelGGL((recon_block_kernel<POW2, FMA, ACC, EMIT>), dim3(oz::ceil_div(N, 256), rows), dim3(256), 0,
                           dev->stream, P + (long long)i0 * ldp, rows, N, ldp, sP, r->ndiag, (float)r->radix,
                           L + (long long)i0 * ldl, sL, ldl, W, r->qw, dA ? dA + i0 : dA, dB,
                           out ? out + (long long)i0 * ldo : out, ldo);
        if (int st = oz::launch_check(dev, "recon_block_kernel")) return st;
    }
    return OZ_OK;
}

template <bool POW2, bool FMA>
int launch_block_mode(oz_dev* dev, int first, int last, const int32_t* P, int M, int N, int ldp, long long sP,
                      const oz1_recon_dev* r, float* L, long long sL, int ldl, const int32_t* dA, const int32_t* dB,
                      double* out, int ldo) {
    if (first && last)
        return launch_block<POW2, FMA, false, false>(dev, P, M, N, ldp, sP, r, L, sL, ldl, dA, dB, out, ldo);
    if (first) return launch_block<POW2, FMA, false, true>(dev, P, M, N, ldp, sP, r, L, sL, ldl, dA, dB, out, ldo);
    if (last) return launch_block<POW2, FMA, true, false>(dev, P, M, N, ldp, sP, r, L, sL, ldl, dA, dB, out, ldo);
    return launch_block<POW2, FMA, true, true>(dev, P, M, N, ldp, sP, r, L, sL, ldl, dA, dB, out, ldo);
}

template <bool POW2, bool FMA, bool SIGNMAG>
int launch_recon(oz_dev* dev, const int32_t* P, int M, int N, int ldp, long long sP, const oz1_recon_dev* r,
                 const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    const uint64_t W = ((uint64_t)r->Whi << 32) | r->Wlo;
    for (int i0 = 0; i0 < M; i0 += 65535) {
        const int rows = min(65535, M - i0);
        hipLaunchKernelGGL((recon_kernel<POW2, FMA, SIGNMAG>), dim3(oz::ceil_div(N, 256), rows), dim3(256), 0,
                           dev->stream, P + (long long)i0 * ldp, rows, N, ldp, sP, r->ndiag, r->nsingle,
                           (float)r->radix, W, r->qw, dA + i0, dB, out + (long long)i0 * ldo, ldo);
        if (int st = oz::launch_check(dev, "recon_kernel")) return st;
    }
    return OZ_OK;
}

// The Horner values are integers, so no intermediate of tfMulR is subnormal, and every |value| is
// below 2^31 r^(p-1) r/(r-1) (|P_d| < 2^31). Below 2^127 / 4097 neither form of tfMulR overflows
// (Dekker's multiplies a limb by 4097), and its TwoProduct form gives the same triples.
bool recon_fma_safe(const oz1_recon_dev* r) {
    const double rad = r->radix;
    const double bits = 31.0 + (r->ndiag - 1) * std::log2(rad) + std::log2(rad / (rad - 1.0)) + std::log2(4097.0);
    return bits < 127.0;
}

// POW2: tfMulP2; otherwise tfMulR, in its TwoProduct form where recon_fma_safe allows
enum RadixForm { kDekker = 0, kTwoProduct = 1, kPow2 = 2 };
RadixForm radix_form(const oz1_recon_dev* r) {
    if ((r->radix & (r->radix - 1)) == 0) return kPow2;
    return recon_fma_safe(r) ? kTwoProduct : kDekker;
}

}  // namespace

extern "C" int oz1_recon_f64(oz_dev* dev, const int32_t* P, int M, int N, int ldp, long long strideP,
                             const oz1_recon_dev* r, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    if (int st = oz::use(dev)) return st;
    if (!P || !r || !dA || !dB || !out || M <= 0 || N <= 0 || ldp < N || ldo < N || r->ndiag < 1 || r->radix < 2 ||
        r->radix > 254 || !(r->Whi >> 31) || r->nsingle < 0 || (r->signmag && r->nsingle) ||
        (r->ndiag > 1 && strideP < (long long)M * ldp))
        return oz::fail(dev, OZ_ERR_ARG, "oz1_recon_f64: invalid arguments");
    const RadixForm form = radix_form(r);
    if (r->signmag)
        return form == kPow2        ? launch_recon<true, false, true>(dev, P, M, N, ldp, strideP, r, dA, dB, out, ldo)
               : form == kTwoProduct ? launch_recon<false, true, true>(dev, P, M, N, ldp, strideP, r, dA, dB, out, ldo)
                                     : launch_recon<false, false, true>(dev, P, M, N, ldp, strideP, r, dA, dB, out, ldo);
    return form == kPow2        ? launch_recon<true, false, false>(dev, P, M, N, ldp, strideP, r, dA, dB, out, ldo)
           : form == kTwoProduct ? launch_recon<false, true, false>(dev, P, M, N, ldp, strideP, r, dA, dB, out, ldo)
                                 : launch_recon<false, false, false>(dev, P, M, N, ldp, strideP, r, dA, dB, out, ldo);
}

extern "C" int oz1_recon_block_f64(oz_dev* dev, const int32_t* P, int M, int N, int ldp, long long strideP,
                                   const oz1_recon_dev* r, int first, int last, float* limbs, long long limb_stride,
                                   int ldl, const int32_t* dA, const int32_t* dB, double* out, int ldo) {
    if (int st = oz::use(dev)) return st;
    if (!P || !r || !limbs || M <= 0 || N <= 0 || ldp < N || ldl < N || r->ndiag < 1 || r->radix < 2 ||
        r->radix > 254 || r->signmag || (r->ndiag > 1 && strideP < (long long)M * ldp) ||
        limb_stride < (long long)M * ldl || (last && (!dA || !dB || !out || ldo < N || !(r->Whi >> 31))))
        return oz::fail(dev, OZ_ERR_ARG, "oz1_recon_block_f64: invalid arguments");
    const RadixForm form = radix_form(r);
    if (form == kPow2)
        return launch_block_mode<true, false>(dev, first, last, P, M, N, ldp, strideP, r, limbs, limb_stride, ldl, dA,
                                              dB, out, ldo);
    if (form == kTwoProduct)
        return launch_block_mode<false, true>(dev, first, last, P, M, N, ldp, strideP, r, limbs, limb_stride, ldl, dA,
                                              dB, out, ldo);
    return launch_block_mode<false, false>(dev, first, last, P, M, N, ldp, strideP, r, limbs, limb_stride, ldl, dA, dB,
                                           out, ldo);
}

// Triple-float FP32 procedures of the splitters and the scheme I reconstruction, and the blocked
// splitter kernel shared by both schemes.
//
// The reference defines its slices, digits and residues through binary32 operations with
// round-to-nearest-even, no fused multiply-add, and denormal inputs and outputs flushed to zero
// (its FP32 model, experiments/src/checks/sfpu_tf_emu.hpp:66-156). Every file that includes this
// header is compiled with -ffp-contract=off and -fgpu-flush-denormals-to-zero, and sets
// `#pragma clang fp contract(off)` before the include, so each operation below is one such binary32
// operation. Zero signs can differ from the model (its products with a zero factor are +0); a zero's
// sign never changes a digit, residue or reconstructed value.
#pragma once
#include <type_traits>

#include "oz_internal.hpp"

namespace {

// split_f64 + tf_load_f64 (reference f64_tf.h:141-172, slice_tf_core.h:67-76): x*2^d as the
// triple-float (hi, mid, lo), built with integer operations on the FP64 words.
__device__ __forceinline__ void load_triple(double x, int32_t d, float& hi, float& mid, float& lo) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(x);
    const uint32_t w1 = (uint32_t)(u >> 32), w0 = (uint32_t)u;
    const uint32_t sgn = w1 & 0x80000000u;
    const int32_t E = (int32_t)((w1 >> 20) & 0x7FFu);
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
    const bool carry = (a == 0x800000u);
    const int32_t eh = carry ? elsb + 180 : elsb + 179;
    const uint32_t mh = carry ? 0u : ((a << 1) & 0x7FFFFFu);
    const int32_t es = elsb + 134;
    const uint32_t hb = (eh > 0 && eh < 255) ? (sgn | ((uint32_t)eh << 23) | mh) : 0u;
    const uint32_t sb = (es > 0 && es < 255) ? (sgn | ((uint32_t)es << 23)) : 0u;
    const uint32_t braw = 0x4B000000u | (((uint32_t)(b + 0x400000)) & 0x7FFFFFu);
    const uint32_t craw = 0x4B000000u | c;
    const float s = __uint_as_float(sb);
    // zero and subnormals (E = 0) give the zero triple; selected at the end, so that no lane branches
    const bool zero = E == 0;
    hi = zero ? 0.0f : __uint_as_float(hb);
    mid = zero ? 0.0f : (__uint_as_float(braw) - 12582912.0f) * s;
    lo = zero ? 0.0f : ((__uint_as_float(craw) - 8388608.0f) * s) * 0.0078125f;
}

// TwoSum (Knuth) and FastTwoSum (Dekker) in the reference's operation order (sfpu_tf_proc.h:61-74).
__device__ __forceinline__ void two_sum(float x, float y, float& s, float& e) {
    s = x + y;
    float bb = s - x;
    float aa = s - bb;
    aa = x - aa;
    bb = y - bb;
    e = aa + bb;
}
__device__ __forceinline__ void fast_two_sum(float a, float b, float& s, float& t) {
    s = a + b;
    const float w = s - a;
    t = b - w;
}

// tfMulP2: the triple times a power of two r, renormalized (sfpu_tf_proc.h:160-169).
__device__ __forceinline__ void tf_mul_pow2(float& hi, float& mid, float& lo, float r) {
    hi = hi * r;
    mid = mid * r;
    lo = lo * r;
    float s3, e4, s5, e6;
    two_sum(mid, lo, s3, e4);
    two_sum(hi, s3, s5, e6);
    hi = s5;
    fast_two_sum(e6, e4, mid, lo);
}

// tfMulP2 on a slicer state, with both TwoSums taken as FastTwoSums; equal to tf_mul_pow2 bit for bit
// on such states. FastTwoSum(a, b) returns TwoSum's pair when |a| >= |b| or a = 0, and r scales the
// limbs exactly. Order of (mid, lo): a loaded triple has |lo| below one unit of mid's last chunk bit,
// or mid = 0; later states take (mid, lo) from FastTwoSum(e6, e4), with |lo| <= ulp(mid)/2. Order of
// (hi, s3): the slicer only subtracts an integer digit from hi, which leaves hi = 0 or a nonzero
// multiple of ulp(old hi) >= 2|mid| > |fl(mid + lo)|. The oracle's orc_check_tf_mul_pow2_fast checks
// the equality and counts order violations on slicer chains (radix 2 to 2^20, every exponent).
__device__ __forceinline__ void tf_mul_pow2_fast(float& hi, float& mid, float& lo, float r) {
    hi = hi * r;
    mid = mid * r;
    lo = lo * r;
    float s3, e4, s5, e6;
    fast_two_sum(mid, lo, s3, e4);
    fast_two_sum(hi, s3, s5, e6);
    hi = s5;
    fast_two_sum(e6, e4, mid, lo);
}

// tfMulR: the triple times a general radix r <= 254, each limb split by Dekker's 4097 so that the
// limb products are exact, then renormalized (sfpu_tf_proc.h:108-141; names of the procedure).
__device__ __forceinline__ void tf_mul_r(float& hi, float& mid, float& lo, float r) {
    const float acc_lo = lo * r;
    float t1 = mid * 4097.0f;
    float t2 = t1 - mid;
    t1 = t1 - t2;                    // upper half of mid
    t2 = mid - t1;                   // lower half of mid
    t1 = t1 * r;
    t2 = t2 * r;
    const float P1 = t1 + t2;        // term
    float keep = P1 - t1;
    float tmp0 = t2 - keep;          // F1
    t1 = hi * 4097.0f;
    t2 = t1 - hi;
    t1 = t1 - t2;                    // upper half of hi
    t2 = hi - t1;                    // lower half of hi
    t1 = t1 * r;
    t2 = t2 * r;
    const float P0 = t1 + t2;        // acc_mid
    keep = P0 - t1;
    const float F0 = t2 - keep;      // acc_hi
    tmp0 = tmp0 + acc_lo;            // G1
    float sa, ea, sb, eb, r0, ec;
    two_sum(P1, tmp0, sa, ea);
    two_sum(F0, sa, sb, eb);
    two_sum(P0, sb, r0, ec);
    const float G = ea + eb;
    hi = r0;
    fast_two_sum(ec, G, mid, lo);
}

// tfMulR with each limb product and its rounding error taken by one multiply and one FMA
// (TwoProduct) instead of Dekker's splitting: 28 operations instead of 43, the same result
// whenever nothing is flushed to zero and nothing overflows.
//   In tf_mul_r the halves of a limb have at most 12 significant bits and a radix r <= 254 at
// most 8, so the half products are exact; P = t1 r + t2 r rounds their exact sum once, so
// P = fl(x r), and the FastTwoSum that follows (|t1 r| >= |t2 r|) leaves F = x r - P exactly.
// fma(x, r, -P) is that same F. The two forms differ only where one of them meets a subnormal
// (flushed) or an infinite intermediate. If the triple's limbs are multiples of 2^e with
// e >= -126, every intermediate of either form is a multiple of 2^e too (sums, products by
// integers and roundings of multiples of 2^e stay multiples of 2^e), so no nonzero intermediate
// is subnormal. Overflow needs |x| 4097 >= 2^128. Callers use this form only where both hold for
// every element of the wave.
__device__ __forceinline__ void tf_mul_r_fma(float& hi, float& mid, float& lo, float r) {
    const float acc_lo = lo * r;
    const float P1 = mid * r;
    float tmp0 = __builtin_fmaf(mid, r, -P1);  // F1
    const float P0 = hi * r;
    const float F0 = __builtin_fmaf(hi, r, -P0);
    tmp0 = tmp0 + acc_lo;  // G1
    float sa, ea, sb, eb, r0, ec;
    two_sum(P1, tmp0, sa, ea);
    two_sum(F0, sa, sb, eb);
    two_sum(P0, sb, r0, ec);
    const float G = ea + eb;
    hi = r0;
    fast_two_sum(ec, G, mid, lo);
}

// The slicer's tfMulR: tf_mul_r_fma with two of its TwoSums taken as FastTwoSums (22 operations).
//   FastTwoSum(a, b) gives TwoSum's sum and exact error whenever |a| >= |b| or a = 0 (and nothing
// overflows or is flushed). (P1, tmp0): tmp0 is the FMA's error of mid r (at most half a unit in the
// last place of P1) plus lo r, and |lo| is at most a unit in the last place of mid (the limbs of
// load_triple and of every renormalization), so |tmp0| is a few units in the last place of P1 while
// a nonzero P1 holds 2^23 of them; P1 = 0 (mid = 0) is exact either way. (P0, sb): sb sums F0 (at
// most half a unit in the last place of P0) and about mid r, and |mid| <= |hi|/2: after a
// renormalization mid is below half a unit in the last place of hi, and after a digit d is taken
// (hi - d, a nonzero multiple of the unit in the last place of the renormalized hi, which bounds mid
// by half of that unit) still at most half of |hi|. So |sb| < |P0| for hi != 0, and P0 = 0 is exact.
// The oracle checks this form against Dekker's, and that both orders hold at every call, over slicer
// chains (orc_check_tf_mul_r_fast). The reconstruction's states do not keep |mid| <= |hi|/2 (adding
// a diagonal sum can cancel hi and leave mid), so it keeps tf_mul_r_fma.
__device__ __forceinline__ void tf_mul_r_fast(float& hi, float& mid, float& lo, float r) {
    const float acc_lo = lo * r;
    const float P1 = mid * r;
    float tmp0 = __builtin_fmaf(mid, r, -P1);  // F1
    const float P0 = hi * r;
    const float F0 = __builtin_fmaf(hi, r, -P0);
    tmp0 = tmp0 + acc_lo;  // G1
    float sa, ea, sb, eb, r0, ec;
    fast_two_sum(P1, tmp0, sa, ea);
    two_sum(F0, sa, sb, eb);
    fast_two_sum(P0, sb, r0, ec);
    const float G = ea + eb;
    hi = r0;
    fast_two_sum(ec, G, mid, lo);
}

// tfMulRadix (sfpu_tf.h:131-134): tfMulP2 for a power-of-two radix, tfMulR otherwise (FMA: its
// TwoProduct form, for callers that meet the conditions of tf_mul_r_fma; FAST: the slicer's forms,
// tf_mul_pow2_fast, and tf_mul_r_fast under the conditions of tf_mul_r_fma).
template <bool POW2, bool FMA = false, bool FAST = false>
__device__ __forceinline__ void tf_mul_radix(float& hi, float& mid, float& lo, float r) {
    if constexpr (POW2 && FAST)
        tf_mul_pow2_fast(hi, mid, lo, r);
    else if constexpr (POW2)
        tf_mul_pow2(hi, mid, lo, r);
    else if constexpr (FMA && FAST)
        tf_mul_r_fast(hi, mid, lo, r);
    else if constexpr (FMA)
        tf_mul_r_fma(hi, mid, lo, r);
    else
        tf_mul_r(hi, mid, lo, r);
}

// tfAddS<3>: the triple plus v (sfpu_tf_proc.h:184-198).
__device__ __forceinline__ void tf_add_s(float& hi, float& mid, float& lo, float v) {
    float tmp0 = hi + v;
    float tmp1 = tmp0 - hi;
    float tmp2 = tmp0 - tmp1;
    tmp2 = hi - tmp2;
    tmp1 = v - tmp1;
    tmp1 = tmp2 + tmp1;
    hi = tmp0;
    tmp0 = mid + tmp1;
    tmp2 = tmp0 - mid;
    float term = tmp0 - tmp2;
    term = mid - term;
    tmp2 = tmp1 - tmp2;
    tmp2 = term + tmp2;
    mid = tmp0;
    lo = lo + tmp2;
}

// ---- Blocked splitter ----------------------------------------------------------------------
// OZ_BLOCK tiles (include/oz_hip.h): 1 KB blocks of 16 plane rows x 64 plane columns, chunk c of
// row r at chunk position c ^ block_swizzle(r).
__device__ __forceinline__ int block_swizzle(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// One wave per block; the wave writes each plane's block with one contiguous 1 KB store (lane l ->
// block bytes 16l..16l+15). GEN supplies the per-element state and, called with s = 0, 1, ... in
// order, the int8 values of plane s for the 16 elements of a lane (GEN::State, GEN::load,
// GEN::planes).
//   TRAN (plane row = column of X): lane l computes plane row l/4, plane columns 16*(l%4)..+15
//   (16 consecutive rows of X in one column; a load instruction reads 4 runs of 16 consecutive
//   doubles) and packs its 16 values into its own stored chunk.
//   !TRAN: lane l computes plane column l of the 16 rows (each load instruction reads one
//   contiguous 512-byte row segment of X); each plane is transposed through a 1 KB LDS image of the
//   block (byte writes, then one 16-byte read per lane). The image is private to the wave, whose
//   LDS operations execute in order, so no barrier is needed.
// The 16 loads of X (and of the deltas) are issued before any element is processed. A block wholly
// inside X (every block but those on its right and bottom edges) loads without bounds checks; an
// edge block clamps its addresses into X and zeroes what lies outside, without branching.
// The low bytes of a, b, c, d in one word (a lowest): two byte permutes make the pairs (a, b) and
// (c, d), a third joins them.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Generators with kDrivesPlanes = true run the plane loop themselves: GEN::run(st, emit) calls
// emit(p, w) for every plane p in order, w[k] holding the bytes of the lane's elements 4k..4k+3
// (element 4k in the low byte). The others are driven plane by plane through GEN::planes.
template <class G, class = void>
struct drives_planes : std::false_type {};
template <class G>
struct drives_planes<G, std::void_t<decltype(G::kDrivesPlanes)>> : std::bool_constant<G::kDrivesPlanes> {};

// Block blk (within a plane, the same for the whole wave) of the operand X; see split_block_kernel.
template <class GEN, bool TRAN>
__device__ __forceinline__ void split_block(const double* __restrict__ X, int rows, int cols, int ld, int mode,
                                            const int32_t* __restrict__ delta, const GEN& gen, int nplanes,
                                            uint4* __restrict__ planes, int kblocks, long long blk,
                                            long long pstride_chunks) {
    const int lane = threadIdx.x & 63;
    const int br = (int)(blk / kblocks), bk = (int)(blk % kblocks);
    double xv[16];
    int32_t dv[16];
    // element e of this lane is X[xr0 + e][xc0]
    const int xr0 = TRAN ? bk * 64 + 16 * (lane & 3) : br * 16;
    const int xc0 = TRAN ? br * 16 + (lane >> 2) : bk * 64 + lane;
    const bool inside = TRAN ? (bk * 64 + 64 <= rows && br * 16 + 16 <= cols) : (br * 16 + 16 <= rows && bk * 64 + 64 <= cols);
    if (inside) {
        const double* p = X + (size_t)xr0 * ld + xc0;
#pragma unroll
        for (int e = 0; e < 16; e++) xv[e] = p[(size_t)e * ld];
#pragma unroll
        for (int e = 0; e < 16; e++) dv[e] = mode == 0 ? delta[xr0 + e] : delta[xc0];
    } else {
        const int xc = min(xc0, cols - 1);
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int xr = min(xr0 + e, rows - 1);
            const bool in = xr0 + e < rows && xc0 < cols;
            const double v = X[(size_t)xr * ld + xc];
            const int32_t d = mode == 0 ? delta[xr] : delta[xc];
            xv[e] = in ? v : 0.0;
            dv[e] = in ? d : 0;
        }
    }
    typename GEN::State st[16];
#pragma unroll
    for (int e = 0; e < 16; e++) gen.load(st[e], xv[e], dv[e]);
    if constexpr (drives_planes<GEN>::value) {
        // The planes (17 x 2 x 64 MiB at C3) are read back only by the product kernel, long after
        // the Infinity Cache has turned over: non-temporal stores (2-6% faster split).
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        if constexpr (TRAN) {
            const int rr = lane >> 2;
            uint4* out = planes + blk * 64 + rr * 4 + ((lane & 3) ^ block_swizzle(rr));
            gen.run(st, [&](int p, const uint32_t* w) {
                __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]},
                                            reinterpret_cast<u32x4*>(out + (long long)p * pstride_chunks));
            });
        } else {
            __shared__ __attribute__((aligned(16))) uint8_t image[4][1024];
            uint8_t* img = image[threadIdx.x >> 6];
            const int colpart = 16 * (lane >> 4), colbyte = lane & 15;
            uint4* out = planes + blk * 64 + lane;
            gen.run(st, [&](int p, const uint32_t* w) {
#pragma unroll
                for (int e = 0; e < 16; e++)
                    img[64 * e + (colpart ^ (16 * block_swizzle(e))) + colbyte] = (uint8_t)(w[e >> 2] >> (8 * (e & 3)));
                __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(img + 16 * lane),
                                            reinterpret_cast<u32x4*>(out + (long long)p * pstride_chunks));
            });
        }
    } else if constexpr (TRAN) {
        // GEN::planes(st, s, emit) computes plane s's 16 values v and calls emit(v, fix) once, where
        // fix(w) maps four packed values to the bytes stored; emit packs and stores them (non-temporal,
        // as above).
        const int rr = lane >> 2;
        uint4* out = planes + blk * 64 + rr * 4 + ((lane & 3) ^ block_swizzle(rr));
        for (int s = 0; s < nplanes; s++) {
            gen.planes(st, s, [&](const int* v, auto fix) {
                typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                __builtin_nontemporal_store(
                    u32x4{fix(pack4(v[0], v[1], v[2], v[3])), fix(pack4(v[4], v[5], v[6], v[7])),
                          fix(pack4(v[8], v[9], v[10], v[11])), fix(pack4(v[12], v[13], v[14], v[15]))},
                    reinterpret_cast<u32x4*>(out + (long long)s * pstride_chunks));
            });
        }
    } else {
        __shared__ __attribute__((aligned(16))) uint8_t image[4][1024];
        uint8_t* img = image[threadIdx.x >> 6];
        // byte of (row e, column lane) inside the block image
        const int colpart = 16 * (lane >> 4), colbyte = lane & 15;
        uint4* out = planes + blk * 64 + lane;
        for (int s = 0; s < nplanes; s++) {
            gen.planes(st, s, [&](const int* v, auto fix) {
#pragma unroll
                for (int e = 0; e < 16; e++) img[64 * e + (colpart ^ (16 * block_swizzle(e))) + colbyte] = (uint8_t)v[e];
                const uint4 w = *reinterpret_cast<const uint4*>(img + 16 * lane);
                typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                __builtin_nontemporal_store(u32x4{fix(w.x), fix(w.y), fix(w.z), fix(w.w)},
                                            reinterpret_cast<u32x4*>(out + (long long)s * pstride_chunks));
            });
        }
    }
}

template <class GEN, bool TRAN>
__global__ void __launch_bounds__(256) split_block_kernel(const double* __restrict__ X, int rows, int cols, int ld,
                                                          int mode, const int32_t* __restrict__ delta, GEN gen,
                                                          int nplanes, uint4* __restrict__ planes, int kblocks,
                                                          long long nblocks, long long pstride_chunks) {
    const long long blk = (long long)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blk >= nblocks) return;
    split_block<GEN, TRAN>(X, rows, cols, ld, mode, delta, gen, nplanes, planes, kblocks, blk, pstride_chunks);
}

// Both operands of a product in one launch: the first ceil(nbA/4) workgroups split A (M x K, row
// deltas) into planes of Mg x Kg in OZ_BLOCK tiles, the others B (K x N, column deltas) into planes of
// B^T, Ng x Kg. The same generator (moduli) serves both.
template <class GEN>
__global__ void __launch_bounds__(256) split_pair_kernel(const double* __restrict__ A, int M, int K, int lda,
                                                         const int32_t* __restrict__ dA, uint4* __restrict__ pA,
                                                         long long nbA, long long sA_chunks,
                                                         const double* __restrict__ B, int N, int ldb,
                                                         const int32_t* __restrict__ dB, uint4* __restrict__ pB,
                                                         long long nbB, long long sB_chunks, int kblocks, GEN gen,
                                                         int nplanes) {
    const long long gA = (nbA + 3) / 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if ((long long)blockIdx.x < gA) {
        const long long blk = (long long)blockIdx.x * 4 + wave;
        if (blk < nbA) split_block<GEN, false>(A, M, K, lda, 0, dA, gen, nplanes, pA, kblocks, blk, sA_chunks);
    } else {
        const long long blk = ((long long)blockIdx.x - gA) * 4 + wave;
        if (blk < nbB) split_block<GEN, true>(B, K, N, ldb, 1, dB, gen, nplanes, pB, kblocks, blk, sB_chunks);
    }
}

// The identity fix: the values are the stored bytes themselves.
struct NoFix {
    __device__ __forceinline__ uint32_t operator()(uint32_t w) const { return w; }
};

// GEN::planes for generators that produce one element's value at a time (GEN::plane).
#define OZ_PLANES_FROM_PLANE                                                            \
    template <class EMIT>                                                               \
    __device__ __forceinline__ void planes(State* st, int s, EMIT&& emit) const {      \
        int v[16];                                                                      \
        _Pragma("unroll") for (int e = 0; e < 16; e++) v[e] = plane(st[e], s);         \
        emit(v, NoFix{});                                                               \
    }

}  // namespace

// A15: Scheme I slicing of FP64 operands into p digit planes.
//
// Semantics (reference ozaki1/kernels/slice_tf_body.h:86-131, slice_tf_sm8.cpp, slice_tf_num.cpp; the
// step is spelled out in experiments/src/checks/sfpu_tf_emu.hpp:193-198). Per element, with exponent
// delta d (= -1 - e for the target 1/2): t = the triple-float of x*2^d; for i = 0..p-1:
//   t = t * radix (tfMulR; tfMulP2 for a power-of-two radix), d_i = clamp(Rnd(t_hi), -dmax, dmax),
//   t_hi -= d_i.
// Slice i is d_i (weight radix^-(i+1)). The digits must equal the reference's bit for bit; they are
// defined by binary32 operations (see oz_tf32.hpp for the rules and the compile flags). The digit is
// stored as a two's-complement int8 (the reference's sign-magnitude byte is a Tensix packing detail;
// the value is the contract).
//
// MI355X design: the blocked splitter of oz_tf32.hpp (one wave per 1 KB OZ_BLOCK block, one 1 KB store
// per plane); the state of an element is its triple, advanced by one digit per plane.
#pragma clang fp contract(off)

#include "oz_tf32.hpp"

namespace {

template <bool POW2>
struct SliceGen {
    float radix, dmax;
    // radix <= 2 dmax + 1: a residual within 1/2 times the radix stays within dmax + 1/2, so the
    // state never grows from plane to plane (the condition under which tf_mul_r_fma may serve)
    bool stable;
    struct State {
        float hi, mid, lo;
        bool fma;  // tf_mul_r_fma gives this element's digits bit for bit
    };
    __device__ __forceinline__ void load(State& st, double x, int32_t d) const {
        load_triple(x, d, st.hi, st.mid, st.lo);
        if constexpr (!POW2) {
            // The limbs are multiples of 2^(E - 1075 + d), the weight of x's last significand bit
            // (the zero triple for E = 0), and |hi| radix <= dmax + 1/2 keeps every later state
            // within dmax + 1/2, far from overflow.
            const int32_t E = (int32_t)(((unsigned long long)__double_as_longlong(x) >> 52) & 0x7FFu);
            st.fma = stable && (E == 0 || E - 1075 + d >= -126) && __builtin_fabsf(st.hi) * radix <= dmax + 0.5f;
        }
    }
    template <bool FMA>
    __device__ __forceinline__ int plane1(State& st) const {
        tf_mul_radix<POW2, FMA, true>(st.hi, st.mid, st.lo, radix);
        float v = __builtin_rintf(st.hi);  // Rnd: nearest, ties to even
        if (v < -dmax)
            v = -dmax;
        else if (v >= dmax)
            v = dmax;
        st.hi = st.hi - v;
        return (int)v;
    }
    // Plane s of the 16 elements. A general radix takes the TwoProduct form of tfMulR when every
    // element of the wave allows it (a wave-uniform branch), Dekker's form otherwise.
    template <class EMIT>
    __device__ __forceinline__ void planes(State* st, int, EMIT&& emit) const {
        int v[16];
        bool fma = !POW2;
        if constexpr (!POW2) {
#pragma unroll
            for (int e = 0; e < 16; e++) fma = fma && st[e].fma;
        }
        if (!POW2 && __all(fma)) {
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = plane1<true>(st[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = plane1<false>(st[e]);
        }
        emit(v, NoFix{});
    }
};

template <bool POW2>
int launch_slices(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int p,
                  float radix, float dmax, int8_t* planes, bool tran, int prow, int pld, long long pstride) {
    const int kblocks = pld / 64;
    const long long nblocks = (long long)(prow / 16) * kblocks;
    const unsigned grid = oz::ceil_div(nblocks, 4);
    const SliceGen<POW2> gen{radix, dmax, radix <= 2.0f * dmax + 1.0f};
    if (tran)
        hipLaunchKernelGGL((split_block_kernel<SliceGen<POW2>, true>), dim3(grid), dim3(256), 0, dev->stream, X, rows,
                           cols, ld, mode, delta, gen, p, reinterpret_cast<uint4*>(planes), kblocks, nblocks,
                           pstride / 16);
    else
        hipLaunchKernelGGL((split_block_kernel<SliceGen<POW2>, false>), dim3(grid), dim3(256), 0, dev->stream, X, rows,
                           cols, ld, mode, delta, gen, p, reinterpret_cast<uint4*>(planes), kblocks, nblocks,
                           pstride / 16);
    return oz::launch_check(dev, "split_block_kernel<SliceGen>");
}

template <bool POW2>
int launch_pair(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA, const double* B, int N,
                int ldb, const int32_t* dB, int p, float radix, float dmax, int8_t* pA, int8_t* pB, int Mg, int Ng,
                int Kg) {
    const int kblocks = Kg / 64;
    const long long nbA = (long long)(Mg / 16) * kblocks, nbB = (long long)(Ng / 16) * kblocks;
    const long long sA = (long long)Mg * Kg / 16, sB = (long long)Ng * Kg / 16;
    const long long grid = (nbA + 3) / 4 + (nbB + 3) / 4;
    if (grid > 0x7FFFFFFFll) return oz::fail(dev, OZ_ERR_ARG, "oz1_split_pair_int8: grid too large");
    const SliceGen<POW2> gen{radix, dmax, radix <= 2.0f * dmax + 1.0f};
    hipLaunchKernelGGL((split_pair_kernel<SliceGen<POW2>>), dim3((unsigned)grid), dim3(256), 0, dev->stream, A, M, K,
                       lda, dA, reinterpret_cast<uint4*>(pA), nbA, sA, B, N, ldb, dB, reinterpret_cast<uint4*>(pB),
                       nbB, sB, kblocks, gen, p);
    return oz::launch_check(dev, "split_pair_kernel<SliceGen>");
}

}  // namespace

extern "C" int oz1_split_int8(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode,
                              const int32_t* delta, int p, int radix, int dmax, int8_t* planes, int layout, int prow,
                              int pld, long long plane_stride) {
    if (int st = oz::use(dev)) return st;
    if (!X || !delta || !planes || rows <= 0 || cols <= 0 || ld < cols || (mode != 0 && mode != 1) ||
        (layout != 2 && layout != 3) || p < 1 || p > 256 || radix < 2 || radix > 254 || dmax < 1 || dmax > 127)
        return oz::fail(dev, OZ_ERR_ARG, "oz1_split_int8: invalid arguments");
    const bool tran = layout == 3;
    const int need_rows = tran ? cols : rows, need_ld = tran ? rows : cols;
    if (prow < need_rows || pld < need_ld || pld % 64 != 0 || prow % 16 != 0 || plane_stride % 1024 != 0 ||
        plane_stride < (long long)prow * pld || ((uintptr_t)planes & 15u))
        return oz::fail(dev, OZ_ERR_ARG, "oz1_split_int8: plane geometry %dx%d (stride %lld) does not fit", prow, pld,
                        plane_stride);
    const bool pow2 = (radix & (radix - 1)) == 0;
    return pow2 ? launch_slices<true>(dev, X, rows, cols, ld, mode, delta, p, (float)radix, (float)dmax, planes, tran,
                                      prow, pld, plane_stride)
                : launch_slices<false>(dev, X, rows, cols, ld, mode, delta, p, (float)radix, (float)dmax, planes, tran,
                                       prow, pld, plane_stride);
}

extern "C" int oz1_split_pair_int8(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA,
                                   const double* B, int N, int ldb, const int32_t* dB, int p, int radix, int dmax,
                                   int8_t* planesA, int8_t* planesB, int Mg, int Ng, int Kg) {
    if (int st = oz::use(dev)) return st;
    if (!A || !B || !dA || !dB || !planesA || !planesB || M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < N || p < 1 ||
        p > 256 || radix < 2 || radix > 254 || dmax < 1 || dmax > 127)
        return oz::fail(dev, OZ_ERR_ARG, "oz1_split_pair_int8: invalid arguments");
    if (Mg < M || Ng < N || Kg < K || Mg % 16 || Ng % 16 || Kg % 64 || ((uintptr_t)planesA & 15u) ||
        ((uintptr_t)planesB & 15u))
        return oz::fail(dev, OZ_ERR_ARG, "oz1_split_pair_int8: plane geometry %dx%d / %dx%d does not fit", Mg, Kg, Ng,
                        Kg);
    return (radix & (radix - 1)) == 0
               ? launch_pair<true>(dev, A, M, K, lda, dA, B, N, ldb, dB, p, (float)radix, (float)dmax, planesA, planesB,
                                   Mg, Ng, Kg)
               : launch_pair<false>(dev, A, M, K, lda, dA, B, N, ldb, dB, p, (float)radix, (float)dmax, planesA,
                                    planesB, Mg, Ng, Kg);
}

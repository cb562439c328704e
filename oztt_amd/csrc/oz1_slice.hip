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
    struct State {
        float hi, mid, lo;
    };
    __device__ __forceinline__ void load(State& st, double x, int32_t d) const { load_triple(x, d, st.hi, st.mid, st.lo); }
    __device__ __forceinline__ int plane(State& st, int) const {
        tf_mul_radix<POW2>(st.hi, st.mid, st.lo, radix);
        float v = __builtin_rintf(st.hi);  // Rnd: nearest, ties to even
        if (v < -dmax)
            v = -dmax;
        else if (v >= dmax)
            v = dmax;
        st.hi = st.hi - v;
        return (int)v;
    }
    OZ_PLANES_FROM_PLANE
};

template <bool POW2>
int launch_slices(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int p,
                  float radix, float dmax, int8_t* planes, bool tran, int prow, int pld, long long pstride) {
    const int kblocks = pld / 64;
    const long long nblocks = (long long)(prow / 16) * kblocks;
    const unsigned grid = oz::ceil_div(nblocks, 4);
    const SliceGen<POW2> gen{radix, dmax};
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

/* oz_hip.h — C ABI of the MI355X (gfx950) device layer of ozTTgemm.
 *
 * The C++20 backends (oztt_amd/csrc/host/) call the device only through these functions; they
 * replace the TT-Metalium program builders and enqueues of the reference (src/backend/ozaki{1,2}/stages.hpp,
 * src/backend/common/scale.hpp, the EnqueueMeshWorkload calls of src/ozaki2.cpp). Each entry point
 * cites the reference stage whose semantics it implements.
 *
 * Conventions
 *   - Every function returns 0 (OZ_OK) on success or a negative oz_status; none throws. The message
 *     of the last failure of a device handle is oz_last_error().
 *   - All launches are ordered on the handle's own HIP stream (default priority); device pointers
 *     are plain addresses from oz_dev_malloc (or any HIP allocation on the same device).
 *   - A handle holds 64 bytes of device counters through which its product kernels hand out their
 *     last tiles (zero between launches; each launch leaves them zero). Launches through one handle
 *     must therefore not overlap in time: use one handle per stream (or per thread), and do not
 *     replay a graph captured from a handle's stream while that handle has other work in flight.
 *   - Matrices are row-major. "Planes" are the per-modulus (Scheme II) or per-slice (Scheme I)
 *     integer matrices; their layout is given with each function.
 *   - Sizes are checked against what the kernels assume before anything is launched; a mismatch
 *     returns OZ_ERR_ARG and launches nothing.
 */
#ifndef OZ_HIP_H
#define OZ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum oz_status {
    OZ_OK = 0,
    OZ_ERR_ARG = -1,     /* invalid argument or shape the kernels do not support */
    OZ_ERR_HIP = -2,     /* HIP runtime failure */
    OZ_ERR_NOMEM = -3,   /* device allocation failed */
    OZ_ERR_RANGE = -4    /* a value outside the exact range of a stage */
};

/* Largest number of moduli (reference digit_limits.h:19, OZ2_MAXS). */
#define OZ2_MAXS 24

typedef struct oz_dev oz_dev;

/* ---- device handle (replaces MeshDevice::create_unit_mesh, context.cpp:155) ---------------- */
int oz_dev_open(int device_id, oz_dev** out);
void oz_dev_close(oz_dev* dev);
const char* oz_last_error(const oz_dev* dev);
int oz_device_count(int* count);
int oz_dev_malloc(oz_dev* dev, size_t bytes, void** ptr);
/* Free and total device memory of the handle's GPU (hipMemGetInfo). */
int oz_mem_info(oz_dev* dev, size_t* free_bytes, size_t* total_bytes);
int oz_dev_free(oz_dev* dev, void* ptr);
int oz_memcpy_h2d(oz_dev* dev, void* dst, const void* src, size_t bytes);
int oz_memcpy_d2h(oz_dev* dev, void* dst, const void* src, size_t bytes);
int oz_fill_u32(oz_dev* dev, void* dst, uint32_t value, size_t count);
/* Page-locked host memory (hipHostMalloc) for staging uploads and downloads: copies from it run at
 * full link speed and asynchronously. */
int oz_host_malloc(oz_dev* dev, size_t bytes, void** ptr);
int oz_host_free(oz_dev* dev, void* ptr);
/* Host-to-device copy ordered on the handle's stream that returns without waiting; src must be
 * page-locked (oz_host_malloc) and stay valid and unchanged until the stream has passed the copy. */
int oz_memcpy_h2d_async(oz_dev* dev, void* dst, const void* src, size_t bytes);
/* Device-to-device copy by a plain streaming kernel (16-byte aligned pointers and size); also the
 * reference transfer for calibrating HBM traffic counters. */
int oz_memcpy_d2d(oz_dev* dev, void* dst, const void* src, size_t bytes);
/* dst (drows x dcols, row-major, leading dimension dcols) = the top-left min(drows, srows) x
 * min(dcols, scols) of src (srows x scols, leading dimension sld), zero elsewhere; stream-ordered.
 * No counterpart in the reference: it lays out the resident operands (ozTTgemm::Matrix) in the
 * zero-padded shapes of the products. */
int oz_pad_copy_f64(oz_dev* dev, double* dst, int drows, int dcols, const double* src, int srows, int scols, int sld);
int oz_sync(oz_dev* dev);
/* Stream-ordered timing (OZ_EVENT_SLOTS event slots per handle). */
#define OZ_EVENT_SLOTS 256
int oz_event_record(oz_dev* dev, int slot);
int oz_event_elapsed_ms(oz_dev* dev, int slot_begin, int slot_end, float* ms);
/* Times product kernels by their own dispatches, with no marker in the stream. After
 * oz_time_products_begin, the first product-kernel launch on the handle (oz_gemm_i8,
 * oz2_gemm_digits, oz1_gemm_diag_i8, oz2_gemm_groups_f8 and the passes built on them) sets event
 * slot_begin at the start of its dispatch, and each such launch sets slot_end at the end of its
 * own, until oz_time_products_end, which reports in *launched whether any ran (0: the events were
 * not touched). An event pair around a launch of tens of microseconds adds a few to it; these do
 * not. No counterpart in the reference (its timing hooks, evaluation_hooks.hpp, bracket whole
 * stages). */
int oz_time_products_begin(oz_dev* dev, int slot_begin, int slot_end);
int oz_time_products_end(oz_dev* dev, int* launched);

/* ---- A5: normalization (reference scale_f64_reader.cpp:129, expdelta.cpp:44, scale_bits.h) --
 * Largest |x| of every row (mode 0, `rows` outputs) or column (mode 1, `cols` outputs) of X
 * (rows x cols, leading dimension ld), compared on the FP64 bit patterns; converted to BF16
 * rounding down (ceil_mode 0), up (1), or up and one more step at a power of two (2);
 * e = ceil(log2(bf16)) (0 for a zero row/column); delta = shift - e.
 * Out-of-range maxima OR bits into *flags (device word): 1 above the largest BF16, 2 nonzero and
 * below 2^-126, 4 Inf/NaN; their delta uses e = 0. */
int oz_scale_f64(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, int ceil_mode, int shift,
                 int32_t* delta, uint32_t* flags);

/* Both operands of a product in one launch: the row maxima of A (M x K, lda) into dA[M] and the
 * column maxima of B (K x N, ldb) into dB[N], each as oz_scale_f64 (mode 0 for A, mode 1 for B, the
 * same ceil_mode and shift), with the range flags of A ORed into flags[0] and those of B into
 * flags[1] (two device words, 4-byte aligned). clear_flags, when not null, names two other device
 * words (4-byte aligned, not overlapping flags) that the launch sets to zero: a caller that
 * alternates between two flag slots, clearing the next pass's slot in this one, needs no launch
 * to clear them. */
int oz_scale_pair_f64(oz_dev* dev, const double* A, int M, int K, int lda, const double* B, int N, int ldb,
                      int ceil_mode, int shift, int32_t* dA, int32_t* dB, uint32_t* flags, uint32_t* clear_flags);

/* ---- A6-A8: Scheme II residues (reference modslice_int8.cpp:60, digits.h:80,165, f64_tf.h:141) -
 * For every element x of X (rows x cols, ld) with exponent delta d (delta[row] for mode 0,
 * delta[col] for mode 1): the triple-float of x*2^d, its nd radix-2^20 digits (nd = 3..5), and
 * for each modulus s the residue r_s == A' (mod m_s), |r_s| <= 127, as int8 (two's complement).
 * A plane is a matrix of `prow` rows and `pld` columns (entries outside the operand are 0):
 *   layout 0 (row):        plane[r][c] = residue of X[r][c], row-major, row stride pld bytes
 *   layout 1 (tran):       plane[c][r] = residue of X[r][c], row-major, row stride pld bytes
 *   layout 2 (block):      as layout 0, stored in OZ_BLOCK tiles (below)
 *   layout 3 (block tran): as layout 1, stored in OZ_BLOCK tiles
 * OZ_BLOCK tiles: 1024-byte blocks of 16 plane rows x 64 plane columns, block (i, j) at byte
 * (i*(pld/64) + j)*1024; inside, plane element (r, c) of the block (r < 16, c < 64) is at byte
 * 64*r + 16*((c/16) ^ oz_block_swizzle(r)) + c%16 with oz_block_swizzle(r) = ((r>>1) ^ (r>>2)) & 3.
 * This is the operand layout of oz_gemm_i8: one 1 KB block is one contiguous direct-to-LDS copy,
 * and the swizzle spreads the rows of each LDS fragment read over all banks.
 * prow and pld must be multiples of 64 (blocked: of 16 and 64); plane_stride is the byte distance
 * between planes (multiple of 1024 for the blocked layouts). */
typedef struct oz2_moduli_dev {
    int S;                 /* number of moduli, 1..OZ2_MAXS */
    int nd;                /* radix-2^20 digits of A', 3..5 */
    float m[OZ2_MAXS];     /* moduli (exact in FP32) */
    float rinv[OZ2_MAXS];  /* FP32 nearest to 1/m (moduli.hpp:686) */
    float c[4][OZ2_MAXS];  /* 2^(20(j+1)) mod m, j = 0..3 (moduli.hpp:694-699) */
} oz2_moduli_dev;
int oz2_split_int8(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                   const oz2_moduli_dev* mo, int8_t* planes, int layout, int prow, int pld, long long plane_stride);
/* Both operands of a product in one launch: oz2_split_int8 of A (M x K, lda, row deltas dA, mode 0)
 * into planesA in layout 2 (S planes of Mg x Kg, plane stride Mg*Kg bytes) and of B (K x N, ldb,
 * column deltas dB, mode 1) into planesB in layout 3 (S planes of Ng x Kg, stride Ng*Kg). Mg >= M and
 * Ng >= N multiples of 16, Kg >= K a multiple of 64, planes 16-byte aligned. */
int oz2_split_pair_int8(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA, const double* B,
                        int N, int ldb, const int32_t* dB, const oz2_moduli_dev* mo, int8_t* planesA, int8_t* planesB,
                        int Mg, int Ng, int Kg);
/* White-box view of A7: the nd digits (top first) of every element as FP32, digits[(r*cols+c)*nd+j]. */
int oz2_digits_f32(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                   int nd, float* digits);

/* ---- A9: exact integer products (reference bmm_int32_spill.cpp:265, ozaki2.cpp:333) ---------
 * C[b] = A[b] * B[b]^T for b < batch: A[b] is an M x K int8 plane and Bt[b] an N x K int8 plane,
 * both in OZ_BLOCK tiles (layout 2 / 3 of oz2_split_int8: 1 KB blocks of 16 rows x 64 K-bytes,
 * K/64 blocks per 16 rows); C[b] is M x N int32, row stride ldc. strideA/strideB/strideC are the
 * distances between batches in bytes (A, B) and elements (C).
 * Exact: |C| <= K*127^2 must fit int32 (the planner guarantees it, moduli.hpp:217-231).
 * Requirements: M % 256 == 0, N % 256 == 0, K % 64 == 0, strideA and strideB multiples of 1024. */
int oz_gemm_i8(oz_dev* dev, const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N, int K, int batch, int ldc,
               long long strideA, long long strideB, long long strideC);

/* ---- A10-A11: CRT reconstruction to FP64 (reference recon_crt.cpp:293, recon_writer.cpp:70) --
 * For each element (i < M, j < N): C' = the integer in (-Mprod/2, Mprod/2] congruent to C_s
 * modulo m_s for every s (C_s read from C + s*strideC, row stride ldc), then
 * out[i*ldo+j] = C' * 2^(eA_i + eB_j - 2b) rounded to nearest-even, where eA_i = shift - dA[i],
 * eB_j = shift - dB[j]; results below 2^-1022 become signed zero (f64_tf.h:45-47).
 * The reconstruction is exact, so it serves both of the reference's one- and two-pass modes. */
typedef struct oz2_crt_dev {
    int S;
    int b;                          /* integer width */
    int shift;                      /* b - 20*(nd-1) */
    int nw;                         /* 32-bit words of the accumulator (host: bits of S*Mprod) */
    uint32_t m[OZ2_MAXS];
    uint32_t y[OZ2_MAXS];           /* (Mprod/m_s)^-1 mod m_s */
    uint32_t Q[OZ2_MAXS][8];        /* Mprod/m_s, little-endian 32-bit words */
    uint32_t Mw[8];                 /* Mprod */
    double Mtop;                    /* Mprod as FP64 (quotient estimate) */
} oz2_crt_dev;
int oz2_crt_f64(oz_dev* dev, const int32_t* C, int M, int N, int ldc, long long strideC, const oz2_crt_dev* crt,
                const int32_t* dA, const int32_t* dB, double* out, int ldo);

/* ---- A9 + A10 fused: products reduced to CRT digits (reference ozaki2.cpp:333-350 followed by
 * the residue step of recon_crt.cpp:293) -------------------------------------------------------
 * The products of oz_gemm_i8 for the S moduli of crt (batch = S), each reduced in the GEMM's
 * epilogue to its CRT digit k_s = (C_s mod m_s) * y_s mod m_s, stored as uint8 in [0, m_s] (a digit
 * 0 may read m_s, which the reconstruction takes as 0):
 * D[s] is M x N bytes, row stride ldd, plane stride strideD bytes (D, ldd and strideD 16-byte
 * aligned). Same operand rules as oz_gemm_i8. Writing one byte instead of four per product is what makes this the production path. */
int oz2_gemm_digits(oz_dev* dev, const int8_t* A, const int8_t* Bt, uint8_t* D, int M, int N, int K, int S, int ldd,
                    long long strideA, long long strideB, long long strideD, const oz2_crt_dev* crt);

/* CRT reconstruction from the digits of oz2_gemm_digits (each in [0, m_s]): same result as
 * oz2_crt_f64 on the products. ldd and strideD (bytes) multiples of 4, D 4-byte aligned. */
int oz2_crt_digits_f64(oz_dev* dev, const uint8_t* D, int M, int N, int ldd, long long strideD,
                       const oz2_crt_dev* crt, const int32_t* dA, const int32_t* dB, double* out, int ldo);

/* ---- A5-A11 in one call: the whole Scheme II INT8 pass on device-resident operands ----------
 * (reference ozaki2.cpp:439-478: scale, slice, products, reconstruction; the plan is the caller's,
 * made on the host as for the C++ backend.) C (M x N, leading dimension ldc) = A B for row-major A
 * (M x K, lda) and B (K x N, ldb): flags[0..1] <- 0; oz_scale_f64 (ceil mode 1, shift crt->shift)
 * of A's rows and B's columns, ORing their range flags into flags[0] and flags[1] (as
 * oz_scale_f64: 1, 2, 4; the caller reads them); oz2_split_int8 of A (layout 2) and B (layout 3);
 * oz2_gemm_digits; oz2_crt_digits_f64. Every launch is ordered on the handle's stream; nothing
 * waits on the host. mo and crt must hold the same INT8 moduli, crt->shift = crt->b - 20 (mo->nd - 1),
 * and K (rounded up to 64) times 127^2 must stay below 2^31. flags: two device words, 4-byte aligned.
 * The intermediates live in `work` (256-byte aligned): the exponent deltas, the S residue planes of
 * A and of B^T and the S digit planes, about S (Mg Kg + Ng Kg + Mg Ng) bytes with Mg, Ng = M, N
 * rounded up to 256 and Kg = K rounded up to 64; oz2_gemm_f64_workspace gives the exact size. */
int oz2_gemm_f64_workspace(int M, int N, int K, int S, size_t* bytes);
int oz2_gemm_f64(oz_dev* dev, const double* A, int lda, const double* B, int ldb, double* C, int ldc, int M, int N,
                 int K, const oz2_moduli_dev* mo, const oz2_crt_dev* crt, uint32_t* flags, void* work,
                 size_t work_bytes);

/* The same pass for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc); it has no counterpart in the reference.
 * It takes no workspace and allocates nothing: the intermediates live in a device array of
 * OZ2_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on until the process ends.
 * Shapes whose workspace (oz2_gemm_f64_workspace) exceeds it are refused with OZ_ERR_ARG; that
 * covers for example 2048 x 2048 x 2048 with up to 21 moduli. Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (several streams or host threads) race and must be
 * serialized by the caller. Otherwise as oz2_gemm_f64. */
#define OZ2_NOALLOC_SCRATCH_BYTES (256u << 20)
int oz2_gemm_f64_noalloc(oz_dev* dev, const double* A, int lda, const double* B, int ldb, double* C, int ldc, int M,
                         int N, int K, const oz2_moduli_dev* mo, const oz2_crt_dev* crt, uint32_t* flags);

/* ==== Scheme II digit formats: residues carried as small digits (reference FP8 route) ========= */

#define OZ2_MAXPLANES 72  /* digit planes (at most 3 per modulus) */
#define OZ2_MAXOUT 96     /* product outputs (at most 4 per modulus) */

/* ---- A18 split (reference modslice_digit.cpp:142-243, sparse_fix.h:48-78, split.hpp:157-279) ---
 * As oz2_split_int8 (same residues r = A' mod m_s, m_s <= 2401), then r split into digits per
 * modulus, planes l, h (and s = h + l for xmode 1; r alone for xmode 3) in modulus order:
 *   xmode 0 (rounded, square or wide modulus): h = Rnd(r*qinv), l = r - q*h;
 *   xmode 1 (Karatsuba): h = Rnd((r + sgn(r)*(q/2 - 1/2))*qinv), l = r - q*h, s = h + l;
 *   xmode 2 (sparse square, q odd): the rounded digits moved into {|x| <= 16} U {even, |x| <= 32};
 *   xmode 3 (one digit, m <= 33): the residue r itself (|r| <= 16), one plane (q is not read).
 * Every operation is one binary32 operation as in the reference. encoding 1 stores e4m3 bytes
 * (gfx950 FP8, exact for these digits), 0 int8 values. Layouts 2 and 3 only (OZ_BLOCK tiles). */
typedef struct oz2_digit_dev {
    oz2_moduli_dev mo;       /* moduli (m <= 2401), rinv, weights, nd */
    int xmode[OZ2_MAXS];     /* 0 rounded, 1 Karatsuba, 2 sparse square, 3 one digit */
    float q[OZ2_MAXS];       /* digit radix */
    float qinv[OZ2_MAXS];    /* 1.0f / q (stages.hpp:223) */
    int encoding;            /* 1 e4m3, 0 int8 */
} oz2_digit_dev;
/* Number of digit planes of a descriptor (2 per modulus, 3 for Karatsuba, 1 for one digit), or -1. */
int oz2_digit_planes(const oz2_digit_dev* dd);
int oz2_split_digits(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta,
                     const oz2_digit_dev* dd, uint8_t* planes, int layout, int prow, int pld, long long plane_stride);
/* Both operands of a product in one launch (the reference splits them in two kernels of the same
 * stage, ozaki2.cpp:228-285): oz2_split_digits of A (M x K, lda, row deltas dA, mode 0) into planesA
 * in layout 2 (planes of Mg x Kg, stride Mg*Kg bytes) and of B (K x N, ldb, column deltas dB, mode 1)
 * into planesB in layout 3 (planes of Ng x Kg, stride Ng*Kg). Mg >= M and Ng >= N multiples of 16,
 * Kg >= K a multiple of 64, planes 16-byte aligned. */
int oz2_split_digits_pair(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA, const double* B,
                          int N, int ldb, const int32_t* dB, const oz2_digit_dev* dd, uint8_t* planesA, uint8_t* planesB,
                          int Mg, int Ng, int Kg);

/* ---- A18 products + composition (reference ozaki2.cpp:228-285 run_digit_modulus, compose.cpp,
 * split.hpp:541-661 product terms and groups) ------------------------------------------------
 * Output o sums npairs digit products over the full K on the FP8 matrix cores (e4m3 x e4m3,
 * FP32 accumulation; exact while |sum| <= bound <= 2^24, which the entry point checks: every
 * partial sum is then an integer that FP32 holds):  P_o = sum_t A[a[t]] * Bt[b[t]]^T  (the reference's concatenation along K).
 * out_kind 0 stores P_o as int32 (M x N per output, element strides, out 16-byte aligned and ldo,
 * strideO multiples of 4); out_kind 1 stores the CRT
 * term w_o = (coef * P_o) mod m as uint16 in [0, m] (m standing for 0), where coef is the composition coefficient
 * times y_s (mod m): for modulus s, sum over its outputs of w_o == D_s * y_s (mod m_s), D_s the
 * composed residue. A and Bt are e4m3 digit planes of oz2_split_digits (layouts 2 and 3);
 * strideA/strideB are the byte distances between planes (multiples of 1024), strideO between
 * outputs in elements. M, N multiples of 256, K of 64. */
typedef struct oz2_group_dev {
    int npairs;              /* 1..4 */
    int modulus;             /* s: the modulus this output composes into */
    unsigned char a[4], b[4];/* digit planes of A and of B, pair t = (a[t], b[t]) */
    uint32_t m;              /* m_s */
    uint32_t coef;           /* (coefficient * y_s) mod m_s */
    float bound;             /* upper bound of |P_o| (sum over pairs of K * |digit| bounds) */
} oz2_group_dev;
typedef struct oz2_groups_dev {
    int nout;                /* outputs, 1..OZ2_MAXOUT */
    int nplanes;             /* digit planes in A and in Bt (every a[t], b[t] is below it) */
    oz2_group_dev g[OZ2_MAXOUT];
} oz2_groups_dev;
int oz2_gemm_groups_f8(oz_dev* dev, const uint8_t* A, const uint8_t* Bt, void* out, int M, int N, int K,
                       const oz2_groups_dev* gd, int out_kind, int ldo, long long strideA, long long strideB,
                       long long strideO);

/* CRT reconstruction from the uint16 terms of oz2_gemm_groups_f8 (out_kind 1): term plane o adds
 * w_o * Q_{modulus(o)}; then as oz2_crt_f64 (moduli up to 2401; crt->nw must hold nterms * M).
 * ldw and strideW in elements, multiples of 4; W 8-byte aligned. */
int oz2_crt_terms_f64(oz_dev* dev, const uint16_t* W, int M, int N, int ldw, long long strideW, int nterms,
                      const unsigned char* term_modulus, const oz2_crt_dev* crt, const int32_t* dA,
                      const int32_t* dB, double* out, int ldo);

/* ==== Scheme I (reference src/ozaki1.cpp run(): scale, slice, diagonal products, Horner) ==== */

/* ---- A15: slicing (reference ozaki1/kernels/slice_tf_body.h:86-131, slice_tf_sm8.cpp) --------
 * For every element x of X (as oz2_split_int8: mode 0 delta per row, 1 per column) the p digits of
 * x*2^delta in radix `radix` with digit bound dmax: t = triple-float(x*2^delta); per digit
 * t *= radix (tfMulR, or tfMulP2 for a power of two), d = clamp(round(t_hi), +-dmax), t_hi -= d.
 * Plane i holds digit i (weight radix^-(i+1)) as int8, in OZ_BLOCK tiles: layout 2 (planes of
 * rows x cols) or layout 3 (transposed, cols x rows); geometry rules as oz2_split_int8's blocked
 * layouts. radix <= 254, dmax <= 127, p <= 256. */
int oz1_split_int8(oz_dev* dev, const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int p,
                   int radix, int dmax, int8_t* planes, int layout, int prow, int pld, long long plane_stride);
/* Both operands of a product in one launch (the reference slices A and B in two kernels of the
 * same stage, ozaki1.cpp run()): oz1_split_int8 of A (M x K, lda, row deltas dA, mode 0) into
 * planesA in layout 2 (p planes of Mg x Kg, stride Mg*Kg bytes) and of B (K x N, ldb, column deltas
 * dB, mode 1) into planesB in layout 3 (p planes of Ng x Kg, stride Ng*Kg). Mg >= M and Ng >= N
 * multiples of 16, Kg >= K a multiple of 64, planes 16-byte aligned. */
int oz1_split_pair_int8(oz_dev* dev, const double* A, int M, int K, int lda, const int32_t* dA, const double* B, int N,
                        int ldb, const int32_t* dB, int p, int radix, int dmax, int8_t* planesA, int8_t* planesB,
                        int Mg, int Ng, int Kg);

/* ---- A16: diagonal partial products (reference ozaki1/gemm.hpp:315, stages.hpp:157) ----------
 * C[d] = sum_{i=0..d} A[i] * Bt[d-i]^T for d < ndiag, exact int32: the d+1 pairs concatenated along
 * K in one accumulation, which requires ndiag*K*dmax^2 < 2^31 for digits |A|, |Bt| <= dmax (the
 * reference's single-K-block INT8 plan, and its int32 sums S_d of the other formats).
 * A[i]: M x K, Bt[i]: N x K int8 in OZ_BLOCK tiles; operand rules as oz_gemm_i8. */
int oz1_gemm_diag_i8(oz_dev* dev, const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N, int K, int ndiag,
                     int dmax, int ldc, long long strideA, long long strideB, long long strideC);

/* ---- A17: reconstruction (reference recon_tf_i32in.cpp:116-157, recon_f64_writer.cpp:148-160) -
 * out[i][j] = S * radix^-(L+2) * 2^-(dA[i]+dB[j]) with S = sum_d radix^(L-d) P_d (L = ndiag-1)
 * evaluated by Horner in triple-float exactly as the reference does, then assembled to FP64 with
 * the 64-bit significand W = Whi:Wlo of radix^-(L+2) = W * 2^qw. P[d] is read from
 * P + d*strideP (row stride ldp). signmag = 1: P_d enters as sign * (|P_d| & ~0xFF) and
 * sign * (|P_d| & 0xFF) (INT8 products); 0: as (P_d & ~0xFF) and (P_d & 0xFF), except the first
 * nsingle diagonals, which enter whole (their |P_d| <= 2^24). */
typedef struct oz1_recon_dev {
    int ndiag;      /* L + 1 */
    int radix;      /* 2..254 */
    int signmag;    /* 1: split of the INT8 products; 0: two's-complement split */
    int nsingle;    /* leading diagonals read whole (signmag = 0 only) */
    uint32_t Whi, Wlo;
    int32_t qw;
} oz1_recon_dev;
int oz1_recon_f64(oz_dev* dev, const int32_t* P, int M, int N, int ldp, long long strideP, const oz1_recon_dev* r,
                  const int32_t* dA, const int32_t* dB, double* out, int ldo);
/* The reconstruction run K block by K block (reference ozaki1/kernels/recon_tf_f32in.cpp:54-89 and
 * recon_f64_writer.cpp, ozaki1/plan.hpp:104-109: FP32 products whose int32 sum over all of K could
 * overflow). P holds one K block's diagonal sums, exact integers of at most 2^24 that enter whole;
 * after the first block (first = 0) the limbs carried in `limbs` (hi, mid, lo planes of M x N floats,
 * leading dimension ldl, limb_stride elements apart) are added in the order lo, mid, hi. Every block
 * but the last (last = 0) writes the limbs back; the last assembles C as oz1_recon_f64 does.
 * r->signmag must be 0 (nsingle is not read: every diagonal enters whole). */
int oz1_recon_block_f64(oz_dev* dev, const int32_t* P, int M, int N, int ldp, long long strideP,
                        const oz1_recon_dev* r, int first, int last, float* limbs, long long limb_stride, int ldl,
                        const int32_t* dA, const int32_t* dB, double* out, int ldo);

#ifdef __cplusplus
}
#endif
#endif /* OZ_HIP_H */

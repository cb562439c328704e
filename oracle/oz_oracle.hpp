// oz_oracle — CPU restatement of the reference ozTTgemm numerics. TEST INFRASTRUCTURE ONLY.
//
// Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load this
// library, and only as a checker: the product path (oztt_amd/) never links, calls or falls
// back to it. Every function cites the reference file:line whose behaviour it restates.
//
// Parity status of each function (how it is pinned, see tests/test_oracle.py):
//   orc_inputs, orc_hash_f64      reference input hashes ahash/bhash (dgemm_ref.log:6,12,18)
//   orc_scale                     closed-form bit rules + marker KATs (scale_bits.h:22-62)
//   orc_split_f64                 exactness hi+mid+lo == x*2^d (binary128) over random and edge inputs
//   orc_oz2_digits/residues       digits.h:44 KAT, ModRound KATs (sfpu_tf_proc.h:271,303,312),
//                                 residue-class invariants, and end to end by the output hashes
//   orc_oz2_digit_planes          closed forms (h = round(r/q) or the Karatsuba ceiling, l + q h == r,
//                                 the sparse-set moves checked against an integer restatement; a
//                                 one-digit plane equals orc_oz2_residues), and end to end by the FP8
//                                 output hash (tools/validated/quick.csv:11)
//   orc_gemm_i8                   brute force int64 (its own definition)
//   orc_oz2_crt_ref               reference output hashes (tools/validated/quick.csv:13,
//                                 phi_sweep.log:116,122)
//   orc_oz2_crt_exact             exact integer arithmetic; cross-checked against a binary128 GEMM
//   orc_check_tf_mul_r_forms      checkers, not restatements: the GPU's forms of tfMulR against Dekker's
//   orc_check_tf_mul_r_fast,      in the FP32 model
//   orc_check_tf_mul_pow2_fast
//   orc_oz1_slices/gemm_diag/     reference output hashes of scheme I INT8 (tools/validated/quick.csv:12,
//   recon/int8_gemm               phi_sweep.log chash of I-INT8 4096^3), the slice exactness
//                                 invariant sum_i d_i radix^-(i+1) + residual == x*2^delta, brute force
#pragma once
#include <cstddef>
#include <cstdint>

extern "C" {
// Bit pattern hash of a double array (evaluation/numerics.hpp:46-57).
uint64_t orc_hash_f64(const double* c, size_t n);
// BASELINE input generator (evaluation/numerics.hpp:19-38 with the seed as a parameter): A (na
// elements) first, then B (nb elements); phi < 0 selects the uniform [-1,1) input.
void orc_inputs(unsigned seed, double phi, size_t na, size_t nb, double* a, double* b);

// A5: row (mode 0) or column (mode 1) maxima of |X| on FP64 bits -> BF16 (ceil_mode 0/1/2) ->
// e = ceil(log2) -> delta = shift - e; flags |= 1 (above BF16), 2 (below 2^-126), 4 (Inf/NaN).
// (scale_f64_reader.cpp:106-197, scale_bits.h:34-62, expdelta.cpp:44-90)
void orc_scale(const double* X, int rows, int cols, int ld, int mode, int ceil_mode, int shift, int32_t* delta,
               uint32_t* flags);
// A6: FP64 words -> four FP32 bit patterns hi, braw, craw, s (f64_tf.h:141-172).
void orc_split_f64(uint32_t w1, uint32_t w0, int32_t d, uint32_t* out4);
// A6 + tf_load_f64: the triple-float (hi, mid, lo) the slicer starts from (slice_tf_core.h:67-76).
void orc_load_triple(double x, int32_t d, float* out3);
// A7: the nd radix-2^20 digits of A' for every element, top digit first: digits[(r*cols+c)*nd + j].
// (digits.h:80-112). mode 0: delta per row, mode 1: delta per column.
void orc_oz2_digits(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd,
                    float* digits);
// A8: residues A' mod m_s for S moduli, planes[s][r][c] (digits.h:165-179, modslice_int8.cpp:60-95).
void orc_oz2_residues(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                      const int* m, int8_t* planes);
// The same residues as int16 values, for the moduli of the digit routes (up to 4096).
void orc_oz2_residues16(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                        const int* m, int16_t* planes);
// A18: the residues split into digit planes (modslice_digit.cpp:195-218, sparse_fix.h:53-73):
// per modulus s with digit radix q[s] and mode xmode[s] (0 rounded, 1 Karatsuba, 2 sparse square,
// 3 one digit: the residue itself, one plane),
// planes l, h (and s = h + l for Karatsuba) as int8 values, planes[p][r][c], moduli in order.
void orc_oz2_digit_planes(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int nd, int S,
                          const int* m, const int* q, const int* xmode, int8_t* planes);
// The reference's ModRound on one value (sfpu_tf_proc.h:316-319).
float orc_modround(float d, float m, float rinv);
// A9: C = A*B exactly (int64 accumulation; returns the largest |C| seen). A: MxK, B: KxN, row-major.
int64_t orc_gemm_i8(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K);

// CRT constants of a moduli set at width b (ozaki2/moduli.hpp:615-703): yi[S], rinv[S] (float),
// c[4*S] (2^20j mod m, j=1..4), m16[S], rp0[S*5], rp1[S*5], rp2[S*3] (float), KM (long double ->
// W hi/lo + qw), nsmall[3] (rp0, rp1, rp2).
struct orc_crt_consts {
    int S, b;
    int m[24], yi[24];
    float rinv[24], c[4][24], m16[24];
    float rp0[24][5], rp1[24][5], rp2[24][3];
    uint32_t Whi, Wlo;
    int32_t qw;
    uint32_t nsmall0, nsmall1, nsmall2;
    double KM;
};
void orc_crt_constants(int S, const int* m, int b, orc_crt_consts* out);
// A10-A11 as the reference computes them: per element triple-float CRT with 12-bit reciprocal
// fragments, then the 128-bit fixed-point fold and FP64 assembly (recon_crt.cpp:181-338,
// recon_crt_proc.h, recon_writer.cpp:70-192, recon_elem.h, f64_tf.h:189-400).
// C: S int32 planes [S][M][N]; dA[M], dB[N]: exponent deltas; nd: digits of A'.
void orc_oz2_crt_ref(const int32_t* C, int M, int N, int S, const int* m, int b, int nd, int two_pass,
                     const int32_t* dA, const int32_t* dB, double* out);
// Exact CRT: C' = the unique integer in (-M/2, M/2) with C' = C_s (mod m_s), rounded once to FP64
// (nearest-even) after scaling by 2^(eA+eB-2b); results below the normal range become signed zero.
void orc_oz2_crt_exact(const int32_t* C, int M, int N, int S, const int* m, int b, int nd, const int32_t* dA,
                       const int32_t* dB, double* out);
// C' of one element as two's-complement 256-bit little-endian words (for white-box tests).
void orc_oz2_crt_exact_int(const int32_t* r, int S, const int* m, uint64_t* out4);

// Binary128 reference for a set of output elements: c[t] = sum_k A[i_t,k] B[k,j_t] rounded to FP64.
void orc_gemm_quad_sample(const double* A, const double* B, int M, int N, int K, int nsample, const int* rows,
                          const int* cols, double* out);
// Dot2 compensated FP64 GEMM as the reference evaluator runs it (evaluation/numerics.hpp:58-93),
// OpenMP over row blocks; returns hi and lo parts. rows [r0, r1) only.
void orc_dot2_gemm(const double* A, const double* B, int M, int N, int K, int r0, int r1, double* Chi, double* Clo);

// ---- Scheme I ----
// Slicer (slice_tf_body.h:86-131): p digits of x*2^delta, radix `radix` (tfMulR, or tfMulP2 for a power
// of two), digits clamp(Rnd(t0), +-dmax); planes[i][r][c].
void orc_oz1_slices(const double* X, int rows, int cols, int ld, int mode, const int32_t* delta, int p, int radix,
                    int dmax, int8_t* planes);
// Equivalence check of tfMulR's Dekker form and its TwoProduct form (the GPU's tf_mul_r_fma) on n
// pseudo-random slicer chains (mode 0) or reconstruction Horner chains (mode 1), in the FP32 model;
// returns the covered chains that differ, *covered the covered count (see oz_oracle.cpp).
int64_t orc_check_tf_mul_r_forms(int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                                 int64_t* covered);
int64_t orc_check_tf_mul_r_fast(int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                                int64_t* covered, int64_t* violations);
int64_t orc_check_tf_mul_pow2_fast(int mode, int64_t n, uint64_t seed, int radix, int dmax, int planes,
                                   int64_t* covered, int64_t* violations);
// Diagonal partial products P_d = sum_{i<=d} A_i B_{d-i} (ozaki1/gemm.hpp:315), exact; returns max |P|.
int64_t orc_oz1_gemm_diag(const int8_t* A, const int8_t* B, int32_t* P, int M, int N, int K, int p, int ndiag);
// Horner reconstruction + FP64 assembly (recon_tf_i32in.cpp:116-157, recon_f64_writer.cpp:148-160).
void orc_oz1_recon(const int32_t* P, int M, int N, int ndiag, int radix, int signmag, int nsingle, const int32_t* dA,
                   const int32_t* dB, double* out);
// The reconstruction K block by K block (recon_tf_f32in.cpp:54-89, plan.hpp:104-109): P holds nkb
// blocks of ndiag planes of exact sums of at most 2^24; per block the Horner sum with every P_d
// whole, then from the second block on the previous limbs added (lo, mid, hi); the last block is
// assembled to FP64. Parity unpinned: no reference record runs this plan; pinned by agreement with
// the single-block reconstruction up to its last bits (tests/test_oracle.py).
void orc_oz1_recon_blocks(const int32_t* P, int M, int N, int ndiag, int nkb, int radix, const int32_t* dA,
                          const int32_t* dB, double* out);
// radix^-(L+2) as W = Whi:Wlo (64-bit significand) and 2^qw (ozaki1/plan.hpp:446-460).
void orc_oz1_scale_w(int radix, int L, uint32_t* Whi, uint32_t* Wlo, int32_t* qw);
// Scheme I INT8 end to end with p slices on padded row-major A, B; returns max |P_d|.
int64_t orc_oz1_int8_gemm(const double* A, const double* B, int M, int N, int K, int p, double* out);
}
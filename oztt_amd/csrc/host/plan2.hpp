// Scheme II planning on the host: moduli set, integer width b, number of reconstruction passes,
// digits of A', and the constants the device stages need. Nothing here touches the device.
//
// The decisions restate the reference planner (src/backend/ozaki2/plan.hpp:258-306
// choose_moduli_and_width, moduli.hpp:719-769 ozaki2_choose_moduli, auto_precision.hpp:95-139,
// common/norm_estimate.hpp:21-73): the moduli and b define the residues, which must match the
// reference bit for bit, so every rule, table and floating-point evaluation order is kept.
#pragma once

#include <cstdint>
#include <limits>
#include <optional>
#include <string>
#include <vector>

#include <ozTTgemm/ozTTgemm.hpp>

#include "oz_hip.h"

namespace ozTTgemm::detail {

inline constexpr int kTargetBits = 53;    // FP64 significand (moduli.hpp:62)
inline constexpr int kDefaultBits = 54;   // default cap on b (moduli.hpp:66)
inline constexpr int kMaxModuli = 24;     // OZ2_MAXS (digit_limits.h:19)
inline constexpr int kDigitBits = 20;     // radix 2^20 of the digits of A' (digit_limits.h:29)
inline constexpr int kMaxDigits = 5;      // digit_limits.h:39
inline constexpr int kAccBits = 31;       // INT8 products read back exactly within 2^31-1 (moduli.hpp:57)

// Input statistics used by the precision and pass models (auto_precision.hpp:17-21, :68-75).
struct OperandStats {
    double TA = 0, TB = 0;  // sum over rows of A / columns of B of (power-of-two scale)^2
    double nA = 0, nB = 0;  // ||A||_F^2, ||B||_F^2 (after the power-of-two normalization)
    double nC = 0;          // low-biased Hutchinson estimate of ||C||_F^2
    double wA = 0, wB = 0;  // largest normalized row norm of A / column norm of B (||a_i||_2 / tau_i)
    // rigorous upper bounds on the largest ||a_i||_2 / 2^ceil(log2 max_k |a_ik|) over the rows of A and
    // the same over the columns of B (between 0 and sqrt(K)); not part of the reference's statistics
    double rA = 0, rB = 0;
    bool measured = false;
};

// Carrying methods of a modulus on the digit routes (split.hpp:176-214 OZ2_SPLIT_*): square modulus
// with balanced digits (3 products), Karatsuba (3), wide two-digit (4), n balanced digits (n^2, or
// n(n+1)/2 when m divides the digit cap), square with sparse digits (3), one digit (1).
inline constexpr int kSplitSq = 0, kSplitKar = 1, kSplitWide = 2, kSplitBal = 3, kSplitSqs = 4, kSplitOne = 5;

// One product output of the FP8 route (split.hpp:628-661 oz2_product_groups): the sum of npairs
// digit products over K, A digit plane a[t] times B digit plane b[t] (global plane indices, the
// moduli's planes one after the other), composed into modulus s with coefficient coef (mod m_s).
struct Fp8Output {
    int s = 0, npairs = 0;
    int a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};
    long coef = 0;
    double bound = 0;  // largest |sum| (oz2_group_bound)
};

// Result of the moduli selection (the subset of the reference's Ozaki2Moduli that this build uses).
struct ModuliSet {
    bool ok = false;
    bool acc_ok = true;
    int b = 0;
    std::vector<int> m;
    double log2M = 0;
    int m_cap = 0, ncand = 0;
    std::string acc_fail;  // first failed accumulation condition (empty when all hold)
    // digit routes only (every format but INT8)
    bool digits = false, sparse = false, fold_first = false;
    bool model_set = false;         // chosen by the stage-time model (awe.hpp), not from the table
    std::vector<int> mode, maxg_m;  // carrying method and concatenation bound per modulus
    std::vector<int> q;             // digit radix per modulus
    std::vector<Fp8Output> outputs; // FP8: product outputs in the reference's order (modulus by modulus)
    int maxg = 1, nprod = 0, nplane = 0, nout = 0;
};

// The plan of one Scheme II call: the moduli set of the requested format's route (`route`: what Info
// reports under Transport::Automatic and what the pass choice is made on), the set the device computes
// with (`mo`), the width b, digits of A' and passes. `mo` is `route` for INT8, and for FP8 on its own
// digits (fp8_digits); otherwise an INT8 set of the same width b (or, beyond the INT8 width, the FP8
// route's set); either is then replaced by a smaller set when the operands' own bound on |C'| allows
// one (bound_log2). C is the same (every set reconstructs the exact product A'B').
struct Plan2 {
    std::uint32_t M = 0, N = 0, K = 0;  // padded dimensions
    std::uint32_t S_req = 0;
    Format format = Format::INT8;
    ModuliSet route;
    ModuliSet mo;
    bool fp8_digits = false;  // the products are the FP8 route's e4m3 digit products
    int b = 0, nd = 3, S = 0;  // S: moduli of mo
    bool two_pass = false;
    int shift() const { return b - kDigitBits * (nd - 1); }  // plan.hpp:81 oz2_shift
    OperandStats stats;
    double recon1_log2 = 0;  // one-pass error estimate (log2), -inf when not estimated
    // The CRT window from the operands: log2 of an upper bound on max |C'_ij| (C' = A'B', the exact
    // integer product), +inf when the operands were not measured. When it needs fewer products than
    // the planned window K 2^(2b), `mo` is the set chosen for it (INT8 residues, or the FP8 route's
    // digits) and S_window the number of moduli of the set it replaced (the exact CRT recovers the
    // same C' from any set whose M exceeds 2 max |C'|).
    double bound_log2 = std::numeric_limits<double>::infinity();
    int S_window = 0;  // moduli of the set for the window K 2^(2b) (0: mo is that set)
};

// Statistics of padded row-major A (M x K) and B (K x N): tau sums and norms after the power-of-two
// normalization, and the product-norm estimate. Deterministic and identical to the reference's
// sequential evaluation; rows and columns are distributed over threads without changing any order
// of floating-point operations.
OperandStats measure_stats(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K);

// Cap on b from the statistics (auto_precision.hpp:95-107).
int precision_cap(const OperandStats& st);

// Moduli selection for the INT8 path (moduli.hpp:719-769 with the INT8 route of split.hpp:73).
// window_log2 replaces the CRT window log2 K (|C'| <= 2^(2b + window_log2)); NaN keeps it.
ModuliSet choose_moduli_int8(std::uint32_t K, int num_moduli, int b_cap,
                             double window_log2 = std::numeric_limits<double>::quiet_NaN());
// Moduli selection on the digit route of a format other than INT8 (moduli.hpp:719-769 with the format's
// row of OZ2_ROUTES, split.hpp:66-146): the table selection for FP8 and TF32, the stage-time model's
// set (awe.hpp) for BF16, FP16, BFP8, BFP4 and BFP2. M and N feed only the model's memory estimate.
// The CRT window is log2 K (the library's rule); window_log2 replaces it (used to restate the research
// planner that wrote the reference's accuracy logs, which measured the window from the input).
ModuliSet choose_moduli_digits(Format format, std::uint32_t M, std::uint32_t N, std::uint32_t K, int num_moduli,
                               int b_cap, double window_log2 = std::numeric_limits<double>::quiet_NaN());
// The FP8 set of fewest e4m3 digit products (at most num_moduli moduli) whose M exceeds 2^(2b + 1 +
// window_log2): every subset of one-digit moduli (residues of at most 16 in magnitude, the digit
// itself, one product; the reference's FP8 route does not use them), filled with the route's squares,
// Karatsuba and wide moduli in order of bits per product, then checked and laid out as
// choose_moduli_digits lays out its sets (exact FP32 accumulation, outputs, planes). Not the
// reference's selection: an execution set that gives the same C as the route's (the exact CRT).
ModuliSet choose_moduli_fp8_fewest(std::uint32_t K, int num_moduli, int b, double window_log2);
// The limit on the number of moduli of a format's route when the caller fixes the width b and gives
// no max_moduli (Oz2Route::def_s: 16 for INT8, 14 for FP8, 11 for TF32, 24 otherwise).
std::uint32_t default_moduli(Format format);

// log2 of the expected relative error of one reconstruction pass (auto_precision.hpp:128-139).
double recon1_log2(const ModuliSet& mo, int b, const OperandStats& st);

// The whole plan (plan.hpp:258-306). fixed_b: width fixed by the caller (evaluator only).
// int8_transport (Transport::Int8Residues): FP8 is carried by INT8 residues at the FP8 plan's width
// whenever an INT8 set reaches that width; otherwise FP8 computes the FP8 route's e4m3 digit products
// on the FP8 matrix cores. The other digit formats are carried by INT8 residues either way.
// operand_window: INT8 residues compute with the smallest set that covers the operands' own bound
// on |C'| (Plan2::bound_log2) when that needs fewer moduli than the window K 2^(2b).
// Throws std::runtime_error when no exact configuration exists.
Plan2 plan_scheme2(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K, Format format,
                   std::uint32_t max_moduli, Reconstruction passes, std::optional<unsigned> fixed_b,
                   bool int8_transport = false, bool operand_window = true);

// Device descriptors of the plan.
oz2_moduli_dev split_descriptor(const Plan2& p);
oz2_crt_dev crt_descriptor(const Plan2& p);
// FP8 route: the digit split (e4m3 planes) and the product outputs with their CRT coefficients
// (coefficient * y_s mod m_s, y_s from crt), ordered with the outputs of more pairs first;
// term_modulus receives the modulus of each output in that order.
oz2_digit_dev digit_descriptor(const Plan2& p);
oz2_groups_dev groups_descriptor(const Plan2& p, const oz2_crt_dev& crt, std::vector<unsigned char>& term_modulus);

}  // namespace ozTTgemm::detail

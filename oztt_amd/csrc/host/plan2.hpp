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
    bool measured = false;
};

// Carrying methods of a modulus on the FP8 route (split.hpp:176-214 OZ2_SPLIT_*): square modulus with
// balanced digits (3 products), radix-16 Karatsuba (3), wide two-digit (4), square with sparse digits (3).
inline constexpr int kFp8SplitSq = 0, kFp8SplitKar = 1, kFp8SplitWide = 2, kFp8SplitSqs = 4;

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
    // FP8 route only
    bool fp8 = false, sparse = false, fold_first = false;
    std::vector<int> mode, maxg_m;  // carrying method and concatenation bound per modulus
    std::vector<int> q;             // digit radix per modulus
    std::vector<Fp8Output> outputs; // product outputs in the reference's order (modulus by modulus)
    int maxg = 1, nprod = 0, nplane = 0, nout = 0;
};

// The plan of one Scheme II call: the moduli set of the requested format's route (`route`: what Info
// reports and what the pass choice is made on), the set the device computes with (`mo`), the width b,
// digits of A' and passes. `mo` is `route` except for FP8 carried by INT8 residues (fp8_digits false):
// then `mo` is an INT8 set of the same width b, and C is the same (both sets reconstruct the exact
// product A'B').
struct Plan2 {
    std::uint32_t M = 0, N = 0, K = 0;  // padded dimensions
    std::uint32_t S_req = 0;
    Format format = Format::INT8;
    ModuliSet route;
    ModuliSet mo;
    bool fp8_digits = false;  // the products are the FP8 route's e4m3 digit products (mo == route)
    int b = 0, nd = 3, S = 0;  // S: moduli of mo
    bool two_pass = false;
    int shift() const { return b - kDigitBits * (nd - 1); }  // plan.hpp:81 oz2_shift
    OperandStats stats;
    double recon1_log2 = 0;  // one-pass error estimate (log2), -inf when not estimated
};

// Statistics of padded row-major A (M x K) and B (K x N): tau sums and norms after the power-of-two
// normalization, and the product-norm estimate. Deterministic and identical to the reference's
// sequential evaluation; rows and columns are distributed over threads without changing any order
// of floating-point operations.
OperandStats measure_stats(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K);

// Cap on b from the statistics (auto_precision.hpp:95-107).
int precision_cap(const OperandStats& st);

// Moduli selection for the INT8 path (moduli.hpp:719-769 with the INT8 route of split.hpp:73).
ModuliSet choose_moduli_int8(std::uint32_t K, int num_moduli, int b_cap);
// Moduli selection for the FP8 route (moduli.hpp:719-769 with OZ2_ROUTE_FP8, split.hpp:72-76). The CRT
// window is log2 K (the library's rule); window_log2 replaces it (used to restate the research planner
// that wrote the reference's accuracy logs, which measured the window from the input).
ModuliSet choose_moduli_fp8(std::uint32_t K, int num_moduli, int b_cap,
                            double window_log2 = std::numeric_limits<double>::quiet_NaN());

// log2 of the expected relative error of one reconstruction pass (auto_precision.hpp:128-139).
double recon1_log2(const ModuliSet& mo, int b, const OperandStats& st);

// The whole plan (plan.hpp:258-306). fixed_b: width fixed by the caller (evaluator only).
// fp8_matrix_cores: FP8 computes the FP8 route's e4m3 digit products on the FP8 matrix cores; otherwise
// it is carried by INT8 residues at the FP8 plan's width whenever an INT8 set reaches that width.
// Throws std::runtime_error when no exact configuration exists.
Plan2 plan_scheme2(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K, Format format,
                   std::uint32_t max_moduli, Reconstruction passes, std::optional<unsigned> fixed_b,
                   bool fp8_matrix_cores = false);

// Device descriptors of the plan.
oz2_moduli_dev split_descriptor(const Plan2& p);
oz2_crt_dev crt_descriptor(const Plan2& p);
// FP8 route: the digit split (e4m3 planes) and the product outputs with their CRT coefficients
// (coefficient * y_s mod m_s, y_s from crt), ordered with the outputs of more pairs first;
// term_modulus receives the modulus of each output in that order.
oz2_digit_dev digit_descriptor(const Plan2& p);
oz2_groups_dev groups_descriptor(const Plan2& p, const oz2_crt_dev& crt, std::vector<unsigned char>& term_modulus);

}  // namespace ozTTgemm::detail

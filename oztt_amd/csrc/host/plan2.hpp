// Scheme II planning on the host: moduli set, integer width b, number of reconstruction passes,
// digits of A', and the constants the device stages need. Nothing here touches the device.
//
// The decisions restate the reference planner (src/backend/ozaki2/plan.hpp:258-306
// choose_moduli_and_width, moduli.hpp:719-769 ozaki2_choose_moduli, auto_precision.hpp:95-139,
// common/norm_estimate.hpp:21-73): the moduli and b define the residues, which must match the
// reference bit for bit, so every rule, table and floating-point evaluation order is kept.
#pragma once

#include <cstdint>
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

// Result of the moduli selection (the subset of the reference's Ozaki2Moduli that the INT8 path uses).
struct ModuliSet {
    bool ok = false;
    bool acc_ok = true;
    int b = 0;
    std::vector<int> m;
    double log2M = 0;
    int m_cap = 0, ncand = 0;
    std::string acc_fail;  // first failed accumulation condition (empty when all hold)
};

// The plan of one Scheme II call.
struct Plan2 {
    std::uint32_t M = 0, N = 0, K = 0;  // padded dimensions
    std::uint32_t S_req = 0;
    ModuliSet mo;
    int b = 0, nd = 3, S = 0;
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

// log2 of the expected relative error of one reconstruction pass (auto_precision.hpp:128-139).
double recon1_log2(const ModuliSet& mo, int b, const OperandStats& st);

// The whole plan (plan.hpp:258-306). fixed_b: width fixed by the caller (evaluator only).
// Throws std::runtime_error when no exact configuration exists.
Plan2 plan_scheme2_int8(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
                        std::uint32_t max_moduli, Reconstruction passes, std::optional<unsigned> fixed_b);

// Device descriptors of the plan.
oz2_moduli_dev split_descriptor(const Plan2& p);
oz2_crt_dev crt_descriptor(const Plan2& p);

}  // namespace ozTTgemm::detail

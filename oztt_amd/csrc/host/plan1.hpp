// Scheme I planning on the host: the number of slices p (automatic selection from the input), the
// issue of the diagonal products with its exactness conditions, and the reconstruction constants.
// Nothing here touches the device.
//
// The decisions restate the reference planner (src/backend/ozaki1/auto_precision.hpp:90-527,
// plan.hpp:95-240 and :412-460, format.hpp:60-190, param.hpp:63-101): p defines the slices, which
// must match the reference bit for bit, so every rule and floating-point evaluation order is kept.
#pragma once

#include <cstdint>

namespace ozTTgemm::detail {

// Scheme I constants of a format (param.hpp:63-101, format.hpp:60-126).
struct Oz1Format {
    int radix;             // weight of a digit
    int dmax;              // digit bound (radix / 2 for every format here)
    std::uint32_t ceil;    // rounding of the BF16 maxima: 0 truncate, 1 up, 2 up and powers of two up
    int nshift;            // normalization target 2^nshift
    bool int32_partial;    // the products accumulate in int32 (INT8) rather than exactly in FP32
    std::uint32_t acc_bits;  // bits the accumulator holds exactly: 31 (int32 magnitude) or 24 (FP32)
};
// INT8: sign-magnitude bytes, digits +-127, radix 254, int32 products, maxima rounded up.
inline constexpr Oz1Format kOz1Int8{254, 127, 1u, -1, true, 31u};
// BF16, FP16, TF32 and BFP8: radix 64, digits +-32, FP32 products (the four formats differ only in how
// the reference's matrix engine receives the same digits).
inline constexpr Oz1Format kOz1Bf16{64, 32, 0u, -1, false, 24u};
// FP8 (e4m3): radix 32, digits +-16.
inline constexpr Oz1Format kOz1Fp8{32, 16, 0u, -1, false, 24u};
// BFP4: radix 14, digits +-7.
inline constexpr Oz1Format kOz1Bfp4{14, 7, 0u, -1, false, 24u};
// BFP2: radix 2, digits +-1, target 1 and the scale stepped above exact powers of two.
inline constexpr Oz1Format kOz1Bfp2{2, 1, 2u, 0, false, 24u};

// Diagnostics of the automatic selection (the two model estimates at the chosen p, in bits).
struct Oz1AutoInfo {
    int pmax = 0;
    double bits_indep = 0;    // -log2 sqrt(estimate (1)) at p
    double bits_sampled = 0;  // -log2 sqrt(estimate (2)) at p
};

// Number of slices for padded row-major A (M x K) and B (K x N) (auto_precision.hpp:506-525,
// oz_fp64_p): the p for which both the independent-sign model and the sampled simulation expect a
// relative error of at most 2^-53, found by the reference's search.
int oz1_auto_p(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
               const Oz1Format& f, Oz1AutoInfo* info = nullptr);

// How the diagonal products are issued and accumulated (plan.hpp:95-240).
struct IssuePlan1 {
    bool pairloop = false, pairwise = false, fuse = false, defer = false;
    std::uint32_t Kc = 0, nkb = 0;  // K block length and number of K blocks
};

// Scheme I constants of a public format (0..7 = Format::BF16 .. BFP2).
const Oz1Format& oz1_format(int format);

struct Plan1 {
    std::uint32_t M = 0, N = 0, K = 0;
    int p = 0;  // slices = diagonals
    Oz1Format f{};
    IssuePlan1 issue;
    int nsmall = 0;          // leading diagonals read whole by the reconstruction (plan.hpp:424-430)
    bool signmag = false;    // the reconstruction reads the INT8 products (magnitude split) rather than int32 sums
    std::uint32_t Whi = 0, Wlo = 0;
    std::int32_t qw = 0;     // radix^-(p+1) = (Whi:Wlo) * 2^qw (plan.hpp:434-460)
    Oz1AutoInfo autop;
};

// K block length whose accumulation of (L+1) K_c digit products is exact (format.hpp:136-158).
std::uint32_t oz1_block_k(std::uint32_t K, int L, const Oz1Format& f);

// The whole plan: p (slices, or automatic when 0), issue, reconstruction constants. Throws
// std::runtime_error when the configuration cannot be executed (plan.hpp:177-240). issue.defer false
// for a format with FP32 products means the reconstruction runs K block by K block (recon_limbs).
Plan1 plan_scheme1(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
                   std::uint32_t slices, const Oz1Format& f);

}  // namespace ozTTgemm::detail

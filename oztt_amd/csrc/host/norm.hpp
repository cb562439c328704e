// Operand scaling and the product-norm estimate shared by the precision models of both schemes
// (reference common/norm_estimate.hpp:21-73). Host only.
#pragma once

#include <cstddef>
#include <cstdint>

namespace ozTTgemm::detail {

// Power of two by which a matrix is divided before sums of squares are formed: 2^e with e the
// exponent of the largest magnitude (frexp), clamped to [-1000, 1000]; 1 for an all-zero or
// non-finite maximum (norm_estimate.hpp:21-30).
double pow2_scale(const double* v, std::size_t n);

// Low-biased Hutchinson estimate of ||(rgA A)(rgB B)||_F^2 for row-major A (M x K), B (K x N):
// L = 8 Gaussian vectors from mt19937(12345), sums in x86 extended precision in the reference's
// order, the largest sample dropped and the rest divided by 1 + 2 sqrt(2/L)
// (norm_estimate.hpp:49-73). The loops are distributed over threads without changing any
// floating-point order, so the value is the reference's for any thread count.
double estimate_product_norm(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
                             double rgA, double rgB);

}  // namespace ozTTgemm::detail

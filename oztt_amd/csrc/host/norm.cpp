// See norm.hpp. Compiled with -ffp-contract=off, like the reference (its Makefile:51-53).
#include "norm.hpp"

#include <algorithm>
#include <cstdint>
#include <cmath>
#include <limits>
#include <random>
#include <vector>

namespace ozTTgemm::detail {

static_assert(std::numeric_limits<long double>::digits == 64,
              "the norm estimate accumulates in x86 extended precision, like the reference (bits.hpp:18-19)");

double pow2_scale(const double* v, std::size_t n) {
    // the maximum does not depend on the order of the comparisons: blocks in parallel
    double mx = 0;
#pragma omp parallel for schedule(static) reduction(max : mx)
    for (std::int64_t i = 0; i < (std::int64_t)n; i++) mx = std::max(mx, std::fabs(v[i]));
    if (!(mx > 0) || !std::isfinite(mx)) return 1.0;
    int e;
    std::frexp(mx, &e);
    e = std::min(std::max(e, -1000), 1000);
    return std::ldexp(1.0, e);
}

namespace {

// out[r] = sum_c (X[r][c] * rg) * v[c] for r < rows, each row summed in column order in x86
// extended precision (norm_estimate.hpp:35-44). Four rows are summed together: their chains are
// independent, so the additions overlap instead of waiting on one another; each row's own sequence
// of operations, and so its value, is unchanged.
void matvec_x87(const double* X, std::uint32_t rows, std::uint32_t cols, double rg, const double* v, double* out) {
    const std::int64_t groups = ((std::int64_t)rows + 3) / 4;
#pragma omp parallel for schedule(static)
    for (std::int64_t gi = 0; gi < groups; gi++) {
        const std::uint32_t r0 = (std::uint32_t)gi * 4;
        if (r0 + 4 <= rows) {
            const double* x0 = X + (std::size_t)r0 * cols;
            const double* x1 = x0 + cols;
            const double* x2 = x1 + cols;
            const double* x3 = x2 + cols;
            long double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (std::uint32_t c = 0; c < cols; c++) {
                const long double vc = v[c];
                s0 += (long double)(x0[c] * rg) * vc;
                s1 += (long double)(x1[c] * rg) * vc;
                s2 += (long double)(x2[c] * rg) * vc;
                s3 += (long double)(x3[c] * rg) * vc;
            }
            out[r0] = (double)s0;
            out[r0 + 1] = (double)s1;
            out[r0 + 2] = (double)s2;
            out[r0 + 3] = (double)s3;
        } else {
            for (std::uint32_t r = r0; r < rows; r++) {
                long double s = 0;
                const double* x = X + (std::size_t)r * cols;
                for (std::uint32_t c = 0; c < cols; c++) s += (long double)(x[c] * rg) * v[c];
                out[r] = (double)s;
            }
        }
    }
}

}  // namespace

double estimate_product_norm(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
                             double rgA, double rgB) {
    const std::uint32_t L = 8;
    std::mt19937 rg(12345);
    std::normal_distribution<double> nd(0.0, 1.0);
    std::vector<double> g(N), y(K), q_i(M);
    double cs2 = 0, cmax = 0;
    for (std::uint32_t l = 0; l < L; l++) {
        for (std::uint32_t j = 0; j < N; j++) g[j] = nd(rg);
        matvec_x87(B, K, N, rgB, g.data(), y.data());
        matvec_x87(A, M, K, rgA, y.data(), q_i.data());
        double q = 0;
        for (std::uint32_t i = 0; i < M; i++) q += q_i[i] * q_i[i];
        cs2 += q;
        cmax = std::max(cmax, q);
    }
    return (cs2 - cmax) / (L - 1) / (1.0 + 2.0 * std::sqrt(2.0 / (double)L));
}

}  // namespace ozTTgemm::detail

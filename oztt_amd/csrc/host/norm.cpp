// See norm.hpp. Compiled with -ffp-contract=off, like the reference (its Makefile:51-53).
#include "norm.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <random>
#include <vector>

namespace ozTTgemm::detail {

static_assert(std::numeric_limits<long double>::digits == 64,
              "the norm estimate accumulates in x86 extended precision, like the reference (bits.hpp:18-19)");

double pow2_scale(const double* v, std::size_t n) {
    double mx = 0;
    for (std::size_t i = 0; i < n; i++) mx = std::max(mx, std::fabs(v[i]));
    if (!(mx > 0) || !std::isfinite(mx)) return 1.0;
    int e;
    std::frexp(mx, &e);
    e = std::min(std::max(e, -1000), 1000);
    return std::ldexp(1.0, e);
}

double estimate_product_norm(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
                             double rgA, double rgB) {
    const std::uint32_t L = 8;
    std::mt19937 rg(12345);
    std::normal_distribution<double> nd(0.0, 1.0);
    std::vector<double> g(N), y(K), q_i(M);
    double cs2 = 0, cmax = 0;
    for (std::uint32_t l = 0; l < L; l++) {
        for (std::uint32_t j = 0; j < N; j++) g[j] = nd(rg);
#pragma omp parallel for schedule(static)
        for (std::int64_t k = 0; k < (std::int64_t)K; k++) {
            long double s = 0;
            const double* row = B + (std::size_t)k * N;
            for (std::uint32_t j = 0; j < N; j++) s += (long double)(row[j] * rgB) * g[j];
            y[k] = (double)s;
        }
#pragma omp parallel for schedule(static)
        for (std::int64_t i = 0; i < (std::int64_t)M; i++) {
            long double s = 0;
            const double* row = A + (std::size_t)i * K;
            for (std::uint32_t k = 0; k < K; k++) s += (long double)(row[k] * rgA) * y[k];
            q_i[i] = (double)s;
        }
        double q = 0;
        for (std::uint32_t i = 0; i < M; i++) q += q_i[i] * q_i[i];
        cs2 += q;
        cmax = std::max(cmax, q);
    }
    return (cs2 - cmax) / (L - 1) / (1.0 + 2.0 * std::sqrt(2.0 / (double)L));
}

}  // namespace ozTTgemm::detail

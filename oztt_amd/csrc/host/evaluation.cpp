// Evaluation hooks and utilities; see evaluation.hpp.
#include "evaluation.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <stdexcept>

namespace ozTTgemm::evaluation {
namespace {
thread_local Settings* g_active = nullptr;
}

Scope::Scope(Settings& s) {
    if (g_active) throw std::logic_error("evaluation scopes cannot be nested");
    g_active = &s;
}
Scope::~Scope() { g_active = nullptr; }
Settings* active() noexcept { return g_active; }

void inputs(unsigned seed, double phi, std::size_t na, std::size_t nb, double* a, double* b) {
    std::mt19937 rng(seed);
    if (phi < 0) {
        std::uniform_real_distribution<double> u(-1, 1);
        for (std::size_t i = 0; i < na; i++) a[i] = u(rng);
        for (std::size_t i = 0; i < nb; i++) b[i] = u(rng);
        return;
    }
    std::uniform_real_distribution<double> u(0, 1);
    std::normal_distribution<double> normal(0, 1);
    for (std::size_t i = 0; i < na + nb; i++) {
        const double v = u(rng);  // u is drawn before z (sequenced statements)
        const double z = normal(rng);
        (i < na ? a[i] : b[i - na]) = (v - 0.5) * std::exp(phi * z);
    }
}

std::uint64_t output_hash(const double* c, std::size_t n) {
    std::uint64_t h = 1469598103934665603ull;
    for (std::size_t z = 0; z < n; z++) {
        std::uint64_t u;
        std::memcpy(&u, &c[z], 8);
        for (int sh = 0; sh < 64; sh += 8) {
            h ^= (u >> sh) & 0xFFu;
            h *= 1099511628211ull;
        }
    }
    return h;
}

void gemm_quad_sample(const double* A, const double* B, int M, int N, int K, int nsample, const int* rows,
                      const int* cols, double* out) {
    (void)M;
#pragma omp parallel for schedule(dynamic)
    for (int t = 0; t < nsample; t++) {
        __float128 s = 0;
        const int i = rows[t], j = cols[t];
        for (int k = 0; k < K; k++) s += (__float128)A[(std::size_t)i * K + k] * (__float128)B[(std::size_t)k * N + j];
        out[t] = (double)s;
    }
}

void reference_gemm(const double* A, const double* B, std::uint32_t M, std::uint32_t K, std::uint32_t N,
                    std::uint32_t r0, std::uint32_t r1, double* Chi, double* Clo) {
    // Each element accumulates k = 0, 1, ... in order: p = a*b and its exact error e (one FMA), the
    // TwoSum of the running head with p, and the tail collecting both errors. Rows are independent, so
    // they are spread over the threads; the inner loop runs along a row of B (vectorizable).
    r1 = std::min(r1, M);
#pragma omp parallel for schedule(dynamic, 1)
    for (std::int64_t i = r0; i < (std::int64_t)r1; i++) {
        double* chi = Chi + (std::size_t)(i - r0) * N;
        double* clo = Clo + (std::size_t)(i - r0) * N;
        std::fill(chi, chi + N, 0.0);
        std::fill(clo, clo + N, 0.0);
        for (std::uint32_t k = 0; k < K; k++) {
            const double a = A[(std::size_t)i * K + k];
            const double* b = B + (std::size_t)k * N;
            for (std::uint32_t j = 0; j < N; j++) {
                const double p = a * b[j], e = std::fma(a, b[j], -p);
                const double c0 = chi[j];
                const double t = c0 + p, bb = t - c0;
                clo[j] += ((c0 - (t - bb)) + (p - bb)) + e;
                chi[j] = t;
            }
        }
    }
}

Accuracy accuracy(const double* C, const double* Chi, const double* Clo, std::size_t n) {
    // the reference value renormalized (TwoSum of head and tail); sums of squares scaled by the largest
    // magnitude so that neither overflows nor underflows
    auto ref = [&](std::size_t z, double& h, double& l) {
        const double t = Chi[z] + Clo[z], bb = t - Chi[z];
        h = t;
        l = (Chi[z] - (t - bb)) + (Clo[z] - bb);
    };
    double mx = 0;
    for (std::size_t z = 0; z < n; z++) {
        double h, l;
        ref(z, h, l);
        mx = std::max(mx, std::max(std::fabs(h), std::fabs((C[z] - h) - l)));
    }
    const int sce = (mx > 0 && std::isfinite(mx)) ? -std::ilogb(mx) : 0;
    const int sce1 = std::min(sce, 1023);
    const double sc1 = std::ldexp(1.0, sce1), sc2 = std::ldexp(1.0, sce - sce1);
    double num = 0, den = 0;
    for (std::size_t z = 0; z < n; z++) {
        double h, l;
        ref(z, h, l);
        const double d = (C[z] - h) - l;
        const double ds = (d * sc1) * sc2, gs = (h * sc1) * sc2;
        num += ds * ds;
        den += gs * gs;
    }
    Accuracy a;
    if (!std::isfinite(num) || !std::isfinite(den))
        a.rel_fro = std::numeric_limits<double>::infinity();
    else if (den > 0)
        a.rel_fro = std::sqrt(num) / std::sqrt(den);
    else
        a.rel_fro = num > 0 ? std::numeric_limits<double>::infinity() : 0.0;
    a.ebits = std::isfinite(a.rel_fro) ? (a.rel_fro > 0 ? -std::log2(a.rel_fro) : 99.0) : -1.0;
    return a;
}

}  // namespace ozTTgemm::evaluation

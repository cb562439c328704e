// Scheme I host planning; see plan1.hpp. Compiled with -ffp-contract=off: the floating-point
// expressions below must round exactly like the reference's (its Makefile:51-53 sets the same).
#include "plan1.hpp"

#include <algorithm>
#include <climits>
#include <cstring>
#include <cmath>
#include <exception>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "norm.hpp"

namespace ozTTgemm::detail {
namespace {

// Rows and columns of the sampled estimate: the TOP of largest norm and UNI drawn uniformly from the
// rest, with fixed seeds (auto_precision.hpp:56-61).
constexpr std::uint32_t kTop = 32, kUni = 32;
constexpr std::uint32_t kSeedRows = 20261021u, kSeedCols = 20261022u;

std::uint64_t f64_bits(double x) {
    std::uint64_t u;
    std::memcpy(&u, &x, 8);
    return u;
}

// BF16 of |x| from its FP64 words with rounding `ceil` and the exponent e = ceil(log2) the device
// normalizes with (scale_bits.h:34-62). in_range is false for 0 and for the device's markers.
int dev_exp(double mx, std::uint32_t ceil, bool& in_range) {
    const std::uint64_t u = f64_bits(mx);
    const std::uint32_t h = (std::uint32_t)(u >> 32) & 0x7FFFFFFFu, l = (std::uint32_t)u;
    std::uint16_t b;
    const std::int32_t E = (std::int32_t)((h >> 20) & 0x7FFu);
    if (E == 0x7FF)
        b = 0xFFC0u;
    else {
        const std::int32_t e8 = E - 896;
        if (e8 <= 0)
            b = (h | l) ? 0xFF80u : 0u;
        else if (e8 >= 255)
            b = 0x7F80u;
        else {
            std::uint32_t v = ((std::uint32_t)e8 << 7) | ((h >> 13) & 0x7Fu);
            if (ceil == 1 && ((h & 0x1FFFu) || l)) v += 1u;
            if (ceil == 2 && ((h & 0x1FFFu) || l || !(v & 0x7Fu))) v += 1u;
            b = (std::uint16_t)v;
        }
    }
    const std::uint32_t BE = (b >> 7) & 0xFFu, bm = b & 0x7Fu;
    std::uint32_t bad = 0;
    int e;
    if (BE == 0u)
        e = 0;
    else if (BE == 0xFFu) {
        e = 0;
        bad = 1;
    } else
        e = (int)BE - 127 + (bm ? 1 : 0);
    in_range = b != 0 && bad == 0u;
    return e;
}

// Error-free sum of doubles (auto_precision.hpp:88-93).
inline void two_sum(double a, double b, double& s, double& e) {
    s = a + b;
    const double bb = s - a;
    e = (a - (s - bb)) + (b - bb);
}

// Radix expansion of one element by the device slicer's rule, residual in two doubles
// (auto_precision.hpp:82-112): u = beta*t, d = clamp(round(fl32(u)), +-dmax), t = u - d.
struct Digits {
    double th = 0.0, tl = 0.0;
    double step(double beta, double dmax) {
        const double ph = beta * th, pe = std::fma(beta, th, -ph);
        double uh, ul;
        two_sum(ph, pe + beta * tl, uh, ul);
        const double d = std::min(dmax, std::max(-dmax, std::nearbyint((double)(float)uh)));
        two_sum(uh - d, ul, th, tl);
        return d;
    }
    double value() const { return th + tl; }
};

struct Cfg {
    std::uint32_t M, N, K;
    double beta, dmax;
    std::int32_t nshift;
    std::uint32_t ceil;
    int pmax;
};

// Row/column normalization: exponents, scaled divisors 2^(e-nshift)*rg, squared norms
// (auto_precision.hpp:140-206).
struct Norm {
    double rgA = 1.0, rgB = 1.0;
    std::vector<int> eA, eB;
    std::vector<double> sA, sB, nrA, nrB;
};

Norm normalize(const double* A, const double* B, const Cfg& g) {
    const std::uint32_t M = g.M, N = g.N, K = g.K;
    Norm nm;
    nm.rgA = 1.0 / pow2_scale(A, (std::size_t)M * K);
    nm.rgB = 1.0 / pow2_scale(B, (std::size_t)K * N);
    const double rgA = nm.rgA, rgB = nm.rgB;
    nm.eA.assign(M, 0);
    nm.eB.assign(N, 0);
    nm.sA.assign(M, 0.0);
    nm.sB.assign(N, 0.0);
    nm.nrA.assign(M, 0.0);
    nm.nrB.assign(N, 0.0);
#pragma omp parallel for schedule(static)
    for (std::int64_t m = 0; m < (std::int64_t)M; m++) {
        double mx = 0, nr = 0;
        for (std::uint32_t k = 0; k < K; k++) {
            const double v = A[(std::size_t)m * K + k];
            mx = std::max(mx, std::fabs(v));
            nr += (v * rgA) * (v * rgA);
        }
        bool ok = false;
        const int e = dev_exp(mx, g.ceil, ok);
        if (mx > 0 && ok) {
            nm.eA[m] = e;
            nm.sA[m] = std::ldexp(rgA, e - g.nshift);
        }
        nm.nrA[m] = nr;
    }
    constexpr std::uint32_t CB = 64;
    const std::uint32_t nblk = (N + CB - 1) / CB;
#pragma omp parallel for schedule(static)
    for (std::int64_t bk = 0; bk < (std::int64_t)nblk; bk++) {
        const std::uint32_t n0 = (std::uint32_t)bk * CB, n1 = std::min(N, n0 + CB);
        double mx[CB] = {0}, nr[CB] = {0};
        for (std::uint32_t k = 0; k < K; k++)
            for (std::uint32_t n = n0; n < n1; n++) {
                const double v = B[(std::size_t)k * N + n];
                mx[n - n0] = std::max(mx[n - n0], std::fabs(v));
                nr[n - n0] += (v * rgB) * (v * rgB);
            }
        for (std::uint32_t n = n0; n < n1; n++) {
            bool ok = false;
            const int e = dev_exp(mx[n - n0], g.ceil, ok);
            if (mx[n - n0] > 0 && ok) {
                nm.eB[n] = e;
                nm.sB[n] = std::ldexp(rgB, e - g.nshift);
            }
            nm.nrB[n] = nr[n - n0];
        }
    }
    return nm;
}

// Estimate (1), independent signs: e2r[q] = expected ||E||_F^2 with q slices (auto_precision.hpp:210-267).
std::vector<double> indep(const double* A, const double* B, const Cfg& g, const Norm& nm) {
    const std::uint32_t M = g.M, N = g.N, K = g.K;
    const int pmax = g.pmax;
    const std::size_t P1 = (std::size_t)pmax + 1;
    const double beta = g.beta, dmax = g.dmax, rgA = nm.rgA, rgB = nm.rgB;
    std::vector<double> SA(P1 * K, 0.0), RA(P1 * K, 0.0), SB(P1 * K, 0.0), RB(P1 * K, 0.0), NA(K, 0.0), NB(K, 0.0);
    auto cut = [&](double x, double s, double* S, double* R) {
        Digits t;
        t.th = x;
        double w = 1.0;
        for (int i = 0; i < pmax; i++) {
            const double d = t.step(beta, dmax);
            w /= beta;
            S[(std::size_t)i * K] += (s * d * w) * (s * d * w);
            const double r = s * t.value() * w;
            R[(std::size_t)(i + 1) * K] += r * r;
            if (t.th == 0) break;
        }
    };
#pragma omp parallel for schedule(static)
    for (std::int64_t k = 0; k < (std::int64_t)K; k++) {
        double na = 0, nb = 0;
        for (std::uint32_t m = 0; m < M; m++) {
            const double v = A[(std::size_t)m * K + k];
            na += (v * rgA) * (v * rgA);
            if (v != 0 && nm.sA[m] > 0) cut(std::ldexp(v, g.nshift - nm.eA[m]), nm.sA[m], &SA[k], &RA[k]);
        }
        for (std::uint32_t n = 0; n < N; n++) {
            const double v = B[(std::size_t)k * N + n];
            nb += (v * rgB) * (v * rgB);
            if (v != 0 && nm.sB[n] > 0) cut(std::ldexp(v, g.nshift - nm.eB[n]), nm.sB[n], &SB[k], &RB[k]);
        }
        NA[k] = na;
        NB[k] = nb;
    }
    std::vector<double> G((std::size_t)pmax * pmax, 0.0);
#pragma omp parallel for schedule(dynamic)
    for (int i = 0; i < pmax; i++)
        for (int j = 0; j < pmax; j++) {
            double gij = 0;
            for (std::uint32_t k = 0; k < K; k++) gij += SA[(std::size_t)i * K + k] * SB[(std::size_t)j * K + k];
            G[(std::size_t)i * pmax + j] = gij;
        }
    std::vector<double> e2r(P1, 0.0);
    for (int q = 2; q <= pmax; q++) {
        double e2 = 0;
        for (int i = 0; i < q; i++)
            for (int j = std::max(0, q - i); j < q; j++) e2 += G[(std::size_t)i * pmax + j];
        for (std::uint32_t k = 0; k < K; k++) e2 += RA[(std::size_t)q * K + k] * NB[k] + NA[k] * RB[(std::size_t)q * K + k];
        e2r[q] = e2;
    }
    return e2r;
}

// Estimate (2): simulation of the device result on sampled rows and columns (auto_precision.hpp:272-447).
struct Sampled {
    const Cfg* g = nullptr;
    const Norm* nm = nullptr;
    std::vector<std::uint32_t> iA, iB;
    std::vector<double> wA, wB;
    std::size_t na = 0, nb = 0;
    std::vector<double> XA, YB, Ch, Cl;
    double nC2 = 0.0;

    double e2(int q) const {
        if (na == 0 || nb == 0) return 0.0;
        const std::uint32_t K = g->K;
        const double beta = g->beta, dmax = g->dmax;
        constexpr std::uint32_t NCH = 64;
        std::vector<double> part((std::size_t)NCH * na * nb, 0.0);
        std::exception_ptr failure;
#pragma omp parallel for schedule(dynamic)
        for (std::int64_t c = 0; c < (std::int64_t)NCH; c++) {
            try {
                const std::uint32_t k0 = (std::uint32_t)((std::uint64_t)K * c / NCH),
                                    k1 = (std::uint32_t)((std::uint64_t)K * (c + 1) / NCH);
                std::vector<double> D(na * q), RX(na), RY(nb * (q + 1)), Y(nb);
                double* acc = &part[(std::size_t)c * na * nb];
                for (std::uint32_t k = k0; k < k1; k++) {
                    for (std::size_t a = 0; a < na; a++) {
                        Digits t;
                        t.th = XA[a * K + k];
                        double w = 1.0;
                        for (int i = 0; i < q; i++) {
                            const double d = t.step(beta, dmax);
                            w /= beta;
                            D[a * q + i] = d * w;
                        }
                        RX[a] = t.value() * w;
                    }
                    for (std::size_t b = 0; b < nb; b++) {
                        Digits t;
                        t.th = Y[b] = YB[b * K + k];
                        double w = 1.0;
                        for (int c2 = 1; c2 <= q; c2++) {
                            (void)t.step(beta, dmax);
                            w /= beta;
                            RY[b * (q + 1) + c2] = t.value() * w;
                        }
                    }
                    for (std::size_t a = 0; a < na; a++)
                        for (std::size_t b = 0; b < nb; b++) {
                            double e = RX[a] * Y[b];
                            for (int i = 0; i < q; i++) e += D[a * q + i] * RY[b * (q + 1) + (q - i)];
                            acc[a * nb + b] += e;
                        }
                }
            } catch (...) {
#pragma omp critical(oz1_sampled_e2)
                if (!failure) failure = std::current_exception();
            }
        }
        if (failure) std::rethrow_exception(failure);
        double e2 = 0;
        for (std::size_t a = 0; a < na; a++)
            for (std::size_t b = 0; b < nb; b++) {
                double E = 0;
                for (std::uint32_t c = 0; c < NCH; c++) E += part[((std::size_t)c * na + a) * nb + b];
                // the device's C - E rounded to FP64; within 2^-59 of a midpoint the far side is taken
                const std::size_t ab = a * nb + b;
                double h, r;
                two_sum(Ch[ab], Cl[ab] - nm->sA[iA[a]] * nm->sB[iB[b]] * E, h, r);
                double out = h;
                if (h != 0) {
                    const double h2 = std::nextafter(h, r >= 0 ? INFINITY : -INFINITY);
                    const double gap = 0.5 * std::fabs(h2 - h) - std::fabs(r);
                    if (gap <= std::ldexp(1.0, std::ilogb(h) - 59)) {
                        const double d1 = (h - Ch[ab]) - Cl[ab], d2 = (h2 - Ch[ab]) - Cl[ab];
                        if (std::fabs(d2) > std::fabs(d1)) out = h2;
                    }
                }
                const double dv = (out - Ch[ab]) - Cl[ab];
                e2 += wA[a] * wB[b] * dv * dv;
            }
        return nC2 > 0 ? e2 / nC2 : (e2 > 0 ? INFINITY : 0.0);
    }
};

Sampled sample(const double* A, const double* B, const Cfg& g, const Norm& nm, double nC) {
    const std::uint32_t M = g.M, N = g.N, K = g.K;
    Sampled sm;
    sm.g = &g;
    sm.nm = &nm;
    auto pick = [&](const std::vector<double>& nr, const std::vector<double>& s, std::uint32_t L, std::uint32_t seed,
                    std::vector<std::uint32_t>& idx, std::vector<double>& wt) {
        std::vector<std::uint32_t> ord;
        for (std::uint32_t i = 0; i < L; i++)
            if (s[i] > 0) ord.push_back(i);
        const std::size_t nt = std::min<std::size_t>(kTop, ord.size());
        std::partial_sort(ord.begin(), ord.begin() + nt, ord.end(), [&](std::uint32_t a, std::uint32_t b) {
            return nr[a] > nr[b] || (nr[a] == nr[b] && a < b);
        });
        for (std::size_t i = 0; i < nt; i++) {
            idx.push_back(ord[i]);
            wt.push_back(1.0);
        }
        std::vector<std::uint32_t> rest(ord.begin() + nt, ord.end());
        const std::size_t nu = std::min<std::size_t>(kUni, rest.size());
        std::mt19937 rg(seed);
        for (std::size_t i = 0; i < nu; i++) {
            std::swap(rest[i], rest[i + rg() % (rest.size() - i)]);
            idx.push_back(rest[i]);
            wt.push_back((double)rest.size() / (double)nu);
        }
    };
    pick(nm.nrA, nm.sA, M, kSeedRows, sm.iA, sm.wA);
    pick(nm.nrB, nm.sB, N, kSeedCols, sm.iB, sm.wB);
    const std::size_t na = sm.iA.size(), nb = sm.iB.size();
    sm.na = na;
    sm.nb = nb;
    sm.XA.assign(na * K, 0.0);
    sm.YB.assign(nb * K, 0.0);
    for (std::size_t a = 0; a < na; a++)
        for (std::uint32_t k = 0; k < K; k++)
            sm.XA[a * K + k] = std::ldexp(A[(std::size_t)sm.iA[a] * K + k], g.nshift - nm.eA[sm.iA[a]]);
    for (std::size_t b = 0; b < nb; b++)
        for (std::uint32_t k = 0; k < K; k++)
            sm.YB[b * K + k] = std::ldexp(B[(std::size_t)k * N + sm.iB[b]], g.nshift - nm.eB[sm.iB[b]]);
    sm.Ch.assign(na * nb, 0.0);
    sm.Cl.assign(na * nb, 0.0);
    const double rgA = nm.rgA, rgB = nm.rgB;
#pragma omp parallel for schedule(dynamic)
    for (std::int64_t ab = 0; ab < (std::int64_t)(na * nb); ab++) {
        const std::size_t a = (std::size_t)ab / nb, b = (std::size_t)ab % nb;
        double sh = 0, sl = 0;
        for (std::uint32_t k = 0; k < K; k++) {
            const double u = A[(std::size_t)sm.iA[a] * K + k] * rgA, v = B[(std::size_t)k * N + sm.iB[b]] * rgB;
            const double pr = u * v, pe = std::fma(u, v, -pr);
            double t, te;
            two_sum(sh, pr, t, te);
            sh = t;
            sl += pe + te;
        }
        two_sum(sh, sl, sm.Ch[ab], sm.Cl[ab]);
    }
    double nCs = 0;
    for (std::size_t a = 0; a < na; a++)
        for (std::size_t b = 0; b < nb; b++) nCs += sm.wA[a] * sm.wB[b] * sm.Ch[a * nb + b] * sm.Ch[a * nb + b];
    sm.nC2 = std::max(nC, nCs);
    return sm;
}

// The smallest q at which (1) meets the target, then doubling and bisection on max((1), (2))
// (auto_precision.hpp:455-500).
int search(const std::vector<double>& r1, std::vector<double>& e2sv, const Sampled& sm, int pmax, double tgt) {
    auto f2 = [&](int q) {
        if (e2sv[q] < 0) e2sv[q] = sm.e2(q);
        return std::max(r1[q], e2sv[q]);
    };
    int q0 = pmax;
    for (int q = 2; q <= pmax; q++)
        if (r1[q] <= tgt) {
            q0 = q;
            break;
        }
    int p = q0;
    if (f2(q0) > tgt) {
        int lo = q0, hi = -1;
        for (int step = 1; lo < pmax; step *= 2) {
            const int q = std::min(pmax, lo + step);
            if (f2(q) <= tgt) {
                hi = q;
                break;
            }
            lo = q;
        }
        if (hi < 0)
            p = pmax;
        else {
            while (hi - lo > 1) {
                const int mid = (lo + hi) / 2;
                if (f2(mid) <= tgt)
                    hi = mid;
                else
                    lo = mid;
            }
            p = hi;
        }
    }
    return p;
}

// bits of dmax^2 rounded up (format.hpp:107-112)
std::uint32_t prod_bits(std::uint32_t dmax) {
    const std::uint64_t r2 = (std::uint64_t)dmax * dmax;
    std::uint32_t b = 0;
    while ((1ull << b) < r2) ++b;
    return b;
}

// (L+1) K digit products summed in int32 cannot overflow (format.hpp:176-183)
bool defer_fits(std::uint32_t K, int L, const Oz1Format& f) {
    const std::uint64_t k_eff = (std::uint64_t)(L + 1) * K;
    const std::uint64_t dsq = (std::uint64_t)f.dmax * f.dmax;
    return dsq != 0 && k_eff <= (std::uint64_t)INT32_MAX / dsq;
}

// the FP32 exponent budget of the Horner evaluation (format.hpp:160-171)
bool horner_fits(std::uint32_t K, int L, const Oz1Format& f) {
    const double v = std::log2((double)K) + (double)(L + 1) * std::log2((double)f.radix);
    return v + 12.0 < 128.0;
}

bool exact_check(std::uint32_t K, int L, const Oz1Format& f) {
    const std::uint64_t k_eff = (std::uint64_t)(L + 1) * K;
    std::uint32_t bits = 0;
    while ((1ull << bits) < k_eff) ++bits;
    if (f.acc_bits < bits) return false;
    const std::uint64_t budget = 1ull << (f.acc_bits - bits);
    const std::uint64_t d2 = (std::uint64_t)f.dmax * f.dmax;
    if (d2 > budget) return false;
    return !f.int32_partial || d2 * k_eff <= (std::uint64_t)INT32_MAX;
}

}  // namespace

const Oz1Format& oz1_format(int format) {
    switch (format) {
    case 0: case 1: case 2: case 3: return kOz1Bf16;  // BF16, FP16, TF32, BFP8
    case 4: return kOz1Fp8;
    case 5: return kOz1Int8;
    case 6: return kOz1Bfp4;
    case 7: return kOz1Bfp2;
    default: throw std::invalid_argument("unknown format");
    }
}

std::uint32_t oz1_block_k(std::uint32_t K, int L, const Oz1Format& f) {
    const std::uint32_t pb = prod_bits((std::uint32_t)f.dmax);
    if (f.acc_bits < pb + 1) return 0;
    std::uint64_t keff_max = 1ull << (f.acc_bits - pb);
    if (f.int32_partial) {
        const std::uint64_t d = (std::uint64_t)f.dmax;
        keff_max = std::min<std::uint64_t>(keff_max, (std::uint64_t)INT32_MAX / (d * d));
    }
    const std::uint64_t kc_max = keff_max / (std::uint64_t)(L + 1);
    if (kc_max >= (std::uint64_t)K) return K;
    std::uint32_t best = 0;
    for (std::uint32_t c = 32; c <= kc_max; c += 32)
        if (K % c == 0) best = c;
    return best;
}

int oz1_auto_p(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
               const Oz1Format& f, Oz1AutoInfo* info) {
    Cfg g{M, N, K, (double)f.radix, (double)f.dmax, f.nshift, f.ceil, 0};
    g.pmax = (int)std::ceil(160.0 / std::log2(g.beta)) + 1;
    const int pmax = g.pmax;
    const std::size_t P1 = (std::size_t)pmax + 1;
    const Norm nm = normalize(A, B, g);
    const std::vector<double> e2r = indep(A, B, g, nm);
    const double nC = estimate_product_norm(A, B, M, N, K, nm.rgA, nm.rgB);
    const Sampled sm = sample(A, B, g, nm, nC);
    const double tgt = std::ldexp(1.0, -106);
    std::vector<double> r1(P1, INFINITY), e2sv(P1, -1.0);
    for (int q = 2; q <= pmax; q++) r1[q] = nC > 0 ? e2r[q] / nC : (e2r[q] > 0 ? INFINITY : 0.0);
    const int p = search(r1, e2sv, sm, pmax, tgt);
    if (info) {
        info->pmax = pmax;
        info->bits_indep = -0.5 * std::log2(r1[p]);
        if (e2sv[p] < 0) e2sv[p] = sm.e2(p);
        info->bits_sampled = -0.5 * std::log2(e2sv[p]);
    }
    return p;
}

Plan1 plan_scheme1(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K,
                   std::uint32_t slices, const Oz1Format& f) {
    Plan1 pl;
    pl.M = M;
    pl.N = N;
    pl.K = K;
    pl.f = f;
    pl.p = slices ? (int)slices : oz1_auto_p(A, B, M, N, K, f, &pl.autop);
    const int L = pl.p - 1;
    const std::uint32_t ndiag = (std::uint32_t)pl.p;
    // issue candidates and choice (plan.hpp:130-175)
    const std::uint32_t kc_cat = oz1_block_k(K, L, f), kc_pw = oz1_block_k(K, 0, f);
    const std::uint32_t nkb_cat = kc_cat ? K / kc_cat : 0u, nkb_pw = kc_pw ? K / kc_pw : 0u;
    const std::uint64_t n_cat = kc_cat ? (std::uint64_t)ndiag * nkb_cat : UINT32_MAX;
    const std::uint64_t n_pw = kc_pw ? (std::uint64_t)ndiag * (ndiag + 1) / 2 * nkb_pw : 0u;
    const bool defer_ok = defer_fits(K, L, f);
    const bool fuse_ok = !f.int32_partial && defer_ok;
    IssuePlan1& ip = pl.issue;
    ip.pairloop = fuse_ok && kc_pw && nkb_pw == 1u;
    ip.pairwise = !ip.pairloop && fuse_ok && kc_pw && n_pw < n_cat;
    const bool per_pair = ip.pairwise || ip.pairloop;
    ip.Kc = per_pair ? kc_pw : kc_cat;
    ip.nkb = ip.Kc ? K / ip.Kc : 0u;
    ip.fuse = !ip.pairloop && fuse_ok && (ip.pairwise || ip.nkb > 1);
    ip.defer = ip.pairloop || ip.fuse;
    // feasibility (plan.hpp:177-206)
    if (ip.Kc == 0)
        throw std::runtime_error("Ozaki scheme I: the partial products for k=" + std::to_string(K) + " with " +
                                 std::to_string(pl.p) +
                                 " slices cannot be accumulated without error in this format (no K block length "
                                 "satisfies the exactness condition). Use fewer slices (Options::slices) or a smaller k.");
    if (f.int32_partial && ip.nkb > 1)
        throw std::runtime_error("Ozaki scheme I with Format::INT8 does not support K blocking, but k=" +
                                 std::to_string(K) + " with " + std::to_string(pl.p) + " slices needs " +
                                 std::to_string(ip.nkb) + " K blocks of " + std::to_string(ip.Kc) +
                                 " columns. Use a smaller k, fewer slices (Options::slices) or another format.");
    if (!horner_fits(K, L, f))
        throw std::runtime_error("Ozaki scheme I: the reconstruction would overflow FP32 for k=" + std::to_string(K) +
                                 " with " + std::to_string(pl.p) + " slices (radix " + std::to_string(f.radix) +
                                 "): log2(k) + slices*log2(radix) + 12 must be below 128. Use fewer slices "
                                 "(Options::slices) or a smaller k.");
    if (!exact_check(ip.Kc, per_pair ? 0 : L, f)) throw std::logic_error("scheme I plan: K block violates exactness");
    // The products run as exact int8 x int8 -> int32 accumulations over all pairs and K of a diagonal.
    // That reproduces the reference's int32 sums S_d (deferred reconstruction) and its single-block INT8
    // products. The remaining plan (FP32 products whose sum over all of K could overflow int32:
    // !defer, several K blocks of the concatenated issue) reconstructs K block by K block
    // (plan.hpp:104-109): the driver sums each block's diagonals exactly and carries the Horner limbs.
    pl.signmag = f.int32_partial;
    // reconstruction constants (plan.hpp:424-460)
    if (ip.defer) {
        const std::uint64_t per = (std::uint64_t)K * f.dmax * f.dmax;
        pl.nsmall = per ? (int)std::min<std::uint64_t>((1ull << 24) / per, ndiag) : 0;
    }
    long double w = 1.0L;
    for (int i = 0; i < L + 2; i++) w /= (long double)f.radix;
    int e;
    const long double fr = frexpl(w, &e);
    const unsigned long long W = (unsigned long long)ldexpl(fr, 64);
    pl.Whi = (std::uint32_t)(W >> 32);
    pl.Wlo = (std::uint32_t)W;
    pl.qw = e - 64;
    return pl;
}

}  // namespace ozTTgemm::detail

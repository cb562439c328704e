// Scheme II host planning; see plan2.hpp. Compiled with -ffp-contract=off: the floating-point
// expressions below must round exactly like the reference's (its Makefile:51-53 sets the same).
#include "plan2.hpp"

#include "norm.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>
#include <random>
#include <stdexcept>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace ozTTgemm::detail {
namespace {

// Candidate moduli of the INT8 path: pairwise coprime, descending (moduli.hpp:180-181).
constexpr int kTableInt8[] = {255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217,
                              211, 199, 197, 193, 191, 181, 179, 173, 167, 163, 157, 151};
constexpr int kTableInt8Min = 151;
constexpr int kInt8ModCap = 255;     // OZ2_ROUTE_INT8.mod_cap (split.hpp:73)
constexpr double kWinEps = 1e-9;     // strict window comparison (moduli.hpp:48)
constexpr double kTailTol = 0.25;    // OZ2_TAIL_EXCESS_TOL (moduli.hpp:54)
constexpr double kRecon1EpsLog2 = -70.0, kRecon1Margin = 2.0;  // auto_precision.hpp:126-127

// Largest |r| with K*r^2 <= 2^acc_bits - 1 (moduli.hpp:224-231).
long int8_rmax(std::uint32_t K) {
    const unsigned __int128 lim = ((unsigned __int128)1 << kAccBits) - 1;
    long r = (long)std::floor(std::sqrt((double)lim / (double)K));
    while (r > 0 && (unsigned __int128)K * r * r > lim) --r;
    while ((unsigned __int128)K * (r + 1) * (r + 1) <= lim) ++r;
    return r;
}

bool int8_fits(std::uint32_t K, int m) {
    const unsigned __int128 r = (unsigned)(m / 2);
    return (unsigned __int128)K * r * r <= (((unsigned __int128)1 << kAccBits) - 1);
}

bool coprime_to_all(int v, const std::vector<int>& set) {
    for (int x : set)
        if (std::gcd(x, v) != 1) return false;
    return true;
}

// Replace the last two moduli by one modulus or a coprime pair that covers the window with the
// least excess (moduli.hpp:365-451); for INT8 every modulus is one product, so the preference is
// (fewer moduli, excess within tolerance, smaller product).
void reselect_tail(std::vector<int>& m, double& logM, double need, int m_cap) {
    if (!(m.size() >= 2 && logM > need)) return;
    const std::vector<int> head(m.begin(), m.end() - 2);
    double base = 0.0;
    for (int x : head) base += std::log2((double)x);
    double best = logM;
    int bp = m[m.size() - 2], bq = m.back(), bcost = 2;
    auto over = [&](double l) { return (l - need) > kTailTol ? 1 : 0; };
    auto better = [&](int c, double l) {
        if (c != bcost) return c < bcost;
        if (over(l) != over(best)) return over(l) < over(best);
        return l < best;
    };
    bool head_even = false;
    for (int x : head) head_even = head_even || (x % 2 == 0);
    const int step = head_even ? 2 : 1;
    for (int p = 3; p <= m_cap; p += step) {
        if (!coprime_to_all(p, head)) continue;
        const double lp = base + std::log2((double)p);
        if (lp >= need && better(1, lp)) {
            best = lp;
            bp = p;
            bq = 0;
            bcost = 1;
        }
        for (int q = p + step; q <= m_cap; q += step) {
            if (std::gcd(p, q) != 1 || !coprime_to_all(q, head)) continue;
            const double lq = lp + std::log2((double)q);
            if (lq >= need && better(2, lq)) {
                best = lq;
                bp = p;
                bq = q;
                bcost = 2;
            }
        }
    }
    m = head;
    m.push_back(bp);
    if (bq) m.push_back(bq);
    logM = best;
}

// Upper bound on ||x||_2 / 2^ceil(log2 max|x_k|) for one row or column of n values x (each scaled by
// the same power of two), from their maximum magnitude mx and the sum of squares s2 that
// measure_stats computes. Recursive summation of n rounded squares errs by at most n 2^-53 of the
// sum, and squares below 2^-1022 lose at most 2^-1074 each; the factors below cover both and the
// bound's own rounding. A maximum below 2^-400 (where the lost squares could matter), or a sum that
// is not finite, gives sqrt(n), which holds for any such vector since every |x_k| <= 2^ceil(log2 mx).
double flatness_bound(double mx, double s2, std::uint32_t n) {
    if (!(mx > 0)) return 0.0;
    const double worst = std::sqrt((double)n) * (1.0 + 0x1p-50);
    if (!(mx >= 0x1p-400) || !std::isfinite(s2)) return worst;
    int e;
    const double f = std::frexp(mx, &e);  // mx = f 2^e, 1/2 <= f < 1
    const int te = f == 0.5 ? e - 1 : e;  // 2^te: the least power of two >= mx
    const double s = s2 * (1.0 + (double)n * 0x1p-51) + (double)n * 0x1p-1022;
    return std::min(std::ldexp(std::sqrt(s), -te) * (1.0 + 0x1p-50), worst);
}

}  // namespace

OperandStats measure_stats(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K) {
    OperandStats st;
    const double rgA = 1.0 / pow2_scale(A, (std::size_t)M * K), rgB = 1.0 / pow2_scale(B, (std::size_t)K * N);
    // Row statistics of A and column statistics of B (auto_precision.hpp:24-56). Per-row and per-column
    // values are computed in parallel with the reference's inner order; the sums over rows/columns
    // run sequentially in the reference's order.
    std::vector<double> tA(M), sA(M), tB(N), sB(N), wA(M, 0.0), wB(N, 0.0), rA(M), rB(N);
#pragma omp parallel for schedule(static)
    for (std::int64_t r = 0; r < (std::int64_t)M; r++) {
        double mx = 0, s2 = 0;
        for (std::uint32_t c = 0; c < K; c++) {
            const double v = A[(std::size_t)r * K + c] * rgA;
            mx = std::max(mx, std::fabs(v));
            s2 += v * v;
        }
        double t2 = 0;
        if (mx > 0) {
            const double t = std::exp2(std::ceil(std::log2(mx)));
            t2 = t * t;
            wA[r] = std::sqrt(s2) / t;
        }
        tA[r] = t2;
        sA[r] = s2;
        rA[r] = flatness_bound(mx, s2, K);
    }
    constexpr std::uint32_t CB = 64;  // column block: row-major sweep, per-column order kept
#pragma omp parallel for schedule(static)
    for (std::int64_t cb = 0; cb < (std::int64_t)((N + CB - 1) / CB); cb++) {
        const std::uint32_t c0 = (std::uint32_t)cb * CB, c1 = std::min<std::uint32_t>(N, c0 + CB);
        double mx[CB] = {}, s2[CB] = {};
        for (std::uint32_t r = 0; r < K; r++)
            for (std::uint32_t c = c0; c < c1; c++) {
                const double v = B[(std::size_t)r * N + c] * rgB;
                mx[c - c0] = std::max(mx[c - c0], std::fabs(v));
                s2[c - c0] += v * v;
            }
        for (std::uint32_t c = c0; c < c1; c++) {
            double t2 = 0;
            if (mx[c - c0] > 0) {
                const double t = std::exp2(std::ceil(std::log2(mx[c - c0])));
                t2 = t * t;
                wB[c] = std::sqrt(s2[c - c0]) / t;
            }
            tB[c] = t2;
            sB[c] = s2[c - c0];
            rB[c] = flatness_bound(mx[c - c0], s2[c - c0], K);
        }
    }
    for (std::uint32_t r = 0; r < M; r++) {
        st.TA += tA[r];
        st.nA += sA[r];
        st.wA = std::max(st.wA, wA[r]);
        st.rA = std::max(st.rA, rA[r]);
    }
    for (std::uint32_t c = 0; c < N; c++) {
        st.TB += tB[c];
        st.nB += sB[c];
        st.wB = std::max(st.wB, wB[c]);
        st.rB = std::max(st.rB, rB[c]);
    }
    st.nC = estimate_product_norm(A, B, M, N, K, rgA, rgB);
    st.measured = true;
    return st;
}

int precision_cap(const OperandStats& st) {
    const double k2 = std::min(std::sqrt((st.TA * st.nB + st.TB * st.nA) / std::max(12.0 * st.nC, 1e-300)), 1e18);
    return std::min(kMaxDigits * kDigitBits, kTargetBits + (int)std::ceil(std::log2(std::max(k2, 1.0))));
}

ModuliSet choose_moduli_int8(std::uint32_t K, int num_moduli, int b_cap, double window_log2) {
    ModuliSet o;
    const double W = std::isnan(window_log2) ? std::log2((double)K) : window_log2;
    const int m_cap = (int)std::min<long>(kInt8ModCap, 2 * int8_rmax(K) + 1);
    double logM = 0.0;
    for (int mm : kTableInt8) {
        if ((int)o.m.size() >= num_moduli) break;
        if (mm > m_cap) continue;
        o.m.push_back(mm);
        logM += std::log2((double)mm);
    }
    // extension below the table when K lowers the cap (moduli.hpp:310-327)
    const int want = std::min(num_moduli, kMaxModuli);
    for (int mm = std::min(m_cap, kTableInt8Min - 1); mm >= 3 && (int)o.m.size() < want; --mm) {
        if (!coprime_to_all(mm, o.m)) continue;
        o.m.push_back(mm);
        logM += std::log2((double)mm);
    }
    o.m_cap = m_cap;
    o.ncand = (int)o.m.size();
    // width from the window |C'| <= K 2^(2b) < M/2 (moduli.hpp:338-344)
    const double room = logM - 1.0 - W - kWinEps;
    o.b = std::min(std::min((int)std::floor(room / 2.0), kMaxDigits * kDigitBits), b_cap);
    const double need = 2.0 * o.b + 1.0 + W + kWinEps;
    // drop surplus moduli from the end (moduli.hpp:347-355), then reselect the last two
    while (o.m.size() > 2) {
        const double l2 = std::log2((double)o.m.back());
        if (logM - l2 < need) break;
        o.m.pop_back();
        logM -= l2;
    }
    reselect_tail(o.m, logM, need, m_cap);
    o.log2M = logM;
    const int s = (int)o.m.size();
    o.ok = (logM >= need) && s > 0 && s <= kMaxModuli && s <= num_moduli && o.b > 0;
    for (int i = 0; i < s; ++i)
        for (int j = i + 1; j < s; ++j)
            if (std::gcd(o.m[i], o.m[j]) != 1) o.ok = false;
    for (int mm : o.m)
        if (!int8_fits(K, mm)) {
            if (o.acc_fail.empty())
                o.acc_fail = "the product bound K*floor(m/2)^2 of modulus " + std::to_string(mm) +
                             " exceeds the exact int32 range 2^31-1";
            o.ok = o.acc_ok = false;
        }
    return o;
}

double recon1_log2(const ModuliSet& mo, int b, const OperandStats& st) {
    if (!(st.nC > 0) || !(st.TA > 0) || !(st.TB > 0)) return -INFINITY;
    double l2m = 0;
    for (int m : mo.m) l2m += std::log2((double)m);
    return kRecon1EpsLog2 + l2m - 2.0 * b + 0.5 * (std::log2(st.TA) + std::log2(st.TB) - std::log2(st.nC));
}

Plan2 plan_scheme2(const double* A, const double* B, std::uint32_t M, std::uint32_t N, std::uint32_t K, Format format,
                   std::uint32_t max_moduli, Reconstruction passes, std::optional<unsigned> fixed_b,
                   bool int8_transport, bool operand_window) {
    // Every format plans on its own route as the reference does (INT8 residues, or the FP8, TF32, BF16,
    // FP16, BFP8, BFP4 or BFP2 digit route): its moduli, width b and pass choice are the reference's.
    // INT8 and FP8 then compute on their own matrix instructions (FP8: the route's e4m3 digits) unless
    // the caller asks for INT8 residues; the other six formats run INT8 residues of the same A' and B'
    // at that width b: on MI355X their digits are int8 values anyway (BFP8, BFP4, BFP2 and TF32 have no
    // matrix instructions of their own; BF16/FP16 run at half the INT8 rate), and the digit routes need
    // two to four digit products per modulus where INT8 needs one per modulus of a set a few moduli
    // larger. The exact reconstruction makes C a function of the width b alone, so the output is the
    // same whichever set computes it.
    if ((int)format < 0 || (int)format > (int)Format::BFP2) throw std::invalid_argument("unknown format");
    const bool int8 = format == Format::INT8, fp8 = format == Format::FP8;
    Plan2 p;
    p.M = M;
    p.N = N;
    p.K = K;
    p.format = format;
    int b_cap = kDefaultBits;
    const bool b_fixed = fixed_b.has_value();
    if (b_fixed)
        b_cap = (int)*fixed_b;
    else {
        p.stats = measure_stats(A, B, M, N, K);
        b_cap = precision_cap(p.stats);
    }
    // limit on the number of moduli (plan.hpp:281): the caller's, else the route's default with a fixed
    // width (16 for INT8, 14 for FP8, 11 for TF32, 24 otherwise; split.hpp:73-98), else 24
    p.S_req = max_moduli ? max_moduli : (b_fixed ? default_moduli(format) : (std::uint32_t)kMaxModuli);
    if (b_fixed && passes == Reconstruction::Automatic) p.stats = measure_stats(A, B, M, N, K);
    p.route = int8 ? choose_moduli_int8(K, (int)p.S_req, b_cap)
                   : choose_moduli_digits(format, M, N, K, (int)p.S_req, b_cap);
    const ModuliSet& r = p.route;
    if (!r.ok) {
        if (!r.acc_ok)
            throw std::runtime_error("Ozaki II: the padded inner dimension K=" + std::to_string(K) +
                                     " is too large for this format: " + r.acc_fail +
                                     ". Use a smaller K or a different format; Options::max_moduli does not change "
                                     "this limit.");
        std::string cause;
        if ((std::uint32_t)r.ncand < std::min<std::uint32_t>(p.S_req, kMaxModuli))
            cause = "Every candidate modulus is in use, so a larger Options::max_moduli does not help.";
        else if (p.S_req < (std::uint32_t)kMaxModuli)
            cause = "The limit of " + std::to_string(p.S_req) + " moduli is too small; raise Options::max_moduli.";
        else
            cause = "The maximum of 24 moduli is not enough; use a smaller K or a different format.";
        throw std::runtime_error("Ozaki II: the available moduli do not cover the CRT window for the padded inner "
                                 "dimension K=" +
                                 std::to_string(K) + ". " + cause);
    }
    if (!b_fixed && r.b < kTargetBits)
        throw std::runtime_error("Ozaki II: for the padded inner dimension K=" + std::to_string(K) + " the " +
                                 std::to_string(r.m.size()) + " selected moduli cover a width of only " +
                                 std::to_string(r.b) + " bits, below the 53 bits of FP64-equivalent accuracy; "
                                 "raise Options::max_moduli or use a smaller K.");
    p.b = r.b;
    p.mo = r;
    p.fp8_digits = fp8;
    if (!int8 && (!fp8 || int8_transport)) {
        // INT8 residues of the same A' and B' (the shift b - 20 (nd - 1) is the same): a set of up to
        // 24 moduli whose window holds width b
        ModuliSet x = choose_moduli_int8(K, kMaxModuli, p.b);
        if (x.ok && x.b == p.b) {
            p.mo = std::move(x);
            p.fp8_digits = false;
        } else if (!fp8) {
            // a width beyond what 24 INT8 moduli hold (about 85 bits), which only extreme inputs or a
            // fixed width ask for: the FP8 route's e4m3 digits carry the same width b (moduli up to
            // 2401, two or three digits each, at most 100 bits), so C is still the one of the format's
            // own plan; a width that neither transport holds is refused, never lowered
            ModuliSet f = choose_moduli_digits(Format::FP8, M, N, K, kMaxModuli, p.b);
            if (!(f.ok && f.b == p.b))
                throw std::runtime_error("Ozaki II: the " + std::string(format_name(format)) + " plan needs a width of " +
                                         std::to_string(p.b) + " bits at the padded inner dimension K=" +
                                         std::to_string(K) + ", beyond what this device's INT8 residues (" +
                                         std::to_string(x.ok ? x.b : 0) + " bits) and FP8 digits (" +
                                         std::to_string(f.ok ? f.b : 0) + " bits) carry exactly. Use a smaller "
                                         "Options::max_moduli or a smaller K.");
            p.mo = std::move(f);
            p.fp8_digits = true;
        }
    }
    // The CRT window from the operands themselves. The reference sizes M for the worst case
    // |C'_ij| <= K 2^(2b). With |A'_ik| <= 2^b |a_ik| / 2^ceil(log2 max_k |a_ik|) + 2 (the row's own
    // power of two is at most the one its delta was taken from; the digits round by less than 2) and
    // the same for the columns of B, Cauchy-Schwarz gives |C'_ij| <= ||A'_i||_2 ||B'_j||_2
    // <= (2^b rA + 2 sqrt K)(2^b rB + 2 sqrt K), where rA, rB <= sqrt K, and far below it unless rows
    // or columns are flat. Any set of moduli whose product exceeds twice that recovers the same exact
    // C', so when a smaller set covers it, that set computes (C is bit for bit the same): fewer INT8
    // moduli, or on the FP8 route a set of fewer digit products. On the FP8 route the set with the
    // fewest digit products for the window is searched for too (choose_moduli_fp8_fewest: it also
    // takes moduli of at most 33, whose residues are e4m3 digits themselves, one product each, which
    // the reference's FP8 route leaves out). Operands that were not measured (a fixed width and pass
    // count: the evaluator's table) keep the planned set, as the reference computes it.
    const double logK = std::log2((double)K);
    double w = logK;
    if (p.stats.measured) {
        const double sk = std::ldexp(2.0 * std::sqrt((double)K) * (1.0 + 0x1p-50), -p.b);
        const double wb = std::log2(p.stats.rA + sk) + std::log2(p.stats.rB + sk) + 1e-12;
        p.bound_log2 = 2.0 * p.b + wb;
        w = std::min(wb, logK);
    }
    if (operand_window && p.stats.measured) {
        auto take = [&](ModuliSet&& t, bool fewer) {
            if (t.ok && t.b == p.b && fewer) {
                if (!p.S_window) p.S_window = (int)p.mo.m.size();
                p.mo = std::move(t);
            }
        };
        if (!p.fp8_digits) {
            if (w < logK) {
                ModuliSet t = choose_moduli_int8(K, kMaxModuli, p.b, w);
                const bool fewer = t.m.size() < p.mo.m.size();
                take(std::move(t), fewer);
            }
        } else {
            // the fewest-products set, else (when it cannot be formed within the moduli limit) the
            // route's own rules for the operands' window
            auto fits = [](const ModuliSet& t) { return t.nplane <= OZ2_MAXPLANES && t.nout <= OZ2_MAXOUT; };
            ModuliSet t = choose_moduli_fp8_fewest(K, (int)p.S_req, p.b, w);
            if (!(t.ok && t.b == p.b && fits(t)) && w < logK)
                t = choose_moduli_digits(Format::FP8, M, N, K, (int)p.S_req, p.b, w);
            const bool fewer = t.nprod < p.mo.nprod && fits(t);
            take(std::move(t), fewer);
        }
    }
    p.S = (int)p.mo.m.size();
    if (p.fp8_digits && (p.mo.nplane > OZ2_MAXPLANES || p.mo.nout > OZ2_MAXOUT))
        throw std::runtime_error("Ozaki II: the FP8 plan needs more digit planes or outputs than the device tables hold");
    // passes (plan.hpp:245-252)
    p.recon1_log2 = p.stats.measured ? recon1_log2(r, p.b, p.stats) : -INFINITY;
    if (passes != Reconstruction::Automatic)
        p.two_pass = passes == Reconstruction::TwoPass;
    else
        p.two_pass = !(p.recon1_log2 <= -(kTargetBits + kRecon1Margin));
    p.nd = (p.b > 4 * kDigitBits) ? 5 : ((p.b > 3 * kDigitBits) ? 4 : 3);
    return p;
}

oz2_moduli_dev split_descriptor(const Plan2& p) {
    oz2_moduli_dev d{};
    d.S = p.S;
    d.nd = p.nd;
    for (int s = 0; s < p.S; s++) {
        const int m = p.mo.m[s];
        d.m[s] = (float)m;
        d.rinv[s] = (float)(1.0 / (double)m);  // correctly rounded binary64 then binary32 (see below)
        for (int j = 0; j < 4; j++) {
            long r = 1 % m;
            for (int e = 0; e < kDigitBits * (j + 1); e++) r = (r * 2) % m;
            d.c[j][s] = (float)r;
        }
    }
    return d;
}

oz2_crt_dev crt_descriptor(const Plan2& p) {
    oz2_crt_dev d{};
    d.S = p.S;
    d.b = p.b;
    d.shift = p.shift();
    // Mprod and Q_s = Mprod / m_s as little-endian 32-bit words (at most 24 * 8 = 192 bits)
    auto mul_small = [](std::vector<std::uint32_t>& w, std::uint32_t k) {
        std::uint64_t c = 0;
        for (auto& x : w) {
            const std::uint64_t t = (std::uint64_t)x * k + c;
            x = (std::uint32_t)t;
            c = t >> 32;
        }
        if (c) w.push_back((std::uint32_t)c);
    };
    std::vector<std::uint32_t> Mw{1};
    for (int m : p.mo.m) mul_small(Mw, (std::uint32_t)m);
    // accumulator width: (terms+1)*M plus a sign bit; a term is a CRT digit (below m_s, one per
    // modulus) or, on the FP8 route, one product output's share of it
    std::vector<std::uint32_t> bound = Mw;
    mul_small(bound, (std::uint32_t)(std::max(p.S, p.mo.nout) + 1));
    int bits = 32 * ((int)bound.size() - 1) + (32 - __builtin_clz(bound.back())) + 1;
    d.nw = std::max(3, (bits + 31) / 32);
    if (d.nw > 8) throw std::runtime_error("Ozaki II: the CRT modulus exceeds the 256-bit reconstruction width");
    for (std::size_t w = 0; w < Mw.size() && w < 8; w++) d.Mw[w] = Mw[w];
    double mt = 0;
    for (int w = 7; w >= 0; w--) mt = mt * 4294967296.0 + (double)d.Mw[w];
    d.Mtop = mt;
    for (int s = 0; s < p.S; s++) {
        const std::uint32_t m = (std::uint32_t)p.mo.m[s];
        d.m[s] = m;
        // Q = M / m (exact), long division from the top word
        std::uint64_t r = 0;
        for (int w = 7; w >= 0; w--) {
            const std::uint64_t cur = (r << 32) | d.Mw[w];
            d.Q[s][w] = (std::uint32_t)(cur / m);
            r = cur % m;
        }
        // y = (Q mod m)^-1 mod m
        std::uint64_t qm = 0;
        for (int w = 7; w >= 0; w--) qm = ((qm << 32) | d.Q[s][w]) % m;
        std::uint32_t y = 0;
        for (std::uint32_t t = 1; t < m; t++)
            if ((qm * t) % m == 1) {
                y = t;
                break;
            }
        d.y[s] = y;
    }
    return d;
}

oz2_digit_dev digit_descriptor(const Plan2& p) {
    oz2_digit_dev d{};
    d.mo = split_descriptor(p);
    for (int s = 0; s < p.S; s++) {
        const int mode = p.mo.mode[s];
        // digit-making modes of the slicer (split.hpp:218-227 oz2_xmode): rounded digits for the square
        // and wide methods, Karatsuba, sparse square, and the residue itself for a one-digit modulus
        d.xmode[s] = mode == kSplitKar ? 1 : (mode == kSplitSqs ? 2 : (mode == kSplitOne ? 3 : 0));
        d.q[s] = (float)p.mo.q[s];
        d.qinv[s] = 1.0f / (float)p.mo.q[s];  // stages.hpp:223
    }
    d.encoding = 1;
    return d;
}

oz2_groups_dev groups_descriptor(const Plan2& p, const oz2_crt_dev& crt, std::vector<unsigned char>& term_modulus) {
    oz2_groups_dev g{};
    const std::vector<Fp8Output>& outs = p.mo.outputs;
    g.nout = (int)outs.size();
    g.nplanes = p.mo.nplane;
    // heavier outputs (more pairs) are dispatched first; ties keep the reference's order
    std::vector<int> order(outs.size());
    for (std::size_t i = 0; i < order.size(); i++) order[i] = (int)i;
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return outs[x].npairs > outs[y].npairs; });
    term_modulus.assign(outs.size(), 0);
    for (std::size_t j = 0; j < order.size(); j++) {
        const Fp8Output& o = outs[order[j]];
        oz2_group_dev& d = g.g[j];
        d.npairs = o.npairs;
        d.modulus = o.s;
        for (int t = 0; t < o.npairs; t++) {
            d.a[t] = (unsigned char)o.a[t];
            d.b[t] = (unsigned char)o.b[t];
        }
        const std::uint64_t m = (std::uint64_t)p.mo.m[o.s];
        d.m = (std::uint32_t)m;
        d.coef = (std::uint32_t)(((std::uint64_t)o.coef % m) * crt.y[o.s] % m);
        d.bound = (float)o.bound;
        term_modulus[j] = (unsigned char)o.s;
    }
    return g;
}

}  // namespace ozTTgemm::detail

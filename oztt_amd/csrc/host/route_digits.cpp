// Scheme II moduli selection on the digit routes (every format but INT8); see plan2.hpp.
//
// A format other than INT8 carries a residue modulo m as small balanced digits that its products
// multiply exactly. The reference's route of each format (src/backend/ozaki2/split.hpp:66-146
// OZ2_ROUTES: modulus cap, digit bound, digit count, sparse digits, one-digit moduli) fixes how
// each modulus is carried (split.hpp:148-728) and which moduli are usable; the moduli are then
// taken from a table (FP8, TF32; moduli.hpp:170-213, :246-300) or chosen by the reference's
// stage-time model of its Tenstorrent stages (BF16, FP16, BFP8, BFP4, BFP2; awe.hpp). The set and
// the width b it covers are what Info reports and what the pass choice is made on; the FP8 set is
// also what the FP8 matrix cores compute with. So every rule, table, coefficient, search order and
// floating-point comparison is kept. Compiled with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "plan2.hpp"

namespace ozTTgemm::detail {
namespace {

constexpr double kWinEps = 1e-9, kTailTol = 0.25;
constexpr double kExact24 = 16777216.0, kCompose22 = 4194304.0;
constexpr long kComposeSplit = 4096;  // radix of the 2^12 split of the composition
constexpr int kMaxProd = 32;          // digit products of one modulus at most (digit_limits.h:23)

// Rows of the stage-time model (split.hpp:66-73).
enum ModelRow { kNoModel = 0, kModelBfp4 = 1, kModelBfp2 = 2, kModelBf16 = 3, kModelFp16 = 4, kModelBfp8 = 5 };

// One format's route (split.hpp:48-64 Oz2Route, rows :78-146).
struct Route {
    int mod_cap;     // largest modulus
    int dmax;        // bound on |digit|
    int nrdig;       // digits of a residue: 2, or up to 5 balanced ternary digits (BFP2)
    unsigned def_s;  // moduli limit with a fixed width and no max_moduli
    int smax;        // bound of the sparse e4m3 digits (FP8), 0 when unused
    int model;       // row of the stage-time model, kNoModel: table selection
    bool one;        // small moduli carried as one digit
};
constexpr Route kRouteFp8 = {2401, 16, 2, 14u, 32, kNoModel, false};
constexpr Route kRouteTf32 = {4096, 32, 2, 11u, 0, kNoModel, false};
constexpr Route kRouteBf16 = {4096, 32, 2, 24u, 0, kModelBf16, true};
constexpr Route kRouteFp16 = {4096, 32, 2, 24u, 0, kModelFp16, true};
constexpr Route kRouteBfp8 = {4096, 32, 2, 24u, 0, kModelBfp8, true};
constexpr Route kRouteBfp4 = {3375, 7, 2, 24u, 0, kModelBfp4, false};
constexpr Route kRouteBfp2 = {243, 1, 5, 24u, 0, kModelBfp2, false};

const Route& route_of(Format f) {
    switch (f) {
    case Format::FP8: return kRouteFp8;
    case Format::TF32: return kRouteTf32;
    case Format::BF16: return kRouteBf16;
    case Format::FP16: return kRouteFp16;
    case Format::BFP8: return kRouteBfp8;
    case Format::BFP4: return kRouteBfp4;
    case Format::BFP2: return kRouteBfp2;
    default: throw std::invalid_argument("internal error: INT8 has no digit route");
    }
}

// Candidate tables (moduli.hpp:184-213), descending and pairwise coprime.
constexpr int kTableF8[] = {1089, 1024, 961, 841, 625, 529, 511, 509, 503, 499,
                            491,  487,  481, 479, 467, 463, 461, 457, 449, 443};
constexpr int kTableF8S[] = {2401, 2209, 1849, 1681, 1521, 1369, 1024, 961, 841, 625, 529, 361,
                             289,  121,  509,  503,  499,  491,  487,  479, 467, 463, 461, 457};
constexpr int kTableB8[] = {4096, 3969, 3721, 3481, 3025, 2809, 2209, 1849,
                            1681, 1369, 961,  841,  529,  361,  289,  169};
constexpr int kTableB4[] = {225, 196, 169, 121, 223, 211, 199, 197, 193, 191, 181,
                            179, 173, 167, 163, 157, 151, 149, 139, 137, 131, 127};
constexpr int kTableB2[] = {243, 242, 241, 239, 235, 233, 229, 227, 223, 221,
                            217, 211, 199, 197, 193, 191, 181, 179, 173, 167};

// ---- how a modulus is carried (split.hpp:233-728) -----------------------------------------------

// The digit shape of a selection: the route's digits after the fallback of FP8 to dense digits.
struct Shape {
    int dmax, n, smax;
    bool one;
};

bool e4m3_int(long v) {
    if (v < 0) v = -v;
    if (v == 0) return true;
    int e = 0;
    for (long x = v; x; x >>= 1) ++e;
    return e <= 4 || (v % (1L << (e - 4))) == 0;
}
// the e4m3 integers up to smax hold every residue class modulo q
bool sparse_covers(int q, int smax) {
    if (q <= 0 || smax <= 0 || q > 2 * smax + 1) return false;
    std::vector<char> hit(q, 0);
    int n = 0;
    for (int x = -smax; x <= smax; ++x)
        if (e4m3_int(x)) {
            const int r = ((x % q) + q) % q;
            n += !hit[r];
            hit[r] = 1;
        }
    return n == q;
}
// the sparse-digit split of a residue modulo q^2, q odd (split.hpp:266-279)
void sqs_split(long r, int q, long& l, long& h) {
    long h0 = (2 * r + (r >= 0 ? q : -q)) / (2 * q);
    long t = r - (long)q * h0;
    const long st = t > 0 ? 1 : (t < 0 ? -1 : 0);
    if ((t & 1) && (t >= 17 || t <= -17)) {
        t -= st * q;
        h0 += st;
    }
    const long sh = h0 > 0 ? 1 : (h0 < 0 ? -1 : 0);
    if ((h0 & 1) && (h0 >= 17 || h0 <= -17)) h0 -= sh * q;
    l = t;
    h = h0;
}
// largest |l| and |h| of the sparse split over |r| <= floor(q^2/2) + 1, for q <= 64 tabulated once
void sqs_bounds(int q, int& dl, int& dh) {
    auto count = [](int qq, int& a, int& b) {
        const long R = (long)qq * qq / 2 + 1;
        a = b = 0;
        for (long r = -R; r <= R; ++r) {
            long l, h;
            sqs_split(r, qq, l, h);
            a = std::max<int>(a, (int)std::labs(l));
            b = std::max<int>(b, (int)std::labs(h));
        }
    };
    if (q > 0 && q <= 64) {
        static const std::vector<std::pair<int, int>> table = [&] {
            std::vector<std::pair<int, int>> t(65, {0, 0});
            for (int qq = 1; qq <= 64; ++qq) count(qq, t[qq].first, t[qq].second);
            return t;
        }();
        dl = table[q].first;
        dh = table[q].second;
        return;
    }
    count(q, dl, dh);
}

// Bound on |r| after the slicer's last ModRound (split.hpp:330-349): at most floor(m/2 + e) with e
// the FP32 rounding of that reduction's input, and at most floor(m/2) + 1.
long resid_bound(int m) {
    long c0 = 1 % m;
    for (int i = 0; i < kDigitBits; ++i) c0 = (c0 * 2) % m;
    const long c1 = (c0 * c0) % m, c2 = (c1 * c0) % m;
    const double u = std::ldexp(1.0, -23) * (1.0 + std::ldexp(1.0, -23));
    const double d0 = 524288.0 + 65536.0 + 1.0;
    const double s3 = d0 + (double)(m / 2) * (double)(c0 + c1);
    const double s4 = m / 2.0 + 2.0 + (double)(m / 2) * (double)c2;
    return std::min<long>((long)std::floor(m / 2.0 + std::max(s3, s4) * u), m / 2 + 1);
}
long bal_cap(int dmax, int n) {
    long c = 1;
    for (int i = 0; i < n; ++i) c *= 2L * dmax + 1;
    return c;
}
// smallest n <= nmax of balanced digits that holds every residue; nmax + 1 if none
int bal_ndig(int m, int dmax, int nmax) {
    const long R = resid_bound(m);
    for (int n = 1; n <= nmax; ++n) {
        const long c = bal_cap(dmax, n);
        if (m <= c && 2 * R + 1 <= c) return n;
    }
    return nmax + 1;
}
int digit_bound_rnd(int m, int q) { return std::max((m / 2 + q / 2) / q, q / 2); }
int digit_bound_kar16(int m) { return std::max((m / 2 + 15) / 16, 15); }
int kar_base(int dmax) { return (dmax && dmax < 15) ? dmax + 1 : 16; }
int digit_bound_kar(int m, int B) { return std::max<int>((int)((resid_bound(m) + B - 1) / B), B - 1); }
int isqrt(int m) {
    int r = (int)std::sqrt((double)m);
    while ((long)(r + 1) * (r + 1) <= m) ++r;
    while ((long)r * r > m) --r;
    return r;
}
int is_square(int m) {
    const int r = isqrt(m);
    return (long)r * r == m ? r : 0;
}
// the radix near sqrt(m) with the smallest rounded digits
int digit_base_rnd(int m) {
    const int r = isqrt(m);
    int best = r + 1, bb = digit_bound_rnd(m, r + 1);
    for (int q = r; q <= r + 3; ++q)
        if (const int v = digit_bound_rnd(m, q); v < bb) {
            bb = v;
            best = q;
        }
    return best;
}

// Carrying method of modulus m (split.hpp:430-450). Sparse squares only where the caller passes smax.
int split_mode(int m, const Shape& S, bool sparse = false) {
    if (S.n > 2) return kSplitBal;
    if (S.one && S.dmax && resid_bound(m) <= S.dmax) return kSplitOne;
    const bool narrow = S.dmax && S.dmax < 15;
    if (const int q = is_square(m)) {
        if (sparse && S.smax && S.dmax && digit_bound_rnd(m, q) > S.dmax && (q & 1) && sparse_covers(q, S.smax))
            return kSplitSqs;
        if (!narrow || digit_bound_rnd(m, q) <= S.dmax) return kSplitSq;
    }
    if (narrow) {
        if (digit_bound_kar(m, kar_base(S.dmax)) <= S.dmax) return kSplitKar;
        if (digit_bound_rnd(m, digit_base_rnd(m)) <= S.dmax) return kSplitWide;
        if (bal_ndig(m, S.dmax, 3) <= 3) return kSplitBal;
        return kSplitWide;  // not carriable: usable() rejects it
    }
    if (digit_bound_kar16(m) <= (S.dmax ? std::min(16, S.dmax) : 16)) return kSplitKar;
    return kSplitWide;
}
int bal_digits(int m, const Shape& S) {
    if (S.n > 2) return bal_ndig(m, S.dmax, S.n);
    return split_mode(m, S) == kSplitBal ? 3 : 0;
}
int digit_base(int m, const Shape& S) {
    if (S.n > 2) return 2 * S.dmax + 1;
    switch (split_mode(m, S)) {
    case kSplitOne: return 1;
    case kSplitBal: return 2 * S.dmax + 1;
    case kSplitSq: return is_square(m);
    case kSplitKar: return kar_base(S.dmax);
    default: return digit_base_rnd(m);
    }
}
// bound on the dense digits; dmax + 1 for a balanced-digit modulus that needs too many digits
int digit_bound(int m, const Shape& S) {
    if (S.n > 2) return bal_ndig(m, S.dmax, S.n) <= S.n ? S.dmax : S.dmax + 1;
    switch (split_mode(m, S)) {
    case kSplitOne: return (int)resid_bound(m);
    case kSplitBal: return bal_ndig(m, S.dmax, 3) <= 3 ? S.dmax : S.dmax + 1;
    case kSplitKar: return (S.dmax && S.dmax < 15) ? digit_bound_kar(m, kar_base(S.dmax)) : digit_bound_kar16(m);
    default: return digit_bound_rnd(m, digit_base(m, S));
    }
}
bool usable(int m, const Shape& S) {
    if (split_mode(m, S, true) == kSplitSqs) return true;
    return digit_bound(m, S) <= S.dmax;
}
int digit_planes(int m, const Shape& S) {
    if (const int n = bal_digits(m, S)) return n;
    const int mode = split_mode(m, S);
    return mode == kSplitOne ? 1 : (mode == kSplitKar ? 3 : 2);
}
// bound on |digit| of plane 0 (l), 1 (h) or 2 (s) of modulus m (split.hpp:482-501)
int plane_bound(int m, int plane, const Shape& S) {
    if (S.one && !S.smax) {
        const int mode = split_mode(m, S), R = (int)resid_bound(m);
        if (mode == kSplitOne) return R;
        if (mode == kSplitKar) {
            const int h = (R + 15) / 16;
            return plane == 0 ? 15 : (plane == 1 ? h : std::max(h, 15));
        }
        const int q = digit_base(m, S);
        return plane == 0 ? q / 2 : (R + q / 2) / q;
    }
    if (!S.smax) return S.dmax;
    if (split_mode(m, S, true) == kSplitSqs) {
        int dl, dh;
        sqs_bounds(is_square(m), dl, dh);
        return plane == 0 ? dl : dh;
    }
    return digit_bound(m, S);
}

// A digit product (plane a of A times plane b of B) and its composition coefficient with its 2^12
// multiple, both reduced modulo m (split.hpp:541-597).
struct Term {
    int a, b;
    long lo, hi;
};
int product_terms(int m, const Shape& S, Term* t) {
    auto rm = [m](long v) {
        const long r = v % m;
        return r < 0 ? r + m : r;
    };
    auto sm = [&](long v) {  // symmetric representative in (-m/2, m/2]
        const long r = rm(v);
        return r > m / 2 ? r - m : r;
    };
    int k = 0;
    if (const int n = bal_digits(m, S)) {  // coefficients q^(i+j); the terms i+j >= n vanish when m | q^n
        const long q = 2L * S.dmax + 1;
        const bool drop = bal_cap(S.dmax, n) % m == 0;
        if ((drop ? n * (n + 1) / 2 : n * n) > kMaxProd)
            throw std::runtime_error("internal error: modulus " + std::to_string(m) + " needs more than " +
                                     std::to_string(kMaxProd) + " digit products");
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < n; ++j) {
                if (drop && i + j >= n) continue;
                long c = 1;
                for (int e = 0; e < i + j; ++e) c = rm(c * q);
                t[k++] = {i, j, sm(c), sm(c * kComposeSplit)};
            }
        return k;
    }
    const int mode = split_mode(m, S), q = digit_base(m, S);
    if (mode == kSplitOne) {
        t[k++] = {0, 0, 1, rm(kComposeSplit)};
        return k;
    }
    if (mode == kSplitKar) {  // coefficients 1 - B, B^2 - B, B
        const long B = q;
        const bool narrow = S.dmax && S.dmax < 15;
        for (const long c : {1 - B, B * B - B, B}) {
            const long v = narrow ? sm(c) : rm(c);
            t[k] = {k, k, v, narrow ? sm(v * kComposeSplit) : rm(v * kComposeSplit)};
            ++k;
        }
        return k;
    }
    const long c[4] = {rm(1), rm(q), rm(q), rm((long)q * q)};  // squares and wide moduli: 1, q, q (, q^2)
    const int pa[4] = {0, 1, 0, 1}, pb[4] = {0, 0, 1, 1};
    const int n = mode == kSplitWide ? 4 : 3;
    for (int j = 0; j < n; ++j) t[k++] = {pa[j], pb[j], c[j], rm(c[j] * kComposeSplit)};
    return k;
}
int digit_prods(int m, const Shape& S) {
    Term t[kMaxProd];
    return product_terms(m, S, t);
}

// Digit products of equal weight concatenated along K in runs of at most maxg (split.hpp:628-661).
struct Group {
    int a0, b0, g;
    long lo, hi;
};
int product_groups(int m, const Shape& S, int maxg, Group* gr) {
    Term t[kMaxProd];
    const int n = product_terms(m, S, t), np = digit_planes(m, S);
    int k = 0;
    for (int key = 0; key <= 2 * (np - 1); ++key) {
        int as[kMaxProd], na = 0;
        long lo = 0, hi = 0;
        for (int j = 0; j < n; ++j)
            if (t[j].a + t[j].b == key) {
                if (na && (t[j].lo != lo || t[j].hi != hi)) return 0;
                as[na++] = t[j].a;
                lo = t[j].lo;
                hi = t[j].hi;
            }
        std::sort(as, as + na);
        for (int i = 0; i < na;) {
            int g = 1;
            while (i + g < na && g < maxg && as[i + g] == as[i] + g) ++g;
            gr[k++] = {as[i], np - 1 - (key - as[i]), g, lo, hi};
            i += g;
        }
    }
    return k;
}
int nout(int m, const Shape& S, int maxg) {
    Group gr[kMaxProd];
    return product_groups(m, S, maxg, gr);
}
// bound on |output| of a group: the B plane at position b0 + t holds digit np - 1 - (b0 + t)
double group_bound(int m, const Group& g, double K, const Shape& S) {
    const int np = digit_planes(m, S);
    double sb = 0;
    for (int t = 0; t < g.g; ++t) sb += K * plane_bound(m, g.a0 + t, S) * plane_bound(m, np - 1 - (g.b0 + t), S);
    return sb;
}
// concatenation bound: g K d_l d_h + cap <= 2^24 (split.hpp:684-690)
int maxg_for(int m, std::uint32_t K, int cap, const Shape& S) {
    const double pb =
        (double)plane_bound(m, 0, S) * plane_bound(m, std::min(1, digit_planes(m, S) - 1), S);
    return std::max(1, (int)std::floor((kExact24 - cap) / ((double)K * pb)));
}

// Planes of the reference's composition stage for a largest output count mx of a composed modulus
// (split.hpp:703-716), and its DRAM estimate (:718-728).
double compose_planes(bool composes, int mx) {
    if (!composes) return 0;
    const int max_nout = std::max(mx, 3), chunk = max_nout > 12 ? 5 : max_nout;
    return chunk < max_nout ? chunk + (max_nout + chunk - 1) / chunk : max_nout;
}
double dram_one_group(double nplane, double P, double cplanes, double S, double out, double F) {
    const double Q = (cplanes + S) * out;
    return nplane * P + (Q > F ? Q - F : 0.0) + (double)(512ull << 20);
}

// ---- the stage-time model (awe.hpp) ---------------------------------------------------------------
// Coefficients per model row at K = 3520, 7040, 14080 (awe_coef.inc, the reference's fitted data):
// gp per matrix product and go per output (products), co per output and cs per modulus
// (composition), sop per slicer operation and spl per digit plane (slicing), and the
// reconstruction max(R0, ra + rb S).
struct Coef {
    double K, gp, go, co, cs, sop, spl, R0, ra, rb;
};
constexpr Coef kCoef[5][3] = {
    {{3520, 0.15104, 0.32008, 0.22464, 0.019534, 0.03579, 0.0079022, 17.049, 0.48024, 1.1506},
     {7040, 1.283, 0.85997, 0.88145, 0.047905, 0.14311, 0.032002, 68.235, 1.3607, 4.6024},
     {14080, 14.296, 1.2996, 3.3835, 2.3497, 0.5724, 0.12698, 276.15, 63.034, 15.008}},
    {{3520, 0.14101, 0.32003, 0.24895, 0.021648, 0.033222, 0.0073353, 17.049, 0.48025, 1.1506},
     {7040, 1.2571, 0.86005, 1.0826, 0.058839, 0.13282, 0.029702, 68.36, 1.3632, 4.6108},
     {14080, 14.01, 1.3, 4.6058, 3.1984, 0.53118, 0.11783, 277.15, 63.262, 15.062}},
    {{3520, 0.18, 0.32, 0.22216, 0.019318, 0.035712, 0.007885, 17.05, 0.48028, 1.1507},
     {7040, 1.6623, 0.86117, 0.89522, 0.048653, 0.14382, 0.032161, 68.35, 1.363, 4.6101},
     {14080, 18.496, 1.2997, 3.7014, 2.5704, 0.57273, 0.12705, 278.85, 63.651, 15.155}},
    {{3520, 0.1811, 0.32017, 0.22564, 0.019621, 0.035752, 0.56545, 17.17, 0.48366, 1.1588},
     {7040, 1.6436, 0.86032, 0.91946, 0.049971, 0.14307, 2.2615, 68.45, 1.365, 4.6168},
     {14080, 18.324, 1.3003, 3.6652, 2.5453, 0.57267, 9.0297, 275.92, 62.982, 14.996}},
    {{3520, 0.16493, 0.31987, 0.22434, 0.019508, 0.03577, 0.0078979, 17.04, 0.48, 1.15},
     {7040, 1.4367, 0.85984, 0.89468, 0.048624, 0.14306, 0.031991, 67.988, 1.3558, 4.5857},
     {14080, 16.021, 1.3, 3.4905, 2.424, 0.57235, 0.12697, 274.29, 62.61, 14.907}},
};
// Bytes of one 32 x 32 tile of the format whose route has the model row (BFP4, BFP2, BF16, FP16,
// BFP8 in row order): what the model's memory estimate counts per digit plane.
constexpr double kSliceTile[5] = {576, 320, 2048, 2048, 1088};
constexpr double kOneRecon = 0.062;           // reconstruction surcharge of a one-digit modulus, times rb
constexpr double kDramFree = 31.0e9;          // free device memory the model assumes
constexpr size_t kVecMax = 200000;            // count vectors enumerated at most
constexpr long kNodeMax = 400000;             // assignment nodes per vector
constexpr long kNodeBudget = 10000000;        // assignment nodes in total when the bound is not the greedy one
constexpr double kOverNeedBits = 16.0;        // a class's count stops this far above the window
constexpr double kUbSlack = 1.05;             // cost bound: this times the greedy solution

// The row's coefficients at K: interpolated in log K between the two nearest fitted rows (power law
// for positive values), extrapolated beyond them.
Coef coef_at(int row, std::uint32_t K) {
    const Coef* t = kCoef[row - 1];
    const double x = std::log2((double)K);
    const int i = x > std::log2(t[1].K) ? 1 : 0;
    const double x0 = std::log2(t[i].K), x1 = std::log2(t[i + 1].K), f = (x - x0) / (x1 - x0);
    auto ip = [f](double a, double b) {
        if (a > 0 && b > 0) return std::exp(std::log(a) + f * (std::log(b) - std::log(a)));
        return a + f * (b - a);
    };
    const Coef& a = t[i];
    const Coef& b = t[i + 1];
    return {(double)K,        ip(a.gp, b.gp),   ip(a.go, b.go), ip(a.co, b.co), ip(a.cs, b.cs),
            ip(a.sop, b.sop), ip(a.spl, b.spl), ip(a.R0, b.R0), ip(a.ra, b.ra), ip(a.rb, b.rb)};
}
double recon_time(const Coef& c, int S) { return std::max(c.R0, c.ra + c.rb * S); }
// slicer operations for a modulus's digits beyond the 19 up to its residue
int slice_ops(int m, const Shape& S) {
    switch (split_mode(m, S, true)) {
    case kSplitBal: return 7 * (bal_digits(m, S) - 1);
    case kSplitOne: return 0;
    case kSplitKar: return 12;
    case kSplitSqs: return 13;
    default: return 6;
    }
}

// Moduli of equal modelled cost form a class; est[t] are the bits of its t largest members that are
// pairwise coprime, taken greedily.
struct Cand {
    int m;
    double bits;
    int np = 0;
    short pr[4] = {0, 0, 0, 0};  // distinct prime factors of m
};
struct Class {
    int nprod, nout, npl, ops;
    bool one;
    double cost;
    std::vector<Cand> v;
    std::vector<double> est;
};

// The distinct prime factors of m <= 4096 (at most four), from a smallest-factor table built once.
int distinct_primes(int m, int* out) {
    static const std::vector<short> spf = [] {
        std::vector<short> t(4097, 0);
        for (int i = 2; i <= 4096; ++i)
            if (!t[i])
                for (int j = i; j <= 4096; j += i)
                    if (!t[j]) t[j] = (short)i;
        return t;
    }();
    int n = 0;
    while (m > 1) {
        const int p = spf[m];
        out[n++] = p;
        while (m % p == 0) m /= p;
    }
    return n;
}

std::vector<Class> model_classes(std::uint32_t K, const Coef& C, int cap, const Shape& S) {
    std::vector<Class> ks;
    for (int m = cap; m >= 2; --m) {
        if (!usable(m, S)) continue;
        const int mg = maxg_for(m, K, cap, S), pl = digit_planes(m, S), np = digit_prods(m, S);
        const int no = nout(m, S, mg), op = slice_ops(m, S);
        const bool one = split_mode(m, S, true) == kSplitOne;
        // outputs that stop being exact FP32 integers with the modulus added, or a reduce-first
        // composition sum at or beyond 2^22, exclude the modulus
        Group gr[kMaxProd];
        const int ng = product_groups(m, S, mg, gr);
        double csum = 0, gmax = 0;
        for (int j = 0; j < ng; ++j) {
            csum += std::fabs((double)gr[j].lo);
            gmax = std::max(gmax, group_bound(m, gr[j], (double)K, S));
        }
        if (!ng || gmax + cap > kExact24 || csum * (m / 2.0 + 2.0) >= kCompose22) continue;
        auto it = std::find_if(ks.begin(), ks.end(), [&](const Class& x) {
            return x.nprod == np && x.nout == no && x.npl == pl && x.ops == op && x.one == one;
        });
        if (it == ks.end()) {
            const double cost = one ? C.gp * np + C.go * no + C.sop * (19 + op) + C.spl * pl + kOneRecon * C.rb
                                    : C.gp * np + (C.go + C.co) * no + C.cs + C.sop * (19 + op) + C.spl * pl;
            ks.push_back({np, no, pl, op, one, cost, {}, {}});
            it = ks.end() - 1;
        }
        Cand cand{m, std::log2((double)m)};
        int pr[5];
        cand.np = distinct_primes(m, pr);
        for (int t = 0; t < cand.np; ++t) cand.pr[t] = (short)pr[t];
        it->v.push_back(cand);
    }
    for (Class& k : ks) {
        std::vector<int> got;
        k.est.assign(1, 0.0);
        for (const Cand& c : k.v)
            if (std::all_of(got.begin(), got.end(), [&](int g) { return std::gcd(g, c.m) == 1; })) {
                got.push_back(c.m);
                k.est.push_back(k.est.back() + c.bits);
            }
    }
    std::sort(ks.begin(), ks.end(), [](const Class& a, const Class& b) {
        const double ra = a.cost / a.v[0].bits, rb = b.cost / b.v[0].bits;
        return ra != rb ? ra < rb : a.cost < b.cost;
    });
    return ks;
}

struct Model {
    const std::vector<Class>& ks;
    Coef C;
    double need, tol;
    int max_moduli;
    std::vector<double> minrate;  // smallest cost per bit among classes c and later
    double P, out, F;             // memory estimate: one digit plane of A and of B, one output plane, the operands
    // S moduli with npl digit planes fit the assumed free memory without row bands
    bool fits(int S, int npl, int mxo) const {
        return dram_one_group(npl, P, compose_planes(mxo > 0, mxo), S, out, F) <= kDramFree;
    }
};

struct CountVec {
    double T;
    std::vector<int> n;
};

// Count vectors (moduli per class) whose modelled time is below the bound and whose bit estimate
// reaches the window, collected at the leaves of a pruned depth-first walk in walk order.
void enumerate(const Model& s, double incumbent, bool check_dram, bool& dram_cut, std::vector<CountVec>& vecs,
               std::vector<int>& n, int c, int S, double cost, double est, int npl, int mxo) {
    const int NC = (int)s.ks.size();
    if (vecs.size() >= kVecMax) return;
    if (c == NC) {
        if (est >= s.need && S > 0) {
            const double T = cost + recon_time(s.C, S);
            if (T < incumbent) {
                if (!check_dram || s.fits(S, npl, mxo))
                    vecs.push_back({T, n});
                else
                    dram_cut = true;
            }
        }
        return;
    }
    if (cost + std::max(0.0, s.need - est) * s.minrate[c] + recon_time(s.C, S) >= incumbent) return;
    const Class& k = s.ks[c];
    const int maxn = std::min<int>((int)k.est.size() - 1, s.max_moduli - S);
    for (int t = 0; t <= maxn; ++t) {
        n[c] = t;
        const double e2 = est + k.est[t], ct = cost + t * k.cost;
        if (ct + recon_time(s.C, S + t) >= incumbent) break;
        if (t > 0 && ct + std::max(0.0, s.need - e2) * s.minrate[c + 1] + recon_time(s.C, S + t) >= incumbent)
            continue;
        enumerate(s, incumbent, check_dram, dram_cut, vecs, n, c + 1, S + t, ct, e2, npl + t * k.npl,
                  (t && !k.one) ? std::max(mxo, k.nout) : mxo);
        if (e2 >= s.need + kOverNeedBits) break;
    }
    n[c] = 0;
}

// Pairwise coprime moduli for one count vector with bits in [need, need + tol], the smallest excess
// first; classes are filled in the order `ord`, the walk stops after kNodeMax nodes or at an excess
// of at most 1e-4 bits. A candidate is coprime to the picked moduli when none of its prime factors
// divides one of them (`uses` counts the picked moduli per prime).
// Sums of `left` consecutive candidates' bits of a class, v[j].bits + v[j+1].bits + ... added in that
// order, for every start j; made once per class and count and kept across count vectors.
struct RunSums {
    const std::vector<Class>& ks;
    std::vector<std::vector<std::vector<double>>> t = std::vector<std::vector<std::vector<double>>>(ks.size());
    const std::vector<double>& of(int c, int left) {
        auto& byleft = t[c];
        if ((int)byleft.size() <= left) byleft.resize(left + 1);
        std::vector<double>& r = byleft[left];
        if (r.empty()) {
            const std::vector<Cand>& v = ks[c].v;
            r.assign(v.size(), 0.0);
            for (int j = 0; j + left <= (int)v.size(); ++j) {
                double u = 0;
                for (int q = 0; q < left; ++q) u += v[j + q].bits;
                r[j] = u;
            }
        }
        return r;
    }
};

struct Assign {
    const Model& s;
    const std::vector<int>& ord;
    RunSums& runs;
    std::vector<int> cnt;
    std::vector<double> ubrest, lbrest;  // most / fewest bits the classes ord[i..] can add
    std::vector<int> pick, best;
    double bestex = 1e300;
    long nodes = 0;
    std::vector<short> uses = std::vector<short>(4097, 0);

    bool coprime(const Cand& c) const {
        for (int t = 0; t < c.np; ++t)
            if (uses[c.pr[t]]) return false;
        return true;
    }

    void walk(int i, int start, int left, double bits) {
        const int NC = (int)s.ks.size();
        if (++nodes > kNodeMax || bestex <= 1e-4) return;
        if (i == NC) {
            const double ex = bits - s.need;
            if (ex >= 0 && ex <= s.tol && ex < bestex) {
                bestex = ex;
                best = pick;
            }
            return;
        }
        if (left == 0) {
            walk(i + 1, 0, i + 1 < NC ? cnt[i + 1] : 0, bits);
            return;
        }
        const std::vector<Cand>& v = s.ks[ord[i]].v;
        if (left == 1) {
            // the candidates that overshoot the window even with the fewest bits of the later classes
            // are skipped; they form a prefix (v descends, rounding is monotone), found by bisection,
            // and none of them could end the loop (ubrest >= lbrest)
            int lo = start, hi = (int)v.size();
            while (lo < hi) {
                const int mid = (lo + hi) / 2;
                if (bits + v[mid].bits + lbrest[i + 1] > s.need + s.tol)
                    lo = mid + 1;
                else
                    hi = mid;
            }
            start = lo;
        }
        const std::vector<double>& run = runs.of(ord[i], left);
        for (int j = start; j + left <= (int)v.size(); ++j) {
            if (bits + run[j] + ubrest[i + 1] < s.need) return;
            if (bits + v[j].bits + lbrest[i + 1] > s.need + s.tol && left == 1) continue;
            if (!coprime(v[j])) continue;
            pick.push_back(v[j].m);
            for (int t = 0; t < v[j].np; ++t) ++uses[v[j].pr[t]];
            walk(i, j + 1, left - 1, bits + v[j].bits);
            for (int t = 0; t < v[j].np; ++t) --uses[v[j].pr[t]];
            pick.pop_back();
            if (nodes > kNodeMax || bestex <= 1e-4) return;
        }
    }
};

std::vector<int> assign(const Model& s, const std::vector<int>& ord, RunSums& runs, const CountVec& vec, long& nodes) {
    const int NC = (int)s.ks.size();
    Assign a{s, ord, runs, std::vector<int>(NC), std::vector<double>(NC + 1, 0.0), std::vector<double>(NC + 1, 0.0)};
    for (int i = 0; i < NC; ++i) a.cnt[i] = vec.n[ord[i]];
    for (int i = NC - 1; i >= 0; --i) {
        const std::vector<Cand>& v = s.ks[ord[i]].v;
        double ub = 0, lb = 0;
        for (int j = 0; j < a.cnt[i] && j < (int)v.size(); ++j) {
            ub += v[j].bits;
            lb += v[v.size() - 1 - j].bits;
        }
        a.ubrest[i] = a.ubrest[i + 1] + ub;
        a.lbrest[i] = a.lbrest[i + 1] + lb;
    }
    a.walk(0, 0, NC ? a.cnt[0] : 0, 0.0);
    nodes = a.nodes;
    return a.best;
}

// The count vectors below the bound in order of modelled time, then the first that has a set; with
// budget > 0 no vector is started once the assignment nodes exceed it.
std::vector<int> model_search(const Model& s, double ub, bool check_dram, bool& dram_cut, long budget) {
    const int NC = (int)s.ks.size();
    std::vector<CountVec> vecs;
    std::vector<int> n(NC, 0);
    enumerate(s, ub, check_dram, dram_cut, vecs, n, 0, 0, 0.0, 0.0, 0, 0);
    std::stable_sort(vecs.begin(), vecs.end(), [](const CountVec& a, const CountVec& b) { return a.T < b.T; });
    std::vector<int> ord(NC);
    std::iota(ord.begin(), ord.end(), 0);
    std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return s.ks[a].v.size() < s.ks[b].v.size(); });
    RunSums runs{s.ks};
    long spent = 0;
    for (const CountVec& vec : vecs) {
        if (budget > 0 && spent > budget) break;
        long nodes = 0;
        std::vector<int> best = assign(s, ord, runs, vec, nodes);
        spent += nodes;
        if (!best.empty()) {
            std::sort(best.begin(), best.end(), std::greater<int>());
            return best;
        }
    }
    return {};
}

// Cost bound: kUbSlack times the greedy set in order of cost per bit, skipping a modulus after which
// the remaining slots could not reach the window even at the cap. `plain`: the greedy set reached the
// window without a skip (the search then needs no node budget).
double model_bound(const Model& s, int cap, bool& plain) {
    std::vector<std::pair<double, std::pair<int, double>>> all;  // (cost per bit, (m, cost))
    for (const Class& k : s.ks)
        for (const Cand& c : k.v) all.push_back({k.cost / c.bits, {c.m, k.cost}});
    std::stable_sort(all.begin(), all.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
    const double maxbits = std::log2((double)cap);
    std::vector<int> got;
    double bits = 0, cost = 0;
    bool skipped = false;
    for (const auto& a : all) {
        if (bits >= s.need || (int)got.size() >= s.max_moduli) break;
        const int m = a.second.first;
        if (!std::all_of(got.begin(), got.end(), [&](int g) { return std::gcd(g, m) == 1; })) continue;
        const double lb = std::log2((double)m);
        if (bits + lb + (s.max_moduli - (int)got.size() - 1) * maxbits < s.need) {
            skipped = true;
            continue;
        }
        got.push_back(m);
        bits += lb;
        cost += a.second.second;
    }
    plain = bits >= s.need && !skipped;
    return bits >= s.need ? (cost + recon_time(s.C, (int)got.size())) * kUbSlack + 1e-9 : 1e300;
}

// The model's set for the window `need` (descending; empty when none is found).
std::vector<int> model_choose(std::uint32_t M, std::uint32_t N, std::uint32_t K, int row, int cap, const Shape& S,
                              double need, int max_moduli) {
    const Coef C = coef_at(row, K);
    const std::vector<Class> ks = model_classes(K, C, cap, S);
    if (ks.empty()) return {};
    const int NC = (int)ks.size();
    const double ops = (double)M * K + (double)K * N;
    Model s{ks, C, need, kTailTol, max_moduli, std::vector<double>(NC + 1, 1e300),
            ops / 1024.0 * kSliceTile[row - 1], (double)M * N * 4.0, ops * 8.0};
    for (int c = NC - 1; c >= 0; --c) s.minrate[c] = std::min(s.minrate[c + 1], ks[c].cost / ks[c].v[0].bits);
    bool plain = false;
    const double ub = model_bound(s, cap, plain);
    bool dram_cut = false;
    std::vector<int> best = model_search(s, ub, true, dram_cut, plain ? 0 : kNodeBudget);
    // nothing found and the memory condition dropped vectors: search again without it (the reference
    // then runs in row bands)
    if (best.empty() && dram_cut) {
        bool unused = false;
        best = model_search(s, ub, false, unused, kNodeBudget);
    }
    return best;
}

// ---- the selection (moduli.hpp:719-769) -----------------------------------------------------------

// Reselect the last two moduli (moduli.hpp:365-451): fewer products, excess within the tolerance,
// fewer outputs and planes, smaller product.
void reselect_tail(std::vector<int>& m, double& logM, double need, std::uint32_t K, int cap, const Shape& S) {
    if (!(m.size() >= 2 && logM > need)) return;
    const std::vector<int> head(m.begin(), m.end() - 2);
    double base = 0.0;
    for (int x : head) base += std::log2((double)x);
    auto cop_head = [&](int mm) {
        return std::all_of(head.begin(), head.end(), [&](int x) { return std::gcd(mm, x) == 1; });
    };
    std::vector<char> use(cap + 1, 0);
    std::vector<int> np(cap + 1, 0), lay(cap + 1, 0);
    for (int mm = 3; mm <= cap; ++mm)
        if (usable(mm, S)) {
            use[mm] = 1;
            np[mm] = digit_prods(mm, S);
            lay[mm] = 1000 * nout(mm, S, maxg_for(mm, K, cap, S)) + digit_planes(mm, S);
        }
    auto ok = [&](int mm) { return mm >= 3 && mm <= cap && use[mm]; };
    double best = logM;
    int bp = m[m.size() - 2], bq = m.back();
    int bcost = np[bp] + np[bq], blay = lay[bp] + lay[bq];
    auto over = [&](double l) { return (l - need) > kTailTol ? 1 : 0; };
    auto better = [&](int c, int l2, double l) {
        if (c != bcost) return c < bcost;
        if (over(l) != over(best)) return over(l) < over(best);
        return l2 < blay || (l2 == blay && l < best);
    };
    const bool head_even = std::any_of(head.begin(), head.end(), [](int x) { return x % 2 == 0; });
    const int step = head_even ? 2 : 1;
    for (int p = 3; p <= cap; p += step) {
        if (!ok(p) || !cop_head(p)) continue;
        const double lp = base + std::log2((double)p);
        if (lp >= need && better(np[p], lay[p], lp)) {
            best = lp;
            bp = p;
            bq = 0;
            bcost = np[p];
            blay = lay[p];
        }
        for (int q = p + step; q <= cap; q += step) {
            if (!ok(q) || std::gcd(p, q) != 1 || !cop_head(q)) continue;
            const double lq = lp + std::log2((double)q);
            const int c = np[p] + np[q], l2 = lay[p] + lay[q];
            if (lq >= need && better(c, l2, lq)) {
                best = lq;
                bp = p;
                bq = q;
                bcost = c;
                blay = l2;
            }
        }
    }
    m = head;
    m.push_back(bp);
    if (bq) m.push_back(bq);
    logM = best;
}

}  // namespace

std::uint32_t default_moduli(Format format) { return format == Format::INT8 ? 16u : route_of(format).def_s; }

// The checks and the layout of a selected set (moduli.hpp:472-606): pairwise coprimality and the
// window, the exact FP32 accumulation of the digit products, the concatenation bounds and the
// composition conditions, then the carrying method, digit radix, planes and (FP8) product outputs of
// every modulus. o.m and o.b are set; o.ok is false when a condition fails. fp64_terms: the set runs
// on this build's FP8 kernel, whose epilogue reduces every output exactly in FP64 (no FP32
// composition stage): an output needs only |P_o| <= 2^24 (exact FP32 sums), without the reference's
// margin of a modulus for its FP32 composition and without its composition-sum conditions.
static void finish_set(ModuliSet& o, Format format, std::uint32_t K, const Shape& S, int num_moduli, double logM,
                       double need, bool fp64_terms = false) {
    o.log2M = logM;
    const int s = (int)o.m.size();
    o.ok = (logM >= need) && s > 0 && s <= kMaxModuli && s <= num_moduli && o.b > 0;
    for (int i = 0; i < s; ++i)
        for (int j = i + 1; j < s; ++j)
            if (std::gcd(o.m[i], o.m[j]) != 1) o.ok = false;
    auto fail = [&](const std::string& why) {
        if (o.acc_fail.empty()) o.acc_fail = why;
        o.ok = o.acc_ok = false;
    };
    // FP32 accumulation of the digit products (moduli.hpp:472-500)
    int deff = S.dmax;
    if (S.smax || S.one) {
        deff = 0;
        for (int mm : o.m)
            for (int pl = 0; pl < digit_planes(mm, S); ++pl) deff = std::max(deff, plane_bound(mm, pl, S));
    }
    if ((double)K * deff * deff > kExact24)
        fail("the digit products K*" + std::to_string(deff) + "^2 exceed the exact FP32 integers 2^24");
    if (S.one)
        for (int mm : o.m)
            if (split_mode(mm, S, true) == kSplitOne) {
                const double R = (double)resid_bound(mm);
                if ((double)K * R * R + (fp64_terms ? 0 : mm) > kExact24)
                    fail("the one-digit products of modulus " + std::to_string(mm) +
                         " exceed the exact FP32 integers 2^24");
            }
    // concatenation bounds and the composition conditions (moduli.hpp:503-578)
    int mmax = 0;
    for (int mm : o.m) mmax = std::max(mmax, mm);
    o.maxg_m.assign(s, 1);
    for (int i = 0; i < s; ++i)
        if (split_mode(o.m[i], S, true) != kSplitOne) o.maxg_m[i] = maxg_for(o.m[i], K, fp64_terms ? 0 : mmax, S);
    auto sync = [&] { o.maxg = *std::max_element(o.maxg_m.begin(), o.maxg_m.end()); };
    if (s) sync();
    auto groups = [&](int i, Group* gr) { return product_groups(o.m[i], S, o.maxg_m[i], gr); };
    auto compose_sum = [&](int i, bool fold) {
        Group gr[kMaxProd];
        const int ng = groups(i, gr);
        double sum = 0;
        for (int j = 0; j < ng; ++j)
            sum += fold ? std::fabs((double)gr[j].lo) * ((double)o.m[i] / 2.0 + 2.0)
                        : std::floor(group_bound(o.m[i], gr[j], (double)K, S) / (double)kComposeSplit + 0.5) *
                                  std::fabs((double)gr[j].hi) +
                              (double)(kComposeSplit / 2) * std::fabs((double)gr[j].lo);
        return sum;
    };
    auto gbound = [&](int i) {
        Group gr[kMaxProd];
        const int ng = groups(i, gr);
        double g = 0;
        for (int j = 0; j < ng; ++j) g = std::max(g, group_bound(o.m[i], gr[j], (double)K, S));
        return g;
    };
    if (fp64_terms) {
        for (int attempt = 0; attempt < 2 && s; ++attempt) {
            bool grouped_ok = true;
            for (int i = 0; i < s; ++i) {
                Group gr[kMaxProd];
                if (groups(i, gr) == 0) grouped_ok = false;
            }
            if (o.maxg > 1 && !grouped_ok) {
                o.maxg_m.assign(s, 1);
                sync();
                continue;
            }
            for (int i = 0; i < s; ++i) {
                Group gr[kMaxProd];
                if (groups(i, gr) == 0 || gbound(i) > kExact24)
                    fail("an output of modulus " + std::to_string(o.m[i]) + " exceeds the exact FP32 integers 2^24");
            }
            break;
        }
    }
    for (int attempt = 0; attempt < 2 && s && !fp64_terms; ++attempt) {
        bool can_fold = true, grouped_ok = true;
        for (int i = 0; i < s; ++i) {
            Group gr[kMaxProd];
            if (groups(i, gr) == 0) grouped_ok = false;
            if (gbound(i) + o.m[i] > kExact24 || compose_sum(i, true) >= kCompose22) can_fold = false;
        }
        if (o.maxg > 1 && (!can_fold || !grouped_ok)) {
            o.maxg_m.assign(s, 1);
            sync();
            continue;
        }
        o.fold_first = can_fold;
        if (!can_fold)
            for (int i = 0; i < s; ++i)
                if (compose_sum(i, false) >= kCompose22)
                    fail("the composition sum of modulus " + std::to_string(o.m[i]) + " exceeds 2^22");
        break;
    }
    // per-modulus layout (moduli.hpp:583-606); on the FP8 route also the product outputs: group
    // (a0, b0, g) pairs A digit a0+t with B digit np-1-(b0+t) (B's planes are read in reversed order)
    const bool fp8 = format == Format::FP8;
    for (int i = 0; i < s; ++i) {
        const int mm = o.m[i], np = digit_planes(mm, S);
        o.mode.push_back(split_mode(mm, S, true));
        o.q.push_back(digit_base(mm, S));
        o.nprod += digit_prods(mm, S);
        Group gr[kMaxProd];
        const int ng = groups(i, gr);
        for (int j = 0; fp8 && j < ng; ++j) {
            Fp8Output out;
            out.s = i;
            out.npairs = gr[j].g;
            for (int u = 0; u < gr[j].g; ++u) {
                out.a[u] = o.nplane + gr[j].a0 + u;
                out.b[u] = o.nplane + np - 1 - (gr[j].b0 + u);
            }
            out.coef = gr[j].lo;
            out.bound = group_bound(mm, gr[j], (double)K, S);
            o.outputs.push_back(out);
        }
        o.nplane += np;
        o.nout += ng;
    }
}

ModuliSet choose_moduli_digits(Format format, std::uint32_t M, std::uint32_t N, std::uint32_t K, int num_moduli,
                               int b_cap, double window_log2) {
    const Route& rt = route_of(format);
    ModuliSet o;
    o.digits = true;
    Shape S{rt.dmax, rt.nrdig, rt.smax, rt.one};
    int cap = rt.mod_cap;
    const double W = std::isnan(window_log2) ? std::log2((double)K) : window_log2;
    // sparse digits only while K smax^2 + the cap stays within 2^24 (moduli.hpp:724-731)
    if (S.smax && S.dmax && (double)K * S.smax * S.smax + cap > kExact24) {
        S.smax = 0;
        cap = std::min(cap, (2 * S.dmax + 1) * (2 * S.dmax + 1));
    }
    o.sparse = S.smax != 0;
    // candidate table (moduli.hpp:246-261)
    const int* tb;
    int ntb;
    if (S.n > 2) {
        tb = kTableB2;
        ntb = (int)std::size(kTableB2);
    } else if (S.smax) {
        tb = kTableF8S;
        ntb = (int)std::size(kTableF8S);
    } else if (S.dmax > 16) {
        tb = kTableB8;
        ntb = (int)std::size(kTableB8);
    } else if (S.dmax < 16) {
        tb = kTableB4;
        ntb = (int)std::size(kTableB4);
    } else {
        tb = kTableF8;
        ntb = (int)std::size(kTableF8);
    }
    // initial candidates: the model's set for the window of b_cap, else the table (moduli.hpp:267-300)
    double logM = 0.0;
    if (rt.model) {
        const double need_model = 2.0 * std::min(b_cap, kMaxDigits * kDigitBits) + 1.0 + W + kWinEps;
        o.m = model_choose(M, N, K, rt.model, cap, S, need_model, std::min(num_moduli, kMaxModuli));
        o.model_set = !o.m.empty();
        for (int mm : o.m) logM += std::log2((double)mm);
    }
    if (!o.model_set)
        for (int t = 0; t < ntb && (int)o.m.size() < num_moduli; ++t) {
            const int mm = tb[t];
            if (mm > cap || !usable(mm, S)) continue;
            o.m.push_back(mm);
            logM += std::log2((double)mm);
        }
    o.m_cap = cap;
    o.ncand = (int)o.m.size();
    // width from the window |C'| <= K 2^(2b) < M/2 (moduli.hpp:314-318)
    o.b = std::min(std::min((int)std::floor((logM - 1.0 - W - kWinEps) / 2.0), kMaxDigits * kDigitBits), b_cap);
    const double need = 2.0 * o.b + 1.0 + W + kWinEps;
    // a table set drops surplus moduli from the end and reselects its last two; a model set is kept
    if (!o.model_set) {
        while (o.m.size() > 2) {
            const double l2 = std::log2((double)o.m.back());
            if (logM - l2 < need) break;
            o.m.pop_back();
            logM -= l2;
        }
        reselect_tail(o.m, logM, need, K, cap, S);
    }
    finish_set(o, format, K, S, num_moduli, logM, need);
    return o;
}

ModuliSet choose_moduli_fp8_fewest(std::uint32_t K, int num_moduli, int b, double window_log2) {
    // The FP8 route's digit shape at this K, with moduli whose residues are e4m3 digits themselves
    // (|r| <= 16: one plane, one product) allowed.
    const Route& rt = kRouteFp8;
    Shape S{rt.dmax, rt.nrdig, rt.smax, true};
    int cap = rt.mod_cap;
    // sparse digits while their products stay exact FP32 integers (the reference also keeps room for a
    // modulus, for its FP32 composition, which this build's FP64 epilogue does not need: K = 16384 keeps
    // them)
    if (S.smax && S.dmax && (double)K * S.smax * S.smax > kExact24) {
        S.smax = 0;
        cap = std::min(cap, (2 * S.dmax + 1) * (2 * S.dmax + 1));
    }
    const double need = 2.0 * b + 1.0 + window_log2 + kWinEps;
    struct Cand {
        int m, prods;
        double bits;
        int np, pf[4];  // distinct prime factors
    };
    struct Cands {
        std::vector<Cand> one, multi;
    };
    // The candidates depend only on the digit shape, which is one of two (sparse digits or not): built
    // once each. One-digit moduli: the largest one-digit power of each small prime; the others in
    // order of bits per product.
    auto build = [](const Shape& Sh, int cp) {
        Cands c;
        for (int m = cp; m >= 2; --m) {
            if (!usable(m, Sh)) continue;
            Cand x{m, digit_prods(m, Sh), std::log2((double)m), 0, {0, 0, 0, 0}};
            x.np = distinct_primes(m, x.pf);
            if (split_mode(m, Sh, true) != kSplitOne) {
                c.multi.push_back(x);
                continue;
            }
            if (x.np != 1) continue;
            bool largest = true;  // no larger one-digit power of the same prime
            for (const Cand& y : c.one) largest = largest && y.pf[0] != x.pf[0];
            if (largest) c.one.push_back(x);
        }
        std::stable_sort(c.multi.begin(), c.multi.end(),
                         [](const Cand& x, const Cand& y) { return x.bits / x.prods > y.bits / y.prods; });
        return c;
    };
    static const Cands sparse_cands = build(Shape{rt.dmax, rt.nrdig, rt.smax, true}, rt.mod_cap);
    static const Cands dense_cands =
        build(Shape{rt.dmax, rt.nrdig, 0, true}, std::min(rt.mod_cap, (2 * rt.dmax + 1) * (2 * rt.dmax + 1)));
    const Cands& cands = S.smax ? sparse_cands : dense_cands;
    const std::vector<Cand>&one = cands.one, &multi = cands.multi;
    // every subset of the one-digit moduli, filled up to the window with the others in that order;
    // the sets in order of fewest products, then fewest moduli, then widest
    struct Sol {
        int prods;
        double bits;
        std::vector<int> m;
    };
    std::vector<Sol> sols;
    const int n1 = (int)one.size();
    std::vector<char> used(4097, 0);  // primes taken by the set being filled
    for (unsigned mask = 0; mask < (1u << n1); ++mask) {
        Sol x{0, 0.0, {}};
        std::vector<int> taken;
        auto take = [&](const Cand& c) {
            x.m.push_back(c.m);
            x.prods += c.prods;
            x.bits += c.bits;
            for (int t = 0; t < c.np; ++t) {
                used[c.pf[t]] = 1;
                taken.push_back(c.pf[t]);
            }
        };
        for (int i = 0; i < n1; ++i)
            if (mask >> i & 1) take(one[i]);
        for (const Cand& c : multi) {
            if (x.bits >= need || (int)x.m.size() >= std::min(num_moduli, kMaxModuli)) break;
            bool cop = true;
            for (int t = 0; t < c.np; ++t) cop = cop && !used[c.pf[t]];
            if (cop) take(c);
        }
        for (int q : taken) used[q] = 0;
        if (x.bits >= need) sols.push_back(std::move(x));
    }
    std::stable_sort(sols.begin(), sols.end(), [](const Sol& x, const Sol& y) {
        if (x.prods != y.prods) return x.prods < y.prods;
        if (x.m.size() != y.m.size()) return x.m.size() < y.m.size();
        return x.bits > y.bits;
    });
    ModuliSet best;
    for (std::size_t t = 0; t < sols.size() && t < 64; ++t) {
        ModuliSet o;
        o.digits = true;
        o.sparse = S.smax != 0;
        o.m = sols[t].m;
        std::sort(o.m.begin(), o.m.end(), std::greater<int>());
        o.m_cap = cap;
        o.ncand = (int)(one.size() + multi.size());
        o.b = b;
        double logM = 0.0;
        for (int mm : o.m) logM += std::log2((double)mm);
        finish_set(o, Format::FP8, K, S, num_moduli, logM, need, true);
        if (o.ok && o.nplane <= OZ2_MAXPLANES && o.nout <= OZ2_MAXOUT) return o;
        if (t == 0) best = std::move(o);
    }
    return best;
}

}  // namespace ozTTgemm::detail

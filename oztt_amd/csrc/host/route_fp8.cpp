// Scheme II moduli selection on the FP8 (e4m3) route; see plan2.hpp.
//
// Restates the reference's FP8 path (src/backend/ozaki2/split.hpp:72-76 OZ2_ROUTE_FP8 and the
// per-modulus carrying rules :176-728; moduli.hpp:184-197 tables, :225-845 selection): residues
// modulo m <= 2401 are carried as two e4m3 digits (|digit| <= 16, or the sparse set of exactly
// representable integers up to 32 while K*32^2 + 2401 <= 2^24), three or four digit products per
// modulus. The selected set and width b define the FP8 result, so the rules, tables and
// floating-point comparisons are kept. Compiled with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <string>
#include <vector>

#include "plan2.hpp"

namespace ozTTgemm::detail {
namespace {

constexpr int kDigitMax = 16;   // dense digit bound of e4m3 (OZ2_ROUTE_FP8.digit_bound)
constexpr int kSparseMax = 32;  // sparse digit bound (OZ2_ROUTE_FP8.sparse_max)
constexpr int kModCap = 2401;   // OZ2_ROUTE_FP8.mod_cap
constexpr double kWinEps = 1e-9, kTailTol = 0.25;
constexpr double kExact24 = 16777216.0, kCompose22 = 4194304.0;
constexpr long kComposeSplit = 4096;  // OZ2_COMPOSE_SPLIT = 2^12

// Candidate tables: dense digits (the FP8 table of GEMMul8) and sparse squares (moduli.hpp:188-197).
constexpr int kTableF8[] = {1089, 1024, 961, 841, 625, 529, 511, 509, 503, 499,
                            491,  487,  481, 479, 467, 463, 461, 457, 449, 443};
constexpr int kTableF8S[] = {2401, 2209, 1849, 1681, 1521, 1369, 1024, 961, 841, 625, 529, 361,
                             289,  121,  509,  503,  499,  491,  487,  479, 467, 463, 461, 457};

// e4m3 represents the integer v exactly (at most 4 significant bits).
bool e4m3_int(long v) {
    if (v < 0) v = -v;
    if (v == 0) return true;
    int e = 0;
    for (long x = v; x; x >>= 1) ++e;
    return e <= 4 || (v % (1L << (e - 4))) == 0;
}
bool in_sparse(long x, int smax) { return (x < 0 ? -x : x) <= smax && e4m3_int(x); }

// the sparse digit set covers every residue class modulo q
bool sparse_covers(int q, int smax) {
    if (q <= 0 || smax <= 0 || q > 2 * smax + 1) return false;
    std::vector<char> hit(q, 0);
    int n = 0;
    for (int x = -smax; x <= smax; ++x)
        if (in_sparse(x, smax)) {
            const int r = ((x % q) + q) % q;
            if (!hit[r]) {
                hit[r] = 1;
                ++n;
            }
        }
    return n == q;
}

// the sparse-digit split of a residue modulo q^2 (q odd), split.hpp:266-279
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
// largest |l| and |h| over |r| <= floor(q^2/2)+1
void sqs_bounds(int q, int& dl, int& dh) {
    const long m = (long)q * q, R = m / 2 + 1;
    dl = dh = 0;
    for (long r = -R; r <= R; ++r) {
        long l, h;
        sqs_split(r, q, l, h);
        dl = std::max<int>(dl, (int)(l < 0 ? -l : l));
        dh = std::max<int>(dh, (int)(h < 0 ? -h : h));
    }
}

int isqrt(int m) {
    int r = (int)std::sqrt((double)m);
    while ((long)(r + 1) * (r + 1) <= m) ++r;
    while ((long)r * r > m) --r;
    return r;
}
int is_square(int m) {
    const int r = isqrt(m);
    return ((long)r * r == m) ? r : 0;
}
// digit bound of balanced digits with radix q by rounding to nearest
int digit_bound_rnd(int m, int q) {
    const int rs = m / 2, h = (rs + q / 2) / q;
    return std::max(h, q / 2);
}
// digit bound of radix-16 Karatsuba
int digit_bound_kar(int m) { return std::max((m / 2 + 15) / 16, 15); }
int digit_base_rnd(int m) {
    const int r = isqrt(m);
    int best = r + 1, bb = digit_bound_rnd(m, r + 1);
    for (int qq = r; qq <= r + 3; ++qq) {
        const int v = digit_bound_rnd(m, qq);
        if (v < bb) {
            bb = v;
            best = qq;
        }
    }
    return best;
}

// carrying method of modulus m on the FP8 route (split.hpp:407-429 with d = 16, two digits)
int split_mode(int m, int smax) {
    if (const int q = is_square(m)) {
        if (smax && digit_bound_rnd(m, q) > kDigitMax && (q & 1) && sparse_covers(q, smax)) return kFp8SplitSqs;
        return kFp8SplitSq;
    }
    if (digit_bound_kar(m) <= kDigitMax) return kFp8SplitKar;
    return kFp8SplitWide;
}
int digit_base(int m, int smax) {
    const int mode = split_mode(m, smax);
    if (mode == kFp8SplitSq || mode == kFp8SplitSqs) return is_square(m);
    return mode == kFp8SplitKar ? 16 : digit_base_rnd(m);
}
int digit_bound(int m, int smax) {
    const int mode = split_mode(m, smax);
    if (mode == kFp8SplitKar) return digit_bound_kar(m);
    return digit_bound_rnd(m, digit_base(m, smax));
}
bool usable(int m, int smax) { return split_mode(m, smax) == kFp8SplitSqs || digit_bound(m, smax) <= kDigitMax; }
int planes(int m, int smax) { return split_mode(m, smax) == kFp8SplitKar ? 3 : 2; }
// bound on |digit| of plane 0 (l) or 1 (h) (split.hpp:482-501)
int plane_bound(int m, int plane, int smax) {
    if (!smax) return kDigitMax;
    if (split_mode(m, smax) == kFp8SplitSqs) {
        int dl, dh;
        sqs_bounds(is_square(m), dl, dh);
        return plane == 0 ? dl : dh;
    }
    return digit_bound(m, smax);
}

struct Term {
    int a, b;
    long lo, hi;  // coefficient and its 2^12 multiple, both in [0, m)
};
// digit products and their coefficients (split.hpp:541-597)
int product_terms(int m, int smax, Term* t) {
    auto rm = [&](long v) {
        const long r = v % m;
        return r < 0 ? r + m : r;
    };
    const int mode = split_mode(m, smax), q = digit_base(m, smax);
    int k = 0;
    if (mode == kFp8SplitKar) {
        const long B = q, c[3] = {rm(1 - B), rm(B * B - B), rm(B)};
        for (int j = 0; j < 3; ++j) t[k++] = {j, j, c[j], rm(c[j] * kComposeSplit)};
        return k;
    }
    const long c[4] = {rm(1), rm(q), rm(q), rm((long)q * q)};
    const int pa[4] = {0, 1, 0, 1}, pb[4] = {0, 0, 1, 1};
    const int n = mode == kFp8SplitWide ? 4 : 3;
    for (int j = 0; j < n; ++j) t[k++] = {pa[j], pb[j], c[j], rm(c[j] * kComposeSplit)};
    return k;
}
struct Group {
    int a0, b0, g;
    long lo, hi;
};
// products of equal weight concatenated along K in runs of at most maxg (split.hpp:628-661)
int product_groups(int m, int smax, int maxg, Group* gr) {
    Term t[4];
    const int n = product_terms(m, smax, t), np = planes(m, smax);
    int k = 0;
    for (int key = 0; key <= 2 * (np - 1); ++key) {
        int as[4], na = 0;
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
double group_bound(int m, const Group& g, double K, int smax) {
    const int np = planes(m, smax);
    double sb = 0;
    for (int t = 0; t < g.g; ++t) sb += K * plane_bound(m, g.a0 + t, smax) * plane_bound(m, np - 1 - (g.b0 + t), smax);
    return sb;
}
// concatenation bound: g K d_l d_h + cap <= 2^24 (split.hpp:684-690)
int maxg_for(int m, std::uint32_t K, int cap, int smax) {
    const double pb = (double)plane_bound(m, 0, smax) * plane_bound(m, std::min(1, planes(m, smax) - 1), smax);
    return std::max(1, (int)std::floor((kExact24 - cap) / ((double)K * pb)));
}

}  // namespace

ModuliSet choose_moduli_fp8(std::uint32_t K, int num_moduli, int b_cap, double window_log2) {
    ModuliSet o;
    o.fp8 = true;
    int mod_cap = kModCap, smax = kSparseMax;
    const double W = std::isnan(window_log2) ? std::log2((double)K) : window_log2;
    // sparse digits only while K*32^2 + the cap stays within 2^24 (moduli.hpp:724-731)
    if ((double)K * smax * smax + mod_cap > kExact24) {
        smax = 0;
        mod_cap = std::min(mod_cap, (2 * kDigitMax + 1) * (2 * kDigitMax + 1));
    }
    o.sparse = smax != 0;
    const int m_cap = mod_cap;
    double logM = 0.0;
    const int* tb = smax ? kTableF8S : kTableF8;
    const int ntb = smax ? (int)std::size(kTableF8S) : (int)std::size(kTableF8);
    for (int t = 0; t < ntb; ++t) {
        const int mm = tb[t];
        if ((int)o.m.size() >= num_moduli) break;
        if (mm > m_cap || !usable(mm, smax)) continue;
        o.m.push_back(mm);
        logM += std::log2((double)mm);
    }
    o.m_cap = m_cap;
    o.ncand = (int)o.m.size();
    const double room = logM - 1.0 - W - kWinEps;
    o.b = std::min(std::min((int)std::floor(room / 2.0), kMaxDigits * kDigitBits), b_cap);
    const double need = 2.0 * o.b + 1.0 + W + kWinEps;
    // trim the tail (moduli.hpp:347-355)
    while (o.m.size() > 2) {
        const double l2 = std::log2((double)o.m.back());
        if (logM - l2 < need) break;
        o.m.pop_back();
        logM -= l2;
    }
    // reselect the last two (moduli.hpp:365-451): fewer products, excess within tolerance, fewer
    // outputs and planes, smaller product
    if (o.m.size() >= 2 && logM > need) {
        const std::vector<int> head(o.m.begin(), o.m.end() - 2);
        double base = 0.0;
        for (int x : head) base += std::log2((double)x);
        auto cop_head = [&](int mm) {
            for (int x : head)
                if (std::gcd(mm, x) != 1) return false;
            return true;
        };
        std::vector<char> use_c(m_cap + 1, 0);
        std::vector<int> np_c(m_cap + 1, 0), lay_c(m_cap + 1, 0);
        for (int mm = 3; mm <= m_cap; ++mm)
            if (usable(mm, smax)) {
                Term t[4];
                Group gr[4];
                use_c[mm] = 1;
                np_c[mm] = product_terms(mm, smax, t);
                lay_c[mm] = 1000 * product_groups(mm, smax, maxg_for(mm, K, m_cap, smax), gr) + planes(mm, smax);
            }
        auto usable_c = [&](int mm) { return mm >= 3 && mm <= m_cap && use_c[mm]; };
        double best = logM;
        int bp = o.m[o.m.size() - 2], bq = o.m.back();
        int bcost = np_c[bp] + np_c[bq], blay = lay_c[bp] + lay_c[bq];
        auto over = [&](double l) { return (l - need) > kTailTol ? 1 : 0; };
        auto better = [&](int c, int lay, double l) {
            if (c != bcost) return c < bcost;
            if (over(l) != over(best)) return over(l) < over(best);
            return lay < blay || (lay == blay && l < best);
        };
        bool head_even = false;
        for (int x : head) head_even = head_even || (x % 2 == 0);
        const int step = head_even ? 2 : 1;
        for (int p2 = 3; p2 <= m_cap; p2 += step) {
            if (!usable_c(p2) || !cop_head(p2)) continue;
            const double lp = base + std::log2((double)p2);
            if (lp >= need && better(np_c[p2], lay_c[p2], lp)) {
                best = lp;
                bp = p2;
                bq = 0;
                bcost = np_c[p2];
                blay = lay_c[p2];
            }
            for (int q = p2 + step; q <= m_cap; q += step) {
                if (!usable_c(q) || std::gcd(p2, q) != 1 || !cop_head(q)) continue;
                const double lq = lp + std::log2((double)q);
                const int c = np_c[p2] + np_c[q], lay = lay_c[p2] + lay_c[q];
                if (lq >= need && better(c, lay, lq)) {
                    best = lq;
                    bp = p2;
                    bq = q;
                    bcost = c;
                    blay = lay;
                }
            }
        }
        o.m = head;
        o.m.push_back(bp);
        if (bq) o.m.push_back(bq);
        logM = best;
    }
    o.log2M = logM;
    const int s = (int)o.m.size();
    o.ok = (logM >= need) && s > 0 && s <= kMaxModuli && s <= num_moduli && o.b > 0;
    for (int i = 0; i < s; ++i)
        for (int j = i + 1; j < s; ++j)
            if (std::gcd(o.m[i], o.m[j]) != 1) o.ok = false;
    // accumulation of the digit products in FP32 (moduli.hpp:472-500)
    int deff = kDigitMax;
    if (smax) {
        deff = 0;
        for (int mm : o.m)
            for (int pl = 0; pl < planes(mm, smax); ++pl) deff = std::max(deff, plane_bound(mm, pl, smax));
    }
    if ((double)K * deff * deff > kExact24) {
        o.acc_fail = "the digit products K*" + std::to_string(deff) + "^2 exceed the exact FP32 integers 2^24";
        o.ok = o.acc_ok = false;
    }
    // concatenation bounds and the composition conditions (moduli.hpp:503-578)
    int mmax = 0;
    for (int mm : o.m) mmax = std::max(mmax, mm);
    o.maxg_m.assign(s, 1);
    for (int i = 0; i < s; ++i) o.maxg_m[i] = maxg_for(o.m[i], K, mmax, smax);
    auto sync = [&] {
        o.maxg = 1;
        for (int g : o.maxg_m) o.maxg = std::max(o.maxg, g);
    };
    sync();
    auto compose_sum = [&](int i, bool fold) {
        Group gr[4];
        const int ng = product_groups(o.m[i], smax, o.maxg_m[i], gr);
        double sum = 0;
        for (int j = 0; j < ng; ++j)
            sum += fold ? std::fabs((double)gr[j].lo) * ((double)o.m[i] / 2.0 + 2.0)
                        : std::floor(group_bound(o.m[i], gr[j], (double)K, smax) / (double)kComposeSplit + 0.5) *
                                  std::fabs((double)gr[j].hi) +
                              (double)(kComposeSplit / 2) * std::fabs((double)gr[j].lo);
        return sum;
    };
    auto gbound_of = [&](int i) {
        Group gr[4];
        const int ng = product_groups(o.m[i], smax, o.maxg_m[i], gr);
        double g = 0;
        for (int j = 0; j < ng; ++j) g = std::max(g, group_bound(o.m[i], gr[j], (double)K, smax));
        return g;
    };
    for (int attempt = 0; attempt < 2; ++attempt) {
        bool can_fold = true, grouped_ok = true;
        for (int i = 0; i < s; ++i) {
            Group gr[4];
            if (product_groups(o.m[i], smax, o.maxg_m[i], gr) == 0) grouped_ok = false;
            if (gbound_of(i) + o.m[i] > kExact24 || compose_sum(i, true) >= kCompose22) can_fold = false;
        }
        if (o.maxg > 1 && (!can_fold || !grouped_ok)) {
            o.maxg_m.assign(s, 1);
            sync();
            continue;
        }
        o.fold_first = can_fold;
        if (!can_fold)
            for (int i = 0; i < s; ++i)
                if (compose_sum(i, false) >= kCompose22) {
                    if (o.acc_fail.empty())
                        o.acc_fail = "the composition sum of modulus " + std::to_string(o.m[i]) + " exceeds 2^22";
                    o.ok = o.acc_ok = false;
                }
        break;
    }
    // per-modulus layout (moduli.hpp:583-606) and the product outputs: group (a0, b0, g) pairs A digit
    // a0+t with B digit np-1-(b0+t) (the B planes are read in reversed order, LAYOUT_B_PERM)
    o.nprod = o.nplane = o.nout = 0;
    for (int i = 0; i < s; ++i) {
        Term t[4];
        Group gr[4];
        const int np = planes(o.m[i], smax);
        o.mode.push_back(split_mode(o.m[i], smax));
        o.q.push_back(digit_base(o.m[i], smax));
        o.nprod += product_terms(o.m[i], smax, t);
        const int ng = product_groups(o.m[i], smax, o.maxg_m[i], gr);
        for (int j = 0; j < ng; ++j) {
            Fp8Output out;
            out.s = i;
            out.npairs = gr[j].g;
            for (int u = 0; u < gr[j].g; ++u) {
                out.a[u] = o.nplane + gr[j].a0 + u;
                out.b[u] = o.nplane + np - 1 - (gr[j].b0 + u);
            }
            out.coef = gr[j].lo;
            out.bound = group_bound(o.m[i], gr[j], (double)K, smax);
            o.outputs.push_back(out);
        }
        o.nplane += np;
        o.nout += ng;
    }
    return o;
}

}  // namespace ozTTgemm::detail

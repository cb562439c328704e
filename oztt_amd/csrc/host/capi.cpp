// C entry points of libozTTgemm.so for callers without C++ (the Python mirror in oztt_amd/, the
// tests and bench.py): the public Context API, the evaluation hooks and utilities, and a view of
// the Scheme II planner. Each function returns 0 on success or one of the OZT_E* codes, mapping the
// C++ exception types of the public API, and copies the exception's message into err.
#include <cstring>
#include <limits>
#include <new>
#include <optional>
#include <stdexcept>

#include <ozTTgemm/ozTTgemm.hpp>

#include "evaluation.hpp"
#include "plan1.hpp"
#include "plan2.hpp"

namespace {
enum { OZT_OK = 0, OZT_EINVAL = 1, OZT_ERUNTIME = 2, OZT_ENOMEM = 3, OZT_EOTHER = 4 };

void put(char* err, std::size_t len, const char* msg) {
    if (err && len) {
        std::strncpy(err, msg, len - 1);
        err[len - 1] = 0;
    }
}

template <class F>
int guarded(char* err, std::size_t len, F&& f) {
    try {
        f();
        return OZT_OK;
    } catch (const std::invalid_argument& e) {
        put(err, len, e.what());
        return OZT_EINVAL;
    } catch (const std::bad_alloc& e) {
        put(err, len, e.what());
        return OZT_ENOMEM;
    } catch (const std::runtime_error& e) {
        put(err, len, e.what());
        return OZT_ERUNTIME;
    } catch (const std::exception& e) {
        put(err, len, e.what());
        return OZT_EOTHER;
    }
}

ozTTgemm::Options make_options(int scheme, int format, unsigned slices, unsigned max_moduli, int recon, int transport) {
    ozTTgemm::Options o;
    o.scheme = static_cast<ozTTgemm::Scheme>(scheme);
    o.format = static_cast<ozTTgemm::Format>(format);
    o.slices = slices;
    o.max_moduli = max_moduli;
    o.reconstruction = static_cast<ozTTgemm::Reconstruction>(recon);
    o.transport = static_cast<ozTTgemm::Transport>(transport);
    return o;
}
}  // namespace

extern "C" {

struct ozt_info {
    int scheme, format;
    unsigned slices, moduli, integer_bits, reconstruction_passes;
    unsigned long long padded_m, padded_n, padded_k;
};

struct ozt_eval {
    unsigned fixed_bits;
    int warmup, repeats;
    double phase_ms[5];
    double whole_ms;
    int whole_checked;
    unsigned partial_products;
    double product_ops;
    double gemm_launch_ms;
    int gemm_launches;
    unsigned max_band_rows;  // input: cap on the rows of a band (0: bands only when memory requires)
    int plan_reused;         // resident operands: the plan kept from an earlier call was used
    unsigned force_kc;       // input: Scheme I block-by-block reconstruction with this K block (0: as planned)
    int replay_drop_phase;   // input: self-test of the whole-pass check (-1: off)
    int whole_sentinel;      // the checking replay rewrote the sentinel-filled output with the first pass's bits
    unsigned whole_steps[5];     // steps per phase issued by the checking replay
    unsigned expected_steps[5];  // steps per phase the plan calls for
    int fp8_matrix_cores;        // input: Scheme II FP8 on the FP8 matrix cores also under Transport::Int8Residues
    int full_window;             // input: Scheme II INT8 residues with the set for the window K 2^(2b)
};

struct ozt_plan2 {
    int ok, b, S, nd, two_pass, m_cap;
    int m[24];
    double log2M, recon1_log2;
    double TA, TB, nA, nB, nC, wA, wB;
    int b_cap;
    // the route's plan (FP8: the reference's FP8 moduli; INT8: as above)
    int rS, rsparse, rfold_first, rmaxg, rnprod, rnplane, rnout;
    int rm[24], rmode[24], rmaxg_m[24];
    double rlog2M;
    int fp8_digits;  // the device computes the FP8 route's e4m3 digit products (else the residues of m[])
    int rmodel_set;  // the route's set was chosen by the stage-time model (not from the table)
    double bound_log2;  // log2 of the operands' bound on max |C'| (+inf when not measured)
    int S_window;       // moduli of the set for the window K 2^(2b) that m[] replaced (0: none)
    int nprod;          // products the device computes: S, or the FP8 route's digit products
    int nplane;         // digit planes per operand on the FP8 route (0 for INT8 residues)
};

static void fill_route(const ozTTgemm::detail::ModuliSet& r, ozt_plan2* out) {
    out->rS = (int)r.m.size();
    out->rsparse = r.sparse;
    out->rfold_first = r.fold_first;
    out->rmaxg = r.maxg;
    out->rnprod = r.nprod;
    out->rnplane = r.nplane;
    out->rnout = r.nout;
    for (int s = 0; s < out->rS && s < 24; s++) {
        out->rm[s] = r.m[s];
        out->rmode[s] = s < (int)r.mode.size() ? r.mode[s] : 0;
        out->rmaxg_m[s] = s < (int)r.maxg_m.size() ? r.maxg_m[s] : 1;
    }
    out->rlog2M = r.log2M;
    out->rmodel_set = r.model_set;
}

int ozt_context_new(int device_id, const char* kernel_dir, void** out, char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        ozTTgemm::DeviceOptions d;
        d.device_id = device_id;
        if (kernel_dir) d.kernel_directory = kernel_dir;
        *out = new ozTTgemm::Context(d);
    });
}

void ozt_context_free(void* ctx) { delete static_cast<ozTTgemm::Context*>(ctx); }

static void fill_info(const ozTTgemm::Info& i, ozt_info* o) {
    if (!o) return;
    o->scheme = (int)i.scheme;
    o->format = (int)i.format;
    o->slices = i.slices;
    o->moduli = i.moduli;
    o->integer_bits = i.integer_bits;
    o->reconstruction_passes = i.reconstruction_passes;
    o->padded_m = i.padded_m;
    o->padded_n = i.padded_n;
    o->padded_k = i.padded_k;
}

int ozt_gemm(void* ctx, const double* a, std::size_t na, const double* b, std::size_t nb, double* c, std::size_t nc,
             std::size_t m, std::size_t n, std::size_t k, int scheme, int format, unsigned slices, unsigned max_moduli,
             int recon, int transport, ozt_info* info, char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        auto* cx = static_cast<ozTTgemm::Context*>(ctx);
        const auto i = cx->gemm({a, na}, {b, nb}, {c, nc}, m, n, k, make_options(scheme, format, slices, max_moduli, recon, transport));
        fill_info(i, info);
    });
}

// ---- resident operands (ozTTgemm::Matrix) -----------------------------------------------------
void* ozt_matrix_new() { return new (std::nothrow) ozTTgemm::Matrix(); }
void ozt_matrix_free(void* m) { delete static_cast<ozTTgemm::Matrix*>(m); }
void ozt_matrix_dims(void* m, std::size_t* rows, std::size_t* cols) {
    const auto* x = static_cast<const ozTTgemm::Matrix*>(m);
    *rows = x->rows();
    *cols = x->cols();
}

int ozt_upload(void* ctx, const double* x, std::size_t n, std::size_t rows, std::size_t cols, void* m, char* err,
               std::size_t errlen) {
    return guarded(err, errlen, [&] {
        *static_cast<ozTTgemm::Matrix*>(m) = static_cast<ozTTgemm::Context*>(ctx)->upload({x, n}, rows, cols);
    });
}

int ozt_download(void* ctx, void* m, double* out, std::size_t n, char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        static_cast<ozTTgemm::Context*>(ctx)->download(*static_cast<const ozTTgemm::Matrix*>(m), {out, n});
    });
}

static void fill_eval(const ozTTgemm::evaluation::Settings& s, ozt_eval* evo);

// C = A B for resident A and B: into the host array c (nc elements) when cm is null, else into the
// Matrix cm. evo, when not null, runs the call under the evaluation hooks.
// The evaluation settings a caller passed in (the inputs of ozt_eval).
static ozTTgemm::evaluation::Settings settings_of(const ozt_eval* evo) {
    ozTTgemm::evaluation::Settings s;
    s.fixed_bits = evo->fixed_bits;
    s.warmup = evo->warmup;
    s.repeats = evo->repeats;
    s.max_band_rows = evo->max_band_rows;
    s.force_kc = evo->force_kc;
    s.replay_drop_phase = evo->replay_drop_phase;
    s.fp8_matrix_cores = evo->fp8_matrix_cores != 0;
    s.full_window = evo->full_window != 0;
    return s;
}

int ozt_gemm_resident(void* ctx, void* a, void* b, double* c, std::size_t nc, void* cm, int scheme, int format,
                      unsigned slices, unsigned max_moduli, int recon, int transport, ozt_info* info, ozt_eval* evo,
                      char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        auto* cx = static_cast<ozTTgemm::Context*>(ctx);
        const auto& A = *static_cast<const ozTTgemm::Matrix*>(a);
        const auto& B = *static_cast<const ozTTgemm::Matrix*>(b);
        const auto o = make_options(scheme, format, slices, max_moduli, recon, transport);
        auto run = [&] {
            return cm ? cx->gemm(A, B, *static_cast<ozTTgemm::Matrix*>(cm), o) : cx->gemm(A, B, {c, nc}, o);
        };
        ozTTgemm::Info i;
        if (evo) {
            ozTTgemm::evaluation::Settings s = settings_of(evo);
            {
                ozTTgemm::evaluation::Scope scope(s);
                i = run();
            }
            fill_eval(s, evo);
        } else {
            i = run();
        }
        fill_info(i, info);
    });
}

int ozt_eval_gemm(void* ctx, const double* a, std::size_t na, const double* b, std::size_t nb, double* c,
                  std::size_t nc, std::size_t m, std::size_t n, std::size_t k, int scheme, int format, unsigned slices,
                  unsigned max_moduli, int recon, int transport, ozt_info* info, ozt_eval* evo, char* err,
                  std::size_t errlen) {
    return guarded(err, errlen, [&] {
        ozTTgemm::evaluation::Settings s = settings_of(evo);
        auto* cx = static_cast<ozTTgemm::Context*>(ctx);
        ozTTgemm::Info i;
        {
            ozTTgemm::evaluation::Scope scope(s);
            i = cx->gemm({a, na}, {b, nb}, {c, nc}, m, n, k, make_options(scheme, format, slices, max_moduli, recon, transport));
        }
        fill_info(i, info);
        fill_eval(s, evo);
    });
}

static void fill_eval(const ozTTgemm::evaluation::Settings& s, ozt_eval* evo) {
    for (int p = 0; p < 5; p++) evo->phase_ms[p] = s.phase_ms[p];
    evo->whole_ms = s.whole_ms;
    evo->whole_checked = s.whole_checked ? 1 : 0;
    evo->partial_products = s.partial_products;
    evo->product_ops = s.product_ops;
    evo->gemm_launch_ms = s.gemm_launch_ms;
    evo->gemm_launches = s.gemm_launches;
    evo->plan_reused = s.plan_reused ? 1 : 0;
    evo->whole_sentinel = s.whole_sentinel ? 1 : 0;
    for (int p = 0; p < 5; p++) {
        evo->whole_steps[p] = s.whole_steps[p];
        evo->expected_steps[p] = s.expected_steps[p];
    }
}

int ozt_is_available(int format) { return ozTTgemm::is_available(static_cast<ozTTgemm::Format>(format)) ? 1 : 0; }
const char* ozt_format_name(int format) { return ozTTgemm::format_name(static_cast<ozTTgemm::Format>(format)); }

// Scheme II planner on padded row-major A (M x K) and B (K x N) for `format`; int8_transport: the plan
// of Transport::Int8Residues.
int ozt_plan_scheme2(const double* A, const double* B, unsigned M, unsigned N, unsigned K, int format, unsigned max_moduli,
              int recon, unsigned fixed_b, int int8_transport, int full_window, ozt_plan2* out, char* err,
              std::size_t errlen) {
    return guarded(err, errlen, [&] {
        std::optional<unsigned> fb;
        if (fixed_b) fb = fixed_b;
        const auto p = ozTTgemm::detail::plan_scheme2(A, B, M, N, K, static_cast<ozTTgemm::Format>(format), max_moduli,
                                                        static_cast<ozTTgemm::Reconstruction>(recon), fb,
                                                        int8_transport != 0, full_window == 0);
        std::memset(out, 0, sizeof(*out));
        out->fp8_digits = p.fp8_digits;
        out->ok = p.mo.ok;
        out->b = p.b;
        out->S = p.S;
        out->nd = p.nd;
        out->two_pass = p.two_pass;
        out->m_cap = p.mo.m_cap;
        for (int s = 0; s < p.S && s < 24; s++) out->m[s] = p.mo.m[s];
        out->log2M = p.mo.log2M;
        out->recon1_log2 = p.recon1_log2;
        out->TA = p.stats.TA;
        out->TB = p.stats.TB;
        out->nA = p.stats.nA;
        out->nB = p.stats.nB;
        out->nC = p.stats.nC;
        out->wA = p.stats.wA;
        out->wB = p.stats.wB;
        out->b_cap = p.stats.measured ? ozTTgemm::detail::precision_cap(p.stats) : 0;
        out->bound_log2 = p.bound_log2;
        out->S_window = p.S_window;
        out->nprod = p.fp8_digits ? p.mo.nprod : p.S;
        out->nplane = p.fp8_digits ? p.mo.nplane : 0;
        fill_route(p.route, out);
    });
}

// The device descriptors of a Scheme II FP8 plan on the FP8 matrix cores (digit split, product outputs,
// CRT, term moduli): for the route's own set (the window K 2^(2b), as the reference plans it), or with
// execution_set for the set the public call computes with (the operands' window, fewest products).
int ozt_plan2_fp8_device(const double* A, const double* B, unsigned M, unsigned N, unsigned K, unsigned max_moduli,
                         int recon, unsigned fixed_b, int execution_set, oz2_digit_dev* dd, oz2_groups_dev* gd,
                         oz2_crt_dev* crt, unsigned char* term_modulus, char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        std::optional<unsigned> fb;
        if (fixed_b) fb = fixed_b;
        const auto p = ozTTgemm::detail::plan_scheme2(A, B, M, N, K, ozTTgemm::Format::FP8, max_moduli,
                                                        static_cast<ozTTgemm::Reconstruction>(recon), fb, false,
                                                        execution_set != 0);
        if (!p.fp8_digits) throw std::runtime_error("the FP8 plan does not run on FP8 digits");
        *crt = ozTTgemm::detail::crt_descriptor(p);
        *dd = ozTTgemm::detail::digit_descriptor(p);
        std::vector<unsigned char> tm;
        *gd = ozTTgemm::detail::groups_descriptor(p, *crt, tm);
        std::memcpy(term_modulus, tm.data(), tm.size());
    });
}

// Moduli selection alone on the digit route of `format` (not INT8; no input statistics); M and N feed
// the stage-time model's memory estimate; window_log2 <= 0 selects log2 K.
int ozt_choose_moduli_route(int format, unsigned M, unsigned N, unsigned K, int num_moduli, int b_cap,
                            double window_log2, ozt_plan2* out, char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        const auto mo = ozTTgemm::detail::choose_moduli_digits(
            static_cast<ozTTgemm::Format>(format), M, N, K, num_moduli, b_cap,
            window_log2 > 0 ? window_log2 : std::numeric_limits<double>::quiet_NaN());
        std::memset(out, 0, sizeof(*out));
        out->ok = mo.ok;
        out->b = mo.b;
        out->S = (int)mo.m.size();
        out->m_cap = mo.m_cap;
        for (int s = 0; s < out->S && s < 24; s++) out->m[s] = mo.m[s];
        out->log2M = mo.log2M;
        fill_route(mo, out);
    });
}

// FP8-route moduli selection alone (no input statistics); window_log2 <= 0 selects log2 K.
int ozt_choose_moduli_fp8(unsigned K, int num_moduli, int b_cap, double window_log2, ozt_plan2* out) {
    const auto mo = ozTTgemm::detail::choose_moduli_digits(
        ozTTgemm::Format::FP8, K, K, K, num_moduli, b_cap,
        window_log2 > 0 ? window_log2 : std::numeric_limits<double>::quiet_NaN());
    std::memset(out, 0, sizeof(*out));
    out->ok = mo.ok;
    out->b = mo.b;
    out->S = (int)mo.m.size();
    out->m_cap = mo.m_cap;
    for (int s = 0; s < out->S && s < 24; s++) out->m[s] = mo.m[s];
    out->log2M = mo.log2M;
    fill_route(mo, out);
    return 0;
}

// Moduli selection alone (no input statistics).
int ozt_choose_moduli_int8(unsigned K, int num_moduli, int b_cap, ozt_plan2* out) {
    const auto mo = ozTTgemm::detail::choose_moduli_int8(K, num_moduli, b_cap);
    std::memset(out, 0, sizeof(*out));
    out->ok = mo.ok;
    out->b = mo.b;
    out->S = (int)mo.m.size();
    out->m_cap = mo.m_cap;
    for (int s = 0; s < out->S && s < 24; s++) out->m[s] = mo.m[s];
    out->log2M = mo.log2M;
    return 0;
}

// Scheme I planner on padded row-major A (M x K) and B (K x N) with the constants of `format`.
struct ozt_plan1 {
    int p, pmax, nsmall;
    unsigned Kc, nkb;
    int pairloop, pairwise, fuse, defer;
    unsigned Whi, Wlo;
    int qw;
    double bits_indep, bits_sampled;
};
int ozt_plan1(const double* A, const double* B, unsigned M, unsigned N, unsigned K, unsigned slices, int format,
              ozt_plan1* out, char* err, std::size_t errlen) {
    return guarded(err, errlen, [&] {
        const auto& f = ozTTgemm::detail::oz1_format(format);
        const auto pl = ozTTgemm::detail::plan_scheme1(A, B, M, N, K, slices, f);
        std::memset(out, 0, sizeof(*out));
        out->p = pl.p;
        out->pmax = pl.autop.pmax;
        out->nsmall = pl.nsmall;
        out->Kc = pl.issue.Kc;
        out->nkb = pl.issue.nkb;
        out->pairloop = pl.issue.pairloop;
        out->pairwise = pl.issue.pairwise;
        out->fuse = pl.issue.fuse;
        out->defer = pl.issue.defer;
        out->Whi = pl.Whi;
        out->Wlo = pl.Wlo;
        out->qw = pl.qw;
        out->bits_indep = pl.autop.bits_indep;
        out->bits_sampled = pl.autop.bits_sampled;
    });
}

void ozt_eval_inputs(unsigned seed, double phi, std::size_t na, std::size_t nb, double* a, double* b) {
    ozTTgemm::evaluation::inputs(seed, phi, na, nb, a, b);
}
unsigned long long ozt_eval_hash(const double* c, std::size_t n) { return ozTTgemm::evaluation::output_hash(c, n); }
void ozt_eval_reference_gemm(const double* A, const double* B, unsigned M, unsigned K, unsigned N, unsigned r0,
                             unsigned r1, double* Chi, double* Clo) {
    ozTTgemm::evaluation::reference_gemm(A, B, M, K, N, r0, r1, Chi, Clo);
}
void ozt_eval_accuracy(const double* C, const double* Chi, const double* Clo, std::size_t n, double* rel_fro,
                       double* ebits) {
    const auto a = ozTTgemm::evaluation::accuracy(C, Chi, Clo, n);
    *rel_fro = a.rel_fro;
    *ebits = a.ebits;
}
void ozt_eval_quad_sample(const double* A, const double* B, int M, int N, int K, int nsample, const int* rows,
                          const int* cols, double* out) {
    ozTTgemm::evaluation::gemm_quad_sample(A, B, M, N, K, nsample, rows, cols, out);
}

}  // extern "C"

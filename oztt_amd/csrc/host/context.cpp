// Public interface: argument validation, zero padding, device lifetime, dispatch, cropping.
// Semantics of the reference's context.cpp:19-194: the same checks in the same order, the same
// exception types, padding of m and n to multiples of 64 and k to a multiple of 32, inputs copied
// before the lock so that C may alias A or B, one process-wide lock, the device opened lazily.
// Resident operands (Matrix, an extension) keep device copies in the padded layouts of the
// products, a host copy for the planner, and the plans of the pairs they were multiplied in.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <filesystem>
#include <limits>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>

#include "backend.hpp"
#include "evaluation.hpp"

namespace ozTTgemm {
namespace {
// Serializes device use by all contexts of the process. Recursive: a resident Matrix frees its
// device memory under it, and may be released while the lock is held.
std::recursive_mutex runtime_mutex;
std::atomic<std::uint64_t> next_matrix_id{1};

// ---- Call validation -----------------------------------------------------------------------------
// The contract is the reference's (context.cpp:17-117): a call is rejected with
// std::invalid_argument before the device is opened and before C is written, and its checks run in
// three rounds, in this order: the options; the shape (span sizes against m, n, k, element counts
// that fit the address space, padded extents that fit the device's 32-bit indices); the values
// (finite, and every nonzero row maximum of A and column maximum of B a normal BF16 value, because
// the device normalizes each row of A and each column of B by its maximum held as BF16).

// The option rules, applied in this order; the first one violated is reported.
struct OptionRule {
    bool (*violated)(const Options&);
    const char* message;
};
constexpr OptionRule kOptionRules[] = {
    // enum values are checked as numbers: a caller can pass any integer through a cast
    {[](const Options& o) { return o.scheme != Scheme::I && o.scheme != Scheme::II; },
     "options.scheme is not an Ozaki scheme"},
    {[](const Options& o) { return !is_available(o.format); }, "options.format is not a format of this build"},
    {[](const Options& o) {
         return o.reconstruction != Reconstruction::Automatic && o.reconstruction != Reconstruction::OnePass &&
                o.reconstruction != Reconstruction::TwoPass;
     },
     "options.reconstruction is not a reconstruction mode"},
    {[](const Options& o) { return o.transport != Transport::Automatic && o.transport != Transport::Int8Residues; },
     "options.transport is not a transport"},
    {[](const Options& o) { return o.slices > 256; }, "options.slices must be 0 (automatic) or 1..256"},
    {[](const Options& o) { return o.max_moduli > 24; }, "options.max_moduli must be 0 (automatic) or 1..24"},
    {[](const Options& o) {
         return o.scheme == Scheme::I && (o.max_moduli != 0 || o.reconstruction != Reconstruction::Automatic ||
                                          o.transport != Transport::Automatic);
     },
     "options.max_moduli, options.reconstruction and options.transport are Ozaki II settings"},
    {[](const Options& o) { return o.scheme == Scheme::II && o.slices != 0; }, "options.slices is an Ozaki I setting"},
    {[](const Options& o) { return !detail::scheme_available(o.format, o.scheme); },
     "this build has no such scheme for options.format"},
};

void require_options(const Options& o) {
    for (const OptionRule& rule : kOptionRules)
        if (rule.violated(o)) throw std::invalid_argument(rule.message);
}

// rows x cols elements of 8 bytes: zero extents, and matrices whose bytes overflow size_t, are rejected.
std::size_t element_count(std::size_t rows, std::size_t cols) {
    std::size_t elements = 0, bytes = 0;
    if (rows == 0 || cols == 0 || __builtin_mul_overflow(rows, cols, &elements) ||
        __builtin_mul_overflow(elements, sizeof(double), &bytes))
        throw std::invalid_argument("a matrix extent is zero or the matrix exceeds the address space");
    return elements;
}

// extent rounded up to a multiple of q (64 for m and n, 32 for k); the padded extents index the
// device with 32-bit signed integers.
std::uint32_t padded_extent(std::size_t extent, std::size_t q) {
    constexpr std::size_t kIndexLimit = (std::size_t)std::numeric_limits<std::int32_t>::max();
    if (extent == 0 || extent > kIndexLimit - q)
        throw std::invalid_argument("a matrix extent exceeds the device's 32-bit index range");
    return (std::uint32_t)((extent + q - 1) / q * q);
}

struct CallShape {
    std::uint32_t mp, np, kp;  // padded extents
    std::size_t mn;            // elements of C
};

CallShape require_shape(std::size_t na, std::size_t nb, std::optional<std::size_t> nc, std::size_t m, std::size_t n,
                        std::size_t k) {
    const std::size_t want_a = element_count(m, k), want_b = element_count(k, n);
    if (na != want_a || nb != want_b) throw std::invalid_argument("the sizes of a and b do not match m, n, k");
    const std::size_t mn = element_count(m, n);
    if (nc && *nc != mn) throw std::invalid_argument("the size of c does not match m x n");
    return {padded_extent(m, 64), padded_extent(n, 64), padded_extent(k, 32), mn};
}

}  // namespace

namespace detail {
// What the value rules need to know of one operand (rows x cols, row-major), from one scan over it
// with the rows split among threads. A maximum is admissible when it is zero or a normal BF16 value.
struct OperandScan {
    std::size_t first_bad_row = 0;    // first row with a non-finite value or an inadmissible maximum (rows: none)
    bool first_bad_nonfinite = false; // that row holds a non-finite value
    bool finite = true;               // no NaN or infinity anywhere
    bool cols_ok = true;              // every column maximum is admissible
};
OperandScan scan_operand(const double* x, std::size_t rows, std::size_t cols) {
    constexpr double kBf16Max = 0x1.fep127, kBf16MinNormal = 0x1p-126;
    auto admissible = [](double v) { return v == 0 || (v >= kBf16MinNormal && v <= kBf16Max); };
    std::vector<unsigned char> row_state(rows);  // 0 fine, 1 non-finite value, 2 inadmissible maximum
    std::vector<double> colmax(cols, 0);
#pragma omp parallel
    {
        std::vector<double> cm(cols, 0);
#pragma omp for schedule(static) nowait
        for (std::int64_t i = 0; i < (std::int64_t)rows; ++i) {
            const double* r = x + (std::size_t)i * cols;
            double mx = 0;
            bool fin = true;
            for (std::size_t j = 0; j < cols; ++j) {
                const double v = std::abs(r[j]);
                fin = fin && std::isfinite(v);
                mx = std::max(mx, v);
                cm[j] = std::max(cm[j], v);
            }
            row_state[(std::size_t)i] = !fin ? 1 : admissible(mx) ? 0 : 2;
        }
#pragma omp critical
        for (std::size_t j = 0; j < cols; ++j) colmax[j] = std::max(colmax[j], cm[j]);
    }
    OperandScan s;
    s.first_bad_row = rows;
    for (std::size_t i = rows; i-- > 0;)
        if (row_state[i]) {
            s.first_bad_row = i;
            s.first_bad_nonfinite = row_state[i] == 1;
        }
    for (unsigned char st : row_state) s.finite = s.finite && st != 1;
    for (double v : colmax) s.cols_ok = s.cols_ok && std::isfinite(v) && admissible(v);
    return s;
}

// The value round, in the reference's order: A row by row (a row's non-finite values before its
// maximum), then the finiteness of all of B, then B's column maxima.
void require_values(const OperandScan& a, std::size_t a_rows, const OperandScan& b) {
    static const char* const kRange =
        "every nonzero row maximum of A and column maximum of B must lie in [2^-126, the largest BF16]";
    if (a.first_bad_row < a_rows)
        throw std::invalid_argument(a.first_bad_nonfinite ? "A holds a NaN or an infinity" : kRange);
    if (!b.finite) throw std::invalid_argument("B holds a NaN or an infinity");
    if (!b.cols_ok) throw std::invalid_argument(kRange);
}

}  // namespace detail

namespace {

CallShape validate(const Options& options, std::span<const double> a, std::span<const double> b,
                   std::optional<std::size_t> c_size, std::size_t m, std::size_t n, std::size_t k) {
    require_options(options);
    const CallShape shape = require_shape(a.size(), b.size(), c_size, m, n, k);
    detail::require_values(detail::scan_operand(a.data(), m, k), m, detail::scan_operand(b.data(), k, n));
    return shape;
}

}  // namespace

namespace detail {
// The opened GPU, shared by a Context and its resident matrices; it is closed by the last of them
// (always under runtime_mutex).
struct DeviceHandle {
    oz_dev* dev = nullptr;
    ~DeviceHandle() {
        if (dev) oz_dev_close(dev);
    }
};
}  // namespace detail

using detail::DeviceHandle;
using detail::OperandScan;
using detail::scan_operand;

struct Matrix::State {
    std::uint64_t id = 0;
    std::shared_ptr<DeviceHandle> device;  // the GPU of the Context that made it (identifies that Context)
    std::size_t rows = 0, cols = 0;
    // host copy (row-major rows x cols) and its facts; a result has them only once it is needed
    std::unique_ptr<double[]> host;
    bool have_host = false;
    OperandScan facts;
    // device copies: the first one (src, leading dimension src_ld) and the zero-padded layouts
    // (prow x pcol, leading dimension pcol) made from it; src is one of them or the raw upload
    struct Copy {
        std::uint32_t prow, pcol;
        double* p;
    };
    double* raw = nullptr;
    const double* src = nullptr;
    std::size_t src_ld = 0;
    std::vector<Copy> copies;
    // zero-padded host copies for the planner, by layout
    std::vector<std::pair<std::pair<std::uint32_t, std::uint32_t>, std::unique_ptr<double[]>>> padded_host;

    ~State() {
        std::lock_guard lock(runtime_mutex);
        if (device && device->dev) {
            for (auto& c : copies) oz_dev_free(device->dev, c.p);
            if (raw) oz_dev_free(device->dev, raw);
        }
        copies.clear();
        device.reset();
    }
};

std::size_t Matrix::rows() const noexcept { return s_ ? s_->rows : 0; }
std::size_t Matrix::cols() const noexcept { return s_ ? s_->cols : 0; }

struct Context::Impl {
    explicit Impl(DeviceOptions o) : options(std::move(o)) {
        if (options.device_id < 0) throw std::invalid_argument("device_id must be nonnegative");
        if (!options.kernel_directory.empty() && !std::filesystem::is_directory(options.kernel_directory))
            throw std::invalid_argument("kernel_directory does not name a directory");
    }
    Info execute(std::span<const double> a, std::span<const double> b, std::span<double> c, std::size_t m,
                 std::size_t n, std::size_t k, const Options& options, const CallShape& v);
    void open();
    // resident operands (under the lock)
    const double* layout(Matrix::State& x, std::uint32_t prow, std::uint32_t pcol);
    void fetch_host(Matrix::State& x);
    const double* padded_host(Matrix::State& x, std::uint32_t prow, std::uint32_t pcol);
    Info resident(Matrix::State& A, Matrix::State& B, std::span<double>* c, std::shared_ptr<Matrix::State>* cslot,
                  const Options& opts);

    // plans of resident pairs, most recent last
    struct CachedPlan {
        std::uint64_t a, b;
        Scheme scheme;
        Format format;
        std::uint32_t slices, max_moduli;
        Reconstruction reconstruction;
        Transport transport;
        std::shared_ptr<const void> plan;
    };
    static constexpr std::size_t kPlanCacheSize = 16;
    std::vector<CachedPlan> plans;

    DeviceOptions options;
    std::shared_ptr<DeviceHandle> handle;
    detail::Device device;
};

Context::Context(DeviceOptions options) : impl_(std::make_unique<Impl>(std::move(options))) {}

Context::~Context() {
    std::lock_guard lock(runtime_mutex);
    if (impl_->device.dev) {
        impl_->device.ws.reset();  // frees the workspace
        impl_->device.dev = nullptr;
        impl_->handle.reset();  // closes the GPU unless resident matrices still hold it
    }
}

void Context::Impl::open() {
    if (device.dev) return;
    oz_dev* d = nullptr;
    const int st = oz_dev_open(options.device_id, &d);
    if (st != OZ_OK)
        throw std::runtime_error("could not open HIP device " + std::to_string(options.device_id) +
                                 " (no MI355X visible, or the device id is out of range)");
    handle = std::make_shared<DeviceHandle>();
    handle->dev = d;
    device.dev = d;
    device.ws = std::make_unique<detail::Workspace>(d);
}

Info Context::Impl::execute(std::span<const double> a, std::span<const double> b, std::span<double> c, std::size_t m,
                            std::size_t n, std::size_t k, const Options& opts, const CallShape& v) {
    const auto mp = v.mp, np = v.np, kp = v.kp;
    std::lock_guard lock(runtime_mutex);
    open();
    // zero-padded copies into the page-locked staging buffers (rows in parallel); they are complete
    // before C is written, so C may alias A or B
    auto* ap = static_cast<double*>(device.ws->host(detail::kHostA, sizeof(double) * element_count(mp, kp)));
    auto* bp = static_cast<double*>(device.ws->host(detail::kHostB, sizeof(double) * element_count(kp, np)));
    const double* ad = a.data();
    const double* bd = b.data();
#pragma omp parallel for schedule(static)
    for (std::int64_t i = 0; i < (std::int64_t)mp; ++i) {
        double* row = ap + (std::size_t)i * kp;
        if ((std::size_t)i < m) {
            std::copy_n(ad + (std::size_t)i * k, k, row);
            std::fill(row + k, row + kp, 0.0);
        } else {
            std::fill(row, row + kp, 0.0);
        }
    }
#pragma omp parallel for schedule(static)
    for (std::int64_t i = 0; i < (std::int64_t)kp; ++i) {
        double* row = bp + (std::size_t)i * np;
        if ((std::size_t)i < k) {
            std::copy_n(bd + (std::size_t)i * n, n, row);
            std::fill(row + n, row + np, 0.0);
        } else {
            std::fill(row, row + np, 0.0);
        }
    }
    const detail::Problem problem{mp, np, kp, ap, bp, opts};
    const detail::Output output = detail::backend_for(opts.format, opts.scheme)(device, problem);
    const double* vals = output.values;
    double* cd = c.data();
#pragma omp parallel for schedule(static)
    for (std::int64_t i = 0; i < (std::int64_t)m; ++i) std::copy_n(vals + (std::size_t)i * np, n, cd + (std::size_t)i * n);
    Info info = output.info;
    info.padded_m = mp;
    info.padded_n = np;
    info.padded_k = kp;
    return info;
}

Info Context::gemm(std::span<const double> a, std::span<const double> b, std::span<double> c, std::size_t m,
                   std::size_t n, std::size_t k, const Options& options) {
    const CallShape v = validate(options, a, b, c.size(), m, n, k);
    return impl_->execute(a, b, c, m, n, k, options, v);
}

std::vector<double> Context::multiply(std::span<const double> a, std::span<const double> b, std::size_t m,
                                      std::size_t n, std::size_t k, const Options& options) {
    const CallShape v = validate(options, a, b, std::nullopt, m, n, k);
    std::vector<double> c(v.mn);
    impl_->execute(a, b, c, m, n, k, options, v);
    return c;
}

// ---- resident operands ------------------------------------------------------------------------

// x's device copy in the zero-padded layout prow x pcol, made from its first device copy on first use.
const double* Context::Impl::layout(Matrix::State& x, std::uint32_t prow, std::uint32_t pcol) {
    for (const auto& c : x.copies)
        if (c.prow == prow && c.pcol == pcol) return c.p;
    void* p = nullptr;
    detail::device_check(device.dev, oz_dev_malloc(device.dev, sizeof(double) * (std::size_t)prow * pcol, &p),
                         "resident matrix");
    x.copies.push_back({prow, pcol, static_cast<double*>(p)});
    detail::device_check(device.dev,
                         oz_pad_copy_f64(device.dev, static_cast<double*>(p), (int)prow, (int)pcol, x.src, (int)x.rows,
                                         (int)x.cols, (int)x.src_ld),
                         "resident matrix layout");
    return static_cast<double*>(p);
}

// x's host copy and its facts (a result is downloaded the first time they are needed).
void Context::Impl::fetch_host(Matrix::State& x) {
    if (x.have_host) return;
    // (new double[]: no zero-filling of buffers that are overwritten anyway)
    std::unique_ptr<double[]> buf(new double[x.rows * x.src_ld]);
    detail::device_check(device.dev,
                         oz_memcpy_d2h(device.dev, buf.get(), x.src, sizeof(double) * x.rows * x.src_ld), "download");
    x.host.reset(new double[x.rows * x.cols]);
#pragma omp parallel for schedule(static)
    for (std::int64_t i = 0; i < (std::int64_t)x.rows; ++i)
        std::copy_n(buf.get() + (std::size_t)i * x.src_ld, x.cols, x.host.get() + (std::size_t)i * x.cols);
    x.facts = scan_operand(x.host.get(), x.rows, x.cols);
    x.have_host = true;
}

// x's host copy zero-padded to prow x pcol: what the planner reads.
const double* Context::Impl::padded_host(Matrix::State& x, std::uint32_t prow, std::uint32_t pcol) {
    for (const auto& e : x.padded_host)
        if (e.first == std::make_pair(prow, pcol)) return e.second.get();
    fetch_host(x);
    std::unique_ptr<double[]> v(new double[(std::size_t)prow * pcol]);
#pragma omp parallel for schedule(static)
    for (std::int64_t i = 0; i < (std::int64_t)prow; ++i) {
        double* row = v.get() + (std::size_t)i * pcol;
        if ((std::size_t)i < x.rows) {
            std::copy_n(x.host.get() + (std::size_t)i * x.cols, x.cols, row);
            std::fill(row + x.cols, row + pcol, 0.0);
        } else {
            std::fill(row, row + pcol, 0.0);
        }
    }
    x.padded_host.emplace_back(std::make_pair(prow, pcol), std::move(v));
    return x.padded_host.back().second.get();
}

Info Context::Impl::resident(Matrix::State& A, Matrix::State& B, std::span<double>* c,
                             std::shared_ptr<Matrix::State>* cslot, const Options& opts) {
    require_options(opts);
    const std::size_t m = A.rows, k = A.cols, n = B.cols;
    if (B.rows != k) throw std::invalid_argument("the extents do not match: a is m x k and b must be k x n");
    const CallShape shape = require_shape(m * k, k * n, c ? std::optional<std::size_t>(c->size()) : std::nullopt, m, n, k);
    const std::uint32_t mp = shape.mp, np = shape.np, kp = shape.kp;
    std::lock_guard lock(runtime_mutex);
    // a Context's matrices hold its device handle, which no other Context shares (and a Context
    // that made no Matrix has none yet)
    if (!handle || A.device != handle || B.device != handle)
        throw std::invalid_argument("the Matrix belongs to another Context");
    // the plan of this pair and these options, if an earlier call made one (not when the
    // evaluation hooks fix the width b or the FP8 transport)
    evaluation::Settings* es = evaluation::active();
    const bool cacheable = !es || (es->fixed_bits == 0 && !es->fp8_matrix_cores && !es->full_window);
    std::shared_ptr<const void> plan;
    if (cacheable)
        for (std::size_t i = plans.size(); i-- > 0;) {
            const CachedPlan& e = plans[i];
            if (e.a == A.id && e.b == B.id && e.scheme == opts.scheme && e.format == opts.format &&
                e.slices == opts.slices && e.max_moduli == opts.max_moduli && e.reconstruction == opts.reconstruction &&
                e.transport == opts.transport) {
                plan = e.plan;
                std::rotate(plans.begin() + (std::ptrdiff_t)i, plans.begin() + (std::ptrdiff_t)i + 1, plans.end());
                break;
            }
        }
    // the value round of gemm(), on the scans of the operands' host copies
    fetch_host(A);
    fetch_host(B);
    detail::require_values(A.facts, m, B.facts);
    const double* ah = plan ? nullptr : padded_host(A, mp, kp);
    const double* bh = plan ? nullptr : padded_host(B, kp, np);
    const double* ad = layout(A, mp, kp);
    const double* bd = layout(B, kp, np);
    // a resident result: the device memory of c's previous matrix when nobody else holds it
    std::shared_ptr<Matrix::State> out;
    double* cdev = nullptr;
    if (cslot) {
        out = std::make_shared<Matrix::State>();
        out->id = next_matrix_id++;
        out->device = handle;
        out->rows = m;
        out->cols = n;
        const std::shared_ptr<Matrix::State>& old = *cslot;
        if (old && old.use_count() == 1 && old->device == handle && old.get() != &A && old.get() != &B)
            for (const auto& cp : old->copies)
                if (cp.prow == mp && cp.pcol == np) cdev = cp.p;  // moves to out once the call succeeded
        if (!cdev) {
            void* p = nullptr;
            detail::device_check(device.dev, oz_dev_malloc(device.dev, sizeof(double) * (std::size_t)mp * np, &p),
                                 "resident result");
            cdev = static_cast<double*>(p);
            out->copies.push_back({mp, np, cdev});  // out frees it if the call fails
        }
        out->src = cdev;
        out->src_ld = np;
    }
    detail::Problem problem{mp, np, kp, ah, bh, opts, ad, bd, cdev, plan};
    const detail::Output output = detail::backend_for(opts.format, opts.scheme)(device, problem);
    if (cslot && out->copies.empty()) {  // the previous matrix's memory: hand it over
        auto& oc = (*cslot)->copies;
        oc.erase(std::find_if(oc.begin(), oc.end(), [&](const Matrix::State::Copy& cp) { return cp.p == cdev; }));
        out->copies.push_back({mp, np, cdev});
    }
    if (es) es->plan_reused = plan != nullptr;
    if (!plan && cacheable) {
        if (plans.size() == kPlanCacheSize) plans.erase(plans.begin());
        plans.push_back({A.id, B.id, opts.scheme, opts.format, opts.slices, opts.max_moduli, opts.reconstruction,
                         opts.transport, output.plan});
    }
    if (c) {
        const double* vals = output.values;
        double* cd = c->data();
#pragma omp parallel for schedule(static)
        for (std::int64_t i = 0; i < (std::int64_t)m; ++i)
            std::copy_n(vals + (std::size_t)i * np, n, cd + (std::size_t)i * n);
    }
    if (cslot) cslot->swap(out);  // the previous matrix (now in out) is released here
    Info info = output.info;
    info.padded_m = mp;
    info.padded_n = np;
    info.padded_k = kp;
    return info;
}

Matrix Context::upload(std::span<const double> x, std::size_t rows, std::size_t cols) {
    if (x.size() != element_count(rows, cols))
        throw std::invalid_argument("matrix span size does not match rows x cols");
    padded_extent(rows, 64);  // index range of either role
    padded_extent(cols, 64);
    auto st = std::make_shared<Matrix::State>();
    st->facts = scan_operand(x.data(), rows, cols);
    if (!st->facts.finite) throw std::invalid_argument("the matrix holds a NaN or an infinity");
    st->id = next_matrix_id++;
    st->rows = rows;
    st->cols = cols;
    st->host.reset(new double[x.size()]);
    const double* xd = x.data();
    double* hd = st->host.get();
#pragma omp parallel for schedule(static)
    for (std::int64_t i = 0; i < (std::int64_t)rows; ++i)
        std::copy_n(xd + (std::size_t)i * cols, cols, hd + (std::size_t)i * cols);
    st->have_host = true;
    {
        std::lock_guard lock(runtime_mutex);
        impl_->open();
        st->device = impl_->handle;
        oz_dev* d = impl_->device.dev;
        void* p = nullptr;
        detail::device_check(d, oz_dev_malloc(d, sizeof(double) * x.size(), &p), "upload");
        st->raw = static_cast<double*>(p);
        detail::device_check(d, oz_memcpy_h2d(d, p, x.data(), sizeof(double) * x.size()), "upload");
        st->src = st->raw;
        st->src_ld = cols;
    }
    Matrix mx;
    mx.s_ = std::move(st);
    return mx;
}

Info Context::gemm(const Matrix& a, const Matrix& b, std::span<double> c, const Options& options) {
    if (!a.s_ || !b.s_) throw std::invalid_argument("empty Matrix");
    return impl_->resident(*a.s_, *b.s_, &c, nullptr, options);
}

Info Context::gemm(const Matrix& a, const Matrix& b, Matrix& c, const Options& options) {
    if (!a.s_ || !b.s_) throw std::invalid_argument("empty Matrix");
    // a and b keep their states alive even when c is one of them
    const std::shared_ptr<Matrix::State> ka = a.s_, kb = b.s_;
    return impl_->resident(*ka, *kb, nullptr, &c.s_, options);
}

void Context::download(const Matrix& x, std::span<double> out) {
    if (!x.s_) throw std::invalid_argument("empty Matrix");
    if (out.size() != x.s_->rows * x.s_->cols) throw std::invalid_argument("span size does not match the Matrix");
    std::lock_guard lock(runtime_mutex);
    if (!impl_->handle || x.s_->device != impl_->handle)
        throw std::invalid_argument("the Matrix belongs to another Context");
    impl_->fetch_host(*x.s_);
    std::copy_n(x.s_->host.get(), out.size(), out.begin());
}

}  // namespace ozTTgemm

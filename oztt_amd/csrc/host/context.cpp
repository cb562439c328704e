// Public interface: argument validation, zero padding, device lifetime, dispatch, cropping.
// Semantics of the reference's context.cpp:19-194: the same checks in the same order, the same
// exception types, padding of m and n to multiples of 64 and k to a multiple of 32, inputs copied
// before the lock so that C may alias A or B, one process-wide lock, the device opened lazily.
#include <algorithm>
#include <cmath>
#include <filesystem>
#include <limits>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>

#include "backend.hpp"

namespace ozTTgemm {
namespace {
std::mutex runtime_mutex;  // serializes device use by all contexts of the process

std::size_t checked_product(std::size_t a, std::size_t b) {
    if (a == 0 || b == 0 || a > std::numeric_limits<std::size_t>::max() / sizeof(double) / b)
        throw std::invalid_argument("matrix dimensions are zero or overflow the address space");
    return a * b;
}
std::uint32_t padded(std::size_t value, std::size_t quantum) {
    constexpr std::size_t limit = std::numeric_limits<std::int32_t>::max();
    if (value == 0 || value > limit - quantum)
        throw std::invalid_argument("matrix dimension exceeds the supported device index range");
    return static_cast<std::uint32_t>((value + quantum - 1) / quantum * quantum);
}
// Every nonzero row maximum of A and column maximum of B must be a normal BF16 value, because the
// device normalizes by BF16 maxima (context.cpp:37-63).
void check_values(std::span<const double> a, std::span<const double> b, std::size_t m, std::size_t n, std::size_t k) {
    constexpr double maximum = 0x1.fep127, minimum = 0x1p-126;
    const auto check_max = [&](double x) {
        if (x != 0 && (x < minimum || x > maximum))
            throw std::invalid_argument(
                "each nonzero row maximum of A and column maximum of B must be in [2^-126, max_BF16]");
    };
    for (std::size_t i = 0; i < m; ++i) {
        double mx = 0;
        for (std::size_t j = 0; j < k; ++j) {
            const double x = a[i * k + j];
            if (!std::isfinite(x)) throw std::invalid_argument("A contains NaN or infinity");
            mx = std::max(mx, std::abs(x));
        }
        check_max(mx);
    }
    std::vector<double> maxima(n, 0);
    for (std::size_t i = 0; i < k; ++i)
        for (std::size_t j = 0; j < n; ++j) {
            const double x = b[i * n + j];
            if (!std::isfinite(x)) throw std::invalid_argument("B contains NaN or infinity");
            maxima[j] = std::max(maxima[j], std::abs(x));
        }
    for (double x : maxima) check_max(x);
}
// Enum values are checked too: a caller can pass any integer through a cast (context.cpp:82-100).
void check_options(const Options& o) {
    if (o.scheme != Scheme::I && o.scheme != Scheme::II) throw std::invalid_argument("unknown Ozaki scheme");
    if (!is_available(o.format)) throw std::invalid_argument("format is unknown or was not built");
    if (o.reconstruction != Reconstruction::Automatic && o.reconstruction != Reconstruction::OnePass &&
        o.reconstruction != Reconstruction::TwoPass)
        throw std::invalid_argument("unknown reconstruction mode");
    if (o.slices > 256) throw std::invalid_argument("slices must be zero (automatic) or at most 256");
    if (o.max_moduli > 24) throw std::invalid_argument("max_moduli exceeds the supported bound of 24");
    if (o.scheme == Scheme::I && (o.max_moduli != 0 || o.reconstruction != Reconstruction::Automatic))
        throw std::invalid_argument("max_moduli and reconstruction apply only to Ozaki II");
    if (o.scheme == Scheme::II && o.slices != 0) throw std::invalid_argument("slices applies only to Ozaki I");
    if (!detail::scheme_available(o.format, o.scheme))
        throw std::invalid_argument("this scheme is not built for the requested format");
}
struct Checked {
    std::uint32_t mp, np, kp;
    std::size_t c_size;
};
Checked validate(const Options& options, std::span<const double> a, std::span<const double> b,
                 std::optional<std::size_t> c_size, std::size_t m, std::size_t n, std::size_t k) {
    check_options(options);
    if (a.size() != checked_product(m, k) || b.size() != checked_product(k, n))
        throw std::invalid_argument("matrix span sizes do not match m, n, k");
    const std::size_t mn = checked_product(m, n);
    if (c_size && *c_size != mn) throw std::invalid_argument("matrix span sizes do not match m, n, k");
    const Checked v{padded(m, 64), padded(n, 64), padded(k, 32), mn};
    check_values(a, b, m, n, k);
    return v;
}
}  // namespace

struct Context::Impl {
    explicit Impl(DeviceOptions o) : options(std::move(o)) {
        if (options.device_id < 0) throw std::invalid_argument("device_id must be nonnegative");
        if (!options.kernel_directory.empty() && !std::filesystem::is_directory(options.kernel_directory))
            throw std::invalid_argument("kernel_directory does not name a directory");
    }
    Info execute(std::span<const double> a, std::span<const double> b, std::span<double> c, std::size_t m,
                 std::size_t n, std::size_t k, const Options& options, const Checked& v);
    DeviceOptions options;
    detail::Device device;
};

Context::Context(DeviceOptions options) : impl_(std::make_unique<Impl>(std::move(options))) {}

Context::~Context() {
    std::lock_guard lock(runtime_mutex);
    if (impl_->device.dev) {
        impl_->device.ws.reset();  // frees the workspace
        oz_dev_close(impl_->device.dev);
        impl_->device.dev = nullptr;
    }
}

Info Context::Impl::execute(std::span<const double> a, std::span<const double> b, std::span<double> c, std::size_t m,
                            std::size_t n, std::size_t k, const Options& opts, const Checked& v) {
    const auto mp = v.mp, np = v.np, kp = v.kp;
    std::lock_guard lock(runtime_mutex);
    if (!device.dev) {
        oz_dev* d = nullptr;
        const int st = oz_dev_open(options.device_id, &d);
        if (st != OZ_OK)
            throw std::runtime_error("could not open HIP device " + std::to_string(options.device_id) +
                                     " (no MI355X visible, or the device id is out of range)");
        device.dev = d;
        device.ws = std::make_unique<detail::Workspace>(d);
    }
    // zero-padded copies into the page-locked staging buffers (rows in parallel); they are complete
    // before C is written, so C may alias A or B
    auto* ap = static_cast<double*>(device.ws->host(detail::kHostA, sizeof(double) * checked_product(mp, kp)));
    auto* bp = static_cast<double*>(device.ws->host(detail::kHostB, sizeof(double) * checked_product(kp, np)));
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
    const Checked v = validate(options, a, b, c.size(), m, n, k);
    return impl_->execute(a, b, c, m, n, k, options, v);
}

std::vector<double> Context::multiply(std::span<const double> a, std::span<const double> b, std::size_t m,
                                      std::size_t n, std::size_t k, const Options& options) {
    const Checked v = validate(options, a, b, std::nullopt, m, n, k);
    std::vector<double> c(v.c_size);
    impl_->execute(a, b, c, m, n, k, options, v);
    return c;
}

}  // namespace ozTTgemm

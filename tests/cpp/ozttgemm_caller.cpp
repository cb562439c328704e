// A C++ caller of the public interface, compiled against include/ozTTgemm/ozTTgemm.hpp and linked
// with libozTTgemm.so exactly as a user of the reference library would build it. It runs the cases
// of the reference's own correctness program (tests/correctness.cpp) and its usage example
// (examples/gemm.cpp):
//   --host-only  the argument checks of correctness.cpp:49-85 (they never open the device) and the
//                defaults of Options and Info;
//   (default)    also the device cases of correctness.cpp:259-308: every format with both schemes on
//                64^3 uniform and 3x5x7 nonnegative inputs; Scaled, ZeroA, Cancellation,
//                ZeroRowAndColumn, SmallestMaximum and LargestMaximum with both schemes; fixed
//                slices; output aliasing an input; 5056x64x32; forced two passes; too few moduli
//                rejected with C untouched; BF16 64x64x32768, which crosses the exact accumulator's
//                K block; each within 8 eps (relative Frobenius error) of a long-double product.
//                Then the usage example (2x3 times 3x2, exact) and the evaluation hooks: a replayed
//                whole pass is bit-identical and checked, and a replay with a phase left out fails
//                the check.
// Prints one line per case; exit status 0 when every case passes, 1 otherwise.
#include <ozTTgemm/ozTTgemm.hpp>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <iostream>
#include <limits>
#include <random>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "evaluation.hpp"

namespace {

using ozTTgemm::Format;
using ozTTgemm::Options;
using ozTTgemm::Reconstruction;
using ozTTgemm::Scheme;

constexpr Format kFormats[] = {Format::BF16, Format::FP16, Format::TF32, Format::BFP8,
                               Format::FP8,  Format::INT8, Format::BFP4, Format::BFP2};

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};
void expect(bool ok, const std::string& what) {
    if (!ok) throw Failure(what);
}

// The call must throw exactly `E` (std::invalid_argument for bad input, std::runtime_error for a
// configuration that cannot run; an invalid_argument is not accepted as the latter).
template <class E>
void expect_throw(const std::function<void()>& call, const std::string& what) {
    try {
        call();
    } catch (const std::invalid_argument& e) {
        if constexpr (std::is_same_v<E, std::invalid_argument>) return;
        throw Failure(what + ": reported as invalid input (" + e.what() + ")");
    } catch (const std::runtime_error& e) {
        if constexpr (std::is_same_v<E, std::runtime_error>) return;
        throw Failure(what + ": reported as a runtime error (" + e.what() + ")");
    }
    throw Failure(what + ": accepted");
}

bool bits_equal(const std::vector<double>& x, const std::vector<double>& y) {
    return x.size() == y.size() && std::memcmp(x.data(), y.data(), sizeof(double) * x.size()) == 0;
}

// ---- host-only: the argument checks ------------------------------------------------------------
void argument_checks(ozTTgemm::Context& ctx) {
    Options dflt;
    expect(dflt.scheme == Scheme::II && dflt.format == Format::BFP8 && dflt.slices == 0 && dflt.max_moduli == 0 &&
               dflt.reconstruction == Reconstruction::Automatic,
           "Options defaults");
    expect(std::string(ozTTgemm::format_name(Format::INT8)) == "INT8" &&
               std::string(ozTTgemm::format_name(Format::BFP2)) == "BFP2",
           "format_name");
    std::vector<double> a(4, 1.0), b(4, 1.0), c(4, 123.0);
    Options o;
    o.format = Format::INT8;
    using IA = std::invalid_argument;
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 0, 2, 2, o); }, "zero extent");
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 3, 2, o); }, "span sizes that do not match");
    expect_throw<IA>([&] { (void)ctx.multiply(a, b, 2, 2, 3, o); }, "multiply with mismatched spans");
    auto with = [&](auto change) {
        Options x = o;
        change(x);
        return x;
    };
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) { x.scheme = static_cast<Scheme>(7); })); },
                     "unknown scheme");
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) { x.format = static_cast<Format>(99); })); },
                     "unknown format");
    expect_throw<IA>(
        [&] {
            ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) { x.reconstruction = static_cast<Reconstruction>(5); }));
        },
        "unknown reconstruction");
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) { x.slices = 10; })); },
                     "slices under scheme II");
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) { x.max_moduli = 25; })); },
                     "max_moduli above 24");
    expect_throw<IA>(
        [&] {
            ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) {
                         x.scheme = Scheme::I;
                         x.reconstruction = Reconstruction::TwoPass;
                     }));
        },
        "reconstruction under scheme I");
    expect_throw<IA>(
        [&] {
            ctx.gemm(a, b, c, 2, 2, 2, with([](Options& x) {
                         x.scheme = Scheme::I;
                         x.slices = 257;
                     }));
        },
        "more than 256 slices");
    a[0] = std::numeric_limits<double>::quiet_NaN();
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, o); }, "NaN in A");
    a[0] = 1;
    b[3] = -std::numeric_limits<double>::infinity();
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, o); }, "infinity in B");
    b[3] = 1;
    std::fill(a.begin(), a.end(), 0x1p-130);
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, o); }, "row maximum below 2^-126");
    std::fill(a.begin(), a.end(), 1.0);
    b[1] = 0x1p128;
    expect_throw<IA>([&] { ctx.gemm(a, b, c, 2, 2, 2, o); }, "column maximum above the largest BF16");
    expect(std::all_of(c.begin(), c.end(), [](double x) { return x == 123.0; }), "rejected calls left C untouched");
    expect_throw<IA>([] { ozTTgemm::Context bad(ozTTgemm::DeviceOptions{-1, {}}); }, "negative device id");
}

// ---- device cases ------------------------------------------------------------------------------
enum class Input { Uniform, ZeroA, Nonnegative, Scaled, Cancellation, ZeroRowAndColumn, SmallestMax, LargestMax };
const char* input_name(Input p) {
    switch (p) {
    case Input::Uniform: return "uniform";
    case Input::ZeroA: return "zero-A";
    case Input::Nonnegative: return "nonnegative";
    case Input::Scaled: return "scaled";
    case Input::Cancellation: return "cancellation";
    case Input::ZeroRowAndColumn: return "zero-row-column";
    case Input::SmallestMax: return "smallest-maximum";
    case Input::LargestMax: return "largest-maximum";
    }
    return "?";
}

// Inputs of the pattern (the reference's check(), correctness.cpp:188-236), from a seeded generator.
void make_inputs(Input p, std::size_t m, std::size_t n, std::size_t k, std::vector<double>& a, std::vector<double>& b) {
    std::mt19937_64 gen(2024);
    std::uniform_real_distribution<double> u(-1.0, 1.0);
    a.resize(m * k);
    b.resize(k * n);
    for (double& x : a) x = u(gen);
    for (double& x : b) x = u(gen);
    switch (p) {
    case Input::Uniform: break;
    case Input::ZeroA: std::fill(a.begin(), a.end(), 0.0); break;
    case Input::Nonnegative:
        for (double& x : a) x = std::fabs(x);
        for (double& x : b) x = std::fabs(x);
        break;
    case Input::Scaled:  // rows of A and columns of B spread over 2^-15..2^15 and 2^-13..2^13
        for (std::size_t i = 0; i < m; ++i)
            for (std::size_t j = 0; j < k; ++j) a[i * k + j] = std::ldexp(a[i * k + j], (int)(i % 31) - 15);
        for (std::size_t i = 0; i < k; ++i)
            for (std::size_t j = 0; j < n; ++j) b[i * n + j] = std::ldexp(b[i * n + j], (int)(j % 27) - 13);
        break;
    case Input::Cancellation:  // +1 -1 +1 ... times ones: exact cancellation
        for (std::size_t i = 0; i < m; ++i)
            for (std::size_t j = 0; j < k; ++j) a[i * k + j] = (j & 1) ? -1.0 : 1.0;
        std::fill(b.begin(), b.end(), 1.0);
        break;
    case Input::ZeroRowAndColumn:
        for (std::size_t j = 0; j < k; ++j) a[j] = 0.0;
        for (std::size_t i = 0; i < k; ++i) b[i * n] = 0.0;
        break;
    case Input::SmallestMax:
        std::fill(a.begin(), a.end(), 0x1p-126);
        std::fill(b.begin(), b.end(), 1.0);
        break;
    case Input::LargestMax:
        std::fill(a.begin(), a.end(), 0x1.fep127);
        std::fill(b.begin(), b.end(), 1.0);
        break;
    }
}

// Relative Frobenius error of c against the long-double product (absolute when the product is 0).
double error_vs_long_double(const std::vector<double>& a, const std::vector<double>& b, const std::vector<double>& c,
                            std::size_t m, std::size_t n, std::size_t k) {
    std::vector<long double> row(n);
    long double err = 0, norm = 0;
    for (std::size_t i = 0; i < m; ++i) {
        std::fill(row.begin(), row.end(), 0.0L);
        for (std::size_t l = 0; l < k; ++l) {
            const long double x = a[i * k + l];
            const double* br = &b[l * n];
            for (std::size_t j = 0; j < n; ++j) row[j] += x * br[j];
        }
        for (std::size_t j = 0; j < n; ++j) {
            expect(std::isfinite(c[i * n + j]), "non-finite output");
            const long double d = c[i * n + j] - row[j];
            err += d * d;
            norm += row[j] * row[j];
        }
    }
    return norm > 0 ? (double)std::sqrt(err / norm) : (double)std::sqrt(err);
}

void gemm_case(ozTTgemm::Context& ctx, const Options& o, std::size_t m, std::size_t n, std::size_t k, Input p) {
    std::vector<double> a, b;
    make_inputs(p, m, n, k, a, b);
    std::vector<double> c(m * n, 123.0);
    const ozTTgemm::Info info = ctx.gemm(a, b, c, m, n, k, o);
    const double err = error_vs_long_double(a, b, c, m, n, k);
    const std::string name = std::string(o.scheme == Scheme::I ? "I " : "II ") + ozTTgemm::format_name(o.format) +
                             " " + std::to_string(m) + "x" + std::to_string(n) + "x" + std::to_string(k) + " " +
                             input_name(p);
    std::cout << name << " error=" << err << " slices=" << info.slices << " moduli=" << info.moduli
              << " passes=" << info.reconstruction_passes << '\n';
    expect(err <= 8 * std::numeric_limits<double>::epsilon(), name + ": error above 8 eps");
    expect(info.scheme == o.scheme && info.format == o.format, name + ": Info names another scheme or format");
    expect(info.padded_m == (m + 63) / 64 * 64 && info.padded_n == (n + 63) / 64 * 64 &&
               info.padded_k == (k + 31) / 32 * 32,
           name + ": padded extents");
    if (o.scheme == Scheme::I && o.slices) expect(info.slices == o.slices, name + ": fixed slices not used");
    if (o.reconstruction == Reconstruction::TwoPass) expect(info.reconstruction_passes == 2, name + ": passes");
}

void device_cases(ozTTgemm::Context& ctx) {
    for (Format f : kFormats) {
        if (!ozTTgemm::is_available(f)) continue;
        for (Scheme s : {Scheme::I, Scheme::II}) {
            Options o;
            o.scheme = s;
            o.format = f;
            gemm_case(ctx, o, 64, 64, 64, Input::Uniform);
            gemm_case(ctx, o, 3, 5, 7, Input::Nonnegative);
        }
    }
    for (Scheme s : {Scheme::I, Scheme::II}) {
        Options o;
        o.scheme = s;
        o.format = Format::BF16;
        gemm_case(ctx, o, 65, 67, 97, Input::Scaled);
        gemm_case(ctx, o, 9, 11, 17, Input::ZeroA);
        gemm_case(ctx, o, 3, 5, 64, Input::Cancellation);
        gemm_case(ctx, o, 3, 5, 7, Input::ZeroRowAndColumn);
        gemm_case(ctx, o, 1, 1, 1, Input::SmallestMax);
        gemm_case(ctx, o, 1, 1, 1, Input::LargestMax);
    }
    {  // fixed slices (the reference's value for its first format, BF16: 10)
        Options o;
        o.scheme = Scheme::I;
        o.format = Format::BF16;
        o.slices = 10;
        gemm_case(ctx, o, 3, 5, 7, Input::Uniform);
    }
    {  // C aliases A: the inputs are consumed before C is written
        std::vector<double> x{1, 2, 3, 4};
        const std::vector<double> id{1, 0, 0, 1};
        Options o;
        o.format = Format::BF16;
        ctx.gemm(x, id, x, 2, 2, 2, o);
        expect(x == std::vector<double>({1, 2, 3, 4}), "output aliasing an input");
        std::cout << "aliased output ok\n";
    }
    {
        Options o;
        o.format = Format::BF16;
        gemm_case(ctx, o, 5056, 64, 32, Input::Uniform);
        o.reconstruction = Reconstruction::TwoPass;
        gemm_case(ctx, o, 64, 64, 64, Input::Uniform);
    }
    {  // two moduli cannot reach an FP64-equivalent width: a runtime error, C untouched
        Options o;
        o.format = Format::BF16;
        o.max_moduli = 2;
        std::vector<double> a(64 * 64, 1.0), b(64 * 64, 1.0), c(64 * 64, 123.0);
        expect_throw<std::runtime_error>([&] { ctx.gemm(a, b, c, 64, 64, 64, o); }, "max_moduli = 2");
        expect(std::all_of(c.begin(), c.end(), [](double x) { return x == 123.0; }), "rejected plan left C untouched");
        std::cout << "too few moduli rejected\n";
    }
    {  // BF16 scheme I with K = 32768: beyond one exact FP32 accumulation block
        Options o;
        o.scheme = Scheme::I;
        o.format = Format::BF16;
        gemm_case(ctx, o, 64, 64, 32768, Input::Nonnegative);
    }
}

// The usage example of the reference (examples/gemm.cpp): default options, 2x3 times 3x2.
void usage_example(ozTTgemm::Context& ctx) {
    ozTTgemm::Options options;  // Scheme II, BFP8
    const std::vector<double> a{1, 2, 3, 4, 5, 6};
    const std::vector<double> b{7, 8, 9, 10, 11, 12};
    const auto c = ctx.multiply(a, b, 2, 2, 3, options);
    expect(c == std::vector<double>({58, 64, 139, 154}), "usage example");
    std::cout << "usage example: " << c[0] << ' ' << c[1] << " / " << c[2] << ' ' << c[3] << '\n';
}

// The evaluation hooks (correctness.cpp:88-172): a checked whole-pass replay gives the bits of a
// plain call; a replay with the reconstruction left out fails the check.
void evaluation_hooks(ozTTgemm::Context& ctx) {
    namespace ev = ozTTgemm::evaluation;
    std::vector<double> a, b;
    make_inputs(Input::Uniform, 64, 64, 64, a, b);
    std::vector<double> plain(64 * 64), replayed(64 * 64);
    for (Scheme s : {Scheme::I, Scheme::II}) {
        Options o;
        o.scheme = s;
        o.format = Format::INT8;
        ctx.gemm(a, b, plain, 64, 64, 64, o);
        ev::Settings st;
        st.repeats = 2;
        {
            ev::Scope scope(st);
            ctx.gemm(a, b, replayed, 64, 64, 64, o);
        }
        expect(ev::active() == nullptr, "the evaluation scope ended");
        expect(bits_equal(plain, replayed), "evaluation hooks changed the result");
        expect(st.whole_checked && st.whole_sentinel && st.whole_ms > 0, "whole-pass replay checked and timed");
        expect(st.phase_ms[ev::Slice] > 0 && st.phase_ms[ev::Gemm] > 0 && st.phase_ms[ev::Recon] > 0,
               "phases timed");
        ev::Settings broken;
        broken.repeats = 2;
        broken.replay_drop_phase = ev::Recon;
        {
            ev::Scope scope(broken);
            ctx.gemm(a, b, replayed, 64, 64, 64, o);
        }
        expect(!broken.whole_checked && broken.whole_ms == 0, "a replay without reconstruction was accepted");
        expect(bits_equal(plain, replayed), "the self-test changed the returned result");
        std::cout << "evaluation hooks ok (scheme " << (s == Scheme::I ? "I" : "II") << ")\n";
    }
}

}  // namespace

int main(int argc, char** argv) {
    const bool host_only = argc == 2 && std::string(argv[1]) == "--host-only";
    if (argc > 2 || (argc == 2 && !host_only)) {
        std::cerr << "usage: ozttgemm_caller [--host-only]\n";
        return 2;
    }
    try {
        ozTTgemm::Context ctx;  // opens the device only on the first valid call
        argument_checks(ctx);
        std::cout << "argument checks passed\n";
        if (host_only) return 0;
        device_cases(ctx);
        usage_example(ctx);
        evaluation_hooks(ctx);
        std::cout << "all cases passed\n";
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "FAILED: " << e.what() << '\n';
        return 1;
    }
}

// Ozaki scheme II driver (INT8 residues; the FP8 format plans its width on the FP8 route and computes
// with INT8 residues, see plan2.hpp): one FP64 GEMM on the GPU.
//
// Pipeline of the reference's ozaki2.cpp:439-478: plan (moduli, width b, passes) -> upload the FP64
// operands -> scale (row/column maxima, exponent deltas) -> slice (int8 residue planes per
// modulus) -> products (one exact int32 GEMM per modulus) -> CRT reconstruction to FP64 -> read
// back and check the range flags. The reference splits the output into row bands when its 32 GB
// of DRAM is short (plan.hpp:386-444); at the sizes one MI355X (288 GB) serves, every buffer is
// resident at once, so there are no bands.
//
// Device layout (all row-major, zero-padded so that every kernel runs unguarded full tiles):
//   A (M x K f64), B (K x N f64), dA[M], dB[N] int32, flags[2];
//   residue planes of A: S x Mg x Kg int8, of B: S x Ng x Kg int8 (B transposed), both K-major in
//   the GEMM's OZ_BLOCK tiles (1 KB blocks of 16 rows x 64 K-bytes), Mg, Ng multiples of 256 and
//   Kg of 64;
//   CRT digits of the products: S x Mg x Ng uint8; output: M x N f64.
#include <chrono>
#include <cstring>
#include <functional>
#include <stdexcept>

#include "backend.hpp"
#include "evaluation.hpp"
#include "pipeline.hpp"
#include "plan2.hpp"

namespace ozTTgemm::detail {
namespace {

namespace ev = ::ozTTgemm::evaluation;

enum Slot { kA = 0, kB, kDA, kDB, kFlags, kPlanesA, kPlanesB, kProducts, kOut };

std::uint32_t round_up(std::uint32_t v, std::uint32_t q) { return (v + q - 1) / q * q; }

}  // namespace

Output ozaki2_run(Device& D, const Problem& p) {
    oz_dev* dev = D.dev;
    ev::Settings* es = ev::active();
    std::optional<unsigned> fixed_b;
    if (es && es->fixed_bits) fixed_b = es->fixed_bits;
    const Plan2 plan = plan_scheme2(p.a.data(), p.b.data(), p.m, p.n, p.k, p.options.format, p.options.max_moduli,
                                    p.options.reconstruction, fixed_b);
    const std::uint32_t M = p.m, N = p.n, K = p.k, S = (std::uint32_t)plan.S;
    const std::uint32_t Mg = round_up(M, 256), Ng = round_up(N, 256), Kg = round_up(K, 64);
    const oz2_moduli_dev mdesc = split_descriptor(plan);
    const oz2_crt_dev cdesc = crt_descriptor(plan);

    Workspace& ws = *D.ws;
    auto* dAf = static_cast<double*>(ws.get(kA, sizeof(double) * M * (std::size_t)K));
    auto* dBf = static_cast<double*>(ws.get(kB, sizeof(double) * K * (std::size_t)N));
    auto* dltA = static_cast<std::int32_t*>(ws.get(kDA, sizeof(std::int32_t) * M));
    auto* dltB = static_cast<std::int32_t*>(ws.get(kDB, sizeof(std::int32_t) * N));
    auto* flags = static_cast<std::uint32_t*>(ws.get(kFlags, 2 * sizeof(std::uint32_t)));
    const long long strideA = (long long)Mg * Kg, strideB = (long long)Ng * Kg, strideC = (long long)Mg * Ng;
    auto* planesA = static_cast<std::int8_t*>(ws.get(kPlanesA, (std::size_t)S * strideA));
    auto* planesB = static_cast<std::int8_t*>(ws.get(kPlanesB, (std::size_t)S * strideB));
    auto* prod = static_cast<std::uint8_t*>(ws.get(kProducts, (std::size_t)S * strideC));
    auto* out = static_cast<double*>(ws.get(kOut, sizeof(double) * M * (std::size_t)N));

    device_check(dev, oz_memcpy_h2d(dev, dAf, p.a.data(), sizeof(double) * p.a.size()), "upload A");
    device_check(dev, oz_memcpy_h2d(dev, dBf, p.b.data(), sizeof(double) * p.b.size()), "upload B");

    const int shift = plan.shift();
    std::vector<Step> steps;
    steps.push_back({ev::Scale, [=] {
                         device_check(dev, oz_fill_u32(dev, flags, 0u, 2), "flags");
                         // Scheme II rounds the BF16 of the maxima up (ozaki2.cpp:143-146)
                         device_check(dev, oz_scale_f64(dev, dAf, (int)M, (int)K, (int)K, 0, 1, shift, dltA, flags),
                                      "scale A");
                         device_check(dev, oz_scale_f64(dev, dBf, (int)K, (int)N, (int)N, 1, 1, shift, dltB, flags + 1),
                                      "scale B");
                     }});
    steps.push_back({ev::Slice, [=] {
                         device_check(dev,
                                      oz2_split_int8(dev, dAf, (int)M, (int)K, (int)K, 0, dltA, &mdesc, planesA, 2,
                                                     (int)Mg, (int)Kg, strideA),
                                      "slice A");
                         device_check(dev,
                                      oz2_split_int8(dev, dBf, (int)K, (int)N, (int)N, 1, dltB, &mdesc, planesB, 3,
                                                     (int)Ng, (int)Kg, strideB),
                                      "slice B");
                     }});
    steps.push_back({ev::Gemm, [=] {
                         device_check(dev,
                                      oz2_gemm_digits(dev, planesA, planesB, prod, (int)Mg, (int)Ng, (int)Kg, (int)S,
                                                      (int)Ng, strideA, strideB, strideC, &cdesc),
                                      "products");
                     }});
    steps.push_back({ev::Recon, [=] {
                         device_check(dev,
                                      oz2_crt_digits_f64(dev, prod, (int)M, (int)N, (int)Ng, strideC, &cdesc, dltA,
                                                         dltB, out, (int)N),
                                      "reconstruction");
                     }});

    std::vector<double> values = run_pipeline(dev, steps, 2, out, (std::size_t)M * N, flags,
                                              2.0 * M * (double)N * K * S, S);
    Info info{Scheme::II, p.options.format};
    info.moduli = (std::uint32_t)plan.route.m.size();
    info.integer_bits = (std::uint32_t)plan.b;
    info.reconstruction_passes = plan.two_pass ? 2 : 1;
    return {std::move(values), info};
}

}  // namespace ozTTgemm::detail

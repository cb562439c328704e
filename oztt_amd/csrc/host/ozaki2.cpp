// Ozaki scheme II driver (INT8 residues, or the FP8 route's e4m3 digits): one FP64 GEMM on the GPU.
//
// Pipeline of the reference's ozaki2.cpp:439-478: plan (moduli, width b, passes) -> upload the FP64
// operands -> scale (row/column maxima, exponent deltas) -> slice -> products -> CRT reconstruction
// to FP64 -> read back and check the range flags. The reference splits the output into row bands
// when its 32 GB of DRAM is short (plan.hpp:386-444); at the sizes one MI355X (288 GB) serves, every
// buffer is resident at once, so there are no bands.
//   INT8: slice = int8 residue planes per modulus; products = one exact int32 GEMM per modulus,
//   reduced in the epilogue to the CRT digit (uint8); reconstruction from the S digit planes.
//   FP8 (ozaki2.cpp:228-318 run_digit_gemms): slice = e4m3 digit planes (2 or 3 per modulus);
//   products = the digit products on the FP8 matrix cores, one output per group of equal-weight
//   products, each reduced in the epilogue to its share of the CRT digit (uint16), which replaces
//   the reference's composition launch; reconstruction from the output planes.
//
// Device layout (all row-major, zero-padded so that every kernel runs unguarded full tiles):
//   A (M x K f64), B (K x N f64), dA[M], dB[N] int32, flags[2];
//   planes of A: P x Mg x Kg bytes, of B: P x Ng x Kg bytes (B transposed), both K-major in the
//   GEMM's OZ_BLOCK tiles (1 KB blocks of 16 rows x 64 K-bytes), Mg, Ng multiples of 256 and Kg of
//   64 (P = S residue planes, or the FP8 route's digit planes);
//   product digits: S x Mg x Ng uint8 (INT8) or nout x Mg x Ng uint16 (FP8); output: M x N f64.
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
    const std::uint32_t M = p.m, N = p.n, K = p.k;
    Workspace& ws = *D.ws;
    // the operands go up while the host plans (they are page-locked, the copies are asynchronous)
    auto* dAf = static_cast<double*>(ws.get(kA, sizeof(double) * M * (std::size_t)K));
    auto* dBf = static_cast<double*>(ws.get(kB, sizeof(double) * K * (std::size_t)N));
    device_check(dev, oz_memcpy_h2d_async(dev, dAf, p.a, sizeof(double) * M * (std::size_t)K), "upload A");
    device_check(dev, oz_memcpy_h2d_async(dev, dBf, p.b, sizeof(double) * K * (std::size_t)N), "upload B");
    const Plan2 plan = plan_scheme2(p.a, p.b, p.m, p.n, p.k, p.options.format, p.options.max_moduli,
                                    p.options.reconstruction, fixed_b);
    const bool fp8 = p.options.format == Format::FP8;
    const std::uint32_t S = (std::uint32_t)plan.S;
    const std::uint32_t Mg = round_up(M, 256), Ng = round_up(N, 256), Kg = round_up(K, 64);
    const oz2_crt_dev cdesc = crt_descriptor(plan);
    const oz2_moduli_dev mdesc = split_descriptor(plan);
    oz2_digit_dev ddesc{};
    oz2_groups_dev gdesc{};
    std::vector<unsigned char> term_mod;
    if (fp8) {
        ddesc = digit_descriptor(plan);
        gdesc = groups_descriptor(plan, cdesc, term_mod);
    }
    const std::uint32_t nplanes = fp8 ? (std::uint32_t)plan.mo.nplane : S;
    const std::uint32_t nterms = fp8 ? (std::uint32_t)gdesc.nout : S;
    const std::size_t term_bytes = fp8 ? 2 : 1;

    auto* dltA = static_cast<std::int32_t*>(ws.get(kDA, sizeof(std::int32_t) * M));
    auto* dltB = static_cast<std::int32_t*>(ws.get(kDB, sizeof(std::int32_t) * N));
    auto* flags = static_cast<std::uint32_t*>(ws.get(kFlags, 2 * sizeof(std::uint32_t)));
    const long long strideA = (long long)Mg * Kg, strideB = (long long)Ng * Kg, strideC = (long long)Mg * Ng;
    auto* planesA = static_cast<std::int8_t*>(ws.get(kPlanesA, (std::size_t)nplanes * strideA));
    auto* planesB = static_cast<std::int8_t*>(ws.get(kPlanesB, (std::size_t)nplanes * strideB));
    auto* prod = static_cast<std::uint8_t*>(ws.get(kProducts, (std::size_t)nterms * strideC * term_bytes));
    auto* out = static_cast<double*>(ws.get(kOut, sizeof(double) * M * (std::size_t)N));
    auto* uA = reinterpret_cast<std::uint8_t*>(planesA);
    auto* uB = reinterpret_cast<std::uint8_t*>(planesB);
    auto* terms = reinterpret_cast<std::uint16_t*>(prod);

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
    if (fp8) {
        steps.push_back({ev::Slice, [=] {
                             device_check(dev,
                                          oz2_split_digits(dev, dAf, (int)M, (int)K, (int)K, 0, dltA, &ddesc, uA, 2,
                                                           (int)Mg, (int)Kg, strideA),
                                          "slice A");
                             device_check(dev,
                                          oz2_split_digits(dev, dBf, (int)K, (int)N, (int)N, 1, dltB, &ddesc, uB, 3,
                                                           (int)Ng, (int)Kg, strideB),
                                          "slice B");
                         }});
        steps.push_back({ev::Gemm, [=] {
                             device_check(dev,
                                          oz2_gemm_groups_f8(dev, uA, uB, terms, (int)Mg, (int)Ng, (int)Kg, &gdesc, 1,
                                                             (int)Ng, strideA, strideB, strideC),
                                          "products");
                         }});
        steps.push_back({ev::Recon, [=] {
                             device_check(dev,
                                          oz2_crt_terms_f64(dev, terms, (int)M, (int)N, (int)Ng, strideC, (int)nterms,
                                                            term_mod.data(), &cdesc, dltA, dltB, out, (int)N),
                                          "reconstruction");
                         }});
    } else {
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
                                          oz2_gemm_digits(dev, planesA, planesB, prod, (int)Mg, (int)Ng, (int)Kg,
                                                          (int)S, (int)Ng, strideA, strideB, strideC, &cdesc),
                                          "products");
                         }});
        steps.push_back({ev::Recon, [=] {
                             device_check(dev,
                                          oz2_crt_digits_f64(dev, prod, (int)M, (int)N, (int)Ng, strideC, &cdesc, dltA,
                                                             dltB, out, (int)N),
                                          "reconstruction");
                         }});
    }
    // products: one per modulus (INT8) or the FP8 route's digit products (sum of the outputs' pairs)
    const std::uint32_t nprod = fp8 ? (std::uint32_t)plan.mo.nprod : S;

    auto* host = static_cast<double*>(ws.host(kHostC, sizeof(double) * M * (std::size_t)N));
    run_pipeline(dev, steps, 2, out, host, (std::size_t)M * N, flags, 2.0 * M * (double)N * K * nprod, nprod);
    Info info{Scheme::II, p.options.format};
    info.moduli = S;
    info.integer_bits = (std::uint32_t)plan.b;
    info.reconstruction_passes = plan.two_pass ? 2 : 1;
    return {host, info};
}

}  // namespace ozTTgemm::detail

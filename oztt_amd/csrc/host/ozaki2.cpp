// Ozaki scheme II driver (INT8 residues, or the FP8 route's e4m3 digits): one FP64 GEMM on the GPU.
// Every format runs INT8 residues unless the plan keeps the FP8 route's digits (plan_scheme2: FP8
// under Transport::Automatic, and widths beyond the INT8 residues').
//
// Pipeline of the reference's ozaki2.cpp:439-478: plan (moduli, width b, passes) -> upload the FP64
// operands -> scale (row/column maxima, exponent deltas) -> slice -> products -> CRT reconstruction
// to FP64 -> read back and check the range flags. Like the reference (plan.hpp:386-444), the output
// is computed in row bands when the device memory is short: the planes of A and the product terms
// are then per band of rows, while A, B, B's planes and C stay whole (band_rows). Up to about
// 60000^3 (INT8, 18 moduli) one MI355X (288 GB) holds everything at once, and there is one band.
//   INT8: slice = int8 residue planes per modulus; products = one exact int32 GEMM per modulus,
//   reduced in the epilogue to the CRT digit (uint8); reconstruction from the S digit planes.
//   FP8 (ozaki2.cpp:228-318 run_digit_gemms): slice = e4m3 digit planes (2 or 3 per modulus);
//   products = the digit products on the FP8 matrix cores, one output per group of equal-weight
//   products, each reduced in the epilogue to its share of the CRT digit (uint16), which replaces
//   the reference's composition launch; reconstruction from the output planes.
//
// Device layout (all row-major, zero-padded so that every kernel runs unguarded full tiles):
//   A (M x K f64), B (K x N f64), dA[M], dB[N] int32 (range flags: Workspace::flag_slots);
//   planes of A (per band of Mb rows): P x Mbg x Kg bytes, of B: P x Ng x Kg bytes (B transposed), both K-major in the
//   GEMM's OZ_BLOCK tiles (1 KB blocks of 16 rows x 64 K-bytes), Mg, Ng multiples of 256 and Kg of
//   64 (P = S residue planes, or the FP8 route's digit planes);
//   product digits (per band): S x Mbg x Ng uint8 (INT8) or nout x Mbg x Ng uint16 (FP8); output: M x N f64.
#include <chrono>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>

#include "backend.hpp"
#include "evaluation.hpp"
#include "pipeline.hpp"
#include "plan2.hpp"

namespace ozTTgemm::detail {
namespace {

namespace ev = ::ozTTgemm::evaluation;

enum Slot { kA = 0, kB, kDA, kDB, kPlanesA, kPlanesB, kProducts, kOut };

std::uint32_t round_up(std::uint32_t v, std::uint32_t q) { return (v + q - 1) / q * q; }

}  // namespace

Output ozaki2_run(Device& D, const Problem& p) {
    oz_dev* dev = D.dev;
    ev::Settings* es = ev::active();
    std::optional<unsigned> fixed_b;
    if (es && es->fixed_bits) fixed_b = es->fixed_bits;
    const std::uint32_t M = p.m, N = p.n, K = p.k;
    Workspace& ws = *D.ws;
    // the operands go up while the host plans (they are page-locked, the copies are asynchronous);
    // resident operands are already there
    const double* dAf = p.a_dev;
    const double* dBf = p.b_dev;
    if (!dAf) {
        auto* a = static_cast<double*>(ws.get(kA, sizeof(double) * M * (std::size_t)K));
        auto* b = static_cast<double*>(ws.get(kB, sizeof(double) * K * (std::size_t)N));
        device_check(dev, oz_memcpy_h2d_async(dev, a, p.a, sizeof(double) * M * (std::size_t)K), "upload A");
        device_check(dev, oz_memcpy_h2d_async(dev, b, p.b, sizeof(double) * K * (std::size_t)N), "upload B");
        dAf = a;
        dBf = b;
    }
    const std::shared_ptr<const Plan2> planp =
        p.plan ? std::static_pointer_cast<const Plan2>(p.plan)
               : std::make_shared<const Plan2>(plan_scheme2(p.a, p.b, p.m, p.n, p.k, p.options.format,
                                                            p.options.max_moduli, p.options.reconstruction, fixed_b,
                                                            p.options.transport == Transport::Int8Residues &&
                                                                !(es && es->fp8_matrix_cores),
                                                            !(es && es->full_window)));
    const Plan2& plan = *planp;
    const bool fp8 = plan.fp8_digits;
    const std::uint32_t S = (std::uint32_t)plan.S;
    const std::uint32_t Ng = round_up(N, 256), Kg = round_up(K, 64);
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

    // Row bands: A's planes and the product terms are per band; A, B, B's planes, the deltas and C
    // are whole. One band (all of M) unless device memory requires more.
    const std::size_t fixed = sizeof(double) * ((p.a_dev ? 0 : (std::size_t)M * K + (std::size_t)K * N) +
                                                (p.c_dev ? 0 : (std::size_t)M * N)) +
                              (std::size_t)nplanes * Ng * Kg + sizeof(std::int32_t) * (M + N) + 256;
    const std::size_t per_row = (std::size_t)nplanes * Kg + (std::size_t)nterms * Ng * term_bytes;
    const std::uint32_t Mb = band_rows(D, M, fixed, per_row, {kPlanesA, kProducts});
    const std::uint32_t Mbg = round_up(Mb, 256);
    const std::uint32_t nbands = (M + Mb - 1) / Mb;

    auto* dltA = static_cast<std::int32_t*>(ws.get(kDA, sizeof(std::int32_t) * M));
    auto* dltB = static_cast<std::int32_t*>(ws.get(kDB, sizeof(std::int32_t) * N));
    const long long strideA = (long long)Mbg * Kg, strideB = (long long)Ng * Kg, strideC = (long long)Mbg * Ng;
    auto* planesA = static_cast<std::int8_t*>(ws.get(kPlanesA, (std::size_t)nplanes * strideA));
    auto* planesB = static_cast<std::int8_t*>(ws.get(kPlanesB, (std::size_t)nplanes * strideB));
    auto* prod = static_cast<std::uint8_t*>(ws.get(kProducts, (std::size_t)nterms * strideC * term_bytes));
    auto* out = p.c_dev ? p.c_dev : static_cast<double*>(ws.get(kOut, sizeof(double) * M * (std::size_t)N));
    auto* uA = reinterpret_cast<std::uint8_t*>(planesA);
    auto* uB = reinterpret_cast<std::uint8_t*>(planesB);
    auto* terms = reinterpret_cast<std::uint16_t*>(prod);

    const int shift = plan.shift();
    Workspace* wsp = &ws;
    std::vector<Step> steps;
    steps.push_back({ev::Scale, [=] {
                         // the range flags: this pass's slot, and the next pass's cleared (Workspace::flag_slots)
                         const Workspace::FlagSlots fs = wsp->flag_slots();
                         // Scheme II rounds the BF16 of the maxima up (ozaki2.cpp:143-146)
                         device_check(dev,
                                      oz_scale_pair_f64(dev, dAf, (int)M, (int)K, (int)K, dBf, (int)N, (int)N, 1, shift,
                                                        dltA, dltB, fs.use, fs.clear),
                                      "scale");
                         wsp->flags_issued();
                     }});
    // B's planes once, then per band: A's planes, the products, the reconstruction of the band's rows
    // (one band: A's and B's planes in one launch)
    if (fp8 && nbands == 1)
        steps.push_back({ev::Slice, [=] {
                             device_check(dev,
                                          oz2_split_digits_pair(dev, dAf, (int)M, (int)K, (int)K, dltA, dBf, (int)N,
                                                                (int)N, dltB, &ddesc, uA, uB, (int)Mbg, (int)Ng,
                                                                (int)Kg),
                                          "slice");
                         }});
    else if (fp8)
        steps.push_back({ev::Slice, [=] {
                             device_check(dev,
                                          oz2_split_digits(dev, dBf, (int)K, (int)N, (int)N, 1, dltB, &ddesc, uB, 3,
                                                           (int)Ng, (int)Kg, strideB),
                                          "slice B");
                         }});
    else if (nbands > 1)
        steps.push_back({ev::Slice, [=] {
                             device_check(dev,
                                          oz2_split_int8(dev, dBf, (int)K, (int)N, (int)N, 1, dltB, &mdesc, planesB, 3,
                                                         (int)Ng, (int)Kg, strideB),
                                          "slice B");
                         }});
    else  // one band: A's and B's planes in one launch
        steps.push_back({ev::Slice, [=] {
                             device_check(dev,
                                          oz2_split_pair_int8(dev, dAf, (int)M, (int)K, (int)K, dltA, dBf, (int)N,
                                                              (int)N, dltB, &mdesc, planesA, planesB, (int)Mbg,
                                                              (int)Ng, (int)Kg),
                                          "slice");
                         }});
    for (std::uint32_t band = 0; band < nbands; band++) {
        const std::uint32_t r0 = band * Mb, rows = std::min(Mb, M - r0), rowsg = round_up(rows, 256);
        const double* Ab = dAf + (std::size_t)r0 * K;
        const std::int32_t* dAb = dltA + r0;
        double* ob = out + (std::size_t)r0 * N;
        if (fp8) {
            if (nbands > 1)
                steps.push_back({ev::Slice, [=] {
                                     device_check(dev,
                                                  oz2_split_digits(dev, Ab, (int)rows, (int)K, (int)K, 0, dAb, &ddesc,
                                                                   uA, 2, (int)rowsg, (int)Kg, strideA),
                                                  "slice A");
                                 }});
            steps.push_back({ev::Gemm, [=] {
                                 device_check(dev,
                                              oz2_gemm_groups_f8(dev, uA, uB, terms, (int)rowsg, (int)Ng, (int)Kg,
                                                                 &gdesc, 1, (int)Ng, strideA, strideB, strideC),
                                              "products");
                             }});
            steps.push_back({ev::Recon, [=] {
                                 device_check(dev,
                                              oz2_crt_terms_f64(dev, terms, (int)rows, (int)N, (int)Ng, strideC,
                                                                (int)nterms, term_mod.data(), &cdesc, dAb, dltB, ob,
                                                                (int)N),
                                              "reconstruction");
                             }});
        } else {
            if (nbands > 1)
                steps.push_back({ev::Slice, [=] {
                                     device_check(dev,
                                                  oz2_split_int8(dev, Ab, (int)rows, (int)K, (int)K, 0, dAb, &mdesc,
                                                                 planesA, 2, (int)rowsg, (int)Kg, strideA),
                                                  "slice A");
                                 }});
            steps.push_back({ev::Gemm, [=] {
                                 device_check(dev,
                                              oz2_gemm_digits(dev, planesA, planesB, prod, (int)rowsg, (int)Ng,
                                                              (int)Kg, (int)S, (int)Ng, strideA, strideB, strideC,
                                                              &cdesc),
                                              "products");
                             }});
            steps.push_back({ev::Recon, [=] {
                                 device_check(dev,
                                              oz2_crt_digits_f64(dev, prod, (int)rows, (int)N, (int)Ng, strideC,
                                                                 &cdesc, dAb, dltB, ob, (int)N),
                                              "reconstruction");
                             }});
        }
    }
    // products: one per modulus (INT8) or the FP8 route's digit products (sum of the outputs' pairs)
    const std::uint32_t nprod = fp8 ? (std::uint32_t)plan.mo.nprod : S;

    // the pass the configuration calls for: scale once; B's slice once and A's per band (one band:
    // both in one step); one product and one reconstruction step per band; and the regions it writes
    PassShape shape;
    shape.steps[ev::Scale] = 1;
    shape.steps[ev::Slice] = nbands == 1 ? 1 : 1 + nbands;
    shape.steps[ev::Gemm] = nbands;
    shape.steps[ev::Recon] = nbands;
    shape.written = {{dltA, sizeof(std::int32_t) * M},
                     {dltB, sizeof(std::int32_t) * N},
                     {planesA, (std::size_t)nplanes * strideA},
                     {planesB, (std::size_t)nplanes * strideB},
                     {prod, (std::size_t)nterms * strideC * term_bytes},
                     {out, sizeof(double) * M * (std::size_t)N}};
    auto* host = p.c_dev ? nullptr : static_cast<double*>(ws.host(kHostC, sizeof(double) * M * (std::size_t)N));
    run_pipeline(dev, steps, shape, out, host, (std::size_t)M * N, ws, 2.0 * M * (double)N * K * nprod, nprod);
    Info info{Scheme::II, p.options.format};
    // the format's route under Transport::Automatic (the reference's Info: for BF16, FP16, TF32, BFP8,
    // BFP4 and BFP2 also when INT8 residues carry it); the moduli that computed under Int8Residues
    info.moduli = (std::uint32_t)(p.options.transport == Transport::Int8Residues ? plan.mo.m.size()
                                                                                 : plan.route.m.size());
    info.integer_bits = (std::uint32_t)plan.b;
    info.reconstruction_passes = plan.two_pass ? 2 : 1;
    return {host, info, planp};
}

}  // namespace ozTTgemm::detail

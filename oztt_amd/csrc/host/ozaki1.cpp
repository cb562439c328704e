// Ozaki scheme I driver: one FP64 GEMM on the GPU, for every format.
//
// Pipeline of the reference's src/ozaki1.cpp run(): number of slices p (given, or chosen from the
// input, auto_precision.hpp:506) and the issue plan (plan.hpp:223) -> upload the FP64 operands ->
// scale (row/column maxima to BF16, deltas nshift - e) -> p slices per operand (radix 254 for INT8,
// 64 for BF16/FP16/TF32/BFP8, 32 for FP8, 14 for BFP4, 2 for BFP2) -> the diagonal partial products
// P_d = sum_{i<=d} A_i B_{d-i} -> Horner reconstruction in triple-float and FP64 assembly.
//
// The digits of every format are integers of at most 7 bits, so all products run on the INT8 matrix
// cores: one exact int32 accumulation per diagonal over its d+1 pairs concatenated along K. For INT8
// that is the reference's single-K-block plan (plan.hpp:187-195); for the FP32-product formats it is
// the exact int32 sum S_d the reference accumulates over pairs and K blocks before its deferred
// reconstruction (plan.hpp:95-128), so the reconstruction reads the same integers. When those sums
// could overflow int32 over all of K (FP32-product formats, plan issue.defer false), the reference
// reconstructs K block by K block (plan.hpp:104-109): here each block's diagonals are summed exactly
// (at most 2^24), and the reconstruction adds the limbs carried from the previous blocks, as the
// reference's FP32-input kernel does. The reference's panels reduce to one launch per stage on one
// MI355X; its row bands (plan.hpp:386-444) remain for problems beyond the device memory (A's slices
// and the partial sums are then per band, band_rows).
//
// Device layout: A (M x K f64), B (K x N f64), dA[M], dB[N] int32 (the range flags: Workspace::flag_slots);
// slices of A: p planes of Mbg x Kg int8 per band of rows, of B: p planes of Ng x Kg (B transposed), both in the GEMM's
// OZ_BLOCK tiles (Mbg, Ng multiples of 256, Kg of 64); partial sums (per band): p planes of Mbg x Ng
// int32; output: M x N f64.
#include <memory>
#include <stdexcept>

#include "backend.hpp"
#include "evaluation.hpp"
#include "pipeline.hpp"
#include "plan1.hpp"

namespace ozTTgemm::detail {
namespace {

namespace ev = ::ozTTgemm::evaluation;

enum Slot { kA = 0, kB, kDA, kDB, kSlicesA, kSlicesB, kPartial, kOut, kLimbs };

std::uint32_t round_up(std::uint32_t v, std::uint32_t q) { return (v + q - 1) / q * q; }

}  // namespace

Output ozaki1_run(Device& D, const Problem& p) {
    oz_dev* dev = D.dev;
    const Oz1Format& f = oz1_format((int)p.options.format);
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
    const std::shared_ptr<const Plan1> planp =
        p.plan ? std::static_pointer_cast<const Plan1>(p.plan)
               : std::make_shared<const Plan1>(plan_scheme1(p.a, p.b, p.m, p.n, p.k, p.options.slices, f));
    const Plan1& plan = *planp;
    const std::uint32_t P = (std::uint32_t)plan.p;
    const std::uint32_t Ng = round_up(N, 256);
    // K blocks: one (the whole K) unless the FP32-product format's sums over all of K could overflow
    // int32 (issue.defer false); then each block's diagonals are summed exactly and the
    // reconstruction carries its limbs from block to block (plan.hpp:104-109). The evaluation hook
    // force_kc selects that mode with a given block length.
    IssuePlan1 issue = plan.issue;
    ev::Settings* es = ev::active();
    if (es && es->force_kc && !f.int32_partial && K % es->force_kc == 0) {
        issue.Kc = es->force_kc;
        issue.nkb = K / es->force_kc;
        issue.defer = false;
    }
    const bool by_block = !f.int32_partial && !issue.defer;
    const std::uint32_t Kc = by_block ? issue.Kc : K, nkb = by_block ? issue.nkb : 1u;
    const std::uint32_t Kbg = round_up(Kc, 64);  // a block's K in the GEMM's tiles
    if ((std::uint64_t)P * Kbg * f.dmax * f.dmax > 0x7FFFFFFFull)
        throw std::logic_error("scheme I plan: the padded K breaks the int32 exactness of a diagonal");
    const oz1_recon_dev rdesc{(int)P, f.radix, plan.signmag ? 1 : 0, plan.nsmall, plan.Whi, plan.Wlo, plan.qw};

    // Row bands: A's slices and the partial sums are per band of rows; A, B, B's slices (of every K
    // block), the deltas, the limbs and C are whole. One band (all of M) unless device memory
    // requires more.
    const std::size_t fixed = sizeof(double) * ((p.a_dev ? 0 : (std::size_t)M * K + (std::size_t)K * N) +
                                                (p.c_dev ? 0 : (std::size_t)M * N)) +
                              (std::size_t)nkb * P * Ng * Kbg + sizeof(std::int32_t) * (M + N) +
                              (by_block ? 3 * sizeof(float) * (std::size_t)M * N : 0) + 256;
    const std::size_t per_row = (std::size_t)P * Kbg + sizeof(std::int32_t) * (std::size_t)P * Ng;
    const std::uint32_t Mb = band_rows(D, M, fixed, per_row, {kSlicesA, kPartial});
    const std::uint32_t Mbg = round_up(Mb, 256);
    const std::uint32_t nbands = (M + Mb - 1) / Mb;

    auto* dltA = static_cast<std::int32_t*>(ws.get(kDA, sizeof(std::int32_t) * M));
    auto* dltB = static_cast<std::int32_t*>(ws.get(kDB, sizeof(std::int32_t) * N));
    const long long strideA = (long long)Mbg * Kbg, strideB = (long long)Ng * Kbg, strideP = (long long)Mbg * Ng;
    auto* slA = static_cast<std::int8_t*>(ws.get(kSlicesA, (std::size_t)P * strideA));
    auto* slB = static_cast<std::int8_t*>(ws.get(kSlicesB, (std::size_t)nkb * P * strideB));
    auto* part = static_cast<std::int32_t*>(ws.get(kPartial, sizeof(std::int32_t) * (std::size_t)P * strideP));
    auto* out = p.c_dev ? p.c_dev : static_cast<double*>(ws.get(kOut, sizeof(double) * M * (std::size_t)N));
    auto* limbs = by_block ? static_cast<float*>(ws.get(kLimbs, 3 * sizeof(float) * (std::size_t)M * N)) : nullptr;
    const long long limb_stride = (long long)M * N;

    Workspace* wsp = &ws;
    std::vector<Step> steps;
    steps.push_back({ev::Scale, [=] {
                         // the range flags: this pass's slot, and the next pass's cleared (Workspace::flag_slots)
                         const Workspace::FlagSlots fs = wsp->flag_slots();
                         // BF16 of the maxima rounded as the format requires, target 2^nshift (format.hpp:76-101)
                         device_check(dev,
                                      oz_scale_pair_f64(dev, dAf, (int)M, (int)K, (int)K, dBf, (int)N, (int)N,
                                                        (int)f.ceil, f.nshift, dltA, dltB, fs.use, fs.clear),
                                      "scale");
                         wsp->flags_issued();
                     }});
    // B's slices once (per K block: rows kb Kc.. of B), then per band and K block: A's slices (columns
    // kb Kc.. of the band's rows), the diagonal products, the reconstruction. With one K block and one
    // band, A's and B's slices are one launch.
    const bool paired = nkb == 1 && nbands == 1;
    for (std::uint32_t kb = 0; kb < (paired ? 0u : nkb); kb++) {
        const double* Bk = dBf + (std::size_t)kb * Kc * N;
        std::int8_t* slBk = slB + (std::size_t)kb * P * strideB;
        steps.push_back({ev::Slice, [=] {
                             device_check(dev,
                                          oz1_split_int8(dev, Bk, (int)Kc, (int)N, (int)N, 1, dltB, (int)P, f.radix,
                                                         f.dmax, slBk, 3, (int)Ng, (int)Kbg, strideB),
                                          "slice B");
                         }});
    }
    for (std::uint32_t band = 0; band < nbands; band++) {
        const std::uint32_t r0 = band * Mb, rows = std::min(Mb, M - r0), rowsg = round_up(rows, 256);
        const std::int32_t* dAb = dltA + r0;
        double* ob = out + (std::size_t)r0 * N;
        for (std::uint32_t kb = 0; kb < nkb; kb++) {
            const double* Ab = dAf + (std::size_t)r0 * K + (std::size_t)kb * Kc;
            const std::int8_t* slBk = slB + (std::size_t)kb * P * strideB;
            float* lb = limbs ? limbs + (std::size_t)r0 * N : nullptr;
            const int first = kb == 0, last = kb + 1 == nkb;
            if (paired)
                steps.push_back({ev::Slice, [=] {
                                     device_check(dev,
                                                  oz1_split_pair_int8(dev, dAf, (int)M, (int)K, (int)K, dltA, dBf,
                                                                      (int)N, (int)N, dltB, (int)P, f.radix, f.dmax,
                                                                      slA, slB, (int)Mbg, (int)Ng, (int)Kbg),
                                                  "slice A and B");
                                 }});
            else
                steps.push_back({ev::Slice, [=] {
                                     device_check(dev,
                                                  oz1_split_int8(dev, Ab, (int)rows, (int)Kc, (int)K, 0, dAb, (int)P,
                                                                 f.radix, f.dmax, slA, 2, (int)rowsg, (int)Kbg,
                                                                 strideA),
                                                  "slice A");
                                 }});
            steps.push_back({ev::Gemm, [=] {
                                 device_check(dev,
                                              oz1_gemm_diag_i8(dev, slA, slBk, part, (int)rowsg, (int)Ng, (int)Kbg,
                                                               (int)P, f.dmax, (int)Ng, strideA, strideB, strideP),
                                              "diagonal products");
                             }});
            if (by_block)
                steps.push_back({ev::Recon, [=] {
                                     device_check(dev,
                                                  oz1_recon_block_f64(dev, part, (int)rows, (int)N, (int)Ng, strideP,
                                                                      &rdesc, first, last, lb, limb_stride, (int)N,
                                                                      dAb, dltB, ob, (int)N),
                                                  "reconstruction");
                                 }});
            else
                steps.push_back({ev::Recon, [=] {
                                     device_check(dev,
                                                  oz1_recon_f64(dev, part, (int)rows, (int)N, (int)Ng, strideP, &rdesc,
                                                                dAb, dltB, ob, (int)N),
                                                  "reconstruction");
                                 }});
        }
    }
    // P(P+1)/2 slice-pair products of 2*M*N*K operations each
    const unsigned pairs = P * (P + 1) / 2;
    // the pass the configuration calls for: scale once; B's slices once per K block; per band and K
    // block A's slices, the diagonal products and a reconstruction step (one band and one K block:
    // both operands' slices in one step); and the regions it writes
    PassShape shape;
    shape.steps[ev::Scale] = 1;
    shape.steps[ev::Slice] = paired ? 1 : nkb + nbands * nkb;
    shape.steps[ev::Gemm] = nbands * nkb;
    shape.steps[ev::Recon] = nbands * nkb;
    shape.written = {{dltA, sizeof(std::int32_t) * M},
                     {dltB, sizeof(std::int32_t) * N},
                     {slA, (std::size_t)P * strideA},
                     {slB, (std::size_t)nkb * P * strideB},
                     {part, sizeof(std::int32_t) * (std::size_t)P * strideP},
                     {out, sizeof(double) * M * (std::size_t)N}};
    if (limbs) shape.written.push_back({limbs, 3 * sizeof(float) * (std::size_t)M * N});
    auto* host = p.c_dev ? nullptr : static_cast<double*>(ws.host(kHostC, sizeof(double) * M * (std::size_t)N));
    run_pipeline(dev, steps, shape, out, host, (std::size_t)M * N, ws, 2.0 * M * (double)N * K * pairs, pairs);
    Info info{Scheme::I, p.options.format};
    info.slices = P;
    return {host, info, planp};
}

}  // namespace ozTTgemm::detail

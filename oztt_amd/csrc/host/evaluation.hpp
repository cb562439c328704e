// Evaluation hooks: per-phase timing and whole-pass timing of one GEMM call, and the evaluation
// utilities (input generator, output hash, binary128 reference) of the paper evaluator.
//
// Counterpart of the reference's evaluation_hooks.hpp:29-219 and evaluation/numerics.hpp. While a
// Scope is active on the calling thread, a backend
//   - times each phase (scale, slice, gemm, compose, recon) with HIP events around every device
//     step on its stream (in warm passes after the replays, when there are replays),
//   - records every device step of the call; fills every region the pass writes with a sentinel
//     and replays the pass once, counting its steps per phase against the plan's; then replays it
//     `warmup` times untimed and `repeats` times between two events (inputs and intermediates
//     resident in HBM, no host work inside), checks that the output is still bit-identical to the
//     first pass, and reports the average whole-pass time.
// Without a Scope the hooks cost nothing. The library itself never activates one.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace ozTTgemm::evaluation {

enum Phase { Scale = 0, Slice, Gemm, Compose, Recon, PhaseCount };

struct Settings {
    // inputs
    unsigned fixed_bits = 0;  // Scheme II: width b fixed by the caller (0: chosen from the input)
    int warmup = 0;           // untimed whole-pass replays
    int repeats = 0;          // timed whole-pass replays (0: no replay)
    unsigned max_band_rows = 0;  // cap on the rows of a band (0: bands only when memory requires)
    unsigned force_kc = 0;       // Scheme I, FP32-product formats: reconstruct K block by K block with
                                 // blocks of this length (0: as planned; it must divide the padded K)
    int replay_drop_phase = -1;  // self-test of the whole-pass check: its checking replay leaves out the
                                 // steps of this phase (so whole_checked must come out false), and
                                 // nothing is timed; -1 (the default) replays every step
    bool fp8_matrix_cores = false;  // Scheme II FP8: the FP8 route's e4m3 digit products on the FP8 matrix
                                    // cores also under Transport::Int8Residues (same C)
    bool full_window = false;       // Scheme II INT8 residues: compute with the set for the window
                                    // K 2^(2b), not the smaller one the operands' bound allows (same C)
    // outputs
    double phase_ms[PhaseCount] = {};  // device time of each phase: the average of up to 5 warm passes
                                       // after the replays (the first pass when there are none)
    double whole_ms = 0;               // average time of one replayed whole pass
    bool whole_checked = false;        // the replays are sound: whole_sentinel, the replayed steps per
                                       // phase equal the plan's, and the output after the timed
                                       // replays is bit-identical to the first pass
    bool whole_sentinel = false;       // every region the pass writes was filled with a sentinel, and one
                                       // replay then rewrote the whole output with the first pass's bits
    unsigned whole_steps[PhaseCount] = {};     // device steps issued per phase by the checking replay
    unsigned expected_steps[PhaseCount] = {};  // device steps per phase that the plan calls for
    unsigned partial_products = 0;     // low-precision matrix products per call (S or slice pairs)
    double product_ops = 0;            // algorithmic operations of the product phase (2*M*N*K*products)
    double gemm_launch_ms = 0;         // device time of the product launches of one pass, from their own
                                       // dispatches (oz_time_products_begin) in whole-pass replays right
                                       // after the timed ones (up to `repeats` passes, 58 launches in all)
    int gemm_launches = 0;             // product-kernel launches per pass (one per row band)
    bool plan_reused = false;          // resident operands: the call ran the plan kept from an earlier call
};

// Activates `s` for the calling thread until destruction (not nestable).
class Scope {
public:
    explicit Scope(Settings& s);
    ~Scope();
    Scope(const Scope&) = delete;
    Scope& operator=(const Scope&) = delete;
};

Settings* active() noexcept;

// ---- evaluation utilities (reference evaluation/numerics.hpp) ---------------------------------
// Inputs of the paper evaluator with a seed (numerics.hpp:19-38): mt19937(seed); phi < 0 gives
// uniform [-1,1); otherwise x = (u - 0.5) * exp(phi * z), u ~ U(0,1) drawn before z ~ N(0,1); all
// of A (na elements) first, then B.
void inputs(unsigned seed, double phi, std::size_t na, std::size_t nb, double* a, double* b);
// FNV-style hash of the bit patterns (numerics.hpp:46-57).
std::uint64_t output_hash(const double* c, std::size_t n);
// The Dot2 reference GEMM (numerics.hpp:58-93) for rows [r0, r1) of C = A B (A: M x K, B: K x N,
// row-major): head and tail of each compensated dot product, Chi/Clo hold (r1 - r0) x N.
void reference_gemm(const double* A, const double* B, std::uint32_t M, std::uint32_t K, std::uint32_t N,
                    std::uint32_t r0, std::uint32_t r1, double* Chi, double* Clo);
// Relative Frobenius error of C against the Dot2 reference and effective bits -log2 of it
// (numerics.hpp:98-127).
struct Accuracy {
    double rel_fro = 0, ebits = 0;
};
Accuracy accuracy(const double* C, const double* Chi, const double* Clo, std::size_t n);
// Binary128 products for sampled output elements (rows[t], cols[t]).
void gemm_quad_sample(const double* A, const double* B, int M, int N, int K, int nsample, const int* rows,
                      const int* cols, double* out);

}  // namespace ozTTgemm::evaluation

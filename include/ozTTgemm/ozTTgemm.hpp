// SPDX-License-Identifier: Apache-2.0
//
// ozTTgemm for AMD Instinct MI355X: FP64 matrix multiplication with the Ozaki schemes.
//
// Drop-in public interface of the reference library (reference include/ozTTgemm/ozTTgemm.hpp:21-123):
// the same namespace, types, members and defaults, the same validation and exception contract.
// Only the device changes: the low-precision products run on the CDNA4 matrix cores of one MI355X
// through hand-written HIP kernels (include/oz_hip.h), and the splitting and reconstruction run on
// the same GPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <span>
#include <string>
#include <vector>

#define OZTTGEMM_VERSION_MAJOR 0
#define OZTTGEMM_VERSION_MINOR 1
#define OZTTGEMM_VERSION_PATCH 0

namespace ozTTgemm {

// Scheme I: slices and slice-pair products. Scheme II: residues modulo small coprime moduli and
// the Chinese remainder theorem.
enum class Scheme { I, II };

// Format of the low-precision matrix products. The enumerators are those of the reference; a
// format that this build does not implement reports is_available() == false and is rejected.
enum class Format { BF16, FP16, TF32, BFP8, FP8, INT8, BFP4, BFP2 };

// Scheme II reconstruction passes. Automatic: one pass when an error estimate from the input
// statistics allows it, two otherwise.
enum class Reconstruction { Automatic, OnePass, TwoPass };

// Scheme II only, an extension of the reference's interface (which has no such option): how the
// products of a format's plan run on the GPU. Both transports give the same C bit for bit (the
// reconstruction is exact, so C depends on the plan's width b only) and the same plan.
//   Automatic: the format's own digits on its own matrix instructions where this build has them
//     (INT8 residues on the INT8 matrix cores; FP8: the reference's e4m3 digits on the FP8 matrix
//     cores), and INT8 residues at the plan's width for the formats whose digits have no matrix
//     instructions here (BF16, FP16, TF32, BFP8, BFP4, BFP2). Info is the reference's.
//   Int8Residues: INT8 residues at the plan's width for every format. On MI355X this is the fastest
//     transport: the FP8 and INT8 dense rates are equal, and the FP8 route needs two to three times
//     the products of INT8 residues for one width. Info.moduli then counts the INT8 moduli that
//     computed. A width beyond what INT8 residues hold (above about 84 bits) keeps the FP8 digits.
// Either way the set that computes can be smaller than the plan's: when the operands' own bound on
// the integer product A'B' (Cauchy-Schwarz on its rows and columns) needs fewer moduli, or on the
// FP8 digits fewer digit products, than the plan's window K 2^(2b), that set computes; C is the
// same bit for bit.
enum class Transport { Automatic, Int8Residues };

// Options of the scheme that is not selected must keep their defaults.
struct Options {
    Scheme scheme = Scheme::II;
    Format format = Format::BFP8;
    // Scheme I only: 0 chooses the number of slices from the input, 1..256 fixes it.
    std::uint32_t slices = 0;
    // Scheme II only: 0 leaves the number of moduli to the library, 1..24 limits it.
    std::uint32_t max_moduli = 0;
    // Scheme II only.
    Reconstruction reconstruction = Reconstruction::Automatic;
    // Scheme II only (extension, see Transport).
    Transport transport = Transport::Automatic;
};

struct DeviceOptions {
    // HIP device ordinal.
    int device_id = 0;
    // Kept for interface compatibility: the HIP code objects are built into the library, so no
    // kernel directory is needed. A non-empty value must name an existing directory.
    std::string kernel_directory;
};

// What a call used.
struct Info {
    Scheme scheme;
    Format format;
    std::uint32_t slices = 0;                 // scheme I: slices
    std::uint32_t moduli = 0;                 // scheme II: CRT moduli
    std::uint32_t integer_bits = 0;           // scheme II: width b of the scaled operands
    std::uint32_t reconstruction_passes = 0;  // scheme II: 1 or 2 (as planned)
    // Dimensions after zero padding (m and n to multiples of 64, k to a multiple of 32).
    std::size_t padded_m = 0, padded_n = 0, padded_k = 0;
};

// False for formats this build does not implement.
bool is_available(Format format) noexcept;
// "BF16", "FP16", "TF32", "BFP8", "FP8", "INT8", "BFP4" or "BFP2".
const char* format_name(Format format) noexcept;

class Context;

// A matrix kept on the GPU of a Context between calls: an extension of the reference's interface,
// which takes host spans only and moves and plans everything per call. A Matrix is immutable; it is
// made by Context::upload or as the result of Context::gemm, and belongs to that Context (using it
// with another Context throws std::invalid_argument). Copies share the same matrix. It may outlive
// its Context: the GPU stays open until the last Matrix is gone.
class Matrix {
public:
    Matrix() = default;  // empty
    std::size_t rows() const noexcept;
    std::size_t cols() const noexcept;
    explicit operator bool() const noexcept { return static_cast<bool>(s_); }

    struct State;  // opaque

private:
    friend class Context;
    std::shared_ptr<State> s_;
};

// Owns one GPU, opened lazily by the first valid GEMM. Calls through all contexts of a process are
// serialized.
class Context {
public:
    // Throws std::invalid_argument for a negative device_id or a kernel_directory that does not exist.
    explicit Context(DeviceOptions options = {});
    ~Context();
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    Context(Context&&) = delete;
    Context& operator=(Context&&) = delete;

    // C = A*B for contiguous row-major FP64 matrices A[m,k], B[k,n], C[m,n]. Dimensions must be
    // positive and the spans must hold exactly m*k, k*n and m*n elements. Inputs are consumed before
    // C is written, so they may overlap C. Inputs must be finite and every nonzero row maximum of A
    // and column maximum of B must lie in [2^-126, largest finite BF16].
    // Throws std::invalid_argument for invalid input (before the device is used and before C is
    // written), std::runtime_error for configurations that cannot be executed and for failures of
    // the HIP runtime, and std::bad_alloc if host memory runs out. Never prints, never terminates.
    Info gemm(std::span<const double> a, std::span<const double> b, std::span<double> c, std::size_t m, std::size_t n,
              std::size_t k, const Options& options = {});

    // Same as gemm(), returning C as a new vector.
    std::vector<double> multiply(std::span<const double> a, std::span<const double> b, std::size_t m, std::size_t n,
                                 std::size_t k, const Options& options = {});

    // ---- resident operands (extension) -------------------------------------------------------
    // Copies the row-major rows x cols matrix x to the GPU. Throws std::invalid_argument for zero or
    // mismatched dimensions and for NaN or infinite entries, std::runtime_error when the GPU cannot
    // be used.
    Matrix upload(std::span<const double> x, std::size_t rows, std::size_t cols);
    // C = A*B with A = a (m x k) and B = b (k x n) on the GPU: the same result, bit for bit, and the
    // same Info as gemm() on the host copies of a and b, with the same checks (the row maxima of a
    // and the column maxima of b in [2^-126, largest finite BF16]). Nothing is moved over PCIe but C
    // (none of it for the second form), and the plan of the pair (a, b) for these options is kept,
    // so later calls on the same pair skip the host planning.
    Info gemm(const Matrix& a, const Matrix& b, std::span<double> c, const Options& options = {});
    // Same, with C kept on the GPU as a new Matrix in c (its previous matrix, if c was the only
    // holder of it and it has C's shape, lends its device memory).
    Info gemm(const Matrix& a, const Matrix& b, Matrix& c, const Options& options = {});
    // Copies x back into out (rows*cols elements, row-major).
    void download(const Matrix& x, std::span<double> out);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace ozTTgemm

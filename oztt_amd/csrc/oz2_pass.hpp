// The whole Scheme II INT8 device pass of oz2_pass.hip, shared by its entry points: the layout of
// its intermediates in a workspace, the checks of its arguments, and the pass itself.
#pragma once
#include "oz_internal.hpp"

namespace oz2pass {

// Byte offsets, inside the workspace, of the exponent deltas of A's rows and B's columns, the S
// residue planes of A (Mg x Kg) and of B^T (Ng x Kg) and the S digit planes (Mg x Ng); every region
// starts on a 256-byte boundary. Mg, Ng: M, N rounded up to 256; Kg: K rounded up to 64.
struct PassLayout {
    int Mg, Ng, Kg;
    size_t dA, dB, planesA, planesB, digits, total;
};

// The workspace of a pass of M x N x K with S moduli; false for shapes outside the kernels' index range.
bool pass_layout(int M, int N, int K, int S, PassLayout* L);

// The descriptors must describe one plan: the same moduli (INT8: 2..255) in both, the shift of the
// width b with nd digits, and int32 products that stay exact over K (|C_s| <= Kg 127^2 < 2^31).
// Returns a message or nullptr.
const char* check_plan(const oz2_moduli_dev* mo, const oz2_crt_dev* crt, int Kg);

// Pointers, extents and leading dimensions; returns a message or nullptr.
const char* check_args(const double* A, int lda, const double* B, int ldb, const double* C, int ldc, int M, int N,
                       int K, const uint32_t* flags);

// The pass on a workspace of L.total bytes at `work` (checked arguments), ordered on dev's stream.
int run_pass(oz_dev* dev, const double* A, int lda, const double* B, int ldb, double* C, int ldc, int M, int N, int K,
             const oz2_moduli_dev* mo, const oz2_crt_dev* crt, uint32_t* flags, uint8_t* work, const PassLayout& L);

}  // namespace oz2pass

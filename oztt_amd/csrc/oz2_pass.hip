// Scheme II INT8, the whole device pass in one call: for device-resident FP64 operands and a plan
// made on the host (the moduli and CRT descriptors of include/oz_hip.h), C = A B through the same
// stage kernels the C++ backend issues one by one (reference ozaki2.cpp:439-478: scale, slice,
// products, reconstruction):
//   flags <- 0; row maxima of A and column maxima of B -> exponent deltas (oz_scale_pair_f64);
//   residue planes of A and of B^T in OZ_BLOCK tiles (oz2_split_pair_int8);
//   products reduced to CRT digits in the GEMM epilogue (oz2_gemm_digits);
//   exact CRT to FP64 (oz2_crt_digits_f64).
// Every launch is ordered on the handle's stream and nothing waits on the host, so a caller that
// keeps its operands on the GPU can queue many passes back to back.
//
// The intermediates live in a workspace: exponent deltas of A's rows and B's columns, then the S
// residue planes of A (Mg x Kg bytes each), of B^T (Ng x Kg) and the S digit planes (Mg x Ng), with
// Mg, Ng = M, N rounded up to 256 and Kg = K rounded up to 64 (the product kernel's tile grid;
// the splitter writes the padding as zeros). Each region starts on a 256-byte boundary.
#include "oz2_pass.hpp"

namespace oz2pass {

namespace {
size_t round256(size_t v) { return (v + 255) / 256 * 256; }
}  // namespace

bool pass_layout(int M, int N, int K, int S, PassLayout* L) {
    if (M <= 0 || N <= 0 || K <= 0 || S < 1 || S > OZ2_MAXS) return false;
    const long long Mg = ((long long)M + 255) / 256 * 256, Ng = ((long long)N + 255) / 256 * 256;
    const long long Kg = ((long long)K + 63) / 64 * 64;
    if (Mg > 0x7FFFFFFFll || Ng > 0x7FFFFFFFll || Kg > 0x7FFFFFFFll) return false;
    L->Mg = (int)Mg;
    L->Ng = (int)Ng;
    L->Kg = (int)Kg;
    size_t at = 0;
    L->dA = at;
    at += round256(sizeof(int32_t) * (size_t)M);
    L->dB = at;
    at += round256(sizeof(int32_t) * (size_t)N);
    L->planesA = at;
    at += (size_t)S * (size_t)Mg * (size_t)Kg;
    L->planesB = at;
    at += (size_t)S * (size_t)Ng * (size_t)Kg;
    L->digits = at;
    at += (size_t)S * (size_t)Mg * (size_t)Ng;
    L->total = at;
    return true;
}

const char* check_plan(const oz2_moduli_dev* mo, const oz2_crt_dev* crt, int Kg) {
    if (!mo || !crt) return "null plan descriptor";
    if (mo->S < 1 || mo->S > OZ2_MAXS || crt->S != mo->S) return "the moduli and CRT descriptors differ in S";
    if (mo->nd < 3 || mo->nd > 5 || crt->shift != crt->b - 20 * (mo->nd - 1)) return "the CRT shift is not b - 20 (nd - 1)";
    for (int s = 0; s < mo->S; s++)
        if (crt->m[s] < 2 || crt->m[s] > 255 || mo->m[s] != (float)crt->m[s] || crt->y[s] >= crt->m[s])
            return "the descriptors do not hold the same INT8 moduli";
    if ((long long)Kg * 127 * 127 > 0x7FFFFFFFll) return "K is too large for exact int32 products";
    return nullptr;
}

int run_pass(oz_dev* dev, const double* A, int lda, const double* B, int ldb, double* C, int ldc, int M, int N, int K,
             const oz2_moduli_dev* mo, const oz2_crt_dev* crt, uint32_t* flags, uint8_t* work, const PassLayout& L) {
    const int S = mo->S;
    auto* dA = reinterpret_cast<int32_t*>(work + L.dA);
    auto* dB = reinterpret_cast<int32_t*>(work + L.dB);
    auto* pA = reinterpret_cast<int8_t*>(work + L.planesA);
    auto* pB = reinterpret_cast<int8_t*>(work + L.planesB);
    auto* dg = work + L.digits;
    const long long sA = (long long)L.Mg * L.Kg, sD = (long long)L.Mg * L.Ng;
    if (int st = oz_fill_u32(dev, flags, 0u, 2)) return st;
    // Scheme II rounds the BF16 of the maxima up (reference ozaki2.cpp:143-146)
    if (int st = oz_scale_pair_f64(dev, A, M, K, lda, B, N, ldb, 1, crt->shift, dA, dB, flags, nullptr)) return st;
    if (int st = oz2_split_pair_int8(dev, A, M, K, lda, dA, B, N, ldb, dB, mo, pA, pB, L.Mg, L.Ng, L.Kg)) return st;
    if (int st = oz2_gemm_digits(dev, pA, pB, dg, L.Mg, L.Ng, L.Kg, S, L.Ng, sA, (long long)L.Ng * L.Kg, sD, crt))
        return st;
    return oz2_crt_digits_f64(dev, dg, M, N, L.Ng, sD, crt, dA, dB, C, ldc);
}

const char* check_args(const double* A, int lda, const double* B, int ldb, const double* C, int ldc, int M, int N,
                       int K, const uint32_t* flags) {
    if (!A || !B || !C || !flags) return "null pointer";
    if (M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < N || ldc < N) return "invalid extents or leading dimensions";
    if ((uintptr_t)flags & 3) return "flags must be 4-byte aligned";
    return nullptr;
}

}  // namespace oz2pass

using namespace oz2pass;

extern "C" int oz2_gemm_f64_workspace(int M, int N, int K, int S, size_t* bytes) {
    PassLayout L;
    if (!bytes || !pass_layout(M, N, K, S, &L)) return OZ_ERR_ARG;
    *bytes = L.total;
    return OZ_OK;
}

extern "C" int oz2_gemm_f64(oz_dev* dev, const double* A, int lda, const double* B, int ldb, double* C, int ldc, int M,
                            int N, int K, const oz2_moduli_dev* mo, const oz2_crt_dev* crt, uint32_t* flags,
                            void* work, size_t work_bytes) {
    if (int st = oz::use(dev)) return st;
    if (const char* e = check_args(A, lda, B, ldb, C, ldc, M, N, K, flags))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64: %s", e);
    PassLayout L;
    if (!mo || !pass_layout(M, N, K, mo->S, &L))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64: unsupported shape %dx%dx%d", M, N, K);
    if (const char* e = check_plan(mo, crt, L.Kg)) return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64: %s", e);
    if (!work || ((uintptr_t)work & 255) || work_bytes < L.total)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64: the workspace needs %zu bytes on a 256-byte boundary (%zu given)",
                        L.total, work_bytes);
    return run_pass(dev, A, lda, B, ldb, C, ldc, M, N, K, mo, crt, flags, static_cast<uint8_t*>(work), L);
}

// oz2_gemm_f64_noalloc: the whole Scheme II INT8 pass of oz2_gemm_f64 for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc). It takes no workspace and calls no allocating routine: its intermediates live in
// `scratch`, a file-scope device array of OZ2_NOALLOC_SCRATCH_BYTES that every GPU this library
// runs on holds until the process ends.
//
// In host code the array's name is only a stand-in, not a device address. Its address on a GPU is
// looked up once per device, with that device current (hipGetSymbolAddress), kept in `scratch_ptr`,
// and only that address is ever handed to a kernel. Every call on one GPU shares that GPU's array,
// which keeps the previous call's contents; the pass clears what must start at zero (the range
// flags) with a fill kernel and writes every other region in full before reading it. Calls that
// overlap on one GPU (two handles' streams, or two host threads) race for the array.
#include <mutex>

#include "oz2_pass.hpp"

static __device__ __align__(256) unsigned char scratch[OZ2_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};  // device address of `scratch` by device ordinal (null: not looked up yet)

// The device address of `scratch` on the handle's GPU, which oz::use has made current.
int scratch_of(oz_dev* dev, uint8_t** out) {
    if (dev->device < 0 || dev->device >= kMaxDevices)
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64_noalloc: device ordinal %d beyond %d", dev->device, kMaxDevices);
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return oz::fail(dev, OZ_ERR_HIP, "oz2_gemm_f64_noalloc: hipGetSymbolAddress(scratch): %s",
                            e != hipSuccess ? hipGetErrorString(e) : "null address");
        scratch_ptr[dev->device] = p;
    }
    *out = static_cast<uint8_t*>(scratch_ptr[dev->device]);
    return OZ_OK;
}

}  // namespace

extern "C" int oz2_gemm_f64_noalloc(oz_dev* dev, const double* A, int lda, const double* B, int ldb, double* C,
                                    int ldc, int M, int N, int K, const oz2_moduli_dev* mo, const oz2_crt_dev* crt,
                                    uint32_t* flags) {
    using namespace oz2pass;
    if (int st = oz::use(dev)) return st;
    if (const char* e = check_args(A, lda, B, ldb, C, ldc, M, N, K, flags))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64_noalloc: %s", e);
    PassLayout L;
    if (!mo || !pass_layout(M, N, K, mo->S, &L))
        return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64_noalloc: unsupported shape %dx%dx%d", M, N, K);
    if (const char* e = check_plan(mo, crt, L.Kg)) return oz::fail(dev, OZ_ERR_ARG, "oz2_gemm_f64_noalloc: %s", e);
    if (L.total > (size_t)OZ2_NOALLOC_SCRATCH_BYTES)
        return oz::fail(dev, OZ_ERR_ARG,
                        "oz2_gemm_f64_noalloc: %dx%dx%d with %d moduli needs %zu bytes of scratch; the limit is %zu "
                        "(use oz2_gemm_f64 with a workspace)",
                        M, N, K, mo->S, L.total, (size_t)OZ2_NOALLOC_SCRATCH_BYTES);
    uint8_t* work = nullptr;
    if (int st = scratch_of(dev, &work)) return st;
    return run_pass(dev, A, lda, B, ldb, C, ldc, M, N, K, mo, crt, flags, work, L);
}

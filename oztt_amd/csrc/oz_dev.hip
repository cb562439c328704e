// Device handle, memory and timing entry points of the C ABI (include/oz_hip.h).
// One handle owns one HIP stream on one GPU; the C++ context (host/context.cpp) opens it lazily on
// the first valid GEMM, as the reference opens its device (context.cpp:152-161).
#include "oz_internal.hpp"

#include <new>

namespace {
__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t v, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = v;
}

// n16 chunks of 16 bytes; every byte is read once and written once (the HBM reference transfer).
__global__ void copy16_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// Row r of dst: blockIdx.y + j gridDim.y; 256 columns per block along x. Rows and columns outside
// src are zero.
__global__ void pad_copy_f64_kernel(double* __restrict__ dst, int drows, int dcols, const double* __restrict__ src,
                                    int srows, int scols, int sld) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= dcols) return;
    for (int r = blockIdx.y; r < drows; r += gridDim.y)
        dst[(size_t)r * dcols + c] = (r < srows && c < scols) ? src[(size_t)r * sld + c] : 0.0;
}
}  // namespace

extern "C" {

int oz_device_count(int* count) {
    if (!count) return OZ_ERR_ARG;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return OZ_OK;
}

int oz_dev_open(int device_id, oz_dev** out) {
    if (!out || device_id < 0) return OZ_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device_id >= n) return OZ_ERR_HIP;
    oz_dev* d = new (std::nothrow) oz_dev;
    if (!d) return OZ_ERR_NOMEM;
    d->device = device_id;
    if (hipSetDevice(device_id) != hipSuccess || hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess) {
        delete d;
        return OZ_ERR_HIP;
    }
    for (auto& e : d->events) {
        if (hipEventCreate(&e) != hipSuccess) {
            oz_dev_close(d);
            return OZ_ERR_HIP;
        }
    }
    if (hipDeviceGetAttribute(&d->cus, hipDeviceAttributeMultiprocessorCount, device_id) != hipSuccess ||
        hipMalloc(&d->queue, 16 * sizeof(int)) != hipSuccess ||
        hipMemsetAsync(d->queue, 0, 16 * sizeof(int), d->stream) != hipSuccess) {  // ordered before every launch
        oz_dev_close(d);
        return OZ_ERR_HIP;
    }
    *out = d;
    return OZ_OK;
}

void oz_dev_close(oz_dev* dev) {
    if (!dev) return;
    (void)hipSetDevice(dev->device);
    if (dev->stream) (void)hipStreamSynchronize(dev->stream);
    for (auto& e : dev->events)
        if (e) (void)hipEventDestroy(e);
    if (dev->queue) (void)hipFree(dev->queue);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
}

const char* oz_last_error(const oz_dev* dev) { return dev ? dev->error.c_str() : "no device handle"; }

int oz_dev_malloc(oz_dev* dev, size_t bytes, void** ptr) {
    if (int st = oz::use(dev)) return st;
    if (!ptr) return oz::fail(dev, OZ_ERR_ARG, "oz_dev_malloc: null output pointer");
    *ptr = nullptr;
    if (bytes == 0) return OZ_OK;
    return oz::hip_check(dev, hipMalloc(ptr, bytes), "hipMalloc");
}

int oz_mem_info(oz_dev* dev, size_t* free_bytes, size_t* total_bytes) {
    if (int st = oz::use(dev)) return st;
    if (!free_bytes || !total_bytes) return oz::fail(dev, OZ_ERR_ARG, "oz_mem_info: null output pointer");
    return oz::hip_check(dev, hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
}

int oz_dev_free(oz_dev* dev, void* ptr) {
    if (int st = oz::use(dev)) return st;
    if (!ptr) return OZ_OK;
    return oz::hip_check(dev, hipFree(ptr), "hipFree");
}

int oz_memcpy_h2d(oz_dev* dev, void* dst, const void* src, size_t bytes) {
    if (int st = oz::use(dev)) return st;
    if (!bytes) return OZ_OK;
    if (int st = oz::hip_check(dev, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream), "hipMemcpyAsync H2D"))
        return st;
    return oz::hip_check(dev, hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

int oz_memcpy_d2h(oz_dev* dev, void* dst, const void* src, size_t bytes) {
    if (int st = oz::use(dev)) return st;
    if (!bytes) return OZ_OK;
    if (int st = oz::hip_check(dev, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream), "hipMemcpyAsync D2H"))
        return st;
    return oz::hip_check(dev, hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

int oz_host_malloc(oz_dev* dev, size_t bytes, void** ptr) {
    if (int st = oz::use(dev)) return st;
    if (!ptr) return oz::fail(dev, OZ_ERR_ARG, "oz_host_malloc: null output pointer");
    *ptr = nullptr;
    if (bytes == 0) return OZ_OK;
    return oz::hip_check(dev, hipHostMalloc(ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
}

int oz_host_free(oz_dev* dev, void* ptr) {
    if (int st = oz::use(dev)) return st;
    if (!ptr) return OZ_OK;
    return oz::hip_check(dev, hipHostFree(ptr), "hipHostFree");
}

int oz_memcpy_h2d_async(oz_dev* dev, void* dst, const void* src, size_t bytes) {
    if (int st = oz::use(dev)) return st;
    if (!bytes) return OZ_OK;
    return oz::hip_check(dev, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream), "hipMemcpyAsync H2D");
}

int oz_fill_u32(oz_dev* dev, void* dst, uint32_t value, size_t count) {
    if (int st = oz::use(dev)) return st;
    if (!count) return OZ_OK;
    if (!dst) return oz::fail(dev, OZ_ERR_ARG, "oz_fill_u32: null pointer");
    const unsigned blocks = (unsigned)std::min<size_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, dev->stream, (uint32_t*)dst, value, count);
    return oz::launch_check(dev, "fill_u32_kernel");
}

int oz_memcpy_d2d(oz_dev* dev, void* dst, const void* src, size_t bytes) {
    if (int st = oz::use(dev)) return st;
    if (!bytes) return OZ_OK;
    if (!dst || !src || bytes % 16 || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15))
        return oz::fail(dev, OZ_ERR_ARG, "oz_memcpy_d2d: pointers and size must be 16-byte aligned");
    const size_t n16 = bytes / 16;
    const unsigned blocks = (unsigned)std::min<size_t>((n16 + 255) / 256, 8192);
    hipLaunchKernelGGL(copy16_kernel, dim3(blocks), dim3(256), 0, dev->stream, (uint4*)dst, (const uint4*)src, n16);
    return oz::launch_check(dev, "copy16_kernel");
}

int oz_pad_copy_f64(oz_dev* dev, double* dst, int drows, int dcols, const double* src, int srows, int scols,
                    int sld) {
    if (int st = oz::use(dev)) return st;
    if (!dst || drows <= 0 || dcols <= 0 || srows < 0 || scols < 0 || (srows && scols && (!src || sld < scols)))
        return oz::fail(dev, OZ_ERR_ARG, "oz_pad_copy_f64: invalid arguments");
    const dim3 grid((unsigned)((dcols + 255) / 256), (unsigned)std::min(drows, 65535));
    hipLaunchKernelGGL(pad_copy_f64_kernel, grid, dim3(256), 0, dev->stream, dst, drows, dcols, src, srows, scols, sld);
    return oz::launch_check(dev, "pad_copy_f64_kernel");
}

int oz_sync(oz_dev* dev) {
    if (int st = oz::use(dev)) return st;
    return oz::hip_check(dev, hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

int oz_event_record(oz_dev* dev, int slot) {
    if (int st = oz::use(dev)) return st;
    if (slot < 0 || slot >= OZ_EVENT_SLOTS) return oz::fail(dev, OZ_ERR_ARG, "event slot %d out of range", slot);
    return oz::hip_check(dev, hipEventRecord(dev->events[slot], dev->stream), "hipEventRecord");
}

int oz_time_products_begin(oz_dev* dev, int slot_begin, int slot_end) {
    if (int st = oz::use(dev)) return st;
    if (slot_begin < 0 || slot_begin >= OZ_EVENT_SLOTS || slot_end < 0 || slot_end >= OZ_EVENT_SLOTS ||
        slot_begin == slot_end)
        return oz::fail(dev, OZ_ERR_ARG, "oz_time_products_begin: bad event slots %d, %d", slot_begin, slot_end);
    dev->time_begin = slot_begin;
    dev->time_end = slot_end;
    dev->time_launched = false;
    return OZ_OK;
}

int oz_time_products_end(oz_dev* dev, int* launched) {
    if (int st = oz::use(dev)) return st;
    if (launched) *launched = dev->time_launched ? 1 : 0;
    dev->time_begin = dev->time_end = -1;
    dev->time_launched = false;
    return OZ_OK;
}

int oz_event_elapsed_ms(oz_dev* dev, int a, int b, float* ms) {
    if (int st = oz::use(dev)) return st;
    if (a < 0 || a >= OZ_EVENT_SLOTS || b < 0 || b >= OZ_EVENT_SLOTS || !ms) return oz::fail(dev, OZ_ERR_ARG, "bad event slots");
    if (int st = oz::hip_check(dev, hipEventSynchronize(dev->events[b]), "hipEventSynchronize")) return st;
    return oz::hip_check(dev, hipEventElapsedTime(ms, dev->events[a], dev->events[b]), "hipEventElapsedTime");
}

}  // extern "C"

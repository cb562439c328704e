// Internal helpers of the device layer (liboz_hip.so): the device handle, error reporting and
// launch checks shared by the kernel sources.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "oz_hip.h"

struct oz_dev {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t events[OZ_EVENT_SLOTS] = {};
    std::string error;
    int* queue = nullptr;   // tile pool counters of the INT8 product kernel (16 ints, zero between launches)
    int cus = 0;            // compute units: a product launch of at most this many tiles needs no pool
    // oz_time_products_begin: event slots of the product launches to time (-1: none), and whether
    // one has run under the request
    int time_begin = -1, time_end = -1;
    bool time_launched = false;
};

namespace oz {

// Launches a product kernel on the handle's stream. Under oz_time_products_begin the launch carries
// the requested events, which the runtime sets from the dispatch's own start and end
// (hipExtLaunchKernel); the start event only on the first such launch.
template <class F, class... Args>
inline void launch_product(oz_dev* dev, F kernel, dim3 grid, dim3 block, Args... args) {
    hipEvent_t start = nullptr, stop = nullptr;
    if (dev->time_end >= 0) {
        if (dev->time_begin >= 0) start = dev->events[dev->time_begin];
        stop = dev->events[dev->time_end];
        dev->time_begin = -1;
        dev->time_launched = true;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, 0, dev->stream, start, stop, 0, args...);
}

// Records a message on the handle and returns the status (printf-style).
inline int fail(oz_dev* dev, int status, const char* fmt, ...) {
    if (dev) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        dev->error = buf;
    }
    return status;
}

// Checks a HIP call; on failure records "what: hip error" and returns OZ_ERR_HIP.
inline int hip_check(oz_dev* dev, hipError_t e, const char* what) {
    if (e == hipSuccess) return OZ_OK;
    return fail(dev, e == hipErrorOutOfMemory ? OZ_ERR_NOMEM : OZ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Checks the launch that was just issued (configuration errors surface here).
inline int launch_check(oz_dev* dev, const char* kernel) { return hip_check(dev, hipGetLastError(), kernel); }

// Sets the handle's device current for the calling thread.
inline int use(oz_dev* dev) {
    if (!dev) return OZ_ERR_ARG;
    return hip_check(dev, hipSetDevice(dev->device), "hipSetDevice");
}

inline unsigned ceil_div(long long a, long long b) { return (unsigned)((a + b - 1) / b); }

}  // namespace oz

// Host-side helpers of the C-ABI hooks that take host arrays: device buffers of one call, released on every
// return path, and the device-0 selection the reference's unit-test hooks make (engine/faie2fn.cu:2754).
#pragma once

#include "common.cuh"

#include <vector>

namespace fn {

struct DevBufs {
    std::vector<void *> ptrs;
    DevBufs() = default;
    DevBufs(const DevBufs &) = delete;
    DevBufs &operator=(const DevBufs &) = delete;
    ~DevBufs() {
        for (void *p : ptrs) (void) hipFree(p);
    }
    template <typename T> int alloc(T **p, size_t n) {
        *p = nullptr;
        if (n == 0) n = 1;
        hipError_t e = hipMalloc((void **) p, n * sizeof(T));
        if (e != hipSuccess) {
            set_error(std::string("hipMalloc(") + std::to_string(n * sizeof(T)) + " B) -> " + hipGetErrorString(e));
            return -1;
        }
        ptrs.push_back(*p);
        return 0;
    }
    template <typename T> int up(T **p, const T *h, size_t n) {
        if (alloc(p, n)) return -1;
        FN_CK(hipMemcpy(*p, h, n * sizeof(T), hipMemcpyHostToDevice));
        return 0;
    }
};

inline int use_device0() {
    int n = 0;
    FN_CK(hipGetDeviceCount(&n));
    if (n < 1) FN_FAIL("no HIP device");
    FN_CK(hipSetDevice(0));
    return 0;
}

}  // namespace fn

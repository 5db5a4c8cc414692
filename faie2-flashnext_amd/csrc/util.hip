// Device utilities of libfaie2fn: seeded normal fill (synthetic inputs resident in HBM without a host round trip),
// a plain streaming copy (the HBM yardstick the path's kernels are compared with, and the known-size kernel that
// calibrates the FETCH_SIZE / WRITE_SIZE counters), and the per-device status word in which kernels record misuse
// they cannot report on the host (positions and counts that live in device memory).
#include "gdn.h"

#include <mutex>
#include <vector>

namespace fn {

namespace {

__device__ __align__(256) unsigned g_status;  // FN_STATUS_* bits, one word per device

constexpr int kMaxDevices = 64;
unsigned *g_status_addr[kMaxDevices];
std::mutex g_status_mu;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {  // splitmix64 finaliser
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// element pair i gets a Box-Muller pair from the 64-bit hash of (seed, i): independent of the launch shape
__global__ void k_fill_normal(float *p, size_t n, uint64_t seed, float mean, float std) {
    const size_t stride = (size_t) gridDim.x * blockDim.x;
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; 2 * i < n; i += stride) {
        const uint64_t h = mix64(seed ^ mix64(i));
        const float u1 = (float) ((h >> 40) + 1) * (1.0f / 16777217.0f);   // (0, 1)
        const float u2 = (float) ((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        float sn, cs;
        sincosf(6.283185307179586f * u2, &sn, &cs);
        p[2 * i] = mean + std * r * cs;
        if (2 * i + 1 < n) p[2 * i + 1] = mean + std * r * sn;
    }
}

// one 16-byte nontemporal load and store per thread per pass (the shape that streamed fastest on MI355X among
// chunked, unrolled and grid-stride copies)
__global__ void __launch_bounds__(256) k_copy(float4 *__restrict__ dst, const float4 *__restrict__ src, size_t n4) {
    const size_t stride = (size_t) gridDim.x * blockDim.x;
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) st_nt(&dst[i], ld_nt(&src[i]));
}

}  // namespace

int device_cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        n = hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v
                : 256;
    }
    return n;
}

int status_word(unsigned **out) {
    int dev = -1;
    FN_CK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) FN_FAIL("status: device index out of range");
    std::lock_guard<std::mutex> lk(g_status_mu);
    if (!g_status_addr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_status));
        if (e != hipSuccess || !p) FN_FAIL(std::string("status: hipGetSymbolAddress -> ") + hipGetErrorString(e));
        g_status_addr[dev] = static_cast<unsigned *>(p);
    }
    *out = g_status_addr[dev];
    return 0;
}

int status_read(unsigned *bits, bool clear) {
    unsigned *w = nullptr;
    if (status_word(&w)) return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(bits, w, sizeof(unsigned), hipMemcpyDeviceToHost));
    if (clear && *bits) {
        const unsigned zero = 0;
        FN_CK(hipMemcpy(w, &zero, sizeof(unsigned), hipMemcpyHostToDevice));
    }
    return 0;
}

namespace {
std::vector<hipEvent_t> g_stage_ev;
size_t g_stage_next = 0;
}  // namespace

int stage_events(void **ev, int n) {
    if (n < 0 || n > 64 || (n && !ev)) FN_FAIL("stage_events: 0..64 events");
    g_stage_ev.assign(reinterpret_cast<hipEvent_t *>(ev), reinterpret_cast<hipEvent_t *>(ev) + n);
    g_stage_next = 0;
    return 0;
}

void stage_mark(hipStream_t st) {
    if (g_stage_next < g_stage_ev.size()) (void) hipEventRecord(g_stage_ev[g_stage_next++], st);
}

int fill_normal_launch(float *p, size_t n, uint64_t seed, float mean, float std, hipStream_t st) {
    if (!p && n) FN_FAIL("fill: null pointer");
    if (!n) return 0;
    const size_t pairs = (n + 1) / 2;
    const unsigned blocks = (unsigned) std::min<size_t>((pairs + 255) / 256, 8192);
    hipLaunchKernelGGL(k_fill_normal, dim3(blocks), dim3(256), 0, st, p, n, seed, mean, std);
    FN_CK(hipGetLastError());
    return 0;
}

int copy_launch(void *dst, const void *src, size_t bytes, hipStream_t st) {
    if ((!dst || !src) && bytes) FN_FAIL("copy: null pointer");
    if (bytes % 16 || ((uintptr_t) dst | (uintptr_t) src) % 16) FN_FAIL("copy: bytes and pointers must be 16-byte aligned");
    if (!bytes) return 0;
    const size_t n4 = bytes / 16;
    const unsigned blocks = (unsigned) std::min<size_t>((n4 + 255) / 256, 1u << 20);
    hipLaunchKernelGGL(k_copy, dim3(blocks), dim3(256), 0, st, (float4 *) dst, (const float4 *) src, n4);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

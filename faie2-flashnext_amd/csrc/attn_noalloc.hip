// GQA decode with no allocation: the attention of fn_attn_dev, its workspace (RMSNormed queries and the split
// partials) taken from a file-scope device array instead of a caller buffer.  For callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The array lives once per GPU for the life of the process.  Its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and kept per device: on the host, the array's name is only a
// stand-in for that address and is never passed to a kernel or a copy.  Every call on a GPU shares that GPU's
// array, so calls that overlap on one GPU (two streams, two threads) race; calls in one stream order are safe.
// Nothing in the workspace needs to start at zero: every split writes its partial (an empty split writes
// m = -inf, l = 0, o = 0) before the combine reads it, so the array keeps the last call's contents harmlessly.
#include "../../include/faie2fn.h"
#include "gdn.h"

#include <mutex>

#define FN_API extern "C" __attribute__((visibility("default")))

namespace {

static __device__ __align__(256) unsigned char scratch[FN_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices];  // device address of `scratch` on each device, looked up once
std::mutex g_scratch_mu;

int scratch_ptr(void **out) {
    int dev = -1;
    FN_CK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) FN_FAIL("attn_noalloc: device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            FN_FAIL(std::string("attn_noalloc: hipGetSymbolAddress(scratch) -> ") + hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace

FN_API int fn_attn_noalloc_dev(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                               const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                               const float *wk, float *Kc, float *Vc, int nsplit, float *og, void *stream) {
    if (B < 1 || nq < 1 || nt < 1 || hd < 1 || nsplit < 1) FN_FAIL("attn_noalloc: B, nq, nt, hd and nsplit must be >= 1");
    const size_t need = fn::attn_work_bytes(B, nq, nt, hd, nsplit);
    if (need > (size_t) FN_NOALLOC_SCRATCH_BYTES)
        FN_FAIL("attn_noalloc: these shapes need " + std::to_string(need) + " bytes of workspace, above the " +
                std::to_string((size_t) FN_NOALLOC_SCRATCH_BYTES) +
                " built in (fewer sequences, tokens or splits per call, or fn_attn_dev with a caller workspace)");
    void *ws = nullptr;
    if (scratch_ptr(&ws)) return -1;
    fn::AttnDecode p{B, nq, nkv, hd, nrot, nt, max_ctx, nsplit, theta, eps, pos, qg, k, v, wq, wk, Kc, Vc,
                     static_cast<float *>(ws), (size_t) FN_NOALLOC_SCRATCH_BYTES, og};
    return fn::attn_decode_launch(p, (hipStream_t) stream);
}

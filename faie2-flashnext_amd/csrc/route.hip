// fn_bench_route (engine/faie2fn.cu:2875-2913): the MoE routing of the reference model on given router outputs,
// timed as a hipGraph of `iters` calls, its picks and weights returned for a bit-for-bit comparison of variants
// (flashnext/route_fn.py).
//
// Input layout, the reference's: part [ks][MAXT = 8][RSG = 528] float32 split-K partial sums of the stacked router
// + shared-gate GEMV; expert e's logit of token t is part[0][t][e] + part[1][t][e] + ... in split order
// (gval, faie2fn.cu:1245-1250), e < NE = 512.  The routing (faie2fn.cu:1747-1798): p = exp(l - max l), the
// NEU = 10 most probable experts in order probability descending with ties to the lower expert, weights p / sum
// of the picked p (summed in pick order).
//
//   variant 0  k_route_rank: every expert's thread counts the experts ranked above it (a plain O(NE^2) rank)
//   variant 1  k_route_wave: the model forward's routing (route_pick: one wave, NEU wave argmaxes)
// Both take exp of the same logits and add the weights in the same order, so they agree bit for bit; a test holds
// them to that and to the float64 routing of the reference model's restatement.
#include "hostbuf.h"

#define FN_API extern "C" __attribute__((visibility("default")))

namespace {

using fn::route_pick;
using fn::wave_max;

constexpr int R_NE = 512, R_NEU = 10, R_MAXT = 8, R_RSG = 528, R_MAXKS = 64;
constexpr size_t R_KST = (size_t) R_MAXT * R_RSG;  // floats between two splits

// s[j] = the logit of expert e0 + 64 j of token t, j < NJ: the splits in chunks of KC, each chunk's NJ * KC loads
// issued before its adds (which run in split order)
template <int NJ, int KC>
__device__ __forceinline__ void route_logits(const float *__restrict__ part, int ks, int t, int e0, float (&s)[NJ]) {
    const float *q = part + (size_t) t * R_RSG + e0;
    for (int k0 = 0; k0 < ks; k0 += KC) {
        float v[NJ][KC];
#pragma unroll
        for (int i = 0; i < KC; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) v[j][i] = k0 + i < ks ? q[(size_t) (k0 + i) * R_KST + 64 * j] : 0.0f;
#pragma unroll
        for (int i = 0; i < KC; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                if (k0 + i < ks) s[j] = k0 + i == 0 ? v[j][i] : s[j] + v[j][i];
    }
}

// variant 1.   grid nt, 64 threads
__global__ void __launch_bounds__(64) k_route_wave(const float *__restrict__ part, int ks, int32_t *__restrict__ sel,
                                                   float *__restrict__ wsel) {
    __shared__ float l[R_NE];
    const int t = blockIdx.x, lane = threadIdx.x;
    float s[R_NE / 64];
    route_logits<R_NE / 64, 4>(part, ks, t, lane, s);
#pragma unroll
    for (int j = 0; j < R_NE / 64; ++j) l[lane + 64 * j] = s[j];
    __syncthreads();
    route_pick(l, R_NE, R_NEU, 0, sel + t * R_NEU, wsel + t * R_NEU);
}

// variant 0.   grid nt, 512 threads (one per expert)
__global__ void __launch_bounds__(R_NE) k_route_rank(const float *__restrict__ part, int ks,
                                                     int32_t *__restrict__ sel, float *__restrict__ wsel) {
    __shared__ float p[R_NE];
    __shared__ float wmax[R_NE / 64];
    __shared__ float topv[R_NEU];
    __shared__ int topi[R_NEU];
    const int t = blockIdx.x, e = threadIdx.x;
    float ls[1];
    route_logits<1, 8>(part, ks, t, e, ls);
    const float l = ls[0];
    const float m = wave_max(l);
    if ((e & 63) == 0) wmax[e >> 6] = m;
    __syncthreads();
    float mx = wmax[0];
    for (int w = 1; w < R_NE / 64; ++w) mx = fmaxf(mx, wmax[w]);
    const float v = expf(l - mx);
    p[e] = v;
    __syncthreads();
    int r = 0;
    for (int j = 0; j < R_NE; ++j) {
        const float pj = p[j];
        r += pj > v || (pj == v && j < e);
    }
    if (r < R_NEU) {
        topv[r] = v;
        topi[r] = e;
    }
    __syncthreads();
    if (e < R_NEU) {
        float s = 0.0f;
        for (int k = 0; k < R_NEU; ++k) s += topv[k];
        sel[t * R_NEU + e] = topi[e];
        wsel[t * R_NEU + e] = topv[e] / s;
    }
}

struct RouteRes {
    hipStream_t st = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    ~RouteRes() {
        if (ge) (void) hipGraphExecDestroy(ge);
        if (g) (void) hipGraphDestroy(g);
        if (a) (void) hipEventDestroy(a);
        if (b) (void) hipEventDestroy(b);
        if (st) (void) hipStreamDestroy(st);
    }
};

}  // namespace

// part [ks][8][528] (host), nt tokens 1..8, ks 1..64 splits, iters >= 1 calls; sel / wsel [nt][10] (host), ms the
// time per call.  Same arguments and meaning as the reference's; variant 0 or 1 as above.
FN_API int fn_bench_route(int variant, int nt, int ks, const float *parth, int iters, int *selh, float *wselh,
                          float *ms) {
    using fn::DevBufs;
    if (variant != 0 && variant != 1) FN_FAIL("bench_route: variant must be 0 (rank) or 1 (wave)");
    if (nt < 1 || nt > R_MAXT) FN_FAIL("bench_route: nt must be 1..8");
    if (ks < 1 || ks > R_MAXKS) FN_FAIL("bench_route: ks must be 1..64");
    if (iters < 1) FN_FAIL("bench_route: iters must be >= 1");
    if (!parth || !selh || !wselh || !ms) FN_FAIL("bench_route: null pointer");
    if (fn::use_device0()) return -1;
    DevBufs m;
    float *part, *wsel;
    int32_t *sel;
    if (m.up(&part, parth, (size_t) ks * R_KST) || m.alloc(&sel, (size_t) R_MAXT * R_NEU) ||
        m.alloc(&wsel, (size_t) R_MAXT * R_NEU))
        return -1;
    RouteRes r;
    FN_CK(hipStreamCreateWithFlags(&r.st, hipStreamNonBlocking));
    FN_CK(hipStreamBeginCapture(r.st, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < iters; ++i) {
        if (variant == 0)
            hipLaunchKernelGGL(k_route_rank, dim3(nt), dim3(R_NE), 0, r.st, part, ks, sel, wsel);
        else
            hipLaunchKernelGGL(k_route_wave, dim3(nt), dim3(64), 0, r.st, part, ks, sel, wsel);
    }
    const hipError_t launched = hipGetLastError();
    hipError_t ended = hipStreamEndCapture(r.st, &r.g);
    FN_CK(launched);
    FN_CK(ended);
    FN_CK(hipGraphInstantiate(&r.ge, r.g, nullptr, nullptr, 0));
    FN_CK(hipEventCreate(&r.a));
    FN_CK(hipEventCreate(&r.b));
    FN_CK(hipGraphLaunch(r.ge, r.st));
    FN_CK(hipEventRecord(r.a, r.st));
    FN_CK(hipGraphLaunch(r.ge, r.st));
    FN_CK(hipEventRecord(r.b, r.st));
    FN_CK(hipEventSynchronize(r.b));
    FN_CK(hipEventElapsedTime(ms, r.a, r.b));
    *ms /= iters;
    FN_CK(hipMemcpy(selh, sel, (size_t) nt * R_NEU * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(wselh, wsel, (size_t) nt * R_NEU * 4, hipMemcpyDeviceToHost));
    return 0;
}

// C ABI timing hooks of the decode path (declared in include/faie2fn.h): the reference times its GEMV inside the
// library on synthetic inputs (fn_bench_gemv, engine/faie2fn.cu:2823-2860); these do the same for the fused
// DeltaNet block and for GQA decode.  Each builds its inputs in HBM (seeded normal fills), enough distinct layers
// that the working set is cold (at least 1 GiB of state or caches, beyond the 256 MB Infinity Cache), captures one
// pass over the layers as a hipGraph and times `iters` replays with HIP events: microseconds per layer-step.
#include "gdn.h"
#include "hostbuf.h"

#include <algorithm>
#include <cmath>

#define FN_API extern "C" __attribute__((visibility("default")))

using fn::DevBufs;

namespace {

struct Timer {
    hipStream_t st = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    ~Timer() {
        if (ge) (void) hipGraphExecDestroy(ge);
        if (g) (void) hipGraphDestroy(g);
        if (a) (void) hipEventDestroy(a);
        if (b) (void) hipEventDestroy(b);
        if (st) (void) hipStreamDestroy(st);
    }
    // capture pass() on the stream, replay once to warm up, then time iters replays: ms per replay
    template <typename F> int run(F &&pass, int iters, float *ms) {
        FN_CK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        FN_CK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        if (pass(st)) {
            hipGraph_t dead = nullptr;
            (void) hipStreamEndCapture(st, &dead);
            if (dead) (void) hipGraphDestroy(dead);
            return -1;
        }
        FN_CK(hipStreamEndCapture(st, &g));
        FN_CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        FN_CK(hipEventCreate(&a));
        FN_CK(hipEventCreate(&b));
        FN_CK(hipGraphLaunch(ge, st));
        FN_CK(hipEventRecord(a, st));
        for (int i = 0; i < iters; ++i) FN_CK(hipGraphLaunch(ge, st));
        FN_CK(hipEventRecord(b, st));
        FN_CK(hipEventSynchronize(b));
        FN_CK(hipEventElapsedTime(ms, a, b));
        *ms /= iters;
        return 0;
    }
};

// distinct layers so that `per_layer` bytes a layer add up to at least 1 GiB (at most `cap`)
int cold_layers(size_t per_layer, int cap) {
    const size_t want = (1ull << 30) / std::max<size_t>(per_layer, 1) + 1;
    return (int) std::max<size_t>(1, std::min<size_t>(want, (size_t) cap));
}

int fill(float *p, size_t n, uint64_t seed, float mean, float std) {
    return fn::fill_normal_launch(p, n, seed, mean, std, nullptr);
}

}  // namespace

FN_API int fn_bench_gdn(int B, int nkh, int nvh, int nt, int iters, float *us) {
    if (B < 1 || nkh < 1 || nvh < 1 || nvh % nkh || nt < 1 || nt > 8 || iters < 1)
        FN_FAIL("bench_gdn: B >= 1, nvh a multiple of nkh, nt 1..8, iters >= 1");
    if (!us) FN_FAIL("bench_gdn: null pointer");
    if (fn::use_device0()) return -1;
    constexpr int DK = 128;
    const size_t C = (size_t) (2 * nkh + nvh) * DK, SB = (size_t) B * nvh * DK * DK;
    int ring = 4;
    while (ring < nt + 3) ring *= 2;
    const int L = cold_layers(SB * 4, 512);
    DevBufs m;
    float *S, *rg, *qkv, *ab, *z, *out, *cw, *dt, *sa, *nw;
    int32_t *pos;
    if (m.alloc(&S, SB * L) || m.alloc(&rg, (size_t) B * ring * C * L) || m.alloc(&qkv, (size_t) B * nt * C * L) ||
        m.alloc(&ab, (size_t) B * nt * 2 * nvh * L) || m.alloc(&z, (size_t) B * nt * nvh * DK * L) ||
        m.alloc(&out, (size_t) B * nt * nvh * DK * L) || m.alloc(&cw, C * 4 * L) || m.alloc(&dt, (size_t) nvh * L) ||
        m.alloc(&sa, (size_t) nvh * L) || m.alloc(&nw, (size_t) DK * L) || m.alloc(&pos, B))
        return -1;
    if (fill(S, SB * L, 11, 0.0f, 0.02f) || fill(rg, (size_t) B * ring * C * L, 12, 0.0f, 1.0f) ||
        fill(qkv, (size_t) B * nt * C * L, 13, 0.0f, 1.0f) || fill(ab, (size_t) B * nt * 2 * nvh * L, 14, 0.0f, 1.0f) ||
        fill(z, (size_t) B * nt * nvh * DK * L, 15, 0.0f, 1.0f) || fill(cw, C * 4 * L, 16, 0.0f, 0.1f) ||
        fill(dt, (size_t) nvh * L, 17, 0.0f, 0.0f) || fill(sa, (size_t) nvh * L, 18, -1.0f, 0.3f) ||
        fill(nw, (size_t) DK * L, 19, 1.0f, 0.1f))
        return -1;
    FN_CK(hipMemset(pos, 0, (size_t) B * 4));
    FN_CK(hipDeviceSynchronize());
    Timer t;
    float ms = 0.0f;
    const auto pass = [&](hipStream_t st) -> int {
        for (int l = 0; l < L; ++l) {
            fn::GdnBlock p{B, nkh, nvh, DK, DK, 0, 0, nt, ring, 1e-6f, pos, qkv + (size_t) B * nt * C * l,
                           cw + C * 4 * l, rg + (size_t) B * ring * C * l, ab + (size_t) B * nt * 2 * nvh * l,
                           dt + (size_t) nvh * l, sa + (size_t) nvh * l, S + SB * l,
                           z + (size_t) B * nt * nvh * DK * l, nw + (size_t) DK * l,
                           out + (size_t) B * nt * nvh * DK * l};
            if (fn::gdn_block_launch(p, st)) return -1;
        }
        return 0;
    };
    if (t.run(pass, iters, &ms)) return -1;
    *us = ms * 1e3f / L;
    return 0;
}

FN_API int fn_bench_attn(int B, int nq, int nkv, int ctx, int nt, int iters, float *us) {
    if (B < 1 || nkv < 1 || nq < 1 || nq % nkv || nt < 1 || nt > 8 || ctx < nt || iters < 1)
        FN_FAIL("bench_attn: B >= 1, nq a multiple of nkv, nt 1..8, ctx >= nt, iters >= 1");
    const int grp = nq / nkv;
    if (grp != 4 && grp != 8 && grp != 12) FN_FAIL("bench_attn: query heads per kv head must be 4, 8 or 12");
    if (!us) FN_FAIL("bench_attn: null pointer");
    if (fn::use_device0()) return -1;
    constexpr int HD = 256;
    const int max_ctx = (ctx + 63) / 64 * 64;
    const size_t cache = (size_t) B * nkv * max_ctx * HD, qn = (size_t) B * nt * nq * 2 * HD,
                 kn = (size_t) B * nt * nkv * HD, on = (size_t) B * nt * nq * HD;
    const int L = cold_layers(cache * 8, 64);
    const int nsplit = fn::attn_pick_nsplit(B, nkv, nt, ctx);
    const size_t wb = fn::attn_work_bytes(B, nq, nt, HD, nsplit);
    DevBufs m;
    float *K, *V, *qg, *k, *v, *og, *wq, *wk, *work;
    int32_t *pos;
    if (m.alloc(&K, cache * L) || m.alloc(&V, cache * L) || m.alloc(&qg, qn * L) || m.alloc(&k, kn * L) ||
        m.alloc(&v, kn * L) || m.alloc(&og, on * L) || m.alloc(&wq, (size_t) HD * L) || m.alloc(&wk, (size_t) HD * L) ||
        m.alloc(&work, wb / 4 + 1) || m.alloc(&pos, B))
        return -1;
    if (fill(K, cache * L, 21, 0.0f, 1.0f) || fill(V, cache * L, 22, 0.0f, 1.0f) || fill(qg, qn * L, 23, 0.0f, 1.0f) ||
        fill(k, kn * L, 24, 0.0f, 1.0f) || fill(v, kn * L, 25, 0.0f, 1.0f) ||
        fill(wq, (size_t) HD * L, 26, 1.0f, 0.1f) || fill(wk, (size_t) HD * L, 27, 1.0f, 0.1f))
        return -1;
    {
        std::vector<int32_t> p0(B, ctx - nt);  // the nt new tokens at positions ctx - nt .. ctx - 1
        FN_CK(hipMemcpy(pos, p0.data(), (size_t) B * 4, hipMemcpyHostToDevice));
    }
    FN_CK(hipDeviceSynchronize());
    Timer t;
    float ms = 0.0f;
    const auto pass = [&](hipStream_t st) -> int {
        for (int l = 0; l < L; ++l) {
            fn::AttnDecode p{B, nq, nkv, HD, 64, nt, max_ctx, nsplit, 1e7f, 1e-6f, pos, qg + qn * l, k + kn * l,
                             v + kn * l, wq + (size_t) HD * l, wk + (size_t) HD * l, K + cache * l, V + cache * l,
                             work, wb, og + on * l};
            if (fn::attn_decode_launch(p, st)) return -1;
        }
        return 0;
    };
    if (t.run(pass, iters, &ms)) return -1;
    *us = ms * 1e3f / L;
    return 0;
}

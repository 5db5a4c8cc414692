// C ABI of the GGUF weight formats and the projection GEMV (declared in include/faie2fn.h).
//
// The reference's hooks keep their names, signatures and meaning (engine/faie2fn.cu:2751-2935):
// fn_test_dequant decodes GGUF rows bit for bit, fn_test_gemv packs GGUF rows and runs the GEMV, fn_gemv_plan
// reports a launch plan, fn_bench_gemv times the GEMV on random bytes with every call reading a cold copy of the
// weight, fn_gemv_override forces the split-K.  The _dev entry points are the same operations on device buffers,
// asynchronous on a caller stream, for an engine that packs its weights once at load.
#include "gdn.h"
#include "hostbuf.h"
#include "quant.h"

#include <algorithm>

#define FN_API extern "C" __attribute__((visibility("default")))

using fn::DevBufs;
using fn::QLayout;

namespace {

int g_bench_hot = 0;  // fn_bench_gemv: 1 = one copy of the weight, replayed hot in the caches

// releases a stream, graph and events on every return path
struct BenchRes {
    hipStream_t st = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    ~BenchRes() {
        if (ge) (void) hipGraphExecDestroy(ge);
        if (g) (void) hipGraphDestroy(g);
        if (a) (void) hipEventDestroy(a);
        if (b) (void) hipEventDestroy(b);
        if (st) (void) hipStreamDestroy(st);
    }
};

}  // namespace

FN_API int fn_test_dequant(uint32_t type, const uint8_t *Wh, int rows, int cols, float *outh) {
    QLayout L;
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    if (!Wh || !outh) FN_FAIL("dequant: null pointer");
    if (fn::use_device0()) return -1;
    DevBufs m;
    uint8_t *raw, *packed;
    float *out;
    if (m.up(&raw, Wh, L.row_bytes * rows) || m.alloc(&packed, L.bytes) || m.alloc(&out, (size_t) rows * cols))
        return -1;
    if (fn::quant_pack_launch(L, raw, packed, nullptr) || fn::quant_dequant_launch(L, packed, out, nullptr)) return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(outh, out, (size_t) rows * cols * 4, hipMemcpyDeviceToHost));
    return 0;
}

FN_API int fn_test_gemv(uint32_t type, const uint8_t *Wh, int rows, int cols, const float *xh, int nt, float *yh) {
    QLayout L;
    if (nt < 1 || nt > 8) FN_FAIL("gemv: nt must be 1..8");
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    if (!Wh || !xh || !yh) FN_FAIL("gemv: null pointer");
    if (fn::use_device0()) return -1;
    const size_t wb = fn::gemv_work_bytes(L, nt);
    DevBufs m;
    uint8_t *raw, *packed;
    float *x, *y, *work;
    if (m.up(&raw, Wh, L.row_bytes * rows) || m.alloc(&packed, L.bytes) || m.up(&x, xh, (size_t) nt * cols) ||
        m.alloc(&y, (size_t) nt * rows) || m.alloc(&work, wb / 4 + 1))
        return -1;
    if (fn::quant_pack_launch(L, raw, packed, nullptr) || fn::gemv_launch(L, packed, x, nt, y, work, wb, nullptr))
        return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(yh, y, (size_t) nt * rows * 4, hipMemcpyDeviceToHost));
    return 0;
}

FN_API int fn_gemv_plan(uint32_t type, int rows, int cols, int *out) {
    QLayout L;
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    if (!out) FN_FAIL("gemv_plan: null pointer");
    const fn::GemvPlan p = fn::gemv_plan(L);
    // the reference's slots {cv, wpt, ks, tb, nbuf, ntiles, nch}: wpt is the split of a row's columns, here the
    // 16-lane groups that sum a row (lanes per row / 16); tb and nbuf hold this plan's rows per workgroup pass and
    // waves per workgroup
    const int v[7] = {p.gv, p.lpr / 16, p.ks, p.rpw, p.waves, p.grid, p.ngroups};
    std::copy(v, v + 7, out);
    return 0;
}

// wpt: 16-lane groups per row (1, 2 or 4; anything else: automatic), as fn_gemv_plan reports it; ks: split-K;
// tb: this library's kernel choice; warps_per_sm: resident waves per CU a persistent grid is sized for
FN_API void fn_gemv_override(int wpt, int ks, int tb, int warps_per_sm) {
    fn::gemv_override(wpt == 1 || wpt == 2 || wpt == 4 ? 16 * wpt : 0, ks, tb, warps_per_sm);
}
FN_API void fn_gemv_waves(int waves) { fn::gemv_persistent(waves); }
FN_API void fn_bench_hot(int on) { g_bench_hot = on; }

FN_API int fn_bench_gemv(uint32_t type, int rows, int cols, int nt, int iters, float *ms) {
    QLayout L;
    if (nt < 1 || nt > 8 || iters < 1) FN_FAIL("bench_gemv: nt must be 1..8 and iters >= 1");
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    if (!ms) FN_FAIL("bench_gemv: null pointer");
    if (fn::use_device0()) return -1;
    // Cold: every call reads its own copy, the copies together well beyond the 256 MB Infinity Cache, and 512 MiB
    // are written before the timed replay so no weight starts in a cache.
    const size_t tb = L.bytes;
    const int copies = g_bench_hot ? 1
                       : tb * (size_t) iters <= (2ull << 30)
                           ? iters
                           : (int) std::max<size_t>(4, (1ull << 30) / tb + 1);
    const size_t flush_n = 512ull << 20;
    const size_t wb = fn::gemv_work_bytes(L, nt);
    DevBufs m;
    uint8_t *w, *flush;
    float *x, *y, *work;
    if (m.alloc(&w, tb * copies) || m.alloc(&flush, flush_n) || m.alloc(&x, (size_t) nt * cols) ||
        m.alloc(&y, (size_t) nt * rows) || m.alloc(&work, wb / 4 + 1))
        return -1;
    if (fn::fill_normal_launch(reinterpret_cast<float *>(w), tb * copies / 4, 0x5eedull + type, 0.0f, 1.0f, nullptr))
        return -1;
    FN_CK(hipMemset(x, 0, (size_t) nt * cols * 4));
    FN_CK(hipDeviceSynchronize());
    BenchRes r;
    FN_CK(hipStreamCreateWithFlags(&r.st, hipStreamNonBlocking));
    FN_CK(hipStreamBeginCapture(r.st, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < iters; ++i) {
        if (fn::gemv_launch(L, w + tb * (size_t) (i % copies), x, nt, y, work, wb, r.st)) {
            hipGraph_t dead = nullptr;
            (void) hipStreamEndCapture(r.st, &dead);
            if (dead) (void) hipGraphDestroy(dead);
            return -1;
        }
    }
    FN_CK(hipStreamEndCapture(r.st, &r.g));
    FN_CK(hipGraphInstantiate(&r.ge, r.g, nullptr, nullptr, 0));
    FN_CK(hipEventCreate(&r.a));
    FN_CK(hipEventCreate(&r.b));
    FN_CK(hipGraphLaunch(r.ge, r.st));
    if (!g_bench_hot) FN_CK(hipMemsetAsync(flush, 1, flush_n, r.st));
    FN_CK(hipEventRecord(r.a, r.st));
    FN_CK(hipGraphLaunch(r.ge, r.st));
    FN_CK(hipEventRecord(r.b, r.st));
    FN_CK(hipEventSynchronize(r.b));
    FN_CK(hipEventElapsedTime(ms, r.a, r.b));
    *ms /= iters;
    return 0;
}

FN_API size_t fn_gemv_packed_bytes(uint32_t type, int rows, int cols) {
    QLayout L;
    return fn::qlayout(type, rows, cols, L) ? L.bytes : 0;
}

FN_API int fn_gemv_pack_dev(uint32_t type, const uint8_t *raw, int rows, int cols, uint8_t *packed, void *stream) {
    QLayout L;
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    return fn::quant_pack_launch(L, raw, packed, (hipStream_t) stream);
}

FN_API int fn_dequant_dev(uint32_t type, const uint8_t *packed, int rows, int cols, float *out, void *stream) {
    QLayout L;
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    return fn::quant_dequant_launch(L, packed, out, (hipStream_t) stream);
}

FN_API size_t fn_gemv_work_bytes(uint32_t type, int rows, int cols, int nt) {
    QLayout L;
    if (nt < 1 || nt > 8 || !fn::qlayout(type, rows, cols, L)) return 0;
    return fn::gemv_work_bytes(L, nt);
}

FN_API int fn_gemv_dev(uint32_t type, const uint8_t *packed, int rows, int cols, const float *x, int nt, float *y,
                       float *work, size_t work_bytes, void *stream) {
    QLayout L;
    if (!fn::qlayout(type, rows, cols, L)) return -1;
    return fn::gemv_launch(L, packed, x, nt, y, work, work_bytes, (hipStream_t) stream);
}

FN_API int fn_gemv_group_dev(int n, const uint32_t *types, const int *rows, int cols, const uint8_t *const *packed,
                             const float *x, int nt, float *const *y, void *stream) {
    if (n < 1 || n > 4 || !types || !rows || !packed || !y) FN_FAIL("gemv group: 1 to 4 parts");
    QLayout L[4];
    fn::GemvPart g[4];
    for (int i = 0; i < n; ++i) {
        if (!fn::qlayout(types[i], rows[i], cols, L[i])) return -1;
        g[i] = fn::GemvPart{&L[i], packed[i], y[i]};
    }
    return fn::gemv_group_launch(g, n, x, nt, (hipStream_t) stream);
}

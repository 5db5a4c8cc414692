// Path engine: B sequences decoded through a stack of DeltaNet and GQA layers in the reference's hybrid order,
// with engine-owned state, one stream, and the whole step captured as one hipGraph.
//
// It plays the part of the reference's Engine / layer_forward / forward (engine/faie2fn.cu:1937-2031, 2370-2490)
// for this path only: the projections, MoE and hyper-connections around the path are not built, so every layer
// reads its inputs (qkv, ab, z for DeltaNet; qg, k, v for attention) from engine buffers the caller fills, and
// writes its output (out / og) to an engine buffer.  Layer il is attention iff (il + 1) % attn_every == 0
// (faie2fn.cu:76 with attn_every = 4).  State follows the reference's ownership: engine-allocated, zeroed at
// allocation and by fn_reset (faie2fn.cu:2018-2024, 2703-2717); per-sequence positions live in device memory so
// a captured step replays unchanged (faie2fn.cu:1447).
#include "engine.h"
#include "model.h"

#include <chrono>
#include <memory>
#include <vector>

namespace fn {

namespace {

constexpr int DK = 128, HD = 256;

struct Layer {
    bool attn = false;
    // DeltaNet
    float *S = nullptr, *ring = nullptr, *qkv = nullptr, *ab = nullptr, *z = nullptr, *out = nullptr;
    float *conv_w = nullptr, *dt_bias = nullptr, *ssm_a = nullptr, *norm_w = nullptr;
    // attention
    float *Kc = nullptr, *Vc = nullptr, *qg = nullptr, *k = nullptr, *v = nullptr, *og = nullptr;
    float *wq = nullptr, *wk = nullptr;
};

struct Engine {
    int B = 0, nl = 0, attn_every = 4, nkh = 0, nvh = 0, nq = 0, nkv = 0, max_ctx = 0, head_map = 0, gate_act = 0;
    int nsplit = 0, ring = 4;
    float eps = 1e-6f, theta = 1e7f;
    int nrot = 64;
    std::vector<Layer> L;
    int32_t *pos = nullptr;
    float *work = nullptr;
    size_t work_bytes = 0;
    std::vector<std::pair<void *, size_t>> allocs;
    size_t bytes = 0;
    hipStream_t st = nullptr;
    hipGraphExec_t graph = nullptr;
    bool use_graphs = true;
    int n_past = 0;
    double last_ms = 0;

    ~Engine() {
        if (st) (void) hipStreamSynchronize(st);
        if (graph) (void) hipGraphExecDestroy(graph);
        for (auto &a : allocs) (void) hipFree(a.first);
        if (st) (void) hipStreamDestroy(st);
    }
    template <typename T> int alloc(T **p, size_t n) {
        const size_t nb = n * sizeof(T);
        hipError_t e = hipMalloc((void **) p, nb);
        if (e != hipSuccess) {
            *p = nullptr;
            set_error("engine: hipMalloc(" + std::to_string(nb) + " B) -> " + hipGetErrorString(e));
            return -1;
        }
        allocs.push_back({(void *) *p, nb});
        bytes += nb;
        FN_CK(hipMemset(*p, 0, nb));
        return 0;
    }
    size_t C() const { return (size_t) 2 * nkh * DK + (size_t) nvh * DK; }
};

std::unique_ptr<Engine> g_eng;

int enqueue_step(Engine &e) {
    for (int il = 0; il < e.nl; ++il) {
        Layer &l = e.L[il];
        if (!l.attn) {
            GdnBlock p{e.B, e.nkh, e.nvh, DK, DK, e.head_map, e.gate_act, 1, e.ring, e.eps, e.pos, l.qkv, l.conv_w,
                       l.ring, l.ab, l.dt_bias, l.ssm_a, l.S, l.z, l.norm_w, l.out};
            if (gdn_block_launch(p, e.st)) return -1;
        } else {
            AttnDecode p{e.B, e.nq, e.nkv, HD, e.nrot, 1, e.max_ctx, e.nsplit, e.theta, e.eps, e.pos, l.qg, l.k, l.v,
                         l.wq, l.wk, l.Kc, l.Vc, e.work, e.work_bytes, l.og};
            if (attn_decode_launch(p, e.st)) return -1;
        }
    }
    return advance_launch(e.pos, e.B, 1, e.st);
}

int drop_graph(Engine &e) {
    if (e.graph) {
        FN_CK(hipStreamSynchronize(e.st));
        FN_CK(hipGraphExecDestroy(e.graph));
        e.graph = nullptr;
    }
    return 0;
}

int ensure_graph(Engine &e) {
    if (e.graph) return 0;
    hipGraph_t g = nullptr;
    FN_CK(hipStreamBeginCapture(e.st, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_step(e);
    hipGraph_t g2 = nullptr;
    const hipError_t ec = hipStreamEndCapture(e.st, &g2);
    if (rc) {
        if (g2) (void) hipGraphDestroy(g2);
        return -1;
    }
    FN_CK(ec);
    g = g2;
    const hipError_t ei = hipGraphInstantiate(&e.graph, g, nullptr, nullptr, 0);
    (void) hipGraphDestroy(g);
    FN_CK(ei);
    return 0;
}

}  // namespace

int path_init(int B, int nl, int attn_every, int nkh, int nvh, int nq, int nkv, int max_ctx, int head_map,
              int gate_act, int nsplit) {
    g_eng.reset();
    model_free();  // one engine at a time: a path engine replaces a loaded model
    if (B < 1 || nl < 1 || attn_every < 0 || nkh < 1 || nvh < 1 || nvh % nkh) FN_FAIL("path_init: bad DeltaNet shape");
    const bool any_attn = attn_every > 0 && nl >= attn_every;
    if (any_attn && (nq < 1 || nkv < 1 || nq % nkv || max_ctx < 1)) FN_FAIL("path_init: bad attention shape");
    if (head_map != 0 && head_map != 1) FN_FAIL("path_init: head_map must be 0 or 1");
    if (gate_act != 0 && gate_act != 1) FN_FAIL("path_init: gate_act must be 0 or 1");
    auto e = std::make_unique<Engine>();
    e->B = B; e->nl = nl; e->attn_every = attn_every; e->nkh = nkh; e->nvh = nvh; e->nq = nq; e->nkv = nkv;
    e->max_ctx = any_attn ? (max_ctx + 63) / 64 * 64 : 0;
    e->head_map = head_map; e->gate_act = gate_act;
    e->nsplit = any_attn ? (nsplit > 0 ? nsplit : attn_pick_nsplit(B, nkv, 1, e->max_ctx)) : 1;
    FN_CK(hipSetDevice(0));
    FN_CK(hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking));
    unsigned *sw = nullptr;  // the status word's address, looked up now rather than under a graph capture
    if (status_word(&sw)) return -1;
    if (e->alloc(&e->pos, B)) return -1;
    if (any_attn) {
        e->work_bytes = attn_work_bytes(B, nq, 1, HD, e->nsplit);
        if (e->alloc(&e->work, e->work_bytes / 4 + 1)) return -1;
    }
    const size_t C = e->C(), nS = (size_t) B * nvh * DK * DK;
    e->L.resize(nl);
    for (int il = 0; il < nl; ++il) {
        Layer &l = e->L[il];
        l.attn = attn_every > 0 && (il + 1) % attn_every == 0;
        if (!l.attn) {
            if (e->alloc(&l.S, nS) || e->alloc(&l.ring, (size_t) B * e->ring * C) || e->alloc(&l.qkv, (size_t) B * C) ||
                e->alloc(&l.ab, (size_t) B * 2 * nvh) || e->alloc(&l.z, (size_t) B * nvh * DK) ||
                e->alloc(&l.out, (size_t) B * nvh * DK) || e->alloc(&l.conv_w, C * 4) || e->alloc(&l.dt_bias, nvh) ||
                e->alloc(&l.ssm_a, nvh) || e->alloc(&l.norm_w, DK))
                return -1;
        } else {
            const size_t cache = (size_t) B * nkv * e->max_ctx * HD;
            if (e->alloc(&l.Kc, cache) || e->alloc(&l.Vc, cache) || e->alloc(&l.qg, (size_t) B * nq * 2 * HD) ||
                e->alloc(&l.k, (size_t) B * nkv * HD) || e->alloc(&l.v, (size_t) B * nkv * HD) ||
                e->alloc(&l.og, (size_t) B * nq * HD) || e->alloc(&l.wq, HD) || e->alloc(&l.wk, HD))
                return -1;
        }
    }
    FN_CK(hipDeviceSynchronize());
    g_eng = std::move(e);
    return 0;
}

int path_buffer(int il, int kind, void **ptr, size_t *bytes) {
    if (!g_eng) FN_FAIL("not loaded");
    Engine &e = *g_eng;
    if (!ptr || !bytes) FN_FAIL("path_buffer: null pointer");
    *ptr = nullptr;
    *bytes = 0;
    if (kind == FN_BUF_POS) {
        *ptr = e.pos;
        *bytes = (size_t) e.B * 4;
        return 0;
    }
    if (il < 0 || il >= e.nl) FN_FAIL("path_buffer: layer out of range");
    const Layer &l = e.L[il];
    const size_t C = e.C(), B = e.B, nvh = e.nvh;
    const size_t cache = (size_t) e.B * e.nkv * e.max_ctx * HD;
    struct K { int kind; bool attn; float *p; size_t n; };
    const K tab[] = {
        {FN_BUF_S, false, l.S, B * nvh * DK * DK}, {FN_BUF_CONV_RING, false, l.ring, B * e.ring * C},
        {FN_BUF_QKV, false, l.qkv, B * C}, {FN_BUF_AB, false, l.ab, B * 2 * nvh}, {FN_BUF_Z, false, l.z, B * nvh * DK},
        {FN_BUF_OUT, false, l.out, B * nvh * DK}, {FN_BUF_CONV_W, false, l.conv_w, C * 4},
        {FN_BUF_DT_BIAS, false, l.dt_bias, nvh}, {FN_BUF_SSM_A, false, l.ssm_a, nvh}, {FN_BUF_NORM_W, false, l.norm_w, DK},
        {FN_BUF_KC, true, l.Kc, cache}, {FN_BUF_VC, true, l.Vc, cache}, {FN_BUF_QG, true, l.qg, B * e.nq * 2 * HD},
        {FN_BUF_K, true, l.k, B * e.nkv * HD}, {FN_BUF_V, true, l.v, B * e.nkv * HD}, {FN_BUF_OG, true, l.og, B * e.nq * HD},
        {FN_BUF_WQ, true, l.wq, HD}, {FN_BUF_WK, true, l.wk, HD},
    };
    for (const K &k : tab)
        if (k.kind == kind) {
            if (k.attn != l.attn) FN_FAIL(std::string("path_buffer: layer ") + std::to_string(il) + " is " +
                                          (l.attn ? "attention" : "DeltaNet") + " and has no such buffer");
            *ptr = k.p;
            *bytes = k.n * 4;
            return 0;
        }
    FN_FAIL("path_buffer: unknown buffer kind");
}

int path_step(int steps, float *ms) {
    if (!g_eng) FN_FAIL("not loaded");
    Engine &e = *g_eng;
    if (steps < 1) FN_FAIL("path_step: steps must be >= 1");
    // Positions live in device memory (the caller may write them through FN_BUF_POS), so they are read back before
    // each call: every step appends one token per sequence to the attention caches, and a sequence whose last
    // token would land past max_ctx fails the call before anything runs ("context full", the reference's check
    // on its host counter, faie2fn.cu:2468).
    if (e.max_ctx > 0) {
        std::vector<int32_t> ph(e.B);
        FN_CK(hipMemcpy(ph.data(), e.pos, (size_t) e.B * 4, hipMemcpyDeviceToHost));
        for (int b = 0; b < e.B; ++b) {
            if (ph[b] < 0) FN_FAIL("path_step: negative position for sequence " + std::to_string(b));
            if ((long) ph[b] + steps > e.max_ctx)
                FN_FAIL("context full: sequence " + std::to_string(b) + " at position " + std::to_string(ph[b]) +
                        " cannot take " + std::to_string(steps) + " more tokens (max_ctx " +
                        std::to_string(e.max_ctx) + ")");
        }
        unsigned stale = 0;  // bits left by earlier calls outside the engine are not this step's
        if (status_read(&stale, true)) return -1;
    }
    if (e.use_graphs && ensure_graph(e)) return -1;
    hipEvent_t a = nullptr, b = nullptr;
    if (ms) {
        FN_CK(hipEventCreate(&a));
        FN_CK(hipEventCreate(&b));
        FN_CK(hipEventRecord(a, e.st));
    }
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < steps; ++i) {
        if (e.use_graphs) FN_CK(hipGraphLaunch(e.graph, e.st));
        else if (enqueue_step(e)) return -1;
    }
    if (ms) FN_CK(hipEventRecord(b, e.st));
    FN_CK(hipStreamSynchronize(e.st));
    e.last_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (ms) {
        FN_CK(hipEventElapsedTime(ms, a, b));
        *ms /= steps;
        (void) hipEventDestroy(a);
        (void) hipEventDestroy(b);
    }
    // kernels record what they had to clamp; with the check above nothing should be
    unsigned bits = 0;
    if (e.max_ctx > 0) {
        if (status_read(&bits, true)) return -1;
        if (bits & FN_STATUS_POS) FN_FAIL("path_step: a token position fell outside the attention cache");
    }
    e.n_past += steps;
    return 0;
}

int path_reset() {
    if (!g_eng) FN_FAIL("not loaded");
    Engine &e = *g_eng;
    FN_CK(hipStreamSynchronize(e.st));
    for (Layer &l : e.L)
        if (!l.attn) {
            FN_CK(hipMemset(l.S, 0, (size_t) e.B * e.nvh * DK * DK * 4));
            FN_CK(hipMemset(l.ring, 0, (size_t) e.B * e.ring * e.C() * 4));
        }
    FN_CK(hipMemset(e.pos, 0, (size_t) e.B * 4));
    FN_CK(hipDeviceSynchronize());
    e.n_past = 0;
    return 0;
}

int path_use_graphs(int on) {
    if (!g_eng) FN_FAIL("not loaded");
    if (drop_graph(*g_eng)) return -1;
    g_eng->use_graphs = on != 0;
    return 0;
}

void path_free() { g_eng.reset(); }
bool path_loaded() { return (bool) g_eng; }
int path_n_past() { return g_eng ? g_eng->n_past : -1; }
double path_dev_gb() { return g_eng ? g_eng->bytes / 1e9 : -1; }
double path_last_ms() { return g_eng ? g_eng->last_ms : -1; }

}  // namespace fn

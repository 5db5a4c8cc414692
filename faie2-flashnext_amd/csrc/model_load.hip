// fn_load's placement of a FAIE2-FlashNext GGUF model on one GPU (the reference loads the same tensors,
// engine/faie2fn.cu:2524-2696, onto two).
//
// Design: the tensors are rows of one table (TABLE below): the slot a tensor fills, the layer kinds that hold it,
// its form (a GGUF weight to pack, a norm / bias vector, zeroed state) and its shape as symbolic extents of the
// model's dimensions.  Loading is two walks over that table:
//   1. plan (plan_weights): per arena (the model-wide one, then one per layer) resolve every row of the arena's
//      kinds to its GGUF tensors, check shapes and formats, and give each piece its offset (256-byte aligned) -- no
//      device work, so a malformed file fails before the device is touched;
//   2. commit (commit_weights): one device allocation per arena, zeroed; vectors copied (F16 widened exactly on the
//      host); weights streamed through one bounded staging buffer in row chunks, each chunk packed into its planes in
//      place (a row chunk of a packed weight is the layout with its rows cut and its plane offsets moved).
// The activations of MAXT tokens are carved from one allocation the same way.
#include "engine.h"
#include "model_impl.h"
#include "qsa.h"

#include <cmath>
#include <cstring>

namespace fn {

namespace {

// symbolic extents, evaluated against the model's dimensions (ext())
enum Ext : uint8_t {
    X1, X4, XD, XHC, XHCR, XHCD, XCONV, XINNER, XVH, XDS, XQG, XKV, XATTN, XIXQ, XIXD, XHD, XNE, XFFS, XFFE, XVOCAB,
    XNGD, XTAB, XSTATE, XRING, XCACHE, XIXKEYS, XIXBLOCKS, XNGHIST
};

enum Form : uint8_t { QUANT = 1, VEC, ZERO };

struct Row {
    Slot slot;
    unsigned kinds;     // arenas that hold it (K_* bits)
    Form form;
    const char *name;   // GGUF tensor (after "blk.<layer>." in a layer's arena); null for state
    const char *name2;  // stacked below the first tensor (null: none)
    Ext rows, rows2, cols, experts;
};

// every tensor and state buffer of the model.  Stacked pairs are the ones a single product reads: the stream
// inject rows below the low-rank down rows (one hyper-connection read), beta below alpha (the DeltaNet block reads
// [alpha | beta] per token), the indexer's k below its q, and the shared expert's gate logit below the router.
constexpr Row TABLE[] = {
    {TOK_EMBED, K_MODEL, QUANT, "token_embd.weight", nullptr, XVOCAB, X1, XD, X1},
    {LM_HEAD, K_MODEL, QUANT, "output.weight", nullptr, XVOCAB, X1, XD, X1},
    {FIN_NORM, K_MODEL, VEC, "output_hc_norm.weight", nullptr, XHCD, X1, X1, X1},
    {FIN_DOWN, K_MODEL, QUANT, "output_hc_down.weight", nullptr, XHCR, X1, XHCD, X1},
    {FIN_UP, K_MODEL, QUANT, "output_hc_up.weight", nullptr, XHCD, X1, XHCR, X1},
    {NG_TABLE, K_MODEL_NG, QUANT, "per_layer_token_embd.weight", nullptr, XTAB, X1, XNGD, X1},

    {R0_NORM, K_LAYER, VEC, "hc_attn_norm.weight", nullptr, XHCD, X1, X1, X1},
    {R0_DOWN, K_LAYER, QUANT, "hc_attn_down.weight", "hc_attn_inject.weight", XHCR, XHC, XHCD, X1},
    {R0_UP, K_LAYER, QUANT, "hc_attn_up.weight", nullptr, XHCD, X1, XHCR, X1},
    {R1_NORM, K_LAYER, VEC, "hc_ffn_norm.weight", nullptr, XHCD, X1, X1, X1},
    {R1_DOWN, K_LAYER, QUANT, "hc_ffn_down.weight", "hc_ffn_inject.weight", XHCR, XHC, XHCD, X1},
    {R1_UP, K_LAYER, QUANT, "hc_ffn_up.weight", nullptr, XHCD, X1, XHCR, X1},

    {DN_IN, K_DELTA, QUANT, "attn_qkv.weight", nullptr, XCONV, X1, XD, X1},
    {DN_ZPROJ, K_DELTA, QUANT, "attn_gate.weight", nullptr, XINNER, X1, XD, X1},
    {DN_AB, K_DELTA, QUANT, "ssm_alpha.weight", "ssm_beta.weight", XVH, XVH, XD, X1},
    {DN_OUT, K_DELTA, QUANT, "ssm_out.weight", nullptr, XD, X1, XINNER, X1},
    {DN_CONVW, K_DELTA, VEC, "ssm_conv1d.weight", nullptr, XCONV, X1, X4, X1},
    {DN_DT, K_DELTA, VEC, "ssm_dt.bias", nullptr, XVH, X1, X1, X1},
    {DN_A, K_DELTA, VEC, "ssm_a", nullptr, XVH, X1, X1, X1},
    {DN_NORMW, K_DELTA, VEC, "ssm_norm.weight", nullptr, XDS, X1, X1, X1},
    {DN_STATE, K_DELTA, ZERO, nullptr, nullptr, XSTATE, X1, X1, X1},
    {DN_RING, K_DELTA, ZERO, nullptr, nullptr, XRING, X1, X1, X1},

    {AT_QG, K_ATTN, QUANT, "attn_q.weight", nullptr, XQG, X1, XD, X1},
    {AT_K, K_ATTN, QUANT, "attn_k.weight", nullptr, XKV, X1, XD, X1},
    {AT_V, K_ATTN, QUANT, "attn_v.weight", nullptr, XKV, X1, XD, X1},
    {AT_O, K_ATTN, QUANT, "attn_output.weight", nullptr, XD, X1, XATTN, X1},
    {AT_IX, K_ATTN, QUANT, "indexer.q_proj.weight", "indexer.k_proj.weight", XIXQ, XIXD, XD, X1},
    {AT_QNORM, K_ATTN, VEC, "attn_q_norm.weight", nullptr, XHD, X1, X1, X1},
    {AT_KNORM, K_ATTN, VEC, "attn_k_norm.weight", nullptr, XHD, X1, X1, X1},
    {AT_IXQNORM, K_ATTN, VEC, "indexer.q_norm.weight", nullptr, XIXD, X1, X1, X1},
    {AT_IXKNORM, K_ATTN, VEC, "indexer.k_norm.weight", nullptr, XIXD, X1, X1, X1},
    {AT_KCACHE, K_ATTN, ZERO, nullptr, nullptr, XCACHE, X1, X1, X1},
    {AT_VCACHE, K_ATTN, ZERO, nullptr, nullptr, XCACHE, X1, X1, X1},
    {AT_IXKEYS, K_ATTN, ZERO, nullptr, nullptr, XIXKEYS, X1, X1, X1},
    {AT_IXBLOCKS, K_ATTN, ZERO, nullptr, nullptr, XIXBLOCKS, X1, X1, X1},

    {FF_ROUTER, K_LAYER, QUANT, "ffn_gate_inp.weight", "ffn_gate_inp_shexp.weight", XNE, X1, XD, X1},
    {FF_SH_GATE, K_LAYER, QUANT, "ffn_gate_shexp.weight", nullptr, XFFS, X1, XD, X1},
    {FF_SH_UP, K_LAYER, QUANT, "ffn_up_shexp.weight", nullptr, XFFS, X1, XD, X1},
    {FF_SH_DOWN, K_LAYER, QUANT, "ffn_down_shexp.weight", nullptr, XD, X1, XFFS, X1},
    {FF_X_GATE, K_LAYER, QUANT, "ffn_gate_exps.weight", nullptr, XFFE, X1, XD, XNE},
    {FF_X_UP, K_LAYER, QUANT, "ffn_up_exps.weight", nullptr, XFFE, X1, XD, XNE},
    {FF_X_DOWN, K_LAYER, QUANT, "ffn_down_exps.weight", nullptr, XD, X1, XFFE, XNE},

    {NG_KEY, K_NGRAM, QUANT, "ple_key.weight", nullptr, XHCD, X1, XD, X1},
    {NG_VAL, K_NGRAM, QUANT, "ple_value.weight", nullptr, XD, X1, XD, X1},
    {NG_KNORM, K_NGRAM, VEC, "ple_norm_key.weight", nullptr, XHCD, X1, X1, X1},
    {NG_QNORM, K_NGRAM, VEC, "ple_norm_query.weight", nullptr, XHCD, X1, X1, X1},
    {NG_CNORM, K_NGRAM, VEC, "ple_norm_conv.weight", nullptr, XHCD, X1, X1, X1},
    {NG_CONVW, K_NGRAM, VEC, "ple_conv1d.weight", nullptr, XHCD, X1, X4, X1},
    {NG_HIST, K_NGRAM, ZERO, nullptr, nullptr, XNGHIST, X1, X1, X1},
};

struct Ctx {
    const ModelDims &d;
    int max_ctx;
    const Gguf &g, &g2;
    const GTensor *find(const std::string &name) const {
        const GTensor *t = g.find(name);
        return t || !g2.base ? t : g2.find(name);
    }
};

uint64_t ext(Ext e, const Ctx &c, const GTensor *t) {
    const ModelDims &d = c.d;
    const uint64_t HCD = (uint64_t) d.HC * d.D, mc = (uint64_t) c.max_ctx;
    switch (e) {
        case X1: return 1;
        case X4: return 4;
        case XD: return (uint64_t) d.D;
        case XHC: return (uint64_t) d.HC;
        case XHCR: return (uint64_t) d.HCR;
        case XHCD: return HCD;
        case XCONV: return (uint64_t) d.CONVCH;
        case XINNER: return (uint64_t) d.DINNER;
        case XVH: return (uint64_t) d.NVH;
        case XDS: return (uint64_t) d.DS;
        case XQG: return (uint64_t) d.NH * 2 * HDK;
        case XKV: return (uint64_t) d.NKV * HDK;
        case XATTN: return (uint64_t) d.NH * HDK;
        case XIXQ: return (uint64_t) IXH * IXD;
        case XIXD: return IXD;
        case XHD: return HDK;
        case XNE: return (uint64_t) d.NE;
        case XFFS: return (uint64_t) d.FFS;
        case XFFE: return (uint64_t) d.FFE;
        case XVOCAB: return (uint64_t) d.VOCAB;
        case XNGD: return (uint64_t) d.ple_hd;
        case XTAB: return t ? t->ne[1] : 0;  // the n-gram table keeps its own row count (checked against the heads)
        case XSTATE: return (uint64_t) d.NVH * DSK * DSK;
        case XRING: return (uint64_t) RING * d.CONVCH;
        case XCACHE: return (uint64_t) d.NKV * mc * HDK;
        case XIXKEYS: return mc * IXD;
        case XIXBLOCKS: return mc / IXR * IXD;
        case XNGHIST: return (uint64_t) NG_RING * HCD;
    }
    return 0;
}

std::string shape_str(const GTensor *t) {
    return "[" + std::to_string(t->ne[0]) + ", " + std::to_string(t->ne[1]) + ", " + std::to_string(t->ne[2]) + "]";
}

// one row of the table for one arena: its tensors found and checked, its bytes and layout known
int plan_piece(const Ctx &c, const Row &r, const std::string &prefix, Piece &pc) {
    pc = Piece{};
    pc.on = true;
    pc.form = r.form;
    if (r.form == ZERO) {
        pc.n = ext(r.rows, c, nullptr) * ext(r.cols, c, nullptr);
        pc.bytes = pc.n * 4;
        return 0;
    }
    const char *names[2] = {r.name, r.name2};
    const Ext rows[2] = {r.rows, r.rows2};
    for (int i = 0; i < 2 && names[i]; ++i) {
        const std::string nm = prefix + names[i];
        pc.src[i] = c.find(nm);
        if (!pc.src[i]) FN_FAIL("load: tensor " + nm + " missing");
    }
    if (r.form == VEC) {
        const GTensor *t = pc.src[0];
        pc.n = ext(r.rows, c, t) * ext(r.cols, c, t);
        if (t->type != 0 && t->type != 1) FN_FAIL("load: tensor " + prefix + r.name + " must be F32 or F16");
        const uint64_t have = t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
        if (have != pc.n)
            FN_FAIL("load: tensor " + prefix + r.name + " has " + std::to_string(have) + " values, expected " +
                    std::to_string(pc.n));
        pc.bytes = pc.n * 4;
        return 0;
    }
    // a packed weight: every source [cols] x rows (x experts), one format
    const uint64_t cols = ext(r.cols, c, pc.src[0]), nx = ext(r.experts, c, pc.src[0]);
    uint64_t total = 0;
    for (int i = 0; i < 2 && pc.src[i]; ++i) {
        const GTensor *t = pc.src[i];
        const uint64_t want = ext(rows[i], c, t) * nx;
        if (t->ne[0] != cols || t->ne[1] * t->ne[2] * t->ne[3] != want || (nx > 1 && t->ne[2] != nx))
            FN_FAIL("load: tensor " + prefix + names[i] + " has shape " + shape_str(t) + ", expected " +
                    std::to_string(cols) + " columns x " + std::to_string(want) + " rows");
        if (i && t->type != pc.src[0]->type)
            FN_FAIL("load: tensors " + prefix + names[0] + " and " + prefix + names[i] + " differ in type");
        if (!i) pc.rows0 = want;
        total += want;
    }
    if (total > 0x7fffffffu) FN_FAIL("load: tensor " + prefix + names[0] + " has too many rows");
    if (!qlayout(pc.src[0]->type, (int) total, (int) cols, pc.L)) return -1;  // fn_error names the type / shape
    pc.bytes = pc.L.bytes;
    return 0;
}

// plan the pieces of one arena (the rows of its kinds), offsets 256-byte aligned
int plan_arena(const Ctx &c, unsigned kind, const std::string &prefix, Arena &a) {
    a.bytes = 0;
    for (const Row &r : TABLE) {
        if (!(r.kinds & kind)) continue;
        Piece &pc = a.piece[r.slot];
        if (plan_piece(c, r, prefix, pc)) return -1;
        pc.off = a.bytes;
        a.bytes += (pc.bytes + 255) / 256 * 256;
    }
    return 0;
}

// streams GGUF rows through a bounded device staging buffer into their packed planes
struct Stager {
    static constexpr size_t kBytes = 256u << 20;
    uint8_t *buf = nullptr;
    hipStream_t st = nullptr;
    ~Stager() {
        if (buf) (void) hipFree(buf);
    }
    int put(const Piece &pc, uint8_t *packed) {
        if (!buf) FN_CK(hipMalloc((void **) &buf, kBytes));
        uint64_t row_at = 0;
        for (int i = 0; i < 2 && pc.src[i]; ++i) {
            const GTensor *t = pc.src[i];
            const uint64_t nrow = i ? pc.L.rows - pc.rows0 : pc.rows0;
            const uint64_t chunk = std::max<uint64_t>(1, kBytes / pc.L.row_bytes);
            for (uint64_t r = 0; r < nrow; r += chunk) {
                const uint64_t nr = std::min(chunk, nrow - r);
                // the staging buffer is reused: the previous chunk's pack must be done with it
                FN_CK(hipStreamSynchronize(st));
                FN_CK(hipMemcpy(buf, t->data + r * pc.L.row_bytes, nr * pc.L.row_bytes, hipMemcpyHostToDevice));
                QLayout v = pc.L;  // rows [row_at + r, + nr) of the packed weight
                v.rows = (int) nr;
                for (int p = 0; p < v.nplanes; ++p) v.off[p] += (row_at + r) * v.rs[p];
                if (quant_pack_launch(v, buf, packed, st)) return -1;
            }
            row_at += nrow;
        }
        return 0;
    }
};

int put_vec(const Piece &pc, float *dst) {
    const GTensor *t = pc.src[0];
    if (t->type == 0) {
        FN_CK(hipMemcpy(dst, t->data, pc.n * 4, hipMemcpyHostToDevice));
        return 0;
    }
    // IEEE half -> float exactly: normal values rebias the exponent, subnormals scale by 2^-24
    std::vector<float> w(pc.n);
    const uint16_t *hv = reinterpret_cast<const uint16_t *>(t->data);
    for (size_t i = 0; i < pc.n; ++i) {
        const uint32_t b = hv[i], mant = b & 0x3ffu, ex = (b >> 10) & 0x1fu;
        float v;
        if (ex == 0x1f) v = mant ? NAN : INFINITY;
        else if (ex == 0) v = std::ldexp((float) mant, -24);
        else v = std::ldexp((float) (mant | 0x400u), (int) ex - 25);
        w[i] = (b & 0x8000u) ? -v : v;
    }
    FN_CK(hipMemcpy(dst, w.data(), pc.n * 4, hipMemcpyHostToDevice));
    return 0;
}

// one allocation for the arena, zeroed (state starts at zero), then its vectors and packed weights
int commit_arena(Model &m, Arena &a, Stager &sg) {
    if (!a.bytes) return 0;
    const hipError_t e = hipMalloc((void **) &a.base, a.bytes);
    if (e != hipSuccess) {
        a.base = nullptr;
        FN_FAIL("load: hipMalloc(" + std::to_string(a.bytes) + " B) -> " + hipGetErrorString(e));
    }
    m.allocs.push_back(a.base);
    m.bytes += a.bytes;
    FN_CK(hipMemsetAsync(a.base, 0, a.bytes, m.st));
    // the vector copies below run on the null stream, which does not wait for m.st
    FN_CK(hipStreamSynchronize(m.st));
    for (const Piece &pc : a.piece) {
        if (!pc.on) continue;
        if (pc.form == VEC && put_vec(pc, reinterpret_cast<float *>(a.base + pc.off))) return -1;
        if (pc.form == QUANT && sg.put(pc, a.base + pc.off)) return -1;
    }
    FN_CK(hipStreamSynchronize(m.st));
    return 0;
}

// the n-gram hash constants to the device as [multipliers 3][table size per head][first row per head]
int ngram_setup(Model &m) {
    const ModelDims &d = m.d;
    std::vector<uint64_t> h(3 + 2 * (size_t) d.ple_heads);
    for (int i = 0; i < 3; ++i) h[i] = (uint64_t) d.ple_mult[i];
    for (int i = 0; i < d.ple_heads; ++i) {
        h[3 + i] = (uint64_t) d.ple_size[i];
        h[3 + d.ple_heads + i] = (uint64_t) d.ple_off[i];
    }
    FN_CK(hipMemcpy(m.a.ng_tab, h.data(), h.size() * 8, hipMemcpyHostToDevice));
    return 0;
}

// the activations of MAXT tokens in one allocation: (pointer, bytes) pairs carved at 256-byte offsets
int carve_acts(Model &m) {
    const ModelDims &d = m.d;
    const size_t T = MAXT, HCD = (size_t) d.HC * d.D, ldr = (size_t) d.HCR + d.HC;
    Acts &a = m.a;
    m.nsplit = attn_pick_nsplit(1, d.NKV, MAXT, 4 * d.top + 4);
    for (int nt = 1; nt <= MAXT; ++nt)
        m.work_bytes = std::max(m.work_bytes, attn_qsa_work_bytes(1, d.NH, nt, HDK, m.nsplit, m.max_ctx, d.top) + 256);
    const size_t F = 4;
    struct Cut {
        void **p;
        size_t bytes;
    };
    std::vector<Cut> cuts = {
        {(void **) &a.hb[0], T * HCD * F}, {(void **) &a.hb[1], T * HCD * F}, {(void **) &a.hn, T * HCD * F},
        {(void **) &a.lr, std::max<size_t>(HC_KS, d.HC) * T * ldr * F}, {(void **) &a.amv, T * AM_CH * F},
        {(void **) &a.ami, T * AM_CH * 4}, {(void **) &a.t320, T * d.HCR * F}, {(void **) &a.a, T * HCD * F},
        {(void **) &a.x, T * d.D * F}, {(void **) &a.inj, T * d.HC * F}, {(void **) &a.qkv, T * d.CONVCH * F},
        {(void **) &a.zz, T * d.DINNER * F}, {(void **) &a.abv, T * 2 * d.NVH * F}, {(void **) &a.on, T * d.DINNER * F},
        {(void **) &a.qg, T * d.NH * 2 * HDK * F}, {(void **) &a.kk, T * d.NKV * HDK * F},
        {(void **) &a.vv, T * d.NKV * HDK * F}, {(void **) &a.iqk, T * (IXH * IXD + IXD) * F},
        {(void **) &a.og, T * d.NH * HDK * F}, {(void **) &a.y, T * d.D * F}, {(void **) &a.rsgv, T * (d.NE + 1) * F},
        {(void **) &a.shg, T * d.FFS * F}, {(void **) &a.shu, T * d.FFS * F}, {(void **) &a.sha, T * d.FFS * F},
        {(void **) &a.shd, T * d.D * F}, {(void **) &a.act, T * d.NEU * d.FFE * F},
        {(void **) &a.dpart, T * d.NEU * d.D * F}, {(void **) &a.wsel, T * d.NEU * F},
        {(void **) &a.logits, T * d.VOCAB * F}, {(void **) &a.work, m.work_bytes}, {(void **) &a.io, IO_WORDS * 4},
        {(void **) &a.sel, T * d.NEU * 4}, {(void **) &a.pos, 4},
    };
    if (d.ple_layers) {
        cuts.push_back({(void **) &a.ng_emb, T * d.D * F});
        cuts.push_back({(void **) &a.ng_key, T * HCD * F});
        cuts.push_back({(void **) &a.ng_val, T * d.D * F});
        cuts.push_back({(void **) &a.ng_tok, NG_RING * 4});
        cuts.push_back({(void **) &a.ng_tab, (3 + 2 * (size_t) d.ple_heads) * 8});
    }
    size_t total = 0;
    for (const Cut &c : cuts) total += (std::max<size_t>(c.bytes, 16) + 255) / 256 * 256;
    uint8_t *base = nullptr;
    const hipError_t e = hipMalloc((void **) &base, total);
    if (e != hipSuccess) FN_FAIL("load: hipMalloc(" + std::to_string(total) + " B) -> " + hipGetErrorString(e));
    m.allocs.push_back(base);
    m.bytes += total;
    FN_CK(hipMemsetAsync(base, 0, total, m.st));
    FN_CK(hipStreamSynchronize(m.st));
    size_t off = 0;
    for (const Cut &c : cuts) {
        *c.p = base + off;
        off += (std::max<size_t>(c.bytes, 16) + 255) / 256 * 256;
    }
    a.ids = a.io;
    a.status = reinterpret_cast<unsigned *>(a.io + MAXT);
    a.am = a.io + MAXT + 1;
    return 0;
}

}  // namespace

int read_dims(const Gguf &g, ModelDims &d) {
    auto it = g.strs.find("general.architecture");
    if (it == g.strs.end()) FN_FAIL("load: general.architecture missing");
    const std::string a = it->second + ".";
    auto num = [&](const char *k, double dflt = -1) { return g.num(a + k, dflt); };
    auto arr = [&](const char *k) {
        auto it2 = g.iarrays.find(a + k);
        return it2 == g.iarrays.end() ? std::vector<int64_t>{} : it2->second;
    };
    d = ModelDims{};
    d.D = (int) num("embedding_length");
    d.NL = (int) num("block_count");
    d.NH = (int) num("attention.head_count");
    d.NKV = (int) num("attention.head_count_kv");
    d.HD = (int) num("attention.key_length", 256);
    d.NROT = (int) num("rope.dimension_count", 64);
    d.theta = (float) num("rope.freq_base", 1e7);
    d.eps = (float) num("attention.layer_norm_rms_epsilon", 1e-6);
    d.NE = (int) num("expert_count");
    d.NEU = (int) num("expert_used_count");
    d.FFE = (int) num("expert_feed_forward_length");
    d.FFS = (int) num("expert_shared_feed_forward_length", d.FFE);
    d.DS = (int) num("ssm.state_size", 128);
    d.NKH = (int) num("ssm.group_count");
    d.NVH = (int) num("ssm.time_step_rank");
    d.DINNER = (int) num("ssm.inner_size");
    d.conv = (int) num("ssm.conv_kernel", 4);
    d.attn_every = (int) num("full_attention_interval", 4);
    d.HC = (int) num("hyper_connection.count");
    d.HCR = (int) num("hyper_connection.low_rank");
    d.IXH = (int) num("attention.indexer.head_count", IXH);
    d.IXD = (int) num("attention.indexer.key_length", IXD);
    d.top = (int) num("attention.indexer.top_k", 2048) / IXR;
    for (int64_t v : arr("ple.layers")) d.ple.push_back((int) v);
    d.ple_layers = (int) d.ple.size();
    if (d.ple_layers) {
        d.ple_heads = 2 * (int) num("ple.heads_per_ngram", 8);
        d.ple_hd = (int) num("embedding_length_per_layer_input", 160);
        d.ple_eos = (int) num("ple.eos_token_id", -1);
        d.ple_mult = arr("ple.layer_multipliers");
        d.ple_off = arr("ple.head_offsets");
        d.ple_size = arr("ple.head_vocab_sizes");
    }
    const GTensor *te = g.find("token_embd.weight");
    if (!te) FN_FAIL("load: tensor token_embd.weight missing");
    d.VOCAB = (int) te->ne[1];
    d.CONVCH = 2 * d.NKH * d.DS + d.DINNER;
    auto bad = [](const std::string &what) { FN_FAIL("load: model hyperparameters: " + what); };
    if (d.D < 32 || d.D % 32 || d.NL < 1 || d.VOCAB < 1) return bad("embedding_length, block_count or vocabulary");
    if (d.HD != HDK || d.DS != DSK || d.conv != 4) return bad("head dims 256 / 128 and conv kernel 4 are built");
    if (d.IXH != IXH || d.IXD != IXD || d.top < 1) return bad("the indexer is built for 4 heads of 128");
    if (d.NKV < 1 || d.NH % d.NKV || (d.NH / d.NKV != 4 && d.NH / d.NKV != 8 && d.NH / d.NKV != 12))
        return bad("query heads per kv head must be 4, 8 or 12");
    if (d.NROT < 2 || d.NROT > 128 || d.NROT % 4) return bad("rope dimension count");
    if (d.NKH < 1 || d.NVH < 1 || d.NVH % d.NKH || d.DINNER != d.NVH * d.DS) return bad("ssm heads");
    if (d.NE < 1 || d.NE > 1024 || d.NEU < 1 || d.NEU > 32 || d.NEU > d.NE || d.FFE < 32 || d.FFS < 32)
        return bad("experts (at most 1024, at most 32 used)");
    if (d.HC < 1 || d.HC > 16 || d.HCR < 1) return bad("hyper-connections");
    if (d.attn_every < 0) return bad("full_attention_interval");
    if (d.ple_layers) {
        if ((int) num("ple.ngram_size", 3) != 3 || (int) num("ple.conv_kernel", 4) != 4)
            return bad("PLE: n-grams of 3 and conv kernel 4 are built");
        if (d.ple_heads < 2 || d.ple_heads > NG_MAXH || d.ple_hd < 32 || d.ple_hd % 32 || d.ple_heads * d.ple_hd != d.D)
            return bad("PLE: heads x values per head must be the embedding length, values per head a multiple of 32");
        if (d.ple_mult.size() != 3 || (int) d.ple_off.size() != d.ple_heads || (int) d.ple_size.size() != d.ple_heads)
            return bad("PLE: multipliers, head offsets and head sizes");
        for (int i = 0; i < d.ple_heads; ++i)
            if (d.ple_size[i] < 1 || d.ple_off[i] < 0 || d.ple_off[i] + d.ple_size[i] > 0x7fffffffLL)
                return bad("PLE: head table ranges");
        for (int il : d.ple)
            if (il < 0 || il >= d.NL) return bad("PLE: layer index");
    }
    return 0;
}

int plan_weights(Model &m, const Gguf &g, const Gguf &g2) {
    const ModelDims &d = m.d;
    const Ctx c{d, m.max_ctx, g, g2};
    if (plan_arena(c, d.ple_layers ? K_MODEL | K_MODEL_NG : K_MODEL, "", m.top)) return -1;
    m.layers.assign(d.NL, Layer{});
    for (int il = 0; il < d.NL; ++il) {
        Layer &L = m.layers[il];
        L.kind = d.attn_every > 0 && (il + 1) % d.attn_every == 0 ? K_ATTN : K_DELTA;
        for (int p : d.ple)
            if (p == il) L.kind |= K_NGRAM;
        if (plan_arena(c, L.kind, "blk." + std::to_string(il) + ".", L)) return -1;
        // one kernel decodes an expert's gate and up rows together
        if (L.piece[FF_X_GATE].L.type != L.piece[FF_X_UP].L.type)
            FN_FAIL("load: blk." + std::to_string(il) + ". gate and up experts differ in type");
    }
    if (d.ple_layers) {
        const Piece &tab = m.top.piece[NG_TABLE];
        int64_t reach = 0;
        for (int i = 0; i < d.ple_heads; ++i) reach = std::max(reach, d.ple_off[i] + d.ple_size[i]);
        if ((int64_t) tab.L.rows < reach)
            FN_FAIL("load: per_layer_token_embd.weight has " + std::to_string(tab.L.rows) +
                    " rows, the n-gram heads reach " + std::to_string(reach));
    }
    return 0;
}

int commit_weights(Model &m) {
    Stager sg;
    sg.st = m.st;
    if (commit_arena(m, m.top, sg)) return -1;
    for (Layer &L : m.layers)
        if (commit_arena(m, L, sg)) return -1;
    if (carve_acts(m) || (m.d.ple_layers && ngram_setup(m))) return -1;
    FN_CK(hipDeviceSynchronize());
    return 0;
}

}  // namespace fn

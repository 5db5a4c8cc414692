// GGUF weight formats and the GEMV of the projections around the decode path, for gfx950: layouts, plans and the
// dispatch to the per-format instantiations (quant_impl.cuh, quant_t*.hip).
//
// The reference decodes its weights with ggml's arithmetic (engine/faie2fn.cu:343-689) and runs them through a
// tiled, split-K GEMV (faie2fn.cu:690-1042, 2033-2116) whose test hooks are fn_test_dequant / fn_test_gemv
// (faie2fn.cu:2751-2782, 2916-2935).  This file is a gfx950 design of the same operations:
//
//   * packing (quant_pack_launch): every field of a format goes to its own plane (QLayout), so each lane reads
//     its group's quants with 16-byte loads and its scales with 8/2-byte loads, all naturally aligned;
//   * decoding: one lane decodes one group of 32 values into exact small-integer floats q[32] plus, per half of
//     16 values, a scale s and an offset m, such that the GGUF value is fl(s * q - m) rounded once -- the value
//     ggml's dequantize_row_* computes (s * q is exact for every format whose m is not zero);
//   * GEMV: 16 lanes per row, four rows per wave, four waves per workgroup; each lane walks the row's groups
//     with stride 16, keeps the next group's loads in flight while it does the current one's FMAs, and the row
//     sum is a 16-lane DPP reduction.  Short rows split K over workgroups whose partials a second pass adds in a
//     fixed order, so results do not depend on timing.  For formats without an offset the scale multiplies the
//     16-value dot product instead of each weight.
#include "quant_impl.cuh"

namespace fn {

int g_ov_ks = 0, g_ov_lpr = 0, g_ov_kernel = 0, g_ov_wpc = 0;
int g_persist = 1;  // fn_gemv_waves: 1 = grid of the workgroups resident at once, 0 = one workgroup per row tile

namespace {

// GGUF rows -> planes: one thread per (row, block), plain byte copies (load-time work)
__global__ void k_pack(QLayout L, const uint8_t *__restrict__ raw, uint8_t *__restrict__ out) {
    const size_t nb = (size_t) (L.cols / L.qk);
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) L.rows * nb) return;
    const size_t row = i / nb, blk = i % nb;
    const uint8_t *src = raw + row * L.row_bytes + blk * L.bb;
    for (int p = 0; p < L.nplanes; ++p) {
        uint8_t *dst = out + L.off[p] + row * L.rs[p] + blk * L.fbytes[p];
        for (int b = 0; b < L.fbytes[p]; ++b) dst[b] = src[L.foff[p] + b];
    }
}

// y[i] = sum over splits s = 0..ks-1 of part[s][i], in that order
__global__ void k_gemv_reduce(const float *__restrict__ part, int ks, int n, float *__restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = part[i];
    for (int k = 1; k < ks; ++k) s += part[(size_t) k * n + i];
    y[i] = s;
}

const QOps *ops(uint32_t type) {
    for (auto f : {qops_group1, qops_group2, qops_group3, qops_group4, qops_group5})
        if (const void *o = f(type)) return static_cast<const QOps *>(o);
    return nullptr;
}

int rows_check(const QLayout &L, int R, int npairs, int xdiv, const float *x, const float *out) {
    if (R < 1 || L.rows % R || npairs < 1 || npairs > 65535 || xdiv < 1) FN_FAIL("rows: bad shape");
    if (!x || !out) FN_FAIL("rows: null pointer");
    if (((uintptr_t) x | (uintptr_t) out) % 16) FN_FAIL("rows: x and out must be 16-byte aligned");
    return 0;
}


}  // namespace

bool qlayout(uint32_t type, int rows, int cols, QLayout &L) {
    struct F {
        int qk, bb, np, fo[3], fb[3];
    };
    F f{};
    switch (type) {
        case QT_BF16: f = {32, 64, 1, {0, 0, 0}, {64, 0, 0}}; break;
        case QT_Q8_0: f = {32, 34, 2, {2, 0, 0}, {32, 2, 0}}; break;
        case QT_IQ4_NL: f = {32, 18, 2, {2, 0, 0}, {16, 2, 0}}; break;
        case QT_IQ4_XS: f = {256, 136, 2, {8, 0, 0}, {128, 8, 0}}; break;
        case QT_IQ3_S: f = {256, 110, 3, {2, 66, 0}, {64, 44, 2}}; break;
        case QT_IQ2_XXS: f = {256, 66, 2, {2, 0, 0}, {64, 2, 0}}; break;
        case QT_IQ2_XS: f = {256, 74, 3, {2, 66, 0}, {64, 8, 2}}; break;
        case QT_IQ2_S: f = {256, 82, 3, {2, 66, 0}, {64, 16, 2}}; break;
        case QT_IQ3_XXS: f = {256, 98, 2, {2, 0, 0}, {96, 2, 0}}; break;
        case QT_Q2_0: f = {64, 18, 2, {2, 0, 0}, {16, 2, 0}}; break;
        case QT_Q4_K: f = {256, 144, 2, {16, 0, 0}, {128, 16, 0}}; break;
        case QT_Q5_K: f = {256, 176, 3, {48, 16, 0}, {128, 32, 16}}; break;
        case QT_Q6_K: f = {256, 210, 3, {0, 128, 192}, {128, 64, 18}}; break;
        default:
            set_error("unsupported type " + std::to_string(type) +
                      " (this library reads BF16, Q8_0, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_NL, "
                      "IQ4_XS, Q2_0)");
            return false;
    }
    if (rows < 1 || cols < 1 || cols % f.qk) {
        set_error("unsupported shape: rows >= 1 and cols a multiple of " + std::to_string(f.qk) + " for type " +
                  std::to_string(type));
        return false;
    }
    L = QLayout{};
    L.type = type;
    L.rows = rows;
    L.cols = cols;
    L.qk = f.qk;
    L.bb = f.bb;
    L.nplanes = f.np;
    const size_t nb = (size_t) cols / f.qk;
    L.row_bytes = nb * f.bb;
    size_t off = 0;
    for (int p = 0; p < f.np; ++p) {
        L.fbytes[p] = f.fb[p];
        L.foff[p] = f.fo[p];
        L.rs[p] = nb * f.fb[p];
        L.off[p] = off;
        off += (L.rs[p] * rows + 255) / 256 * 256;
    }
    L.bytes = off;
    return true;
}

void gemv_override(int lpr, int ks, int kernel, int waves_per_cu) {
    g_ov_lpr = (lpr == 16 || lpr == 32 || lpr == 64) ? lpr : 0;
    g_ov_ks = std::max(0, ks);
    g_ov_kernel = (kernel >= 1 && kernel <= 4) ? kernel : 0;
    g_ov_wpc = std::max(0, waves_per_cu);
}

void gemv_persistent(int on) { g_persist = on != 0; }

GemvPlan gemv_plan(const QLayout &L, int ks_force) {
    GemvPlan p;
    p.ngroups = L.cols / 32;
    // lanes per row (measured on the projection shapes, nt 1 and 8): a few groups per lane, fewer lanes per row for
    // very tall weights (more row-sets per wave to stream through), and enough lanes in all (rows * lpr / 64 waves)
    // to spread a short weight over the CUs
    // (a forced split: the same rule on the groups of one split and the rows times the splits)
    const int kf = ks_force > 0 ? std::min(ks_force, p.ngroups) : 1;
    const int G = (p.ngroups + kf - 1) / kf;
    const bool q6 = L.type == QT_Q6_K;  // one group in flight per lane and batch: more groups per lane pay off
    int lpr = G >= 160 ? 32 : (G >= 128 ? 64 : (G >= 48 ? (L.rows >= 32768 || (q6 && L.rows >= 4096) ? 16 : 32) : 16));
    while (lpr < 64 && G > lpr && (size_t) L.rows * kf * lpr / 64 < 1024) lpr *= 2;
    p.lpr = g_ov_lpr ? g_ov_lpr : lpr;
    p.rpw = 8 * (64 / p.lpr);
    p.ntiles = (L.rows + p.rpw - 1) / p.rpw;
    p.grid = g_persist ? 0 : p.ntiles;
    p.ks = std::min(ks_force > 0 ? ks_force : g_ov_ks ? g_ov_ks : 1, p.ngroups);
    const int gps = (p.ngroups + p.ks - 1) / p.ks;
    p.ks = (p.ngroups + gps - 1) / gps;  // every split holds at least one group
    return p;
}

size_t gemv_work_bytes(const QLayout &L, int nt) {
    const GemvPlan p = gemv_plan(L);
    return p.ks > 1 ? (size_t) p.ks * nt * L.rows * 4 : 0;
}

int quant_pack_launch(const QLayout &L, const uint8_t *raw, uint8_t *packed, hipStream_t st) {
    if (!raw || !packed) FN_FAIL("pack: null pointer");
    const size_t n = (size_t) L.rows * (L.cols / L.qk);
    hipLaunchKernelGGL(k_pack, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, L, raw, packed);
    FN_CK(hipGetLastError());
    return 0;
}

int quant_dequant_launch(const QLayout &L, const uint8_t *packed, float *out, hipStream_t st) {
    if (!packed || !out) FN_FAIL("dequant: null pointer");
    if ((uintptr_t) out % 16 || (uintptr_t) packed % 16) FN_FAIL("dequant: pointers must be 16-byte aligned");
    const QOps *o = ops(L.type);
    if (!o) FN_FAIL("dequant: unsupported type");
    return o->dequant(L, planes(L, packed), out, st);
}

// the GEMV kernels address each plane of a weight with 32-bit offsets from its base
bool gemv_planes_fit(const QLayout &L) {
    for (int i = 0; i < 3; ++i)
        if (L.rs[i] * (size_t) L.rows > ((size_t) 1 << 32)) return false;
    return true;
}

int gemv_launch(const QLayout &L, const uint8_t *packed, const float *x, int nt, float *y, float *work,
                size_t work_bytes, hipStream_t st, int ks_force) {
    if (nt < 1 || nt > MAXNT) FN_FAIL("gemv: nt must be 1..8");
    if (!packed || !x || !y) FN_FAIL("gemv: null pointer");
    if (!gemv_planes_fit(L)) FN_FAIL("gemv: a plane of the packed weight exceeds 4 GiB");
    if ((uintptr_t) packed % 16 || (uintptr_t) x % 16) FN_FAIL("gemv: weight and x must be 16-byte aligned");
    const GemvPlan pl = gemv_plan(L, ks_force);
    float *out = y;
    if (pl.ks > 1) {
        const size_t need = (size_t) pl.ks * nt * L.rows * 4;
        if (!work || work_bytes < need) FN_FAIL("gemv: work buffer smaller than fn_gemv_work_bytes()");
        out = work;
    }
    const QOps *o = ops(L.type);
    if (!o) FN_FAIL("gemv: unsupported type");
    const int rc = o->gemv(L, pl, planes(L, packed), x, nt, out, st);
    if (rc) return rc;
    if (pl.ks > 1) {
        const int n = nt * L.rows;
        hipLaunchKernelGGL(k_gemv_reduce, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, work, pl.ks, n, y);
        FN_CK(hipGetLastError());
    }
    return 0;
}

int gemv_split_launch(const QLayout &L, const uint8_t *packed, const float *x, int nt, int ks, float *part,
                      int *ks_out, hipStream_t st) {
    if (nt < 1 || nt > MAXNT) FN_FAIL("gemv: nt must be 1..8");
    if (!packed || !x || !part || ks < 1) FN_FAIL("gemv: bad arguments");
    if (!gemv_planes_fit(L)) FN_FAIL("gemv: a plane of the packed weight exceeds 4 GiB");
    if ((uintptr_t) packed % 16 || (uintptr_t) x % 16) FN_FAIL("gemv: weight and x must be 16-byte aligned");
    const GemvPlan pl = gemv_plan(L, ks);
    const QOps *o = ops(L.type);
    if (!o) FN_FAIL("gemv: unsupported type");
    if (ks_out) *ks_out = pl.ks;
    return o->gemv(L, pl, planes(L, packed), x, nt, part, st);
}

int embed_launch(const QLayout &L, const uint8_t *packed, const int32_t *ids, int nt, int copies, float *out,
                 hipStream_t st) {
    if (!packed || !ids || !out || nt < 1 || copies < 1) FN_FAIL("embed: bad arguments");
    if ((uintptr_t) out % 16) FN_FAIL("embed: out must be 16-byte aligned");
    const QOps *o = ops(L.type);
    if (!o) FN_FAIL("embed: unsupported type");
    return o->embed(L, planes(L, packed), ids, nt, copies, out, st);
}

int ngram_gather_launch(const QLayout &L, const uint8_t *packed, const NgramGather &g, int nt, float *out,
                        hipStream_t st) {
    if (!packed || !out || !g.ids || !g.pos || !g.ring || !g.tab || nt < 1 || g.heads < 2)
        FN_FAIL("ngram: bad arguments");
    if (g.ring_mask < nt + 1 || (g.ring_mask & (g.ring_mask + 1))) FN_FAIL("ngram: token ring too short");
    if ((uintptr_t) out % 16) FN_FAIL("ngram: out must be 16-byte aligned");
    const QOps *o = ops(L.type);
    if (!o) FN_FAIL("ngram: unsupported type");
    return o->ngram(L, planes(L, packed), g, nt, out, st);
}

int rows_launch(const QLayout &L, const uint8_t *packed, int R, const int32_t *sel, int npairs, int xdiv,
                const float *x, float *out, hipStream_t st) {
    if (!packed || rows_check(L, R, npairs, xdiv, x, out)) return -1;
    const QOps *o = ops(L.type);
    if (!o) FN_FAIL("rows: unsupported type");
    const PP P = planes(L, packed);
    return o->rows(L, P, P, R, sel, npairs, xdiv, x, out, st, RouteIn{});
}

int swiglu_launch(const QLayout &Lg, const uint8_t *pg, const QLayout &Lu, const uint8_t *pu, int R,
                  const int32_t *sel, int npairs, int xdiv, const float *x, float *act, hipStream_t st,
                  const RouteIn *route) {
    if (!pg || !pu || rows_check(Lg, R, npairs, xdiv, x, act)) return -1;
    if (Lg.type != Lu.type || Lg.rows != Lu.rows || Lg.cols != Lu.cols) FN_FAIL("swiglu: gate and up weights differ");
    const QOps *o = ops(Lg.type);
    if (!o) FN_FAIL("swiglu: unsupported type");
    RouteIn rt{};
    if (route) {
        rt = *route;
        if (!rt.rsg || !rt.sel || !rt.wsel || !rt.shg || !rt.shu || !rt.sha || rt.NE < 1 || rt.NE > 64 * ROUTE_PER ||
            rt.NEU < 1 || rt.NEU > 64 || rt.NEU > rt.NE || xdiv != rt.NEU || npairs % rt.NEU)
            FN_FAIL("swiglu: bad routing arguments");
    }
    return o->swiglu(Lg, planes(Lg, pg), planes(Lu, pu), R, sel, npairs, xdiv, x, act, st, rt);
}

}  // namespace fn


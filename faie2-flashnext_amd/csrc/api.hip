// C ABI of libfaie2fn.so (declared in include/faie2fn.h).
//
// Section 1 keeps the reference's fn_* names and signatures (engine/faie2fn.cu:2492-2935) so its ctypes layer
// (flashnext/fn.py) binds unchanged; fn_load / fn_forward run the model on one GPU (model.hip), fn_bench_route is
// in route.hip.  Sections 2 and 3 are this path's hooks: host arrays in / out (synchronous, device 0,
// the reference's unit-test-hook style, faie2fn.cu:2745) and the device-buffer entry points an engine calls.
#include "engine.h"
#include "model.h"
#include "quant.h"
#include "qsa.h"
#include "hostbuf.h"

#include <cstring>
#include <vector>

#define FN_API extern "C" __attribute__((visibility("default")))

namespace fn {

static std::string g_err;

void set_error(const std::string &msg) { g_err = msg; }
const char *error_cstr() { return g_err.c_str(); }

}  // namespace fn

using fn::DevBufs;
using fn::set_error;
using fn::use_device0;

// ---------------------------------------------------------------------------------------------
// 1. reference API

// The engine entry points act on the loaded model (fn_load) if there is one, else on the path engine (fn_path_init).
FN_API const char *fn_error(void) { return fn::error_cstr(); }
FN_API void fn_free(void) {
    fn::model_free();
    fn::path_free();
}
FN_API int fn_load(const char *shard1, const char *shard2, int max_ctx, int split) {
    (void) split;  // one GPU: every layer on device 0
    return fn::model_load(shard1, shard2, max_ctx);
}
FN_API int fn_split(void) {
    if (fn::model_loaded()) return fn::model_layers();  // no layer on a second device
    return fn::path_loaded() ? 0 : -1;
}
FN_API double fn_dev_gb(int dv) {
    if (fn::model_loaded()) return dv == 0 ? fn::model_dev_gb() : (dv == 1 ? 0.0 : -1.0);
    return dv == 0 ? fn::path_dev_gb() : -1;
}
FN_API int fn_n_past(void) { return fn::model_loaded() ? fn::model_n_past() : fn::path_n_past(); }
FN_API double fn_last_ms(void) { return fn::model_loaded() ? fn::model_last_ms() : fn::path_last_ms(); }
FN_API int fn_reset(void) { return fn::model_loaded() ? fn::model_reset() : fn::path_reset(); }
FN_API int fn_use_graphs(int on) { return fn::model_loaded() ? fn::model_use_graphs(on) : fn::path_use_graphs(on); }
FN_API int fn_forward(const int32_t *tokens, int nt, float *logits, int32_t *argmax) {
    return fn::model_forward(tokens, nt, logits, argmax);
}
FN_API int fn_debug_layers(float *out) { return fn::model_debug_layers(out); }
// The reference's A/B switches for its CUDA forward, accepted so that its scripts bind and run; these three change
// nothing here.  fn_pdl / fn_early: programmatic dependent launch, and GEMVs started beside the kernel before them
// under it, have no HIP counterpart (the forward is one hipGraph on one stream; graph branches for the independent
// GEMVs measured slower).  fn_moe_var: the variant of the reference's expert gate/up tiles; the gate/up kernel here
// has one shape (16 lanes a row, 8 rows a workgroup).
FN_API void fn_pdl(int) {}
FN_API void fn_early(int) {}
FN_API void fn_moe_var(int) {}
// The reference's expert launch shapes (gate/up and down: warps splitting a tile's columns, tiles a block).  dn_wpt
// picks the MoE output kernel by the waves that share one output row: 1 = the 16-row kernel (one wave sums whole
// rows), 2 or more = the 4-row kernel (four waves split each row's items); 0 leaves it, as in the reference, and a
// negative value returns to the automatic choice (not in the reference, which ignores it).  Either kernel gives
// the same bits; a graph captured before keeps its kernel (fn_use_graphs drops the graphs).  gu_wpt, gu_tb, dn_tb:
// no effect (one gate/up shape; rows a workgroup follow from the kernel).
FN_API void fn_moe_override(int, int, int dn_wpt, int) { fn::moe_down_override(dn_wpt); }

FN_API int fn_model_dims(const char *path, int *out, int n) {
    fn::ModelDims d;
    if (!out || n < 1) FN_FAIL("model_dims: null output");
    if (fn::model_inspect(path, &d)) return -1;
    const int v[] = {d.D, d.NL, d.NH, d.NKV, d.HD, d.NROT, d.NE, d.NEU, d.FFE, d.FFS, d.DS, d.NKH, d.NVH, d.DINNER,
                     d.CONVCH, d.attn_every, d.HC, d.HCR, d.IXH, d.IXD, d.top, d.VOCAB, d.ple_layers, d.ple_heads,
                     d.ple_hd};
    const int k = (int) (sizeof(v) / sizeof(v[0]));
    for (int i = 0; i < n; ++i) out[i] = i < k ? v[i] : 0;
    return k;
}

// ---------------------------------------------------------------------------------------------
// 3. device entry points

FN_API int fn_gdn_block_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt, int ring,
                            const int32_t *pos, const float *qkv, const float *conv_w, float *conv_ring,
                            const float *ab, const float *dt_bias, const float *ssm_a, float *S, const float *z,
                            const float *norm_w, float eps, float *out, void *stream) {
    fn::GdnBlock p{B, nkh, nvh, dk, dv, head_map, gate_act, nt, ring, eps, pos, qkv, conv_w, conv_ring, ab,
                   dt_bias, ssm_a, S, z, norm_w, out};
    return fn::gdn_block_launch(p, (hipStream_t) stream);
}

FN_API int fn_gdn_block_xab_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int ring,
                                const int32_t *pos, const float *qkv, const float *conv_w, float *conv_ring,
                                const float *x, int hidden, const uint16_t *w_ab, const float *dt_bias,
                                const float *ssm_a, float *S, const float *z, const float *norm_w, float eps,
                                float *out, void *stream) {
    fn::GdnBlock p{B, nkh, nvh, dk, dv, head_map, gate_act, 1, ring, eps, pos, qkv, conv_w, conv_ring, nullptr,
                   dt_bias, ssm_a, S, z, norm_w, out};
    p.x = x;
    p.wab = w_ab;
    p.hidden = hidden;
    if (!w_ab) FN_FAIL("gdn: null pointer");
    return fn::gdn_block_launch(p, (hipStream_t) stream);
}

FN_API int fn_gdn_verify_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt, int ring,
                             const int32_t *pos, const int32_t *kr, int rnt, const float *rqkv, const float *rab,
                             const float *qkv, const float *conv_w, float *conv_ring, const float *ab,
                             const float *dt_bias, const float *ssm_a, float *S, const float *z, const float *norm_w,
                             float eps, float *out, void *stream) {
    fn::GdnVerify p{{B, nkh, nvh, dk, dv, head_map, gate_act, nt, ring, eps, pos, qkv, conv_w, conv_ring, ab, dt_bias,
                     ssm_a, S, z, norm_w, out},
                    kr, rnt, rqkv, rab};
    return fn::gdn_verify_launch(p, (hipStream_t) stream);
}

FN_API int fn_advance_by_dev(int32_t *pos, const int32_t *kr, int B, void *stream) {
    return fn::advance_by_launch(pos, kr, B, (hipStream_t) stream);
}

FN_API int fn_gdn_core_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int nt, const float *q,
                           const float *k, const float *v, const float *beta, const float *g, float *S, float *o,
                           void *stream) {
    fn::GdnCore p{B, nkh, nvh, dk, dv, head_map, nt, q, k, v, beta, g, S, o};
    return fn::gdn_core_launch(p, (hipStream_t) stream);
}

FN_API size_t fn_attn_work_bytes(int B, int nq, int nt, int hd, int nsplit) {
    if (B < 1 || nq < 1 || nt < 1 || hd < 1 || nsplit < 1) return 0;
    return fn::attn_work_bytes(B, nq, nt, hd, nsplit);
}

FN_API int fn_attn_nsplit(int B, int nkv, int nt, int ctx) { return fn::attn_pick_nsplit(B, nkv, nt, ctx); }

FN_API int fn_attn_dev(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                       const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                       const float *wk, float *Kc, float *Vc, int nsplit, float *work, size_t work_bytes, float *og,
                       void *stream) {
    fn::AttnDecode p{B, nq, nkv, hd, nrot, nt, max_ctx, nsplit, theta, eps, pos, qg, k, v, wq, wk, Kc, Vc, work,
                     work_bytes, og};
    return fn::attn_decode_launch(p, (hipStream_t) stream);
}

FN_API int fn_dev_status(int clear) {
    unsigned bits = 0;
    if (fn::status_read(&bits, clear != 0)) return -1;
    return (int) (bits & 0x7fffffffu);
}

FN_API int fn_advance_dev(int32_t *pos, int B, int nt, void *stream) {
    return fn::advance_launch(pos, B, nt, (hipStream_t) stream);
}

FN_API int fn_fill_normal_dev(float *p, size_t n, uint64_t seed, float mean, float std, void *stream) {
    return fn::fill_normal_launch(p, n, seed, mean, std, (hipStream_t) stream);
}

FN_API int fn_copy_dev(void *dst, const void *src, size_t bytes, void *stream) {
    return fn::copy_launch(dst, src, bytes, (hipStream_t) stream);
}

FN_API int fn_stage_events(void **events, int n) { return fn::stage_events(events, n); }

FN_API size_t fn_attn_qsa_work_bytes(int B, int nq, int nt, int hd, int nsplit, int max_ctx, int top) {
    if (B < 1 || nq < 1 || nt < 1 || hd < 1 || nsplit < 1 || max_ctx < 1 || top < 1) return 0;
    return fn::attn_qsa_work_bytes(B, nq, nt, hd, nsplit, max_ctx, top) + 256;
}

FN_API int fn_attn_qsa_dev(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                           const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                           const float *wk, float *Kc, float *Vc, const float *iqk, const float *wqn, const float *wkn,
                           float *IKc, float *BKc, int top, int nsplit, float *work, size_t work_bytes, float *og,
                           void *stream) {
    fn::AttnDecode p{B, nq, nkv, hd, nrot, nt, max_ctx, nsplit, theta, eps, pos, qg, k, v, wq, wk, Kc, Vc, work,
                     work_bytes, og};
    fn::QsaIndexer ix{B, nt, max_ctx, top, nrot, theta, eps, pos, iqk, wqn, wkn, IKc, BKc};
    return fn::attn_qsa_launch(p, ix, (hipStream_t) stream);
}

FN_API int fn_ix_blocks_dev(int B, int max_ctx, int j0, int j1, const float *IKc, const float *wkn, float *BKc,
                            int nrot, float theta, float eps, void *stream) {
    fn::QsaIndexer ix{B, 1, max_ctx, 512, nrot, theta, eps, nullptr, nullptr, nullptr, wkn, const_cast<float *>(IKc),
                      BKc};
    return fn::qsa_blocks_launch(ix, j0, j1, (hipStream_t) stream);
}

// ---------------------------------------------------------------------------------------------
// 4. path engine

FN_API int fn_path_init(int B, int nl, int attn_every, int nkh, int nvh, int nq, int nkv, int max_ctx, int head_map,
                        int gate_act, int nsplit) {
    return fn::path_init(B, nl, attn_every, nkh, nvh, nq, nkv, max_ctx, head_map, gate_act, nsplit);
}
FN_API int fn_path_buffer(int il, int kind, void **ptr, size_t *bytes) { return fn::path_buffer(il, kind, ptr, bytes); }
FN_API int fn_path_step(int steps, float *ms) { return fn::path_step(steps, ms); }

// ---------------------------------------------------------------------------------------------
// 2. host-array hooks

FN_API int fn_test_gdn(int B, int nkh, int nvh, int dk, int dv, int head_map, int nt, const float *q, const float *k,
                       const float *v, const float *beta, const float *g, float *S, float *o) {
    if (B < 1 || nkh < 1 || nvh < 1 || nt < 1 || dk < 1 || dv < 1) FN_FAIL("gdn: bad shape");
    if (!q || !k || !v || !beta || !g || !S || !o) FN_FAIL("gdn: null pointer");
    if (use_device0()) return -1;
    const size_t nq = (size_t) B * nt * nkh * dk, nv = (size_t) B * nt * nvh * dv, ns = (size_t) B * nt * nvh;
    const size_t nS = (size_t) B * nvh * dk * dv;
    DevBufs m;
    float *dq, *dk_, *dv_, *db, *dg, *dS, *dO;
    if (m.up(&dq, q, nq) || m.up(&dk_, k, nq) || m.up(&dv_, v, nv) || m.up(&db, beta, ns) || m.up(&dg, g, ns) ||
        m.up(&dS, (const float *) S, nS) || m.alloc(&dO, nv))
        return -1;
    if (fn_gdn_core_dev(B, nkh, nvh, dk, dv, head_map, nt, dq, dk_, dv_, db, dg, dS, dO, nullptr)) return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(S, dS, nS * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(o, dO, nv * 4, hipMemcpyDeviceToHost));
    return 0;
}

FN_API int fn_test_gdn_block(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt,
                             const float *qkv, const float *conv_w, float *conv_state, const float *ab,
                             const float *dt_bias, const float *ssm_a, float *S, const float *z, const float *norm_w,
                             float eps, float *out) {
    if (B < 1 || nkh < 1 || nvh < 1 || nt < 1 || dk < 1 || dv < 1) FN_FAIL("gdn: bad shape");
    if (nt > 61) FN_FAIL("gdn: nt must be <= 61 in one call");
    if (!qkv || !conv_w || !conv_state || !ab || !dt_bias || !ssm_a || !S || !z || !norm_w || !out)
        FN_FAIL("gdn: null pointer");
    if (use_device0()) return -1;
    const size_t C = (size_t) 2 * nkh * dk + (size_t) nvh * dv;
    int ring = 4;
    while (ring < nt + 3) ring *= 2;
    // host conv state [B][3][C] -> ring slots of positions -3, -2, -1 (pos = 0 inside the hook)
    std::vector<float> rh((size_t) B * ring * C, 0.0f);
    for (int b = 0; b < B; ++b)
        for (int j = 0; j < 3; ++j)
            std::memcpy(&rh[((size_t) b * ring + ((j - 3) & (ring - 1))) * C], conv_state + ((size_t) b * 3 + j) * C,
                        C * 4);
    std::vector<int32_t> ph(B, 0);
    const size_t nx = (size_t) B * nt * C, nab = (size_t) B * nt * 2 * nvh, nz = (size_t) B * nt * nvh * dv;
    const size_t nS = (size_t) B * nvh * dk * dv;
    DevBufs m;
    int32_t *dpos;
    float *dx, *dw, *dr, *dab, *ddt, *dsa, *dS, *dz, *dnw, *dout;
    if (m.up(&dpos, ph.data(), B) || m.up(&dx, qkv, nx) || m.up(&dw, conv_w, C * 4) || m.up(&dr, rh.data(), rh.size()) ||
        m.up(&dab, ab, nab) || m.up(&ddt, dt_bias, nvh) || m.up(&dsa, ssm_a, nvh) || m.up(&dS, (const float *) S, nS) ||
        m.up(&dz, z, nz) || m.up(&dnw, norm_w, dv) || m.alloc(&dout, nz))
        return -1;
    if (fn_gdn_block_dev(B, nkh, nvh, dk, dv, head_map, gate_act, nt, ring, dpos, dx, dw, dr, dab, ddt, dsa, dS, dz,
                         dnw, eps, dout, nullptr))
        return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(S, dS, nS * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(out, dout, nz * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(rh.data(), dr, rh.size() * 4, hipMemcpyDeviceToHost));
    // ring slots of positions nt-3 .. nt-1 -> [B][3][C]
    for (int b = 0; b < B; ++b)
        for (int j = 0; j < 3; ++j)
            std::memcpy(conv_state + ((size_t) b * 3 + j) * C, &rh[((size_t) b * ring + ((nt - 3 + j) & (ring - 1))) * C],
                        C * 4);
    return 0;
}

FN_API int fn_test_attn(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                        const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                        const float *wk, float *Kc, float *Vc, int nsplit, float *og) {
    if (B < 1 || nq < 1 || nkv < 1 || hd < 1 || nt < 1 || max_ctx < 1) FN_FAIL("attn: bad shape");
    if (!pos || !qg || !k || !v || !wq || !wk || !Kc || !Vc || !og) FN_FAIL("attn: null pointer");
    int maxpos = 0;
    for (int b = 0; b < B; ++b) {
        if (pos[b] < 0 || pos[b] + nt > max_ctx) FN_FAIL("attn: pos[b] + nt must lie in [0, max_ctx]");
        maxpos = std::max(maxpos, pos[b]);
    }
    if (use_device0()) return -1;
    const int mc = (max_ctx + 63) / 64 * 64;  // device cache rows, tile multiple
    if (nsplit <= 0) nsplit = fn::attn_pick_nsplit(B, nkv, nt, maxpos + nt);
    // reference layout [B][max_ctx][nkv][hd] -> key-tiled K / head-major V, rows < pos[b] only
    const size_t per = (size_t) nkv * mc * hd;
    std::vector<float> kh((size_t) B * per, 0.0f), vh((size_t) B * per, 0.0f);
    for (int b = 0; b < B; ++b)
        for (int p = 0; p < pos[b]; ++p)
            for (int g = 0; g < nkv; ++g) {
                const float *ks = Kc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                const float *vs = Vc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                float *kt = &kh[(((size_t) b * nkv + g) * (mc / 64) + p / 64) * 64 * hd + (size_t) (p % 64) * 4];
                for (int c = 0; c < hd / 4; ++c) std::memcpy(kt + (size_t) c * 256, ks + c * 4, 16);
                std::memcpy(&vh[(((size_t) b * nkv + g) * mc + p) * hd], vs, (size_t) hd * 4);
            }
    const size_t nqg = (size_t) B * nt * nq * 2 * hd, nkvn = (size_t) B * nt * nkv * hd, nog = (size_t) B * nt * nq * hd;
    const size_t wb = fn::attn_work_bytes(B, nq, nt, hd, nsplit);
    DevBufs m;
    int32_t *dpos;
    float *dqg, *dk_, *dv_, *dwq, *dwk, *dK, *dV, *dwork, *dog;
    if (m.up(&dpos, pos, B) || m.up(&dqg, qg, nqg) || m.up(&dk_, k, nkvn) || m.up(&dv_, v, nkvn) ||
        m.up(&dwq, wq, hd) || m.up(&dwk, wk, hd) || m.up(&dK, kh.data(), kh.size()) || m.up(&dV, vh.data(), vh.size()) ||
        m.alloc(&dwork, wb / 4 + 1) || m.alloc(&dog, nog))
        return -1;
    if (fn_attn_dev(B, nq, nkv, hd, nrot, theta, eps, nt, mc, dpos, dqg, dk_, dv_, dwq, dwk, dK, dV, nsplit, dwork, wb,
                    dog, nullptr))
        return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(og, dog, nog * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(kh.data(), dK, kh.size() * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(vh.data(), dV, vh.size() * 4, hipMemcpyDeviceToHost));
    // appended rows back into the reference layout
    for (int b = 0; b < B; ++b)
        for (int p = pos[b]; p < pos[b] + nt; ++p)
            for (int g = 0; g < nkv; ++g) {
                float *kd = Kc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                float *vd = Vc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                const float *kt = &kh[(((size_t) b * nkv + g) * (mc / 64) + p / 64) * 64 * hd + (size_t) (p % 64) * 4];
                for (int c = 0; c < hd / 4; ++c) std::memcpy(kd + c * 4, kt + (size_t) c * 256, 16);
                std::memcpy(vd, &vh[(((size_t) b * nkv + g) * mc + p) * hd], (size_t) hd * 4);
            }
    return 0;
}

FN_API int fn_test_attn_qsa(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                            const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                            const float *wk, float *Kc, float *Vc, const float *iqk, const float *wqn, const float *wkn,
                            float *IKc, int top, int nsplit, float *og, float *scores, uint8_t *mask) {
    constexpr int IXD = 128, IXR = 4;
    if (B < 1 || nq < 1 || nkv < 1 || hd < 1 || nt < 1 || max_ctx < 1 || top < 1) FN_FAIL("attn_qsa: bad shape");
    if (!pos || !qg || !k || !v || !wq || !wk || !Kc || !Vc || !iqk || !wqn || !wkn || !IKc || !og)
        FN_FAIL("attn_qsa: null pointer");
    int minpos = max_ctx, maxpos = 0;
    for (int b = 0; b < B; ++b) {
        if (pos[b] < 0 || pos[b] + nt > max_ctx) FN_FAIL("attn_qsa: pos[b] + nt must lie in [0, max_ctx]");
        minpos = std::min(minpos, pos[b]);
        maxpos = std::max(maxpos, pos[b]);
    }
    if (use_device0()) return -1;
    const int mc = (max_ctx + 255) / 256 * 256;
    if (nsplit <= 0) nsplit = fn::attn_pick_nsplit(B, nkv, nt, top * IXR + IXR);  // split the attended keys
    // K/V to the device layouts (rows < pos[b]), raw index keys as they are
    const size_t per = (size_t) nkv * mc * hd;
    std::vector<float> kh((size_t) B * per, 0.0f), vh((size_t) B * per, 0.0f), ikh((size_t) B * mc * IXD, 0.0f);
    for (int b = 0; b < B; ++b) {
        for (int p = 0; p < pos[b]; ++p)
            for (int g = 0; g < nkv; ++g) {
                const float *ks = Kc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                const float *vs = Vc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                float *kt = &kh[(((size_t) b * nkv + g) * (mc / 64) + p / 64) * 64 * hd + (size_t) (p % 64) * 4];
                for (int c = 0; c < hd / 4; ++c) std::memcpy(kt + (size_t) c * 256, ks + c * 4, 16);
                std::memcpy(&vh[(((size_t) b * nkv + g) * mc + p) * hd], vs, (size_t) hd * 4);
            }
        std::memcpy(&ikh[(size_t) b * mc * IXD], IKc + (size_t) b * max_ctx * IXD, (size_t) pos[b] * IXD * 4);
    }
    const size_t nqg = (size_t) B * nt * nq * 2 * hd, nkvn = (size_t) B * nt * nkv * hd, nog = (size_t) B * nt * nq * hd;
    const size_t niqk = (size_t) B * nt * (4 * IXD + IXD), nbk = (size_t) B * (mc / IXR) * IXD;
    const size_t wb = fn_attn_qsa_work_bytes(B, nq, nt, hd, nsplit, mc, top);
    DevBufs m;
    int32_t *dpos;
    float *dqg, *dk_, *dv_, *dwq, *dwk, *dK, *dV, *dwork, *dog, *diqk, *dwqn, *dwkn, *dIK, *dBK;
    if (m.up(&dpos, pos, B) || m.up(&dqg, qg, nqg) || m.up(&dk_, k, nkvn) || m.up(&dv_, v, nkvn) ||
        m.up(&dwq, wq, hd) || m.up(&dwk, wk, hd) || m.up(&dK, kh.data(), kh.size()) || m.up(&dV, vh.data(), vh.size()) ||
        m.alloc(&dwork, wb / 4 + 1) || m.alloc(&dog, nog) || m.up(&diqk, iqk, niqk) || m.up(&dwqn, wqn, IXD) ||
        m.up(&dwkn, wkn, IXD) || m.up(&dIK, ikh.data(), ikh.size()) || m.alloc(&dBK, nbk))
        return -1;
    FN_CK(hipMemset(dwork, 0, wb));
    // block keys complete before this call (the shortest sequence's; longer ones are rebuilt per sequence below)
    for (int b = 0; b < B; ++b) {
        fn::QsaIndexer one{1, 1, mc, top, nrot, theta, eps, nullptr, nullptr, nullptr, dwkn, dIK + (size_t) b * mc * IXD,
                           dBK + (size_t) b * (mc / IXR) * IXD};
        if (fn::qsa_blocks_launch(one, 0, pos[b] / IXR, nullptr)) return -1;
    }
    if (fn_attn_qsa_dev(B, nq, nkv, hd, nrot, theta, eps, nt, mc, dpos, dqg, dk_, dv_, dwq, dwk, dK, dV, diqk, dwqn,
                        dwkn, dIK, dBK, top, nsplit, dwork, wb, dog, nullptr))
        return -1;
    FN_CK(hipDeviceSynchronize());
    FN_CK(hipMemcpy(og, dog, nog * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(kh.data(), dK, kh.size() * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(vh.data(), dV, vh.size() * 4, hipMemcpyDeviceToHost));
    FN_CK(hipMemcpy(ikh.data(), dIK, ikh.size() * 4, hipMemcpyDeviceToHost));
    for (int b = 0; b < B; ++b) {
        for (int p = pos[b]; p < pos[b] + nt; ++p) {
            for (int g = 0; g < nkv; ++g) {
                float *kd = Kc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                float *vd = Vc + (((size_t) b * max_ctx + p) * nkv + g) * hd;
                const float *kt = &kh[(((size_t) b * nkv + g) * (mc / 64) + p / 64) * 64 * hd + (size_t) (p % 64) * 4];
                for (int c = 0; c < hd / 4; ++c) std::memcpy(kd + c * 4, kt + (size_t) c * 256, 16);
                std::memcpy(vd, &vh[(((size_t) b * nkv + g) * mc + p) * hd], (size_t) hd * 4);
            }
            std::memcpy(IKc + ((size_t) b * max_ctx + p) * IXD, &ikh[((size_t) b * mc + p) * IXD], IXD * 4);
        }
    }
    // indexer outputs: scores and the kept-block mask from the key lists
    const size_t bt = (size_t) B * nt, nbmax = (size_t) max_ctx / IXR, aw = fn::attn_work_bytes(B, nq, nt, hd, nsplit);
    const char *iw = reinterpret_cast<const char *>(dwork) + (aw + 255) / 256 * 256;
    const float *dsc = reinterpret_cast<const float *>(iw) + bt * 4 * IXD;
    const int32_t *dkeys = reinterpret_cast<const int32_t *>(dsc + bt * (mc / IXR));
    if (scores) {
        std::vector<float> sh(bt * (mc / IXR));
        FN_CK(hipMemcpy(sh.data(), dsc, sh.size() * 4, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < bt; ++i) std::memcpy(scores + i * nbmax, &sh[i * (mc / IXR)], nbmax * 4);
    }
    if (mask) {
        const size_t ks = (size_t) top * IXR + IXR;
        std::vector<int32_t> kl(bt * ks);
        FN_CK(hipMemcpy(kl.data(), dkeys, kl.size() * 4, hipMemcpyDeviceToHost));
        std::memset(mask, 0, bt * nbmax);
        for (int b = 0; b < B; ++b)
            for (int t = 0; t < nt; ++t) {
                const size_t i = (size_t) b * nt + t;
                const int nb = (pos[b] + t + 1) / IXR;
                if (nb <= top) continue;
                for (int r = 0; r < top; ++r) mask[i * nbmax + kl[i * ks + (size_t) r * IXR] / IXR] = 1;
            }
    }
    return 0;
}

// Internal API of the GGUF weight formats and the GEMV of the projections around the decode path
// (quant.hip).  Type ids are the GGUF ones the reference uses (engine/faie2fn.cu:78-81).
#pragma once

#include "common.cuh"

#include <cstddef>

namespace fn {

enum : uint32_t {
    QT_Q8_0 = 8, QT_Q4_K = 12, QT_Q5_K = 13, QT_Q6_K = 14, QT_IQ2_XXS = 16, QT_IQ2_XS = 17, QT_IQ3_XXS = 18,
    QT_IQ4_NL = 20, QT_IQ3_S = 21, QT_IQ2_S = 22, QT_IQ4_XS = 23, QT_BF16 = 30, QT_Q2_0 = 42,
};

// Packed ("plane") layout of a rows x cols weight.  A GGUF row is a run of blocks, each an array of structs
// (scales and quants interleaved, 2-byte aligned at best).  The packed layout moves every field of the format
// into its own plane, [rows][blocks per row][field bytes], so that each lane of the GEMV reads its group's quants
// and scales with naturally aligned 16/8/2-byte loads.  Bytes are moved, never changed: the packed weight holds
// exactly the GGUF bytes (plus alignment padding between planes).
struct QLayout {
    uint32_t type = 0;
    int rows = 0, cols = 0;
    int qk = 0;                 // values per GGUF block
    int bb = 0;                 // bytes per GGUF block
    int nplanes = 0;
    int fbytes[3] = {0, 0, 0};  // bytes per block in each plane
    int foff[3] = {0, 0, 0};    // offset of each plane's field inside the GGUF block
    size_t rs[3] = {0, 0, 0};   // row stride of each plane
    size_t off[3] = {0, 0, 0};  // byte offset of each plane in the packed buffer
    size_t bytes = 0;           // packed bytes in all
    size_t row_bytes = 0;       // GGUF bytes per row
};

// false (and an fn_error message) for a type this library does not read or a shape it cannot split into whole
// blocks of 32 values
bool qlayout(uint32_t type, int rows, int cols, QLayout &L);

// Launch plan of one GEMV (the values fn_gemv_plan reports, include/faie2fn.h).  It depends on the shape only, never
// on the number of tokens, so token t of an nt-token call gets the same bits as a one-token call on x[t].
struct GemvPlan {
    int gv = 32;      // values per group (a lane's unit of work)
    int waves = 8;    // waves per workgroup
    int ks = 1;       // workgroups along a row (split-K; partials are summed in a second, fixed-order pass)
    int rpw = 32;     // rows per workgroup pass (8 waves x 64 / lpr)
    int lpr = 16;     // lanes per row (16, 32 or 64)
    int ntiles = 0;   // row tiles (workgroups along the rows)
    int ngroups = 0;  // groups per row
    int grid = 0;     // workgroups along the rows: 0 = the ones resident at once (persistent, sized at launch),
                      // else one per row tile (ntiles)
};

// ks_force > 0: that many splits along the row (capped so that every split holds a group), whatever the override
GemvPlan gemv_plan(const QLayout &L, int ks_force = 0);
// benchmarking and tests: force lanes per row (16 / 32 / 64), split-K, the kernel (1 = x staged in chunks of lpr
// groups, the path of an x too large for the LDS; 2 = x staged once; 3 / 4 = x staged once with the deep / short
// walk) and the resident waves per CU a persistent grid is sized for; 0 = automatic
void gemv_override(int lpr, int ks, int kernel, int waves_per_cu);
size_t gemv_work_bytes(const QLayout &L, int nt);
// the reference's fn_gemv_waves switch (faie2fn.cu:2041, 2075, 2793): nonzero = persistent grid (default), 0 = one
// workgroup per row tile
void gemv_persistent(int on);

// GGUF rows (device) -> packed planes (device); stream-ordered
int quant_pack_launch(const QLayout &L, const uint8_t *raw, uint8_t *packed, hipStream_t st);
// packed planes -> float rows [rows][cols], bit for bit the GGUF decode of the format
int quant_dequant_launch(const QLayout &L, const uint8_t *packed, float *out, hipStream_t st);
// y[t][r] = sum_c W[r][c] x[t][c] for t < nt (1..8); x [nt][cols], y [nt][rows]; work: gemv_work_bytes() bytes
// ks_force: as gemv_plan's (1: no split-K whatever fn_gemv_override asks, for callers without a work buffer)
// whether every plane of the packed weight is addressable with 32-bit offsets (the GEMV kernels' form)
bool gemv_planes_fit(const QLayout &L);

int gemv_launch(const QLayout &L, const uint8_t *packed, const float *x, int nt, float *y, float *work,
                size_t work_bytes, hipStream_t st, int ks_force = 0);

// the GEMV with ks splits along the row and no reduce pass: part[k][t][r] = sum over split k's groups, k < *ks_out
// (ks capped so that every split holds a group); the consumer sums the partials in split order.  The split is fixed
// by the call, never by nt, so token t keeps the bits of a one-token call
int gemv_split_launch(const QLayout &L, const uint8_t *packed, const float *x, int nt, int ks, float *part,
                      int *ks_out, hipStream_t st);

// Several weights with the same cols over one x (y_i[t][r] = W_i[r] . x[t]): one launch when their formats form one
// of the sets built as a group (quant_grp.hip) and x of nt tokens fits the LDS, else one GEMV launch per weight.
// A grouped launch sums every row with the group's lanes per row (the GEMV's arithmetic with that lpr), so a
// weight's results may differ in the last bits from its own GEMV's; which path runs depends on the shapes and
// formats only, never on nt.
struct GemvPart {
    const QLayout *L;
    const uint8_t *packed;
    float *y;
};
int gemv_group_launch(const GemvPart *parts, int n, const float *x, int nt, hipStream_t st);

// Rows of a packed weight selected on the device (the model forward's embedding and routed experts):
//   embed_launch: out[t][k * cols + c] = W[ids[t]][c] for k < copies (the GGUF decode, bit for bit);
//   rows_launch: out[p][r] = W[e_p * R + r] . x[p / xdiv] for r < R, p < npairs, e_p = sel[p] (sel null: e_p = 0),
//     x rows of cols floats;
//   swiglu_launch: act[p][r] = silu(Wg[e_p R + r] . x[p / xdiv]) * (Wu[e_p R + r] . x[p / xdiv]).
// Each row is summed by 16 lanes, lane li taking groups li, li + 16, ... in ascending order (the arithmetic of the
// GEMV with 16 lanes per row); x and out 16-byte aligned.
int embed_launch(const QLayout &L, const uint8_t *packed, const int32_t *ids, int nt, int copies, float *out,
                 hipStream_t st);

// The n-gram rows of the per-layer embedding: token t of a call (position p = *pos + t) reads, for each of `heads`
// hash heads, the table row its n-gram context hashes to, decoded into out[t][head cols + c] (cols = the table's
// row length).  The hash of head h: key = XOR over k < order of (uint64) c[k] * mult[k], modulo 2^64, where c[0]
// is the token, c[k] the token k positions back (EOS before the sequence starts and after an EOS), order 2 for the
// first half of the heads and 3 for the second; row = first[h] + key mod size[h].  The call's ids go into the
// token ring (the id of position p at p & ring_mask) that later calls read their context from.
struct NgramGather {
    const int32_t *ids = nullptr;   // the call's token ids [nt]
    const int32_t *pos = nullptr;   // position of the call's first token (device)
    int32_t *ring = nullptr;        // token ring (device), ring_mask + 1 >= nt + 2 entries
    int ring_mask = 0;
    const uint64_t *tab = nullptr;  // device: mult[3], then size[heads], then first[heads]
    int heads = 0, eos = -1;
};
int ngram_gather_launch(const QLayout &L, const uint8_t *packed, const NgramGather &g, int nt, float *out,
                        hipStream_t st);
int rows_launch(const QLayout &L, const uint8_t *packed, int R, const int32_t *sel, int npairs, int xdiv,
                const float *x, float *out, hipStream_t st);
// The routing done inside the expert gate/up kernel (the model forward, one kernel fewer): pair p = t NEU + k
// takes the k-th pick of token t (route_wave over the router logits rsg[t][0 .. NE), row stride NE + 1); the
// workgroups of pair t NEU, row tile 0, write sel[t][..] and wsel[t][..] and the shared expert's SwiGLU
// sha[t][r] = silu(shg[t][r]) * shu[t][r], r < FFS.
struct RouteIn {
    const float *rsg = nullptr;
    int NE = 0, NEU = 0, FFS = 0;
    int32_t *sel = nullptr;
    float *wsel = nullptr;
    const float *shg = nullptr, *shu = nullptr;
    float *sha = nullptr;
};
int swiglu_launch(const QLayout &Lg, const uint8_t *pg, const QLayout &Lu, const uint8_t *pu, int R,
                  const int32_t *sel, int npairs, int xdiv, const float *x, float *act, hipStream_t st,
                  const RouteIn *route = nullptr);

// Hyper-connection write + the next read's per-stream RMSNorm + its down (+ inject) product, one launch (hc.hip):
// v[t][k] = h[t][k] + y[t] inj[t][k] (v = h when y is null; written to hout), hn[t][k] = RMSNorm(v[t][k]) w[k],
// part[k][t][r] = W[r][k D .. (k + 1) D) . hn[t][k] for the R rows of W (HC D columns, BF16).  hc_down_supported:
// the weights and widths it is built for.
bool hc_down_supported(const QLayout &L, int D, int HC);
int hc_down_launch(const float *h, const float *y, const float *inj, const float *w, int D, int HC, float eps,
                   const QLayout &L, const uint8_t *packed, int nt, float *hout, float *hn, float *part,
                   hipStream_t st);

// The MoE output of nt tokens in one launch: y[t][r] = sigmoid(rsg[t][NE]) (Ws[r] . sha[t]) + the sum over k < NEU,
// in order, of wsel[t][k] (We[sel[t][k] R + r] . act[t NEU + k]), r < R; We the stacked experts' down weights
// (rows of cols = FFE values), Ws the shared expert's (R x cols, Q8_0), each dot product with the arithmetic of
// rows_launch.  moe_down_supported: the formats, shapes and expert counts this kernel is built for (its LDS holds a
// token's NEU + 1 x rows), else rows_launch and a GEMV.
bool moe_down_supported(const QLayout &Le, const QLayout &Ls, int R, int NEU);
int moe_down_launch(const QLayout &Le, const uint8_t *pe, const QLayout &Ls, const uint8_t *ps, int R,
                    const int32_t *sel, const float *wsel, int NEU, const float *act, const float *sha, const float *rsg,
                    int NE, int nt, float *y, hipStream_t st);
// benchmarking: the waves that share one output row of moe_down_launch.  1: the 16-row kernel (a wave takes 4 rows
// and every item of the token); 2 or more: the 4-row kernel (4 waves split the items of each row); 0: unchanged;
// negative: automatic (4 rows a workgroup for one token, 16 for several).  Either kernel gives the same bits.
// Launches read it when they are made (a captured graph keeps the kernel it was captured with).
void moe_down_override(int waves_per_row);

}  // namespace fn

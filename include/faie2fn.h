/*
 * faie2fn.h -- C ABI of libfaie2fn.so, the MI355X (gfx950) decode-attention engine of FAIE2-FlashNext.
 *
 * Conventions (the reference's, engine/faie2fn.cu:111-118, 2492-2935; flashnext/fn.py:21-38):
 *   - int entry points return 0 on success and -1 on error; the message is then read with fn_error().  The
 *     pointer fn_error() returns stays valid until the next failing call.
 *   - Calls are synchronous unless their name ends in _dev, and not re-entrant: one caller thread, process-global
 *     state.  A _dev entry point only enqueues work on the HIP stream it is given (NULL = the null stream) and
 *     returns; its pointers are device memory the caller owns.
 *   - Host-array hooks (fn_test_*) take caller-owned, C-contiguous float32/int32 host arrays and copy them to and
 *     from device 0 inside the call, as the reference's unit-test hooks do (faie2fn.cu:2745-2782).
 *   - No torch type appears anywhere: plain pointers, sizes and a void* HIP stream.
 */
#ifndef FAIE2FN_H
#define FAIE2FN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================================================================================================
 * 1. The reference's C API, same names and C signatures (engine/faie2fn.cu, flashnext/fn.py:26-34), so that
 *    flashnext/fn.py's argtypes bind unchanged.  The GEMV hooks (fn_test_dequant, fn_test_gemv, fn_gemv_plan,
 *    fn_bench_gemv, fn_gemv_override, fn_bench_hot) work as in the reference for the formats of section 5.
 *    fn_load / fn_forward / fn_debug_layers run the model on one GPU (section 6); fn_bench_route times the
 *    model's MoE routing.  The engine entry points (fn_reset, fn_use_graphs, fn_n_past, fn_dev_gb, fn_last_ms, fn_split,
 *    fn_free) act on the loaded model, else on the path engine of section 4, and return -1 like the reference's
 *    when neither is loaded.
 * ====================================================================================================== */
const char *fn_error(void);                                                   /* faie2fn.cu:2495 */
void fn_free(void);                                                           /* faie2fn.cu:2497 */
/* One GPU: the model in shard1, and shard2 (NULL, "" or the same file when there is none) whose tensors join
 * shard1's (the reference model keeps the PLE n-gram table there); split is ignored (every layer on device 0,
 * fn_split() then returns the layer count). */
int fn_load(const char *shard1, const char *shard2, int max_ctx, int split);  /* faie2fn.cu:2524 */
int fn_split(void);                                                           /* faie2fn.cu:2698 */
double fn_dev_gb(int dv);                                                     /* faie2fn.cu:2699 */
int fn_n_past(void);                                                          /* faie2fn.cu:2700 */
double fn_last_ms(void);                                                      /* faie2fn.cu:2701 */
int fn_reset(void);                                                           /* faie2fn.cu:2703 */
int fn_use_graphs(int on);                                                    /* faie2fn.cu:2721 */
int fn_forward(const int32_t *tokens, int nt, float *logits, int32_t *argmax);  /* faie2fn.cu:2733 */
int fn_debug_layers(float *out);                                              /* faie2fn.cu:2739 */
/* GGUF rows W (rows x cols of `type`, the file's bytes) -> out [rows][cols] float32, bit for bit ggml's decode. */
int fn_test_dequant(uint32_t type, const uint8_t *W, int rows, int cols, float *out);  /* faie2fn.cu:2751 */
/* Force the plan of GEMVs launched from now on, 0 = automatic.  wpt: the reference's split of a row's columns
 * (its warps per 16-row tile); here the 16-lane groups that sum one row, 1, 2 or 4 (16, 32 or 64 lanes per row;
 * other values: automatic), the quantity fn_gemv_plan reports in out[1], so a forced plan reads back as forced.
 * ks: split-K workgroups per row, as the reference's (out[2]).  tb: not the reference's tiles per block (the
 * workgroups here are fixed at 8 waves) but this library's kernel choice (1 x staged in chunks, 2 x staged once,
 * 3 / 4 x staged once with the deep / short walk).  warps_per_sm: the resident waves per CU a persistent grid is
 * sized for (the reference's target warps per SM).  Lanes per row and ks > 1 change the summation order, the other
 * choices give the same bits.  The model forward's GEMVs take no split-K whatever ks asks (no work buffer). */
void fn_gemv_override(int wpt, int ks, int tb, int warps_per_sm);             /* faie2fn.cu:2786 */
/* The reference's persistent-grid switch: waves != 0 (default) launches the GEMV on the workgroups resident at once,
 * each walking many row tiles; 0 launches one workgroup per row tile.  Same bits either way; fn_gemv_plan's out[5]
 * reports the choice for plans made afterwards. */
void fn_gemv_waves(int waves);                                                /* faie2fn.cu:2793 */
/* The reference's A/B switches for its CUDA forward (programmatic dependent launch, GEMVs started early under it,
 * the gate/up tile variant): accepted so that its scripts bind and run, no effect here (no HIP counterpart; one
 * hipGraph per token count on one stream; one gate/up shape). */
void fn_pdl(int on);                                                          /* faie2fn.cu:2796 */
void fn_early(int on);                                                        /* faie2fn.cu:2798 */
void fn_moe_var(int v);                                                       /* faie2fn.cu:2799 */
/* The expert launch shapes.  dn_wpt picks the MoE output kernel by the waves that share one output row: 1 = 16 rows
 * a workgroup (one wave sums whole rows), 2 or more = 4 rows a workgroup (four waves split each row's items), 0 =
 * unchanged, negative = automatic (4 rows for one token, 16 for several; an extension: the reference ignores values
 * <= 0).  Same bits either way; graphs captured before keep their kernel.  gu_wpt, gu_tb, dn_tb: no effect. */
void fn_moe_override(int gu_wpt, int gu_tb, int dn_wpt, int dn_tb);           /* faie2fn.cu:2801 */
/* Launch plan of a rows x cols weight in the reference's 7 slots {cv, wpt, ks, tb, nbuf, ntiles, nch}:
 * out = {values per group (32), 16-lane groups per row (wpt, as fn_gemv_override takes it), split-K workgroups per
 * row, rows per workgroup pass, waves per workgroup (8), workgroups along the rows (0 = persistent grid: the
 * workgroups resident at once, sized at launch; after fn_gemv_waves(0) one per row tile of rows-per-pass rows),
 * groups per row}.  Like the reference's it depends on the shape only, never on the number of tokens. */
int fn_gemv_plan(uint32_t type, int rows, int cols, int *out);                /* faie2fn.cu:2809 */
void fn_bench_hot(int on);                                                    /* faie2fn.cu:2822 */
/* ms per GEMV call of nt tokens (1..8) on random bytes of the format, iters calls replayed as one hipGraph, each
 * reading its own copy of the weight (copies beyond the 256 MB Infinity Cache, 512 MiB written before the timed
 * replay) unless fn_bench_hot(1). */
int fn_bench_gemv(uint32_t type, int rows, int cols, int nt, int iters, float *ms);  /* faie2fn.cu:2823 */
/* MoE routing (softmax top-10 of 512 router logits, ties to the lower expert, weights renormalized over the picks)
 * of nt tokens 1..8, the logits summed from part [ks][8][528] (ks 1..64 split-K partials, the reference's layout),
 * iters calls replayed as one hipGraph: ms per call, sel / wsel [nt][10].  variant 0 ranks every expert, variant 1
 * is the model forward's one-wave routing; both give the same bits. */
int fn_bench_route(int variant, int nt, int ks, const float *part, int iters, int *sel, float *wsel,
                   float *ms);                                                /* faie2fn.cu:2875 */
/* y [nt][rows] = W x for GGUF rows W and x [nt][cols], nt 1..8 (packed, then the GEMV of section 5). */
int fn_test_gemv(uint32_t type, const uint8_t *W, int rows, int cols, const float *x, int nt,
                 float *y);                                                   /* faie2fn.cu:2916 */

/* ======================================================================================================
 * 2. Path hooks, host arrays (new; the reference reaches this path only through fn_forward, faie2fn.cu:2733,
 *    and its model-free hooks follow the style of faie2fn.cu:2745).  Shapes: B sequences, nt tokens each.
 *    head_map: 0 = tiled (value head h reads key head h % nkh, faie2fn.cu:1374), 1 = grouped (h / (nvh/nkh)).
 *    gate_act: 0 = sigmoid (faie2fn.cu:1424), 1 = silu.  dk = dv = 128 and hd = 256 are the built sizes.
 * ====================================================================================================== */

/* DeltaNet state core, the delta rule of k_gdn (faie2fn.cu:1407-1421) on given normalised q, k:
 *   q, k [B][nt][nkh][dk]; v [B][nt][nvh][dv]; beta, g [B][nt][nvh] (g = log decay, gamma = exp(g));
 *   S [B][nvh][dk][dv] in/out (row = key index); o [B][nt][nvh][dv] out, o = S'^T q / sqrt(dk). */
int fn_test_gdn(int B, int nkh, int nvh, int dk, int dv, int head_map, int nt, const float *q, const float *k,
                const float *v, const float *beta, const float *g, float *S, float *o);

/* Fused DeltaNet block, k_gdn (faie2fn.cu:1366-1431): conv1d k=4 + SiLU, q/k L2-norm, gates, delta rule,
 * gated RMSNorm.  C = 2 nkh dk + nvh dv.
 *   qkv [B][nt][C] (channels [q | k | v], faie2fn.cu:1377); conv_w [C][4] oldest tap first;
 *   conv_state [B][3][C] in/out, raw inputs of the three previous tokens, oldest first;
 *   ab [B][nt][2 nvh] alpha rows then beta rows (faie2fn.cu:1407-1408); dt_bias, ssm_a [nvh] (ssm_a = -exp(A_log));
 *   S [B][nvh][dk][dv] in/out; z [B][nt][nvh dv]; norm_w [dv]; out [B][nt][nvh dv]. */
int fn_test_gdn_block(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt,
                      const float *qkv, const float *conv_w, float *conv_state, const float *ab,
                      const float *dt_bias, const float *ssm_a, float *S, const float *z, const float *norm_w,
                      float eps, float *out);

/* GQA decode, k_qk_norm_rope + k_attn_split (dense) + k_attn_combine (faie2fn.cu:1451-1478, 1612-1690).
 *   pos [B]: tokens already in each sequence's cache; token t of sequence b sits at pos[b] + t.
 *   qg [B][nt][nq][2][hd] query then gate per head (faie2fn.cu:50, 1463, 1686); k, v [B][nt][nkv][hd] new rows;
 *   wq, wk [hd] RMSNorm weights (stored as the effective multiplier); Kc, Vc [B][max_ctx][nkv][hd] in/out in the
 *   reference layout (faie2fn.cu:1461, 1477): rows < pos[b] are read, rows pos[b]..pos[b]+nt-1 are written;
 *   nsplit: KV splits per (sequence, token, kv head), 0 = automatic; og [B][nt][nq][hd] out. */
int fn_test_attn(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                 const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                 const float *wk, float *Kc, float *Vc, int nsplit, float *og);

/* ======================================================================================================
 * 3. Path entry points on device memory (new): what an engine's layer loop calls, asynchronously on its stream.
 *    They are the same kernels as section 2 without copies or allocation.
 * ====================================================================================================== */

/* Fused DeltaNet block on device buffers.  Differences from fn_test_gdn_block:
 *   pos [B] device int32: tokens already seen per sequence (advanced by the caller, e.g. fn_advance_dev);
 *   conv_ring [B][ring][C] device: the raw input of position p sits in slot p & (ring - 1); ring is a power of
 *   two >= 4 and nt <= ring - 3 (ring = 4 serves one-token decode). */
int fn_gdn_block_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt, int ring,
                     const int32_t *pos, const float *qkv, const float *conv_w, float *conv_ring, const float *ab,
                     const float *dt_bias, const float *ssm_a, float *S, const float *z, const float *norm_w,
                     float eps, float *out, void *stream);

/* One decode token of the fused DeltaNet block with the alpha/beta projection fused in: replaces the ab GEMV and
 * the k_gdn launch that follows it (faie2fn.cu:2388-2389) with one launch.  As fn_gdn_block_dev with nt = 1, except
 * that ab is computed inside: ab[b][j] = sum_i w_ab[j][i] * x[b][i] in fp32 (BF16 weights widened exactly),
 *   x [B][hidden] device fp32 (the layer's input, the x the reference's gemv(L.ab, d.x, ...) reads),
 *   w_ab [2 nvh][hidden] device BF16 rows as GGUF stores them (alpha rows 0..nvh-1, then beta rows), the weight
 *   whose GEMV gives ab; hidden a positive multiple of 4, x and w_ab 16-byte aligned. */
int fn_gdn_block_xab_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int ring,
                         const int32_t *pos, const float *qkv, const float *conv_w, float *conv_ring, const float *x,
                         int hidden, const uint16_t *w_ab, const float *dt_bias, const float *ssm_a, float *S,
                         const float *z, const float *norm_w, float eps, float *out, void *stream);

/* A verify step of the fused DeltaNet block with deferred commit (speculative decoding; the reference's engine
 * family verifies drafts by replay-commit, reference DESIGN.md:287-293, and FN's k_gdn already takes nt <= 8
 * tokens of one sequence, faie2fn.cu:1390).  For sequence b, pos[b] is the position of the first new token and
 * the kr[b] tokens before it (0 <= kr[b] <= rnt) are the previous call's accepted ones: the kernel first replays
 * them from their saved inputs rqkv [B][rnt][C] and rab [B][rnt][2 nvh] (the previous call's qkv and ab) into the
 * state, writes S and the ring as the committed state, then runs the nt new tokens on that state in registers
 * only: out [B][nt][nvh dv] gets their outputs, S and the ring never hold them.  One read and one write of S per
 * call, as in plain decode; the new tokens' outputs are bit-identical to decoding them one by one after the
 * committed prefix.  ring >= rnt + 3; kr[b] outside [0, rnt] is clamped into it and recorded (FN_STATUS_KR, fn_dev_status).  Advance pos by the accepted counts with fn_advance_by_dev before the step
 * (the attention layers of the step then append the new tokens at pos, pos + 1, ... as usual). */
int fn_gdn_verify_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt, int ring,
                      const int32_t *pos, const int32_t *kr, int rnt, const float *rqkv, const float *rab,
                      const float *qkv, const float *conv_w, float *conv_ring, const float *ab, const float *dt_bias,
                      const float *ssm_a, float *S, const float *z, const float *norm_w, float eps, float *out,
                      void *stream);

/* pos[b] += kr[b] for b < B, on the stream (k_advance with per-sequence counts). */
int fn_advance_by_dev(int32_t *pos, const int32_t *kr, int B, void *stream);

/* DeltaNet core on device buffers (layouts of fn_test_gdn). */
int fn_gdn_core_dev(int B, int nkh, int nvh, int dk, int dv, int head_map, int nt, const float *q, const float *k,
                    const float *v, const float *beta, const float *g, float *S, float *o, void *stream);

/* GQA decode on device buffers.  Device cache layouts (max_ctx a multiple of 64):
 *   Kc [B][nkv][max_ctx/64][hd/4][64][4] (key-tiled), Vc [B][nkv][max_ctx][hd];
 *   pos [B] device int32 (not advanced here); work: fn_attn_work_bytes() bytes of device scratch. */
int fn_attn_dev(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq, const float *wk,
                float *Kc, float *Vc, int nsplit, float *work, size_t work_bytes, float *og, void *stream);

/* Scratch bytes fn_attn_dev needs for these shapes. */
size_t fn_attn_work_bytes(int B, int nq, int nt, int hd, int nsplit);

/* The split count fn_test_attn uses when given 0, for a context of ctx keys. */
int fn_attn_nsplit(int B, int nkv, int nt, int ctx);

/* GQA decode that allocates nothing.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results (bit for bit) as fn_attn_dev, without work / work_bytes: the workspace is a
 * file-scope device array of FN_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.  Shapes whose
 * fn_attn_work_bytes() exceeds it are rejected with an error.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams or threads) race; calls in one stream order do not. */
#define FN_NOALLOC_SCRATCH_BYTES (32u << 20)
int fn_attn_noalloc_dev(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                        const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                        const float *wk, float *Kc, float *Vc, int nsplit, float *og, void *stream);

/* Misuse the device entry points cannot see on the host, because positions and counts live in device memory (no
 * counterpart in the reference, whose positions are a host counter checked by forward(), faie2fn.cu:2468).  The
 * kernels stay in bounds -- a new token outside the cache is neither appended nor attended past the cache's end, a
 * verify count kr[b] outside [0, rnt] is clamped into it -- and OR a bit into a per-device status word.
 * fn_dev_status synchronizes the current device, returns the bits (>= 0, -1 on error) and, if clear != 0, zeroes
 * the word.  Not to be called while a stream is being captured.  The path engine and the host-array hooks check it
 * themselves and fail with an fn_error() message. */
#define FN_STATUS_POS 1u  /* attention: a new token's position pos[b] + t outside [0, max_ctx) */
#define FN_STATUS_KR 2u   /* verify: kr[b] outside [0, rnt] */
int fn_dev_status(int clear);

/* pos[b] += nt for b < B, on the stream (the reference's k_advance, faie2fn.cu:1905). */
int fn_advance_dev(int32_t *pos, int B, int nt, void *stream);

/* Utilities with no counterpart in the reference (its GEMV bench fills inputs on the host, faie2fn.cu:2836-2840):
 *   fn_fill_normal_dev: p[i] = mean + std * N(0,1), a function of (seed, i) only (splitmix64 + Box-Muller), for
 *   synthetic inputs generated in HBM; fn_copy_dev: plain 16-byte-per-lane streaming copy of bytes (16-aligned),
 *   the yardstick for achievable HBM bandwidth and the known-size kernel for counter calibration. */
int fn_fill_normal_dev(float *p, size_t n, uint64_t seed, float mean, float std, void *stream);
int fn_copy_dev(void *dst, const void *src, size_t bytes, void *stream);

/* Timing hooks of the path (SURVEY's path hooks; the reference's style of fn_bench_gemv, faie2fn.cu:2823): inputs
 * filled in HBM (seeded normal values), enough distinct layers that state or caches are cold (>= 1 GiB), one pass
 * over the layers captured as a hipGraph, `iters` replays timed with HIP events; *us = microseconds per layer-step.
 *   fn_bench_gdn: the fused DeltaNet block (dk = dv = 128, conv k = 4) of B sequences, nt tokens each;
 *   fn_bench_attn: GQA decode (head dim 256, RoPE on 64 dims) of B sequences with nt new tokens at positions
 *   ctx - nt .. ctx - 1 (query heads per kv head 4, 8 or 12).
 * Shapes are checked before any device work. */
int fn_bench_gdn(int B, int nkh, int nvh, int nt, int iters, float *us);
int fn_bench_attn(int B, int nq, int nkv, int ctx, int nt, int iters, float *us);

/* Per-kernel timing without a profiler (no counterpart in the reference, which times kernels under nsys): with
 * n > 0 hipEvent_t handles set, the GQA decode and sparse attention entry points (fn_attn_dev, fn_attn_qsa_dev and
 * the path engine's attention layers) record events[0], events[1], ... on their stream after each of their kernel
 * launches, in launch order, until the list is used up; n = 0 clears the list.  The events must not be recorded
 * while a stream is being captured.  0 or -1 (n outside 0..64). */
int fn_stage_events(void **events, int n);

/* ======================================================================================================
 * 3b. QSA sparse attention (new): the reference's attention layer with its indexer (faie2fn.cu:1480-1607, the
 *     masked k_attn_split :1628-1636, launch order :2396-2402).  Indexer shapes are the reference's: 4 query heads
 *     of 128 dims, one raw index key of 128 dims per token, blocks of 4 keys, RoPE as the attention's.  A query with
 *     more than `top` complete blocks (512 in the reference, faie2fn.cu:60) attends the keys of its `top`
 *     highest-scoring blocks (ties at the threshold: lowest index first) plus the incomplete tail block; otherwise it
 *     attends every key.
 * ====================================================================================================== */

/* As fn_attn_dev, plus: iqk [B][nt][640] (indexer query heads, then the raw index key), wqn, wkn [128] indexer norm
 * weights; IKc [B][max_ctx][128] raw index keys (row pos[b]+t written); BKc block keys, device layout
 * [B][max_ctx/256][32][64][4] (blocks completed by this call written); max_ctx a multiple of 256;
 * work: fn_attn_qsa_work_bytes() bytes. */
int fn_attn_qsa_dev(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                    const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                    const float *wk, float *Kc, float *Vc, const float *iqk, const float *wqn, const float *wkn,
                    float *IKc, float *BKc, int top, int nsplit, float *work, size_t work_bytes, float *og,
                    void *stream);
size_t fn_attn_qsa_work_bytes(int B, int nq, int nt, int hd, int nsplit, int max_ctx, int top);

/* Block keys of blocks [j0, j1) of every sequence from the raw index keys (the reference's k_ix_blocks over a
 * range, faie2fn.cu:1509-1530): for prefill or for rebuilding BKc from IKc. */
int fn_ix_blocks_dev(int B, int max_ctx, int j0, int j1, const float *IKc, const float *wkn, float *BKc, int nrot,
                     float theta, float eps, void *stream);

/* For the sparse step, fn_attn_nsplit(B, nkv, nt, 4 * top + 4) sizes the split of the attended keys. */

/* Host-array hook of the sparse layer step, reference layouts: Kc, Vc [B][max_ctx][nkv][hd], IKc [B][max_ctx][128]
 * in/out (rows < pos[b] read, new rows written).  Block keys of the blocks complete before the call are built from
 * IKc inside the hook.  Optional outputs (NULL to skip): scores [B][nt][max_ctx/4] (entries < nb of queries with
 * nb > top), mask [B][nt][max_ctx/4] (1 = block kept; all 0 for dense queries). */
int fn_test_attn_qsa(int B, int nq, int nkv, int hd, int nrot, float theta, float eps, int nt, int max_ctx,
                     const int32_t *pos, const float *qg, const float *k, const float *v, const float *wq,
                     const float *wk, float *Kc, float *Vc, const float *iqk, const float *wqn, const float *wkn,
                     float *IKc, int top, int nsplit, float *og, float *scores, uint8_t *mask);

/* ======================================================================================================
 * 4. Path engine (new): the reference's Engine + layer_forward + forward (faie2fn.cu:1937-2031, 2370-2490) for
 *    this path only.  B sequences, nl layers; layer il is attention iff (il + 1) % attn_every == 0
 *    (faie2fn.cu:76, attn_every = 4; 0 = DeltaNet only).  All state is engine-owned on device 0 and zeroed.
 *    The projections around the path are not part of this library, so each layer reads its inputs from engine
 *    buffers the caller fills (fn_path_buffer gives their device addresses) and writes its output to one.
 *    Once fn_path_init has run, the reference's engine entry points act on this engine: fn_reset zeroes the
 *    DeltaNet state, conv rings and positions (faie2fn.cu:2703-2717), fn_use_graphs switches hipGraph replay of
 *    the step (default on), fn_n_past counts steps since reset, fn_dev_gb(0) is the engine's device memory in GB,
 *    fn_last_ms is the host wall time of the last fn_path_step, fn_free releases everything.
 * ====================================================================================================== */
int fn_path_init(int B, int nl, int attn_every, int nkh, int nvh, int nq, int nkv, int max_ctx, int head_map,
                 int gate_act, int nsplit);

/* Buffer kinds of fn_path_buffer.  DeltaNet layers: S [B][nvh][128][128], conv ring [B][4][C], qkv [B][C],
 * ab [B][2 nvh], z [B][nvh 128], out [B][nvh 128], conv_w [C][4], dt_bias [nvh], ssm_a [nvh], norm_w [128].
 * Attention layers: Kc, Vc in the fn_attn_dev layouts, qg [B][nq][2][256], k, v [B][nkv][256], og [B][nq][256],
 * wq, wk [256].  FN_BUF_POS (any il): the engine's int32 positions [B]. */
#define FN_BUF_S 0
#define FN_BUF_CONV_RING 1
#define FN_BUF_QKV 2
#define FN_BUF_AB 3
#define FN_BUF_Z 4
#define FN_BUF_OUT 5
#define FN_BUF_CONV_W 6
#define FN_BUF_DT_BIAS 7
#define FN_BUF_SSM_A 8
#define FN_BUF_NORM_W 9
#define FN_BUF_KC 10
#define FN_BUF_VC 11
#define FN_BUF_QG 12
#define FN_BUF_K 13
#define FN_BUF_V 14
#define FN_BUF_OG 15
#define FN_BUF_WQ 16
#define FN_BUF_WK 17
#define FN_BUF_POS 18
int fn_path_buffer(int il, int kind, void **ptr, size_t *bytes);

/* steps decode steps (one token per sequence each) through all layers, then a stream synchronize; with ms
 * non-NULL, the HIP-event time per step on the engine's stream is written there. */
int fn_path_step(int steps, float *ms);

/* ======================================================================================================
 * 5. GGUF weights and the GEMV of the projections around the path (the reference's dequantisers and tiled GEMV,
 *    engine/faie2fn.cu:343-1042, 2033-2116; its callers on the path: the qkv / z / ab projections before k_gdn
 *    and ssm_out after it, the q / k / v projections before the attention and o_proj after it, :2386-2403).
 *    Types are GGUF type ids: 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K, 20 IQ4_NL, 23 IQ4_XS, 30 BF16.  cols must be a
 *    whole number of blocks (32 values, 256 for the K and IQ4_XS formats).  An engine packs each weight once
 *    (fn_gemv_pack_dev: every field of the format in its own aligned plane, the same bytes) and then calls
 *    fn_gemv_dev per token batch.  All _dev pointers must be 16-byte aligned.
 * ====================================================================================================== */

/* Bytes of the packed layout of a rows x cols weight (0 if the type or shape is not supported). */
size_t fn_gemv_packed_bytes(uint32_t type, int rows, int cols);

/* GGUF rows raw [rows][row bytes] (device) -> packed (device, fn_gemv_packed_bytes() bytes). */
int fn_gemv_pack_dev(uint32_t type, const uint8_t *raw, int rows, int cols, uint8_t *packed, void *stream);

/* packed -> out [rows][cols] float32 (device), bit for bit ggml's decode (what fn_test_dequant returns). */
int fn_dequant_dev(uint32_t type, const uint8_t *packed, int rows, int cols, float *out, void *stream);

/* Scratch bytes fn_gemv_dev needs for nt tokens (0 when the plan does not split K). */
size_t fn_gemv_work_bytes(uint32_t type, int rows, int cols, int nt);

/* y [nt][rows] = W x, x [nt][cols], nt 1..8, on device buffers; split-K partials (if any) in work. */
int fn_gemv_dev(uint32_t type, const uint8_t *packed, int rows, int cols, const float *x, int nt, float *y,
                float *work, size_t work_bytes, void *stream);

/* Several packed weights of the same cols over one x (new; the reference runs the projections that read one
 * activation row as separate GEMVs, faie2fn.cu:2386-2403): y[i] [nt][rows[i]] = W_i x for i < n (1..4).  One
 * launch, x staged once per workgroup, when the formats form one of the built sets ({IQ4_XS, IQ3_S, BF16},
 * {IQ4_XS, Q6_K, BF16}, {IQ4_XS, IQ4_XS, Q6_K, BF16}, in any order) and x of nt tokens fits the LDS; otherwise one
 * fn_gemv_dev-like launch per weight.  A grouped launch sums each row over at least 32 lanes, so a weight whose own
 * plan takes 16 lanes per row may differ from fn_gemv_dev in the last bits; the path taken depends on the formats
 * and shapes only, never on nt (token t gets the bits of a one-token call).  No work buffer. */
int fn_gemv_group_dev(int n, const uint32_t *types, const int *rows, int cols, const uint8_t *const *packed,
                      const float *x, int nt, float *const *y, void *stream);

/* ======================================================================================================
 * 6. Model (new beside the reference's fn_load / fn_forward, faie2fn.cu:2524, 2733): what fn_load reads.
 *    Shapes come from the GGUF metadata (<general.architecture>.* keys: embedding_length, block_count,
 *    attention.head_count(_kv), expert_count, expert_used_count, expert_(shared_)feed_forward_length, ssm.*,
 *    hyper_connection.count / low_rank, attention.indexer.*, full_attention_interval, rope.*) and the token
 *    embedding; head_dim 256, DeltaNet head dim 128, conv kernel 4 and the indexer's 4 x 128 are the built sizes.
 *    Tensor names are the reference's (token_embd, output, output_hc_*, blk.N.{hc_attn_*, hc_ffn_*, attn_qkv,
 *    attn_gate, ssm_*, attn_q/k/v/output, attn_q_norm/k_norm, indexer.*, ffn_gate_inp(_shexp), ffn_*_shexp,
 *    ffn_*_exps}); weights in the formats of section 5, norms and conv weights F32 or F16.  The layers listed in
 *    <arch>.ple.layers add the per-layer n-gram embedding first: blk.N.{ple_key, ple_value, ple_norm_key,
 *    ple_norm_query, ple_norm_conv, ple_conv1d} and the table per_layer_token_embd ([ple values per head] x rows,
 *    packed whole into HBM), hashed by ple.{heads_per_ngram, eos_token_id, layer_multipliers, head_offsets,
 *    head_vocab_sizes} and embedding_length_per_layer_input; n-grams of 3 and conv kernel 4 are the built sizes.
 * ====================================================================================================== */

/* Parse a GGUF file (no device work) and write its model shapes to out[0..n): {D, layers, q heads, kv heads,
 * head dim, rope dims, experts, experts used, expert ffn, shared ffn, ssm state, ssm groups, ssm value heads,
 * ssm inner, conv channels, attention interval, hyper-connections, hc low rank, indexer heads, indexer dim,
 * indexer top blocks, vocabulary, PLE layers, PLE heads, PLE values per head}.  Returns the number of values (25)
 * or -1 (fn_error: what is wrong or missing). */
int fn_model_dims(const char *path, int *out, int n);

#ifdef __cplusplus
}
#endif

#endif /* FAIE2FN_H */

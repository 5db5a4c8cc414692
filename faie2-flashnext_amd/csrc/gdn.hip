// Gated-DeltaNet decode for gfx950: the fused block (causal conv1d k=4 + SiLU, q/k L2-norm, gates, delta rule,
// readout, gated RMSNorm) and the bare state core, one workgroup per (sequence, value head).
//
// Semantics follow k_gdn (reference engine/faie2fn.cu:1349-1431).  The kernel is organised for CDNA4, not as a
// translation of the sm_120 one:
//   * 512 threads (eight wave64s) per head in the one-token kernels.  Thread (rg = tid / 32, cg = tid % 32) owns the
//     4 columns 4cg..4cg+3 of the 8 state rows rg, rg + 16, ..., rg + 112, i.e. 8 float4 registers.  The
//     multi-token kernels run 256 threads per head, each owning the two row groups 2rg and 2rg + 1, and reproduce
//     the 512-thread arithmetic bit for bit.  Every wave load and store of S
//     moves two contiguous 512-byte rows with 128-bit accesses, and the eight waves' r-th accesses together sweep
//     rows 16r .. 16r + 15, 8 KiB in a row, so the tile streams through HBM in address order (row groups of 8
//     consecutive rows per thread scatter each sweep over the whole 64 KiB; on MI355X the bare tile pass takes
//     43.8 instead of 49.1 us at B = 64).  S makes exactly one trip HBM -> VGPRs -> HBM per call, with the
//     nontemporal hint on both legs (62.2 -> 52.4 us per B = 64 layer-step; 256 or 1024 threads per head and an
//     XCD-contiguous head order were all slower).
//   * One read pass computes both reductions the step needs, kv = S^T k and sq = S^T q (old S), because
//       S' = g S + k d^T  with  d = beta (v - g kv)    =>    S'^T q = g sq + (k.q) d.
//     The column partials of the 16 row groups are folded with a v_permlane32_swap (2 groups per wave) and
//     one 4 KiB LDS exchange across the eight waves; there is no serial 128-long FMA chain.
//   * Per-lane global access goes through raw buffer descriptors (one VGPR offset per address) and the barriers
//     order LDS only, so a multi-token call keeps the next token's loads in flight across a token (no barrier and
//     no spilled-address reload drains them): the verify step at B = 64, 4 new + 2 replayed tokens, 114 -> 94 us.
//   * q/k are not normalised before the pass: the L2 factors are applied to the 4 per-column sums, so the
//     norm reductions (wave DPP sums) overlap the S loads instead of sitting in front of them.
//   * The causal conv state is a ring of R slots per sequence, R a power of two >= nt + 3: the raw input of
//     position p lives in slot p & (R - 1).  A call reads the slots of positions pos-3..pos-1 and writes only the
//     slots of its own last (up to) three positions, so value heads sharing a key head read their q/k taps with
//     no race and no per-head copies (the reference keeps one copy per value head, faie2fn.cu:1353, 1378-1382).
//     Taps inside the call's own tokens come straight from the qkv input.
#include "gdn.h"

#include <algorithm>

namespace fn {

namespace {

#ifndef GDN_THREADS
#define GDN_THREADS 512
#endif
#ifndef GDN_NT
#define GDN_NT 1
#endif
#ifndef GDN_NT_ST
#define GDN_NT_ST GDN_NT
#endif
#ifndef GDN_WPE
#define GDN_WPE 1
#endif
#ifndef GDN_VERIFY_WPE
// the multi-token kernels (verify, prefill; 256 threads per head) in at most 168 VGPRs: three workgroups per CU
// (B = 64, 4 tokens per call through the committed block: 72.6 -> 67.3 us per layer-step against two per CU)
#define GDN_VERIFY_WPE 3
#endif

#ifndef GDN_ONE_LDS_PAD
// k_gdn<3> (the decode step) fits in 78 VGPRs, which would let three workgroups (six waves per SIMD) share a CU;
// two interleave their state streams better (B = 64: 49.4 against 50.8 us per layer-step on MI355X).  The launch
// reserves this much dynamic LDS, unused, so that three do not fit in the CU's 160 KiB and two do.
#define GDN_ONE_LDS_PAD 57344
#endif

constexpr int DK = 128, DV = 128;
constexpr int THREADS = GDN_THREADS;  // threads per head of the one-token kernels (decode, bare core)
#ifndef GDN_MT_THREADS
// The multi-token kernels run the per-token reduction chain nt + kr times per call, which makes them VALU-bound
// rather than memory-bound: with 256 threads per head the cross-wave sum of the column partials is repeated by half
// as many threads, and three heads share a CU instead of two (B = 64, 4 new + 2 replayed tokens: 92.0 -> 80.7 us
// per layer-step; 8 + 4: 158.8 -> 131.4 us).  The one-token decode stays at 512 (memory-bound: 256 measured equal
// at B = 64 and slower at B = 1, 5.26 against 4.94 us).
#define GDN_MT_THREADS 256
#endif
constexpr int MT_THREADS = GDN_MT_THREADS;  // threads per head of the multi-token kernels (prefill, verify)
static_assert(THREADS == 256 || THREADS == 512, "one state tile per 4 or 8 waves");
static_assert(MT_THREADS == 256 || MT_THREADS == 512, "one state tile per 4 or 8 waves");

// The state tile in registers: 16 row groups g of 8 rows (g, g + 16, ..., g + 112), 32 column groups of 4 columns.
// Row r of group g is at byte offset so(g, column group) + r * 16 rows.
constexpr int NG = 16, GROWS = DK / NG;
__device__ __forceinline__ float4 ld_state(brsrc S, uint32_t so, int r) {
    return bld4<GDN_NT ? 2 : 0>(S, so, (uint32_t) r * NG * DV * 4);
}
// Cache policy of the state tile's stores: nontemporal (2), or nontemporal at system scope (2 | 16) for one-token
// calls whose grid holds more workgroups than are resident at once, where the stores of one round of heads share
// the memory with the loads of the next (B = 64: 49.2 -> 48.9 us per launch; at B = 1, one round, 5.21 -> 5.37 us,
// so those keep the plain hint).  The policy changes no value.
constexpr int ST_NT = GDN_NT_ST ? 2 : 0, ST_NT_SYS = ST_NT | 16;
template <int AUX = ST_NT> __device__ __forceinline__ void st_state(brsrc S, uint32_t so, int r, float4 v) {
    bst4<AUX>(S, so, (uint32_t) r * NG * DV * 4, v);
}

struct GdnArgs {
    int B, nkh, nvh, nt, ring, head_map, gate_act;
    float eps;
    const int32_t *pos;
    const float *qkv, *conv_w;
    float *ring_buf;
    const float *ab, *dt_bias, *ssm_a;
    float *S;
    const float *z, *norm_w;
    float *out;
    const float *q, *k, *v, *beta, *g;  // core variant inputs
    const int32_t *kr;                  // verify: tokens of the previous call to commit first, per sequence
    int rnt;                            // verify: token stride of the replay inputs
    const float *rqkv, *rab;            // verify: the previous call's qkv [B][rnt][C] and ab [B][rnt][2 nvh]
    const float *x;                     // one-token block with the alpha/beta projection fused: x [B][hidden]
    const uint16_t *wab;                //   and the BF16 weight [2 nvh][hidden] (null: ab is given)
    int hidden;
    unsigned *status;                   // verify: per-device status word (FN_STATUS_KR when kr[b] is clamped)
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }

// sigmoid / SiLU on the per-token path with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of the IEEE
// division sequence: within a few ulp of x / (1 + e^-x), and the one-token and multi-token kernels share them
__device__ __forceinline__ float sigmoid_r(float x) { return __builtin_amdgcn_rcpf(1.0f + expf(-x)); }
__device__ __forceinline__ float silu_r(float x) { return x * sigmoid_r(x); }

// Causal depthwise conv (kernel 4, weights oldest tap first) + SiLU (faie2fn.cu:1392-1395) of one channel.
// The raw inputs of the three previous positions ride in registers across the token loop (hist[0] oldest),
// as the reference keeps them (faie2fn.cu:1378-1398); the ring is read once before the loop and written once after.
struct ConvChan {
    float4 w;
    float hist[3];
    float x;  // raw input of the current token
    __device__ __forceinline__ float out() const {
        float acc = w.x * hist[0];
        acc = fmaf(w.y, hist[1], acc);
        acc = fmaf(w.z, hist[2], acc);
        acc = fmaf(w.w, x, acc);
        return silu_r(acc);
    }
    __device__ __forceinline__ void shift(float next) {
        hist[0] = hist[1];
        hist[1] = hist[2];
        hist[2] = x;
        x = next;
    }
};

// The ring of one sequence is a buffer of a.ring rows of C channels; a channel is the lane's byte offset oc = 4 c,
// the slot of position p the row offset slot_off(p).
__device__ __forceinline__ uint32_t slot_off(const GdnArgs &a, int C, int p) {
    return (uint32_t) (p & (a.ring - 1)) * C * 4;
}

// x0: the raw input row of the call's first token
__device__ __forceinline__ void conv_load(ConvChan &cc, const GdnArgs &a, brsrc ring, brsrc x0, int C, uint32_t oc,
                                          int pos) {
    cc.w = bld4(buf(a.conv_w, C * 16), 4 * oc, 0);
#pragma unroll
    for (int j = 0; j < 3; ++j) cc.hist[j] = bld(ring, oc, slot_off(a, C, pos - 3 + j));
    cc.x = bld(x0, oc, 0);
}

// after the last token: raw inputs of this call's own last (up to) three positions into their ring slots
__device__ __forceinline__ void conv_store(const ConvChan &cc, const GdnArgs &a, brsrc ring, int C, uint32_t oc,
                                           int pos) {
    const int last = pos + a.nt - 1;
    bst(ring, oc, slot_off(a, C, last), cc.x);
    if (a.nt >= 2) bst(ring, oc, slot_off(a, C, last - 1), cc.hist[2]);
    if (a.nt >= 3) bst(ring, oc, slot_off(a, C, last - 2), cc.hist[1]);
}

// Gates of one head and token (uniform per head): beta = sigmoid(b), gamma = exp(ssm_a * softplus(a + dt_bias)),
// softplus the identity above 20 (faie2fn.cu:1407-1410).  One function for the one-token and the lane-parallel
// (multi-token) callers, so both compute the same bits.
__device__ __forceinline__ void gdn_gates(float ga, float gb, float dtb, float ssa, float &beta, float &gamma) {
    beta = sigmoidf_(gb);
    const float x = ga + dtb;
    const float sp = x > 20.0f ? x : log1pf(expf(x));
    gamma = expf(sp * ssa);
}

// MODE 0: the bare core; 1: the fused block (every token committed); 3: the fused block for exactly one token (the
// decode step: no token loop, no next-token prefetch, fewer registers); 2: the fused block as a verify step with
// deferred commit -- first the kr[b] tokens of the previous call that the caller accepted are replayed from their
// saved inputs (no output), the state and ring after them are written (the committed state), then the nt new tokens
// run on the state in registers only: their outputs are written, their state is not.
// mid-loop, once token u = n has been shifted in (n >= 1 tokens processed, the last at position end - 1): the raw
// inputs of positions end-3 .. end-1 are hist[0..2]; write the slots of the ones this call processed (the last
// min(n, 3))
__device__ __forceinline__ void conv_store_hist(const ConvChan &cc, const GdnArgs &a, brsrc ring, int C, uint32_t oc,
                                                int end, int n) {
    bst(ring, oc, slot_off(a, C, end - 1), cc.hist[2]);
    if (n >= 2) bst(ring, oc, slot_off(a, C, end - 2), cc.hist[1]);
    if (n >= 3) bst(ring, oc, slot_off(a, C, end - 3), cc.hist[0]);
}

template <int MODE, int NTH = (MODE == 1 || MODE == 2) ? MT_THREADS : THREADS, int SAUX = ST_NT>
__global__ void __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu((MODE == 1 || MODE == 2) ? GDN_VERIFY_WPE : GDN_WPE, 8)))
k_gdn(const GdnArgs a) {
    constexpr int WAVES = NTH / 64;
    // Every thread count computes the 512-thread kernel's arithmetic bit for bit (a verify step must reproduce
    // one-token decode exactly): the column partials of a row group are chained in row order, groups 2m and 2m + 1
    // are added, and the 8 sums are added in m order.  A thread owns CH = 512 / NTH consecutive row groups
    // CH rg + j of column group cg: with 512 threads groups 2m and 2m + 1 sit in lanes l and l ^ 32 of wave m, with
    // 256 threads in one thread.
    constexpr int CH = 512 / NTH;
    constexpr bool FUSED = MODE >= 1, VERIFY = MODE == 2, ONE = MODE == 3;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cg = tid & 31, rg = tid >> 5;
    const int bh = blockIdx.x, b = bh / a.nvh, h = bh - b * a.nvh;
    const int kh = a.head_map == 0 ? h % a.nkh : h / (a.nvh / a.nkh);
    const int C = 2 * a.nkh * DK + a.nvh * DV;
    const bool qk_thr = tid < DK, v_thr = tid >= DK && tid < DK + DV;  // wave-uniform roles

    // The per-token exchange is double-buffered by token parity in multi-token calls: token u + 2 writes a buffer
    // only after every wave has passed token u + 1's barriers, i.e. finished reading token u, so the loop needs no
    // barrier of its own between tokens.
    constexpr int NBUF = ONE ? 1 : 2;
    __shared__ float4 qs4[NBUF][DK / 4], ks4[NBUF][DK / 4];  // raw q, k of the key head (this token)
    __shared__ float vs[NBUF][DV];                            // conv'd v of the value head
    __shared__ float4 red[NBUF][NG / 2][2][DV / 4];           // folded column partials of kv and sq
    __shared__ float nrm[NBUF][2][3];                         // per-wave sums q.q, k.k, q.k (waves 0, 1)
    __shared__ float2 abp[WAVES];                 // fused alpha/beta projection: per-wave partial dots

    // 1. every input of the first token is requested before the state tile, so nothing waits behind S twice:
    //    conv weights, ring taps and raw inputs (waves 0-3), z and the norm weight (wave 0)
    // verify: pos is the position of the first new token; the kr replayed tokens sit at pos - kr .. pos - 1
    const int kr = VERIFY ? max(0, min(a.kr[b], a.rnt)) : 0;  // clamped: never past the replay rows
    if (VERIFY && h == 0 && tid == 0 && kr != a.kr[b]) atomicOr(a.status, FN_STATUS_KR);
    const int ntot = ONE ? 1 : kr + a.nt;
    const int pos = FUSED ? a.pos[b] - kr : 0;  // position of the first token this call processes
    const float *x_b = a.qkv + (size_t) b * a.nt * C;
    const float *rx_b = VERIFY ? a.rqkv + (size_t) b * a.rnt * C : x_b;
    const brsrc ring = buf(a.ring_buf + (size_t) b * a.ring * C, a.ring * C * 4);
    // byte offsets of this thread's channels in a row of C: c0 carries q (waves 0-1) or v (waves 2-3), c1 carries k;
    // of its 4 columns in a row of DV (z, norm weight, output)
    const uint32_t o0 = 4u * (qk_thr ? kh * DK + tid : 2 * a.nkh * DK + h * DV + (tid - DK));
    const uint32_t o1 = 4u * (a.nkh * DK + kh * DK + tid);
    const uint32_t oz = 16u * cg;
    ConvChan c0{}, c1{};
    float4 z4 = f4(0.0f), w4 = f4(0.0f);
    if (FUSED) {
        const brsrc x0 = buf(kr > 0 ? rx_b : x_b, C * 4);  // raw input row of the first token
        if (qk_thr || v_thr) conv_load(c0, a, ring, x0, C, o0, pos);
        if (qk_thr) conv_load(c1, a, ring, x0, C, o1, pos);
        if (wave == 0 && lane < 32) {
            if (kr == 0) z4 = bld4(buf(a.z + (size_t) b * a.nt * a.nvh * DV + (size_t) h * DV, DV * 4), oz, 0);
            w4 = bld4(buf(a.norm_w, DV * 4), oz, 0);
        }
    }
    const bool primary = a.head_map == 0 ? h < a.nkh : (h % (a.nvh / a.nkh)) == 0;
    // fused alpha/beta projection (one token): this head's two rows of the BF16 weight against the sequence's x,
    // requested before the state tile so their wait never includes it; thread tid takes elements 4 tid + 2048 k,
    // the waves' partial dots meet in LDS and are summed in wave order (deterministic)
    const bool xab = ONE && a.wab != nullptr;
    if (xab) {
        const float *xb = a.x + (size_t) b * a.hidden;
        const uint16_t *wa = a.wab + (size_t) h * a.hidden, *wb = a.wab + (size_t) (a.nvh + h) * a.hidden;
        float pa = 0.0f, pb = 0.0f;
        for (int i = 4 * tid; i < a.hidden; i += 4 * NTH) {
            const float4 xv = *reinterpret_cast<const float4 *>(xb + i);
            const uint2 ua = *reinterpret_cast<const uint2 *>(wa + i), ub = *reinterpret_cast<const uint2 *>(wb + i);
            pa = fmaf(bf16_lo(ua.x), xv.x, pa);
            pa = fmaf(bf16_hi(ua.x), xv.y, pa);
            pa = fmaf(bf16_lo(ua.y), xv.z, pa);
            pa = fmaf(bf16_hi(ua.y), xv.w, pa);
            pb = fmaf(bf16_lo(ub.x), xv.x, pb);
            pb = fmaf(bf16_hi(ub.x), xv.y, pb);
            pb = fmaf(bf16_lo(ub.y), xv.z, pb);
            pb = fmaf(bf16_hi(ub.y), xv.w, pb);
        }
        pa = wave_sum(pa);
        pb = wave_sum(pb);
        if (lane == 0) abp[wave] = make_float2(pa, pb);
    }

    // multi-token calls: lane i holds the logits (then the gates) of token u0 + i of each run of 64 tokens, computed
    // once for the run instead of once per token by every thread
    const auto lane_logits = [&](int u0, float &la, float &lb) {
        const int uu = u0 + lane;
        la = lb = 0.0f;
        if (uu < ntot) {
            const float *abt = VERIFY && uu < kr ? a.rab + ((size_t) b * a.rnt + uu) * 2 * a.nvh
                                                 : a.ab + ((size_t) b * a.nt + (uu - kr)) * 2 * a.nvh;
            la = abt[h];
            lb = abt[a.nvh + h];
        }
    };
    float ga = 0.0f, gb = 0.0f, dtb = 0.0f, ssa = 0.0f;  // one token's alpha, beta logits; the head's gate params
    float lbeta = 0.0f, lgamma = 0.0f;                   // gates of token u0 + lane (one token: its gates)
    if (FUSED) {
        if (!ONE) lane_logits(0, ga, gb);
        if (ONE && !xab) {
            const float *ab0 = a.ab + (size_t) b * a.nt * 2 * a.nvh;
            ga = ab0[h];
            gb = ab0[a.nvh + h];
        }
        dtb = a.dt_bias[h];
        ssa = a.ssm_a[h];
    }

    // 2. state tile into registers
    float4 s[CH][GROWS];
    const brsrc Sb = buf(a.S + (size_t) bh * DK * DV, DK * DV * 4);
    const uint32_t so = 16u * (CH * rg * (DV / 4) + cg);  // the thread's float4 of row CH rg; group j is j rows on
#pragma unroll
    for (int j = 0; j < CH; ++j)
#pragma unroll
        for (int r = 0; r < GROWS; ++r) s[j][r] = ld_state(Sb, so + j * DV * 4, r);
    // gates under the tile's loads: of the first 64 tokens (lane-parallel), or of the one token (uniform; with the
    // fused alpha/beta projection they wait for its sums)
    if (FUSED && (!ONE || !xab)) gdn_gates(ga, gb, dtb, ssa, lbeta, lgamma);

    const float scale = 0.08838834764831845f;  // 1/sqrt(128), faie2fn.cu:1352

    // Inputs of token u of this call: its raw conv channels, z (wave 0) and alpha/beta logits.  The next token's are
    // requested one iteration ahead, so a multi-token call (verify, prefill) does not wait a memory round trip per
    // token: the loop's barriers order LDS only (lds_barrier), every one of these is a vector (buffer) load, and no
    // per-lane address is a 64-bit pair the compiler could keep across the loop and spill (a scratch reload waits
    // for every load issued before it, the prefetch included).
    float nx0 = 0.0f, nx1 = 0.0f;  // next token's raw channels
    float4 nz = f4(0.0f);
#define GDN_PREFETCH(U_)                                                                                           \
    do {                                                                                                          \
        const int u_ = (U_);                                                                                      \
        const bool rp_ = VERIFY && u_ < kr;                                                                       \
        const float *xt_ = rp_ ? rx_b + (size_t) u_ * C : x_b + (size_t) (u_ - kr) * C;                           \
        const brsrc xr_ = buf(xt_, C * 4);                                                                        \
        if (qk_thr || v_thr) nx0 = bld(xr_, o0, 0);                                                              \
        if (qk_thr) nx1 = bld(xr_, o1, 0);                                                                        \
        if (wave == 0 && lane < 32 && !rp_)                                                                       \
            nz = bld4(buf(a.z + ((size_t) b * a.nt + (u_ - kr)) * a.nvh * DV + (size_t) h * DV, DV * 4), oz, 0); \
    } while (0)
    if (FUSED) {
        if (!ONE && ntot > 1) GDN_PREFETCH(1);
    }

    // runs of up to 64 tokens: the gates of a run are computed lane-parallel before it
    for (int u0 = 0; u0 < ntot; u0 += 64) {
    if (FUSED && !ONE && u0 > 0) {
        lane_logits(u0, ga, gb);
        gdn_gates(ga, gb, dtb, ssa, lbeta, lgamma);
    }
    for (int u = u0; u < min(u0 + 64, ntot); ++u) {
            // token u: a replayed one (u < kr, inputs from the previous call, no output) or new token t = u - kr
            const bool replay = VERIFY && u < kr;
            const int t = u - kr;
            const int pb = NBUF == 1 ? 0 : (u & 1);  // exchange buffer of this token
            const size_t bt = (size_t) b * a.nt + (replay ? 0 : t);
            if (u > 0) {
                if (FUSED) {
                    if (qk_thr) {
                        c0.shift(nx0);
                        c1.shift(nx1);
                    } else if (v_thr) {
                        c0.shift(nx0);
                    }
                    if (!replay) z4 = nz;
                    if (!ONE && u + 1 < ntot) GDN_PREFETCH(u + 1);
                }
            }
            if (VERIFY && u == kr && kr > 0) {
                // the committed state, before the first new token moves the registers on: S after the replayed tokens,
                // and the ring slots of the replayed positions (the last up to three; after the shift above hist holds
                // the raw inputs of positions pos + kr - 3 .. pos + kr - 1)
#pragma unroll
                for (int j = 0; j < CH; ++j)
#pragma unroll
                    for (int r = 0; r < GROWS; ++r) st_state<SAUX>(Sb, so + j * DV * 4, r, s[j][r]);
                if (qk_thr) {
                    if (primary) {
                        conv_store_hist(c0, a, ring, C, o0, pos + kr, kr);
                        conv_store_hist(c1, a, ring, C, o1, pos + kr, kr);
                    }
                } else if (v_thr) {
                    conv_store_hist(c0, a, ring, C, o0, pos + kr, kr);
                }
            }

            // 3. q, k (waves 0-1, channel i = tid) and v (waves 2-3, channel j = tid - 128)
            if (qk_thr) {
                float q, k;
                if (FUSED) {
                    q = c0.out();
                    k = c1.out();
                } else {
                    q = a.q[(bt * a.nkh + kh) * DK + tid];
                    k = a.k[(bt * a.nkh + kh) * DK + tid];
                }
                reinterpret_cast<float *>(qs4[pb])[tid] = q;
                reinterpret_cast<float *>(ks4[pb])[tid] = k;
                const float sqq = wave_sum(q * q), skk = wave_sum(k * k), sqk = wave_sum(q * k);
                if (lane == 0) {
                    nrm[pb][wave][0] = sqq;
                    nrm[pb][wave][1] = skk;
                    nrm[pb][wave][2] = sqk;
                }
            } else if (v_thr) {
                vs[pb][tid - DK] = FUSED ? c0.out() : a.v[(bt * a.nvh + h) * DV + (tid - DK)];
            }

            lds_barrier();
            // 4. gates (uniform per head): beta = sigmoid(b), gamma = exp(ssm_a * softplus(a + dt_bias)), softplus
            //    the identity above 20 (faie2fn.cu:1407-1410)
            if (xab) {
                ga = abp[0].x;
                gb = abp[0].y;
#pragma unroll
                for (int w = 1; w < WAVES; ++w) {
                    ga += abp[w].x;
                    gb += abp[w].y;
                }
            }
            float beta, gamma;
            if (FUSED && ONE) {
                if (xab) {
                    gdn_gates(ga, gb, dtb, ssa, beta, gamma);
                } else {
                    beta = lbeta;
                    gamma = lgamma;
                }
            } else if (FUSED) {
                beta = readlane(lbeta, u - u0);
                gamma = readlane(lgamma, u - u0);
            } else {
                beta = a.beta[bt * a.nvh + h];
                gamma = expf(a.g[bt * a.nvh + h]);
            }

            // L2 factors x * rsqrt(sum x^2 + 1e-6) (faie2fn.cu:1399-1402); the core takes q, k as given
            float rq = 1.0f, rk = 1.0f;
            const float sqk = nrm[pb][0][2] + nrm[pb][1][2];
            if (FUSED) {
                rq = rsqrtf(nrm[pb][0][0] + nrm[pb][1][0] + 1e-6f);
                rk = rsqrtf(nrm[pb][0][1] + nrm[pb][1][1] + 1e-6f);
            }
            const float kq = sqk * rq * rk;

            // 5. one pass over the registers: column partials of S^T k and S^T q over this thread's rows
            const float *ksf = reinterpret_cast<const float *>(ks4[pb]), *qsf = reinterpret_cast<const float *>(qs4[pb]);
            float4 kvp[CH], sqp[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                kvp[j] = sqp[j] = f4(0.0f);
#pragma unroll
                for (int r = 0; r < GROWS; ++r) {
                    const int row = CH * rg + j + NG * r;
                    const float kr = ksf[row], qr = qsf[row];
                    const float4 sv = s[j][r];
                    kvp[j].x = fmaf(sv.x, kr, kvp[j].x);
                    kvp[j].y = fmaf(sv.y, kr, kvp[j].y);
                    kvp[j].z = fmaf(sv.z, kr, kvp[j].z);
                    kvp[j].w = fmaf(sv.w, kr, kvp[j].w);
                    sqp[j].x = fmaf(sv.x, qr, sqp[j].x);
                    sqp[j].y = fmaf(sv.y, qr, sqp[j].y);
                    sqp[j].z = fmaf(sv.z, qr, sqp[j].z);
                    sqp[j].w = fmaf(sv.w, qr, sqp[j].w);
                }
            }
            // fold row groups 2m and 2m + 1 (lanes l and l ^ 32, or the thread's two groups), then the 8 folded sums
            // through LDS
            float4 kvf, sqf;
            if constexpr (CH == 1) {
                kvf = make_float4(add_xor32(kvp[0].x), add_xor32(kvp[0].y), add_xor32(kvp[0].z), add_xor32(kvp[0].w));
                sqf = make_float4(add_xor32(sqp[0].x), add_xor32(sqp[0].y), add_xor32(sqp[0].z), add_xor32(sqp[0].w));
            } else {
                kvf = make_float4(kvp[0].x + kvp[1].x, kvp[0].y + kvp[1].y, kvp[0].z + kvp[1].z, kvp[0].w + kvp[1].w);
                sqf = make_float4(sqp[0].x + sqp[1].x, sqp[0].y + sqp[1].y, sqp[0].z + sqp[1].z, sqp[0].w + sqp[1].w);
            }
            if (CH == 2 || lane < 32) {
                const int m = CH == 1 ? wave : rg;
                red[pb][m][0][cg] = kvf;
                red[pb][m][1][cg] = sqf;
            }
            lds_barrier();
            float4 kv = red[pb][0][0][cg], sq = red[pb][0][1][cg];
#pragma unroll
            for (int w = 1; w < NG / 2; ++w) {
                const float4 x = red[pb][w][0][cg], y = red[pb][w][1][cg];
                kv.x += x.x; kv.y += x.y; kv.z += x.z; kv.w += x.w;
                sq.x += y.x; sq.y += y.y; sq.z += y.z; sq.w += y.w;
            }

            // 6. delta, readout, update.  kv and sq were taken over raw k and q: scale by rk and rq here.
            const float4 v4 = reinterpret_cast<const float4 *>(vs[pb])[cg];
            float4 d, o;
            d.x = (v4.x - gamma * (kv.x * rk)) * beta;
            d.y = (v4.y - gamma * (kv.y * rk)) * beta;
            d.z = (v4.z - gamma * (kv.z * rk)) * beta;
            d.w = (v4.w - gamma * (kv.w * rk)) * beta;
            o.x = fmaf(gamma, sq.x * rq, kq * d.x) * scale;
            o.y = fmaf(gamma, sq.y * rq, kq * d.y) * scale;
            o.z = fmaf(gamma, sq.z * rq, kq * d.z) * scale;
            o.w = fmaf(gamma, sq.w * rq, kq * d.w) * scale;
            const float4 dk4 = make_float4(d.x * rk, d.y * rk, d.z * rk, d.w * rk);  // k enters raw below
#pragma unroll
            for (int j = 0; j < CH; ++j)
#pragma unroll
                for (int r = 0; r < GROWS; ++r) {
                    const float kr = ksf[CH * rg + j + NG * r];
                    float4 &sv = s[j][r];
                    sv.x = fmaf(kr, dk4.x, gamma * sv.x);
                    sv.y = fmaf(kr, dk4.y, gamma * sv.y);
                    sv.z = fmaf(kr, dk4.z, gamma * sv.z);
                    sv.w = fmaf(kr, dk4.w, gamma * sv.w);
                }

            // 7. output: wave 0 holds every column twice (lanes l and l + 32)
            if (wave == 0 && !replay) {
                if (FUSED) {
                    // gated RMSNorm on = o * rsqrt(mean o^2 + eps) * w * act(z) (faie2fn.cu:1422-1424); the wave sum
                    // counts each column twice, exactly, so halve it
                    const float ss = 0.5f * wave_sum(o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w);
                    const float rn = rsqrtf(ss / DV + a.eps);
                    if (lane < 32) {
                        float4 r;
                        if (a.gate_act == 0) {
                            r.x = o.x * rn * w4.x * sigmoid_r(z4.x);
                            r.y = o.y * rn * w4.y * sigmoid_r(z4.y);
                            r.z = o.z * rn * w4.z * sigmoid_r(z4.z);
                            r.w = o.w * rn * w4.w * sigmoid_r(z4.w);
                        } else {
                            r.x = o.x * rn * w4.x * silu_r(z4.x);
                            r.y = o.y * rn * w4.y * silu_r(z4.y);
                            r.z = o.z * rn * w4.z * silu_r(z4.z);
                            r.w = o.w * rn * w4.w * silu_r(z4.w);
                        }
                        bst4(buf(a.out + bt * a.nvh * DV + (size_t) h * DV, DV * 4), oz, 0, r);
                    }
                } else if (lane < 32) {
                    bst4(buf(a.out + (bt * a.nvh + h) * DV, DV * 4), oz, 0, o);
                }
            }
        }
    }

    // 8. write back: state once; ring slots of this call's last (up to) three positions from the registers.  The
    //    q/k channels of a key head are written by one of its value heads only.  A verify step wrote its committed
    //    state above and leaves the new tokens' state uncommitted.
    if (VERIFY) return;
#pragma unroll
    for (int j = 0; j < CH; ++j)
#pragma unroll
        for (int r = 0; r < GROWS; ++r) st_state<SAUX>(Sb, so + j * DV * 4, r, s[j][r]);
    if (FUSED) {
        if (qk_thr) {
            if (primary) {
                conv_store(c0, a, ring, C, o0, pos);
                conv_store(c1, a, ring, C, o1, pos);
            }
        } else if (v_thr) {
            conv_store(c0, a, ring, C, o0, pos);
        }
    }
}

#undef GDN_PREFETCH

int check_dims(int B, int nkh, int nvh, int dk, int dv, int head_map, int nt) {
    if (B < 1 || nkh < 1 || nvh < 1 || nt < 1) FN_FAIL("gdn: B, nkh, nvh and nt must be >= 1");
    if (dk != DK || dv != DV) FN_FAIL("gdn: only dk = dv = 128 is built");
    if (nvh % nkh) FN_FAIL("gdn: nvh must be a multiple of nkh");
    if (head_map != 0 && head_map != 1) FN_FAIL("gdn: head_map must be 0 (tiled h % nkh) or 1 (grouped)");
    if ((size_t) B * nvh > 0x7fffffffu) FN_FAIL("gdn: too many heads");
    return 0;
}

}  // namespace

int gdn_block_launch(const GdnBlock &p, hipStream_t st) {
    if (check_dims(p.B, p.nkh, p.nvh, p.dk, p.dv, p.head_map, p.nt)) return -1;
    if (p.gate_act != 0 && p.gate_act != 1) FN_FAIL("gdn: gate_act must be 0 (sigmoid) or 1 (silu)");
    if (p.ring < 4 || (p.ring & (p.ring - 1))) FN_FAIL("gdn: ring must be a power of two >= 4");
    if (p.nt > p.ring - 3) FN_FAIL("gdn: nt must be <= ring - 3");
    const bool xab = p.wab != nullptr;
    if (!p.pos || !p.qkv || !p.conv_w || !p.conv_ring || (!xab && !p.ab) || !p.dt_bias || !p.ssm_a || !p.S || !p.z ||
        !p.norm_w || !p.out || (xab && !p.x))
        FN_FAIL("gdn: null pointer");
    if (xab && p.nt != 1) FN_FAIL("gdn: the fused alpha/beta projection takes one token (nt = 1)");
    if (xab && (p.hidden < 4 || p.hidden % 4)) FN_FAIL("gdn: hidden must be a positive multiple of 4");
    if (xab && ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.wab)) & 15))
        FN_FAIL("gdn: x and w_ab must be 16-byte aligned");
    GdnArgs a{};
    a.B = p.B; a.nkh = p.nkh; a.nvh = p.nvh; a.nt = p.nt; a.ring = p.ring; a.head_map = p.head_map;
    a.gate_act = p.gate_act; a.eps = p.eps; a.pos = p.pos; a.qkv = p.qkv; a.conv_w = p.conv_w;
    a.ring_buf = p.conv_ring; a.ab = p.ab; a.dt_bias = p.dt_bias; a.ssm_a = p.ssm_a; a.S = p.S; a.z = p.z;
    a.norm_w = p.norm_w; a.out = p.out; a.x = p.x; a.wab = p.wab; a.hidden = p.hidden;
    if (p.nt == 1 && p.B * p.nvh > 2 * device_cus())  // more heads than one round of resident workgroups (two a CU)
        hipLaunchKernelGGL((k_gdn<3, THREADS, ST_NT_SYS>), dim3(p.B * p.nvh), dim3(THREADS), GDN_ONE_LDS_PAD, st, a);
    else if (p.nt == 1)
        hipLaunchKernelGGL(k_gdn<3>, dim3(p.B * p.nvh), dim3(THREADS), GDN_ONE_LDS_PAD, st, a);
    else
        hipLaunchKernelGGL(k_gdn<1>, dim3(p.B * p.nvh), dim3(MT_THREADS), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

int gdn_core_launch(const GdnCore &p, hipStream_t st) {
    if (check_dims(p.B, p.nkh, p.nvh, p.dk, p.dv, p.head_map, p.nt)) return -1;
    if (!p.q || !p.k || !p.v || !p.beta || !p.g || !p.S || !p.o) FN_FAIL("gdn: null pointer");
    GdnArgs a{};
    a.B = p.B; a.nkh = p.nkh; a.nvh = p.nvh; a.nt = p.nt; a.ring = 4; a.head_map = p.head_map;
    a.q = p.q; a.k = p.k; a.v = p.v; a.beta = p.beta; a.g = p.g; a.S = p.S; a.out = p.o;
    hipLaunchKernelGGL(k_gdn<0>, dim3(p.B * p.nvh), dim3(THREADS), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

namespace fn {

int gdn_verify_launch(const GdnVerify &p, hipStream_t st) {
    const GdnBlock &q = p.blk;
    if (check_dims(q.B, q.nkh, q.nvh, q.dk, q.dv, q.head_map, q.nt)) return -1;
    if (q.gate_act != 0 && q.gate_act != 1) FN_FAIL("gdn: gate_act must be 0 (sigmoid) or 1 (silu)");
    if (q.ring < 4 || (q.ring & (q.ring - 1))) FN_FAIL("gdn: ring must be a power of two >= 4");
    if (p.rnt < 0 || p.rnt > q.ring - 3) FN_FAIL("gdn_verify: rnt (most tokens committed per call) must be <= ring - 3");
    if (!q.pos || !q.qkv || !q.conv_w || !q.conv_ring || !q.ab || !q.dt_bias || !q.ssm_a || !q.S || !q.z ||
        !q.norm_w || !q.out || !p.kr || (p.rnt > 0 && (!p.rqkv || !p.rab)))
        FN_FAIL("gdn_verify: null pointer");
    GdnArgs a{};
    a.B = q.B; a.nkh = q.nkh; a.nvh = q.nvh; a.nt = q.nt; a.ring = q.ring; a.head_map = q.head_map;
    a.gate_act = q.gate_act; a.eps = q.eps; a.pos = q.pos; a.qkv = q.qkv; a.conv_w = q.conv_w;
    a.ring_buf = q.conv_ring; a.ab = q.ab; a.dt_bias = q.dt_bias; a.ssm_a = q.ssm_a; a.S = q.S; a.z = q.z;
    a.norm_w = q.norm_w; a.out = q.out;
    a.kr = p.kr; a.rnt = p.rnt; a.rqkv = p.rqkv; a.rab = p.rab;
    if (status_word(&a.status)) return -1;
    hipLaunchKernelGGL(k_gdn<2>, dim3(q.B * q.nvh), dim3(MT_THREADS), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

// GQA decode attention over an fp32 KV cache for gfx950: q/k RMSNorm + partial RoPE + cache append, split-K
// online softmax, and the split merge with the sigmoid output gate.
//
// Semantics follow k_qk_norm_rope, k_attn_split (indexer mask null = dense) and k_attn_combine (reference
// engine/faie2fn.cu:1436-1478, 1609-1690).  The CDNA4 design:
//   * One workgroup per (sequence, token, kv head, split) serves all GRP query heads of the group, so every K/V
//     byte crosses HBM once per token (the reference runs one block per query head and re-reads K/V GRP times).
//   * The K cache is stored key-tiled: each tile of 64 positions is [hd/4][64][4] floats (64 KiB at hd = 256).
//     Lane l of a wave owns key l of the tile and reads it 16 bytes at a time with fully coalesced 1 KiB wave
//     loads; the query values it multiplies are wave-uniform LDS broadcasts, so q.k costs GRP FMAs per 4 dims per
//     key and needs no cross-lane reduction at all.
//   * V stays row-major; for p.V a lane owns 4 output dims, reads each V row with one coalesced 1 KiB wave load
//     and takes the GRP probabilities of the key as LDS broadcasts.
//   * The four waves of a workgroup walk each 64-key tile together: each requests a quarter of the tile's K
//     (16 chunks of every key) and a quarter of its V rows at the start, with the nontemporal hint, so a tile
//     costs about two load latencies; partial scores meet in LDS, one wave per GRP/4 heads runs the online
//     softmax (DPP wave max), and every wave accumulates p.V over its rows.  (A first version let each wave walk
//     whole tiles alone: eight dependent load batches per tile, 36.5 us at B = 1, L = 4K against 18 us now.)
//   * The workgroup writes one (m, l, o[hd]) partial per query head per split.
//   * The combine kernel merges the splits with the log-sum-exp identity and applies o / L * sigmoid(gate).
// Device cache layouts (max_ctx a multiple of 64):
//   Kc: [B][nkv][max_ctx / 64][hd / 4][64][4]   Vc: [B][nkv][max_ctx][hd]
#include "qsa.h"

#include <algorithm>
#include <cmath>

namespace fn {

namespace {

constexpr int HD = 256;     // head dim built (the reference's, faie2fn.cu:49)
constexpr int TILE = 64;    // keys per tile (= wave size)
constexpr int WAVES = 4;
constexpr int MAXROT = 128;


struct AttnArgs {
    int B, nq, nkv, nt, max_ctx, nsplit, nrot;
    float eps;
    const int32_t *pos;
    const float *qg, *knew, *vnew, *wq, *wk;
    float *Kc, *Vc;
    float *Q;        // [B nt][nkv][HD/4][grp][4]
    float *part_o;   // [B nt][nq][nsplit][HD]
    float *part_ml;  // [B nt][nq][nsplit][2]
    float *og;
    const int32_t *keys;   // visible-key list per query (QSA) or null (dense)
    const int32_t *nkeys;
    int kstride;           // list stride per query
    unsigned *status;      // per-device status word: FN_STATUS_POS when a new token falls outside the cache
    float inv_freq[MAXROT / 2];
};

__device__ __forceinline__ size_t k_index(int max_ctx, int b, int nkv, int g, int p, int d) {
    const size_t tile = ((size_t) b * nkv + g) * (max_ctx / TILE) + p / TILE;
    return ((tile * (HD / 4) + d / 4) * TILE + (p % TILE)) * 4 + (d % 4);
}

// RMSNorm + RoPE of the query heads and the new key (faie2fn.cu:1451-1478), cache append.
// grid (B nt, nq + nkv), HD threads
__global__ void __launch_bounds__(HD) k_attn_prep(const AttnArgs a) {
    __shared__ float buf[HD];
    __shared__ float red[HD / 64];
    const int bt = blockIdx.x, b = bt / a.nt, t = bt - b * a.nt, j = blockIdx.y, d = threadIdx.x;
    const int P = a.pos[b] + t;
    if (P < 0 || P >= a.max_ctx) {  // outside the cache: nothing is written past it; the status word says so
        if (j == 0 && d == 0) atomicOr(a.status, FN_STATUS_POS);
        return;
    }
    const bool isq = j < a.nq;
    const int g = isq ? j / (a.nq / a.nkv) : j - a.nq;
    const float x = isq ? a.qg[((size_t) bt * a.nq + j) * 2 * HD + d] : a.knew[((size_t) bt * a.nkv + g) * HD + d];
    const float ws = wave_sum(x * x);
    if ((d & 63) == 0) red[d >> 6] = ws;
    __syncthreads();
    const float ss = red[0] + red[1] + red[2] + red[3];
    buf[d] = x * rsqrtf(ss / HD + a.eps) * (isq ? a.wq[d] : a.wk[d]);
    __syncthreads();
    float y = buf[d];
    const int half = a.nrot / 2;
    if (d < a.nrot) {
        const int i = d < half ? d : d - half;
        const float x0 = buf[i], x1 = buf[i + half];
        const float ang = (float) P * a.inv_freq[i];  // fp32 angle (faie2fn.cu:1440)
        const float cs = cosf(ang), sn = sinf(ang);
        y = d < half ? x0 * cs - x1 * sn : x1 * cs + x0 * sn;
    }
    if (isq) {
        const int grp = a.nq / a.nkv, hh = j - g * grp;
        a.Q[((((size_t) bt * a.nkv + g) * (HD / 4) + d / 4) * grp + hh) * 4 + (d % 4)] = y;
    } else {
        a.Kc[k_index(a.max_ctx, b, a.nkv, g, P, d)] = y;
        a.Vc[(((size_t) b * a.nkv + g) * a.max_ctx + P) * HD + d] = a.vnew[((size_t) bt * a.nkv + g) * HD + d];
    }
}

// Split-K attention partials.  grid (nsplit, nkv, B nt), WAVES*64 threads.
// The four waves walk one 64-key tile together: wave w reads K chunks 16w..16w+15 of every key (lane = key) and V
// rows 16w..16w+15 (lane = 4 dims), both requested at the start of the tile; the partial scores meet in LDS; wave w
// then runs the online softmax of heads w*GRP/4 .. (w+1)*GRP/4 - 1 (lane = key) and publishes p and the rescale
// factors; each wave accumulates p.V over its 16 rows for all heads.  A tile costs about two load latencies instead
// of eight, which is what a short context or a small batch is bound by.
// RMSNorm of a 256-long row held as one float4 per lane (lane = dims 4l..4l+3): x * rsqrt(mean x^2 + eps) * w
// (faie2fn.cu:1466-1467).  Call from wave-uniform control flow.
__device__ __forceinline__ float4 rms_row(float4 x, float4 w, float eps) {
    const float ss = wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
    const float r = rsqrtf(ss / HD + eps);
    return make_float4(x.x * r * w.x, x.y * r * w.y, x.z * r * w.z, x.w * r * w.w);
}

// RoPE in place on a row stored in LDS as float4 chunks with stride `stride` (chunk c of the row at row4[c *
// stride]): dims d < nrot, pairs (i, i + nrot/2) (faie2fn.cu:1438-1445, 1470-1474), with cos/sin of the fp32 angle
// (float)P * inv_freq[i] taken from cs/sn.  One wave, lane = chunk; every read happens before any write.
__device__ __forceinline__ void rope_row_lds(float4 *row4, int stride, int lane, int nrot, const float *cs,
                                             const float *sn) {
    const float *row = reinterpret_cast<const float *>(row4);
    const int half = nrot / 2;
    float y[4];
    const bool act = 4 * lane < nrot;
    if (act) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = 4 * lane + e, i = d < half ? d : d - half;
            const float x0 = row[(i / 4) * stride * 4 + (i % 4)], x1 = row[((i + half) / 4) * stride * 4 + ((i + half) % 4)];
            y[e] = d < half ? x0 * cs[i] - x1 * sn[i] : x1 * cs[i] + x0 * sn[i];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (act) row4[lane * stride] = make_float4(y[0], y[1], y[2], y[3]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// PREP (one new token per sequence): the workgroup also does k_attn_prep's work for its group -- RMSNorm + RoPE of
// its GRP query heads into LDS, and, in the workgroup whose split holds the new position, of the new key, which it
// appends with the new value to the caches before its first tile load.
// LIST (sparse): the keys a query attends are the first nkeys entries of its key list (ascending positions); tile
// slots index the list and K/V are gathered from the caches.
template <int GRP, bool PREP, bool LIST = false>
__global__ void __launch_bounds__(WAVES * 64) k_attn_split(const AttnArgs a) {
    constexpr int HPW = GRP / WAVES;                 // softmax heads per wave
    constexpr int CPW = HD / 4 / WAVES;              // K chunks (of 4 dims) per wave = 16
    constexpr int RPW = TILE / WAVES;                // V rows per wave = 16
    static_assert(GRP % WAVES == 0, "heads split evenly over the waves");
    constexpr int QB = HD / 4 * GRP * 16, SB = WAVES * GRP * TILE * 4, PB = TILE * GRP * 4, CB = GRP * 4;
    constexpr int MERGE = WAVES * GRP * HD * 4, WALK = QB + SB + PB + CB;
    __shared__ __align__(16) unsigned char smem[WALK > MERGE ? WALK : MERGE];
    __shared__ float mmax[GRP], msum[GRP];
    float4 *qs = reinterpret_cast<float4 *>(smem);                  // [HD/4][GRP]
    float *sp = reinterpret_cast<float *>(smem + QB);               // [WAVES][GRP][TILE] partial scores
    float *pb = reinterpret_cast<float *>(smem + QB + SB);          // [TILE][GRP] probabilities
    float *cr = reinterpret_cast<float *>(smem + QB + SB + PB);     // [GRP] rescale of this tile
    float4 *mo = reinterpret_cast<float4 *>(smem);                  // [WAVES][GRP][HD/4] (after the walk)
    __shared__ float4 kn4[HD / 4], vn4[HD / 4];                      // new key and value (PREP)
    __shared__ float rcs[MAXROT / 2], rsn[MAXROT / 2];                // cos / sin of the RoPE angles (PREP)

    const int sp_i = blockIdx.x, g = blockIdx.y, bt = blockIdx.z, b = bt / a.nt, t = bt - b * a.nt;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // (one new token) Every load of the prologue is requested first, before the position is waited for and before
    // any of them is used (none depends on the position): the RoPE frequency, the wave's query rows and their norm
    // weight, the new key row, its norm weight and the new value row; the sines and cosines then overlap their round
    // trip.  The key row is normalised and the key and value rows go to the LDS by every wave (the same values),
    // unconditionally, so that the compiler does not move their loads under the owner's branch, behind the others.
    float fr = 0.0f;
    float4 wq, xq[HPW], xk, wkv, xv;
    if constexpr (PREP) {
        fr = a.inv_freq[min((int) threadIdx.x, MAXROT / 2 - 1)];
        wq = reinterpret_cast<const float4 *>(a.wq)[lane];
#pragma unroll
        for (int i = 0; i < HPW; ++i)
            xq[i] = reinterpret_cast<const float4 *>(a.qg + ((size_t) bt * a.nq + g * GRP + wave * HPW + i) * 2 * HD)[lane];
        const size_t kv = ((size_t) bt * a.nkv + g) * HD;
        xk = reinterpret_cast<const float4 *>(a.knew + kv)[lane];
        wkv = reinterpret_cast<const float4 *>(a.wk)[lane];
        xv = reinterpret_cast<const float4 *>(a.vnew + kv)[lane];
    }
    const int P = a.pos[b] + t;
    const int32_t *klist = LIST ? a.keys + (size_t) bt * a.kstride : nullptr;
    const int nk = LIST ? a.nkeys[bt] : min(P + 1, a.max_ctx);  // slots 0 .. nk-1 hold visible keys
    const int ntiles = (nk + TILE - 1) / TILE;
    const int per = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tile0 = sp_i * per, tile1 = min(tile0 + per, ntiles);
    const float scale = rsqrtf((float) HD);
    // the new key is visible (inside the cache) and its slot, the last one (nk - 1 = P for the dense walk, the end of
    // the tail for a key list), falls in this split's tiles
    const bool owner = PREP && P >= 0 && P < a.max_ctx && (nk - 1) / TILE >= tile0 && (nk - 1) / TILE < tile1;
    // a new token outside the cache is neither appended nor attended past the cache's end; record it once
    if (PREP && sp_i == 0 && g == 0 && threadIdx.x == 0 && (P < 0 || P >= a.max_ctx)) atomicOr(a.status, FN_STATUS_POS);

    if (PREP) {
        if (threadIdx.x < a.nrot / 2) {
            const float ang = (float) P * fr;  // fp32 angle (faie2fn.cu:1440)
            rcs[threadIdx.x] = cosf(ang);
            rsn[threadIdx.x] = sinf(ang);
        }
#pragma unroll
        for (int i = 0; i < HPW; ++i) qs[lane * GRP + wave * HPW + i] = rms_row(xq[i], wq, a.eps);
        kn4[lane] = rms_row(xk, wkv, a.eps);
        vn4[lane] = xv;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < HPW; ++i) rope_row_lds(qs + wave * HPW + i, GRP, lane, a.nrot, rcs, rsn);
        if (owner && wave == 0) rope_row_lds(kn4, 1, lane, a.nrot, rcs, rsn);
    } else {
        const float4 *Qg = reinterpret_cast<const float4 *>(a.Q + ((size_t) bt * a.nkv + g) * HD * GRP);
        for (int i = threadIdx.x; i < HD / 4 * GRP; i += WAVES * 64) qs[i] = Qg[i];
    }
    const float *Kbase = a.Kc + ((size_t) b * a.nkv + g) * a.max_ctx * HD;
    const float4 *Vbase = reinterpret_cast<const float4 *>(a.Vc + ((size_t) b * a.nkv + g) * a.max_ctx * HD);

    float m[HPW], l[HPW];  // softmax state of this wave's heads (wave-uniform m, per-lane partial l)
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
    }
    float4 o[GRP];
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) o[hh] = f4(0.0f);
    if (owner && wave == 0) {
        // append the new row to the caches; the barrier below orders these stores before every wave's tile loads,
        // so the new key is read back like any other
        const float4 k = kn4[lane];
        const float kk[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) a.Kc[k_index(a.max_ctx, b, a.nkv, g, P, 4 * lane + e)] = kk[e];
        reinterpret_cast<float4 *>(a.Vc + (((size_t) b * a.nkv + g) * a.max_ctx + P) * HD)[lane] = vn4[lane];
    }
    __syncthreads();

    for (int tile = tile0; tile < tile1; ++tile) {
        const int key0 = tile * TILE;
        float4 kf[CPW], vf[RPW];
        if (LIST) {  // gather: this lane's key from its 64-key tile of the key-tiled layout
            const int key = klist[min(key0 + lane, nk - 1)];
            const float4 *Kt = reinterpret_cast<const float4 *>(Kbase + (size_t) (key / TILE) * TILE * HD);
#pragma unroll
            for (int u = 0; u < CPW; ++u) kf[u] = ld_nt(&Kt[(wave * CPW + u) * TILE + (key % TILE)]);
#pragma unroll
            for (int u = 0; u < RPW; ++u) {
                const int row = klist[min(key0 + wave * RPW + u, nk - 1)];
                vf[u] = ld_nt(&Vbase[(size_t) row * (HD / 4) + lane]);
            }
        } else {
            const float4 *Kt = reinterpret_cast<const float4 *>(Kbase + (size_t) tile * TILE * HD);
#pragma unroll
            for (int u = 0; u < CPW; ++u) kf[u] = ld_nt(&Kt[(wave * CPW + u) * TILE + lane]);
#pragma unroll
            for (int u = 0; u < RPW; ++u) {
                const int row = min(key0 + wave * RPW + u, nk - 1);  // clamp past the last key: finite, weight 0
                vf[u] = ld_nt(&Vbase[(size_t) row * (HD / 4) + lane]);
            }
        }
        float s[GRP];
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) s[hh] = 0.0f;
#pragma unroll
        for (int u = 0; u < CPW; ++u) {
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh) {
                const float4 qv = qs[(wave * CPW + u) * GRP + hh];
                s[hh] = fmaf(qv.x, kf[u].x, s[hh]);
                s[hh] = fmaf(qv.y, kf[u].y, s[hh]);
                s[hh] = fmaf(qv.z, kf[u].z, s[hh]);
                s[hh] = fmaf(qv.w, kf[u].w, s[hh]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) sp[(wave * GRP + hh) * TILE + lane] = s[hh];
        __syncthreads();
        // online softmax of this wave's heads over the tile's keys (lane = key)
        const bool valid = key0 + lane < nk;
#pragma unroll
        for (int i = 0; i < HPW; ++i) {
            const int hh = wave * HPW + i;
            float sc = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) sc += sp[(w * GRP + hh) * TILE + lane];
            sc = valid ? sc * scale : -INFINITY;
            const float mn = fmaxf(m[i], wave_max(sc));  // finite: the tile holds >= 1 visible key
            const float corr = expf(m[i] - mn);           // 0 while m is -inf
            const float pr = valid ? expf(sc - mn) : 0.0f;
            l[i] = fmaf(l[i], corr, pr);
            m[i] = mn;
            pb[lane * GRP + hh] = pr;
            if (lane == 0) cr[hh] = corr;
        }
        __syncthreads();
        // p.V over this wave's 16 rows, every head
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
            const float c = cr[hh];
            o[hh].x *= c; o[hh].y *= c; o[hh].z *= c; o[hh].w *= c;
        }
#pragma unroll
        for (int u = 0; u < RPW; ++u) {
            const float *pj = pb + (wave * RPW + u) * GRP;
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh) {
                const float pr = pj[hh];
                o[hh].x = fmaf(pr, vf[u].x, o[hh].x);
                o[hh].y = fmaf(pr, vf[u].y, o[hh].y);
                o[hh].z = fmaf(pr, vf[u].z, o[hh].z);
                o[hh].w = fmaf(pr, vf[u].w, o[hh].w);
            }
        }
    }

    // all waves share each head's running max, so their o sum without rescaling
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        const float lw = wave_sum(l[i]);
        if (lane == 0) {
            mmax[wave * HPW + i] = m[i];
            msum[wave * HPW + i] = lw;
        }
    }
    __syncthreads();  // the walk's LDS is free
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) mo[(wave * GRP + hh) * (HD / 4) + lane] = o[hh];
    __syncthreads();
    const int d = threadIdx.x;
    const float *mof = reinterpret_cast<const float *>(mo);
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        float O = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) O += mof[(w * GRP + hh) * HD + d];
        const size_t pi = ((size_t) bt * a.nq + g * GRP + hh) * a.nsplit + sp_i;
        const bool empty = tile0 >= tile1;
        a.part_o[pi * HD + d] = empty ? 0.0f : O;
        if (d == 0) {
            a.part_ml[pi * 2] = empty ? -INFINITY : mmax[hh];
            a.part_ml[pi * 2 + 1] = empty ? 0.0f : msum[hh];
        }
    }
}

// ---- several new tokens per sequence (verify / chunked prefill): one K/V pass for all of them on the matrix cores
//
// For nt > 1 the nt * GRP query rows of a (sequence, kv head) form a small matrix (R = nt * GRP rows), so the work is
// two thin GEMMs per key block instead of R dot products, and every token reads the same K/V.  k_attn_split_mt reads
// each K/V byte of its split once for all R rows and runs the products on v_mfma_f32_16x16x4f32, in fp32 like the
// single-token kernel.  Both products are taken transposed so that one lane holds one query row throughout:
//   S^T[key][row] = sum_d K[key][d] Q[row][d]      A = K (lane: key l%16, dim slot l/16), B = Q (lane: row l%16)
//   O^T[d][row]  += sum_key V[key][d] P[row][key]  A = V (lane: dim l%16, key slot l/16), B = P (lane: row l%16)
// The S^T result leaves lane l with row l%16 and keys 4(l/16)..4(l/16)+3 of the 16-key block, which is exactly the
// B operand the P.V product needs (key slot l/16 of step s = key 4(l/16)+s), and the O^T result leaves lane l with row
// l%16 too, so the online-softmax rescale of O is a per-lane multiply with no data movement.  The contraction slots
// are free to permute as long as both operands agree: in S^T, step (u, e) pairs dim 16u + 4(l/16) + e of K (lane l
// reads 16-byte chunk 4u + l/16 of its key from the key-tiled cache) with the same dim of Q; in O^T, output tile
// (c, e) maps MFMA row i to dim 64c + 4i + e, so lane l's V load is one float4 (dims 64c + 4(l%16) ...) and its
// accumulators cover 16 consecutive dims 64c + 16(l/16) + 4r + e of its row.
// Work split: KW waves walk the split's 16-key blocks interleaved (wave kw takes blocks kw, kw + KW, ..., so the
// waves of a workgroup together stream whole 64-key tiles), each with its own softmax state, and RW row groups of
// NRW 16-row blocks cover the R rows; the KW partial states merge in LDS with the log-sum-exp identity at the end and
// the workgroup writes the same (m, l, o) partial per (token, head, split) as k_attn_split, for k_attn_combine.
// Token t (row r = t * GRP + h) sees keys < min(pos + t + 1, max_ctx) (faie2fn.cu:1609-1668 per query, causal over
// the new tokens).  One wave per SIMD (up to 512 registers; the O accumulators and the K operands live in AGPRs).
// One row block per wave (R <= 16): two 16-key blocks of K and V in flight while the other is multiplied.  Two row
// blocks: twice the products per block, so half a block in flight suffices, and the walk is software pipelined --
// the softmax step of block i is cut into stages woven between the score products of block i + 1.
// Measured on MI355X (B = 16, 32K context, 16 query / 2 kv heads): with the K/V loads made cache-resident the layer
// step is only 5-6 % faster, so the kernel is bound by the matrix cores and the instructions between them, not by
// HBM: at nt = 8 the products alone take 490 us at the 2.14 GHz this load runs at, the kernel ~700 us.  Two waves per
// SIMD with one row block each were slower (each wave loads K/V for its own 16 rows: twice the loads).
constexpr int MT_OS = HD + 4;  // LDS row stride (floats) of the merge buffer: a wave's 16 rows land on distinct banks
constexpr float MT_SLACK = 8.0f;  // growth of a row's max (natural-log units) that triggers a rescale
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// max / sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (swap16 / swap32: VALU lane swaps, the same bits in every lane)
__device__ __forceinline__ float max_x16_x32(float x) {
    float2 r = swap16(x);
    r = swap32(fmaxf(r.x, r.y));
    return fmaxf(r.x, r.y);
}
__device__ __forceinline__ float sum_x16_x32(float x) {
    float2 r = swap16(x);
    r = swap32(r.x + r.y);
    return r.x + r.y;
}

// K of the 16-key block starting at key kb: lane l takes 16-byte chunk 4u + l/16 of key kb + l%16 (keys past nkmax
// are clamped: finite values, masked later).  KEEP: an ordinary load, whose lines stay in the L2 for the other row
// group of the workgroup, which reads the same block (with the nontemporal hint the second read went back to HBM:
// 1.26x the K/V bytes at 8 new tokens); else nontemporal (each byte is read once).
template <bool KEEP> __device__ __forceinline__ float4 mt_ld(const float4 *p) { return KEEP ? *p : ld_nt(p); }
template <bool KEEP>
__device__ __forceinline__ void mt_load_k(float4 (&k)[16], const float4 *Kb, int kb, int nkmax, int lane) {
    const int key = min(kb + (lane & 15), nkmax - 1);
    const float4 *kt = Kb + (size_t) (key / TILE) * (TILE * HD / 4) + (key % TILE);
#pragma unroll
    for (int u = 0; u < 16; ++u) k[u] = mt_ld<KEEP>(kt + (4 * u + (lane >> 4)) * TILE);
}
// V of the block: v[4s + c] = dims 64c + 4(l%16) .. +3 of key kb + 4(l/16) + s
template <bool KEEP>
__device__ __forceinline__ void mt_load_v(float4 (&v)[16], const float4 *Vb, int kb, int nkmax, int lane) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int row = min(kb + 4 * (lane >> 4) + s, nkmax - 1);
        const float4 *vr = Vb + (size_t) row * (HD / 4) + (lane & 15);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[4 * s + c] = mt_ld<KEEP>(vr + 16 * c);
    }
}

// Scores of one 16-key block for this wave's NRW row blocks and the online-softmax step: p = probabilities (lane l:
// row l%16, keys kb + 4(l/16) + r), o rescaled to the new running max.
// S^T of one 16-key block for this wave's NRW row blocks (lane l: row l%16, keys 4(l/16) .. 4(l/16)+3 of the block).
// Q comes from LDS ([row block][u][lane] float4, lane l = row l%16, chunk 4u + l/16; ds_read_b128 of consecutive
// lanes is conflict-free), one u ahead: the reads of step u + 1 are in flight while the 4 * NRW products of step u
// run.  (Held in registers instead, Q would take 64 of the 256 VGPRs per row block that MFMA operands must come
// from, which two row blocks with their K and V block do not leave.)
template <int NRW>
__device__ __forceinline__ void mt_qk(const float4 (&k)[16], const float4 *qs, int lane, int kb, v4f (&S)[NRW]) {
    v4f s0[NRW], s1[NRW];
    float4 qc[NRW];
    // the read offset goes through an empty asm that also takes the block's first key: opaque and different per
    // block, so the compiler neither hoists the 64 * NRW registers of Q reads out of the walk nor orders them
    int qo = lane;
    asm("" : "+v"(qo) : "v"(kb));
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        s0[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        s1[j] = s0[j];
        qc[j] = qs[(j * 16) * 64 + qo];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        float4 qn[NRW];
#pragma unroll
        for (int j = 0; j < NRW; ++j) qn[j] = qs[(j * 16 + (u + 1) % 16) * 64 + qo];  // u = 15: a harmless re-read
#pragma unroll
        for (int j = 0; j < NRW; ++j) {
            v4f &acc = (u & 1) ? s1[j] : s0[j];
            acc = mfma4(k[u].x, qc[j].x, acc);
            acc = mfma4(k[u].y, qc[j].y, acc);
            acc = mfma4(k[u].z, qc[j].z, acc);
            acc = mfma4(k[u].w, qc[j].w, acc);
        }
#pragma unroll
        for (int j = 0; j < NRW; ++j) qc[j] = qn[j];
    }
#pragma unroll
    for (int j = 0; j < NRW; ++j) S[j] = s0[j] + s1[j];
}

// Online-softmax step of a block whose keys start at kb: p = probabilities of the lane's 4 keys against the row's
// reference max, corr = the factor o and l take (1 unless the reference moved).  The row keeps its reference until a
// block exceeds it by more than MT_SLACK, so p <= e^MT_SLACK and o is rescaled rarely (o / l and the split merge
// only need one reference per row).  exp(d) = 2^(d log2 e) on v_exp_f32: d <= MT_SLACK, and the two roundings
// before the exponential cost at most ~2e-6 relative on the smallest weights (|d| ~ 30), ~1e-7 near the max.
template <int NRW>
__device__ __forceinline__ void mt_softmax(const v4f (&S)[NRW], int kb, float (&m)[NRW], float (&l)[NRW],
                                           const int (&lim)[NRW], int lane, v4f (&p)[NRW], float (&corr)[NRW]) {
    constexpr float LOG2E = 1.4426950408889634f;
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        const float scale = rsqrtf((float) HD);
        const int key = kb + 4 * (lane >> 4);
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = key + r < lim[j] ? S[j][r] * scale : -INFINITY;
        // max over the row's 16 keys (lanes l, l^16, l^32, l^48)
        const float mx = max_x16_x32(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
        const bool first = m[j] == -INFINITY, moved = !first && mx > m[j] + MT_SLACK;
        const float mn = first || moved ? mx : m[j];
        corr[j] = moved ? __builtin_amdgcn_exp2f((m[j] - mn) * LOG2E) : 1.0f;  // o, l are 0 while no key was seen
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[j][r] = sc[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((sc[r] - mn) * LOG2E);
            ps += p[j][r];
        }
        l[j] = fmaf(l[j], corr[j], ps);
        m[j] = mn;
    }
}

// The softmax step of mt_softmax cut into 5 stages per row block (t = 5 j + stage), for interleaving with the next
// block's products; same arithmetic in the same order.
template <int NRW>
struct MtSoft {
    float sc[NRW][4], mx[NRW];
};
template <int NRW>
__device__ __forceinline__ void mt_soft_stage(int t, MtSoft<NRW> &st, const v4f (&S)[NRW], int kb, float (&m)[NRW],
                                              float (&l)[NRW], const int (&lim)[NRW], int lane, v4f (&p)[NRW],
                                              float (&corr)[NRW]) {
    constexpr float LOG2E = 1.4426950408889634f;
    const int j = t / 5, ph = t % 5;
    if (j >= NRW) return;
    if (ph == 0) {
        const float scale = rsqrtf((float) HD);
        const int key = kb + 4 * (lane >> 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) st.sc[j][r] = key + r < lim[j] ? S[j][r] * scale : -INFINITY;
        st.mx[j] = fmaxf(fmaxf(st.sc[j][0], st.sc[j][1]), fmaxf(st.sc[j][2], st.sc[j][3]));
    } else if (ph == 1) {
        const float2 r = swap16(st.mx[j]);
        st.mx[j] = fmaxf(r.x, r.y);
    } else if (ph == 2) {
        const float2 r = swap32(st.mx[j]);
        const float mx = fmaxf(r.x, r.y);
        const bool first = m[j] == -INFINITY, moved = !first && mx > m[j] + MT_SLACK;
        const float mn = first || moved ? mx : m[j];
        corr[j] = moved ? __builtin_amdgcn_exp2f((m[j] - mn) * LOG2E) : 1.0f;
        m[j] = mn;
    } else if (ph == 3) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
            p[j][r] = st.sc[j][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((st.sc[j][r] - m[j]) * LOG2E);
    } else {
#pragma unroll
        for (int r = 2; r < 4; ++r)
            p[j][r] = st.sc[j][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((st.sc[j][r] - m[j]) * LOG2E);
        l[j] = fmaf(l[j], corr[j], ((p[j][0] + p[j][1]) + p[j][2]) + p[j][3]);
    }
}

// mt_qk of the block at kbq into Sn, with the softmax step of the previous block (scores S, first key kb) woven in:
// stage u runs after the products of dim step u, fenced by scheduling barriers (this compiler otherwise puts all of
// the VALU work before or after the products, where nothing overlaps it).
template <int NRW>
__device__ __forceinline__ void mt_qk_soft(const float4 (&k)[16], const float4 *qs, int lane, int kbq, v4f (&Sn)[NRW],
                                           const v4f (&S)[NRW], int kb, float (&m)[NRW], float (&l)[NRW],
                                           const int (&lim)[NRW], v4f (&p)[NRW], float (&corr)[NRW]) {
    MtSoft<NRW> st;
    v4f s0[NRW], s1[NRW];
    float4 qc[NRW];
    int qo = lane;
    asm("" : "+v"(qo) : "v"(kbq));
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        s0[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        s1[j] = s0[j];
        qc[j] = qs[(j * 16) * 64 + qo];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        float4 qn[NRW];
#pragma unroll
        for (int j = 0; j < NRW; ++j) qn[j] = qs[(j * 16 + (u + 1) % 16) * 64 + qo];
#pragma unroll
        for (int j = 0; j < NRW; ++j) {
            v4f &acc = (u & 1) ? s1[j] : s0[j];
            acc = mfma4(k[u].x, qc[j].x, acc);
            acc = mfma4(k[u].y, qc[j].y, acc);
            acc = mfma4(k[u].z, qc[j].z, acc);
            acc = mfma4(k[u].w, qc[j].w, acc);
        }
#pragma unroll
        for (int j = 0; j < NRW; ++j) qc[j] = qn[j];
        __builtin_amdgcn_sched_barrier(0);
        mt_soft_stage<NRW>(u, st, S, kb, m, l, lim, lane, p, corr);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < NRW; ++j) Sn[j] = s0[j] + s1[j];
}

template <int NRW>
__device__ __forceinline__ void mt_rescale(v4f (&o)[NRW][16], const float (&corr)[NRW]) {
    bool rescale = false;
#pragma unroll
    for (int j = 0; j < NRW; ++j) rescale |= corr[j] != 1.0f;
    if (__builtin_amdgcn_ballot_w64(rescale)) {  // x * 1.0f == x: the rows that kept their reference are unchanged
#pragma unroll
        for (int j = 0; j < NRW; ++j)
#pragma unroll
            for (int t = 0; t < 16; ++t) o[j][t] *= corr[j];
    }
}

// o += V^T P^T for one block
template <int NRW>
__device__ __forceinline__ void mt_pv(const float4 (&v)[16], const v4f (&p)[NRW], v4f (&o)[NRW][16]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int j = 0; j < NRW; ++j) {
                o[j][4 * c + 0] = mfma4(v[4 * s + c].x, p[j][s], o[j][4 * c + 0]);
                o[j][4 * c + 1] = mfma4(v[4 * s + c].y, p[j][s], o[j][4 * c + 1]);
                o[j][4 * c + 2] = mfma4(v[4 * s + c].z, p[j][s], o[j][4 * c + 2]);
                o[j][4 * c + 3] = mfma4(v[4 * s + c].w, p[j][s], o[j][4 * c + 3]);
            }
}

// scores, softmax step and P.V of one block, in sequence
template <int NRW>
__device__ __forceinline__ void mt_block(const float4 (&k)[16], const float4 (&v)[16], int kb, const float4 *qs,
                                         v4f (&o)[NRW][16], float (&m)[NRW], float (&l)[NRW], const int (&lim)[NRW],
                                         int lane) {
    v4f S[NRW], p[NRW];
    float corr[NRW];
    mt_qk<NRW>(k, qs, lane, kb, S);
    mt_softmax<NRW>(S, kb, m, l, lim, lane, p, corr);
    mt_rescale<NRW>(o, corr);
    mt_pv<NRW>(v, p, o);
}

// grid (nsplit, nkv, B), RW * KW <= 4 waves; dynamic LDS: max(RW * NRW * 16 KiB of Q, RW * KW * 16 * MT_OS * 4 B);
// KEEP = RW > 1 (row groups share each block through the L2)
template <int NRW, bool KEEP>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_attn_split_mt(const AttnArgs a, int grp, int RW, int KW) {
    extern __shared__ float4 mt_lds[];
    __shared__ float2 mls[WAVES][NRW * 16];
    const int sp_i = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nth = RW * KW * 64, rw = wave / KW, kw = wave - rw * KW;
    const int R = a.nt * grp;
    const int P0 = a.pos[b];
    const int nkmax = min(P0 + a.nt, a.max_ctx);  // keys visible to the last token
    const int ntiles = nkmax > 0 ? (nkmax + TILE - 1) / TILE : 0;
    const int per = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tile0 = min(sp_i * per, ntiles), tile1 = min(tile0 + per, ntiles);
    const int k0 = tile0 * TILE, k1 = min(tile1 * TILE, nkmax);
    const int nblk = k1 > k0 ? (k1 - k0 + 15) / 16 : 0;
    const int nw = nblk > kw ? (nblk - 1 - kw) / KW + 1 : 0;  // this wave's blocks

    // Q of all row blocks into LDS: [row block][u][lane] float4, lane l = (row l%16, chunk 4u + l/16); rows >= R zero
    const float4 *Qg = reinterpret_cast<const float4 *>(a.Q);
    for (int i = tid; i < RW * NRW * 1024; i += nth) {
        const int rb = i >> 10, u = (i >> 6) & 15, l = i & 63;
        const int row = rb * 16 + (l & 15), c = 4 * u + (l >> 4);
        float4 qv = f4(0.0f);
        if (row < R) {
            const int t = row / grp, h = row - t * grp;
            qv = Qg[(((size_t) (b * a.nt + t) * a.nkv + g) * (HD / 4) + c) * grp + h];
        }
        mt_lds[i] = qv;
    }
    __syncthreads();
    const float4 *qs = mt_lds + rw * NRW * 1024;
    const float4 *Kb = reinterpret_cast<const float4 *>(a.Kc + ((size_t) b * a.nkv + g) * a.max_ctx * HD);
    const float4 *Vb = reinterpret_cast<const float4 *>(a.Vc + ((size_t) b * a.nkv + g) * a.max_ctx * HD);
    v4f o[NRW][16];
    float m[NRW], l[NRW];
    int lim[NRW];
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
        const int t = min(((rw * NRW + j) * 16 + (lane & 15)) / grp, a.nt - 1);
        lim[j] = min(min(P0 + t + 1, a.max_ctx), k1);
#pragma unroll
        for (int t2 = 0; t2 < 16; ++t2) o[j][t2] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (nw > 0 && NRW == 1) {
        // one row block: two whole blocks in flight (pairs of blocks; an odd count gets one block past k1, fully
        // masked, to keep the loop free of conditionals, which keeps the wait counts exact: A's loads are awaited
        // while B's 32 are still in flight)
        const int npair = (nw + 1) / 2;
        float4 ka[16], va[16], kb2[16], vb2[16];
        mt_load_k<KEEP>(ka, Kb, k0 + kw * 16, nkmax, lane);
        mt_load_v<KEEP>(va, Vb, k0 + kw * 16, nkmax, lane);
        mt_load_k<KEEP>(kb2, Kb, k0 + (kw + KW) * 16, nkmax, lane);
        mt_load_v<KEEP>(vb2, Vb, k0 + (kw + KW) * 16, nkmax, lane);
        int pr = 0;
        for (; pr + 1 < npair; ++pr) {
            const int kb = k0 + (kw + 2 * pr * KW) * 16;
            mt_block<NRW>(ka, va, kb, qs, o, m, l, lim, lane);
            mt_load_k<KEEP>(ka, Kb, kb + 2 * KW * 16, nkmax, lane);
            mt_load_v<KEEP>(va, Vb, kb + 2 * KW * 16, nkmax, lane);
            mt_block<NRW>(kb2, vb2, kb + KW * 16, qs, o, m, l, lim, lane);
            mt_load_k<KEEP>(kb2, Kb, kb + 3 * KW * 16, nkmax, lane);
            mt_load_v<KEEP>(vb2, Vb, kb + 3 * KW * 16, nkmax, lane);
        }
        const int kb = k0 + (kw + 2 * pr * KW) * 16;
        mt_block<NRW>(ka, va, kb, qs, o, m, l, lim, lane);
        mt_block<NRW>(kb2, vb2, kb + KW * 16, qs, o, m, l, lim, lane);
    } else if (nw > 0) {
        // two row blocks: twice the products per block, so half a block in flight hides the load latency -- the
        // next block's K is requested once its predecessor's scores are done, its V once P.V is done.  Software
        // pipelined: the softmax step of block i (VALU) sits next to the scores of block i + 1 (MFMA) so the two can
        // overlap; the scheduling barriers keep each load where the pipeline puts it (hoisted above the products that
        // still read the previous block, it would hold two blocks' registers at once and spill).
        float4 kf[16], vf[16];
        v4f S[NRW];
        auto kbl = [&](int i) { return k0 + (kw + i * KW) * 16; };  // first key of this wave's block i
        mt_load_k<KEEP>(kf, Kb, kbl(0), nkmax, lane);
        mt_load_v<KEEP>(vf, Vb, kbl(0), nkmax, lane);
        mt_qk<NRW>(kf, qs, lane, kbl(0), S);
        __builtin_amdgcn_sched_barrier(0);
        mt_load_k<KEEP>(kf, Kb, kbl(1), nkmax, lane);  // past the wave's last block when nw = 1: in bounds, unused
        __builtin_amdgcn_sched_barrier(0);
        int i = 0;
        for (; i + 1 < nw; ++i) {
            v4f p[NRW];
            float corr[NRW];
            v4f Sn[NRW];
            mt_qk_soft<NRW>(kf, qs, lane, kbl(i + 1), Sn, S, kbl(i), m, l, lim, p, corr);
#pragma unroll
            for (int j = 0; j < NRW; ++j) S[j] = Sn[j];
            __builtin_amdgcn_sched_barrier(0);
            mt_load_k<KEEP>(kf, Kb, kbl(i + 2), nkmax, lane);
            __builtin_amdgcn_sched_barrier(0);
            mt_rescale<NRW>(o, corr);
            mt_pv<NRW>(vf, p, o);
            __builtin_amdgcn_sched_barrier(0);
            mt_load_v<KEEP>(vf, Vb, kbl(i + 1), nkmax, lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        v4f p[NRW];
        float corr[NRW];
        mt_softmax<NRW>(S, kbl(i), m, l, lim, lane, p, corr);
        mt_rescale<NRW>(o, corr);
        mt_pv<NRW>(vf, p, o);
    }

    // merge the KW key streams of each row group (log-sum-exp), then write the split partials
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        l[j] = sum_x16_x32(l[j]);
        if (lane < 16) mls[wave][j * 16 + lane] = make_float2(m[j], l[j]);
    }
    __syncthreads();  // Q is dead: the LDS becomes the merge buffer
    float *ob = reinterpret_cast<float *>(mt_lds);
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        {
            const int row = lane & 15;
            float M = -INFINITY;
            for (int w = 0; w < KW; ++w) M = fmaxf(M, mls[rw * KW + w][j * 16 + row].x);
            const float sc = m[j] == -INFINITY ? 0.0f : expf(m[j] - M);
            float *dst = ob + (wave * 16 + row) * MT_OS + 16 * (lane >> 4);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<float4 *>(dst + 64 * c + 4 * q) =
                        make_float4(o[j][4 * c][q] * sc, o[j][4 * c + 1][q] * sc, o[j][4 * c + 2][q] * sc,
                                    o[j][4 * c + 3][q] * sc);
        }
        __syncthreads();
        for (int i = tid; i < RW * 16 * 64; i += nth) {
            const int rg = i >> 10, row = (i >> 6) & 15, d4 = i & 63;
            const int rowg = (rg * NRW + j) * 16 + row;
            if (rowg < R) {
                float4 O = f4(0.0f);
                for (int w = 0; w < KW; ++w) {
                    const float4 x = *reinterpret_cast<const float4 *>(ob + ((rg * KW + w) * 16 + row) * MT_OS + 4 * d4);
                    O.x += x.x; O.y += x.y; O.z += x.z; O.w += x.w;
                }
                const int t = rowg / grp, h = rowg - t * grp;
                const size_t pi = ((size_t) (b * a.nt + t) * a.nq + g * grp + h) * a.nsplit + sp_i;
                reinterpret_cast<float4 *>(a.part_o + pi * HD)[d4] = O;
                if (d4 == 0) {
                    float M = -INFINITY, L = 0.0f;
                    for (int w = 0; w < KW; ++w) M = fmaxf(M, mls[rg * KW + w][j * 16 + row].x);
                    for (int w = 0; w < KW; ++w) {
                        const float2 ml = mls[rg * KW + w][j * 16 + row];
                        if (ml.x != -INFINITY) L = fmaf(expf(ml.x - M), ml.y, L);
                    }
                    a.part_ml[pi * 2] = M;
                    a.part_ml[pi * 2 + 1] = L;
                }
            }
        }
        __syncthreads();
    }
}

// merge splits + sigmoid output gate (faie2fn.cu:1670-1690).  grid (nq, B nt), cw * 64 threads, 4 <= cw <= CW.
// Wave w takes splits w, w + cw, ...; lane l owns dims 4l..4l+3 (one coalesced 1 KiB row per split) with NB rows in
// flight.  The first NB rows of every wave, their (m, l) and the gate are all requested at the start, before the
// global max M over the splits is known, so a merge of up to cw * NB splits costs one memory round trip; the waves'
// sums meet in LDS.  The host sizes cw to the split count (combine_waves), so a merge of few splits does not hold
// 16 waves.
constexpr int CW = 16, CNB = 8;
int combine_waves(int nsplit) { return std::min(CW, std::max(4, (nsplit + CNB - 1) / CNB)); }
__global__ void __launch_bounds__(CW * 64) k_attn_combine(const AttnArgs a) {
    constexpr int NB = CNB;
    __shared__ float red[CW];
    __shared__ float4 acc[CW][HD / 4];
    __shared__ float lsum[CW];
    const int h = blockIdx.x, bt = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cw = blockDim.x >> 6;
    const int ns = a.nsplit;
    const size_t base = ((size_t) bt * a.nq + h) * ns;
    const float *ml = a.part_ml + base * 2;
    const float4 *po = reinterpret_cast<const float4 *>(a.part_o + base * HD);
    const float gate = tid < HD ? a.qg[(((size_t) bt * a.nq + h) * 2 + 1) * HD + tid] : 0.0f;
    float4 v[NB];
    float mv[NB], lv[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int s = min(wave + cw * u, ns - 1);
        v[u] = ld_nt(&po[(size_t) s * (HD / 4) + lane]);
        mv[u] = ml[2 * s];
        lv[u] = ml[2 * s + 1];
    }
    float M = -INFINITY;
    for (int s = tid; s < ns; s += cw * 64) M = fmaxf(M, ml[2 * s]);
    M = wave_max(M);
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int w = 1; w < cw; ++w) M = fmaxf(M, red[w]);
    float4 O = f4(0.0f);
    float L = 0.0f;
    for (int s0 = wave;;) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            // splits without keys (m = -inf) and the clamped repeats past the end weigh 0
            const float w = (s0 + cw * u < ns && mv[u] != -INFINITY) ? expf(mv[u] - M) : 0.0f;
            L = fmaf(w, w != 0.0f ? lv[u] : 0.0f, L);
            O.x = fmaf(w, v[u].x, O.x);
            O.y = fmaf(w, v[u].y, O.y);
            O.z = fmaf(w, v[u].z, O.z);
            O.w = fmaf(w, v[u].w, O.w);
        }
        s0 += cw * NB;
        if (s0 >= ns) break;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int s = min(s0 + cw * u, ns - 1);
            v[u] = ld_nt(&po[(size_t) s * (HD / 4) + lane]);
            mv[u] = ml[2 * s];
            lv[u] = ml[2 * s + 1];
        }
    }
    acc[wave][lane] = O;
    if (lane == 0) lsum[wave] = L;
    __syncthreads();
    if (tid < HD) {
        const float *af = reinterpret_cast<const float *>(acc);
        float Lt = 0.0f, Ot = 0.0f;
#pragma unroll
        for (int w = 0; w < cw; ++w) {
            Lt += lsum[w];
            Ot += af[w * HD + tid];
        }
        a.og[((size_t) bt * a.nq + h) * HD + tid] = (Ot / Lt) * sigmoidf_(gate);
    }
}

__global__ void k_advance(int32_t *pos, int B, int nt) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) pos[b] += nt;
}

__global__ void k_advance_by(int32_t *pos, const int32_t *kr, int B) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) pos[b] += kr[b];
}

}  // namespace

size_t attn_work_bytes(int B, int nq, int nt, int hd, int nsplit) {
    const size_t bt = (size_t) B * nt;
    const size_t q = bt * nq * hd, po = bt * nq * nsplit * hd, pm = bt * nq * nsplit * 2;
    return (q + po + pm) * sizeof(float) + 256;
}

// One new token: about 512 workgroups in all (two per CU at the split kernel's occupancy); a context of 256 tiles or
// more keeps at least 4 tiles per workgroup (fewer, larger splits: less partial traffic for the combine), a shorter
// one goes as wide as one tile per workgroup (latency-bound).  Measured on MI355X (B, L -> best nsplit): 1, 4K -> 64;
// 1, 32K -> 128; 1, 128K -> 256; 16, 32K -> 16.
// Several new tokens: k_attn_split_mt's grid has no token dimension and holds one workgroup per CU, so one
// workgroup per CU in all.
int attn_pick_nsplit(int B, int nkv, int nt, int ctx) {
    const int tiles = std::max(1, (ctx + TILE - 1) / TILE);
    if (nt > 1) {
        const long groups = std::max(1L, (long) B * nkv), cus = device_cus();
        return (int) std::max(1L, std::min<long>((cus + groups - 1) / groups, tiles));
    }
    const long groups = std::max(1L, (long) B * nkv);
    long want = std::max(1L, (512 + groups - 1) / groups);
    if (tiles >= 256) want = std::min<long>(want, tiles / 4);
    return (int) std::max(1L, std::min<long>(want, tiles));
}

int attn_decode_launch(const AttnDecode &p, hipStream_t st) {
    if (p.B < 1 || p.nt < 1 || p.nq < 1 || p.nkv < 1) FN_FAIL("attn: B, nt, nq and nkv must be >= 1");
    if (p.hd != HD) FN_FAIL("attn: only head_dim 256 is built");
    if (p.nq % p.nkv) FN_FAIL("attn: nq must be a multiple of nkv");
    if (p.nrot < 0 || p.nrot > std::min(HD, MAXROT) || (p.nrot & 1)) FN_FAIL("attn: nrot must be even and <= 128");
    if (p.max_ctx < TILE || p.max_ctx % TILE) FN_FAIL("attn: max_ctx must be a positive multiple of 64");
    if (p.nsplit < 1) FN_FAIL("attn: nsplit must be >= 1");
    if (!p.pos || !p.qg || !p.k || !p.v || !p.wq || !p.wk || !p.Kc || !p.Vc || !p.work || !p.og)
        FN_FAIL("attn: null pointer");
    if (p.work_bytes < attn_work_bytes(p.B, p.nq, p.nt, p.hd, p.nsplit)) FN_FAIL("attn: workspace too small");
    const int grp = p.nq / p.nkv;
    AttnArgs a{};
    a.B = p.B; a.nq = p.nq; a.nkv = p.nkv; a.nt = p.nt; a.max_ctx = p.max_ctx; a.nsplit = p.nsplit;
    a.nrot = p.nrot; a.eps = p.eps; a.pos = p.pos; a.qg = p.qg; a.knew = p.k; a.vnew = p.v; a.wq = p.wq;
    a.wk = p.wk; a.Kc = p.Kc; a.Vc = p.Vc; a.og = p.og;
    if (p.status) a.status = p.status;
    else if (status_word(&a.status)) return -1;
    const size_t bt = (size_t) p.B * p.nt;
    a.Q = p.work;
    a.part_o = a.Q + bt * p.nq * HD;
    a.part_ml = a.part_o + bt * p.nq * p.nsplit * HD;
    // inv_freq[i] = (float)(1 / theta^(2i/nrot)) computed in double, as the reference (faie2fn.cu:2573-2576)
    for (int i = 0; i < p.nrot / 2; ++i)
        a.inv_freq[i] = (float) (1.0 / std::pow((double) p.theta, (double) (2 * i) / p.nrot));
    if (bt > 65535u * 65535u) FN_FAIL("attn: batch too large");
    const dim3 sg(p.nsplit, p.nkv, (unsigned) bt), sb(WAVES * 64);
    if (grp != 4 && grp != 8 && grp != 12) FN_FAIL("attn: query heads per kv head must be 4, 8 or 12");
    // one new token per sequence: the split kernel does the norm/RoPE/append itself (one launch fewer); several
    // tokens see each other's new keys, so they go through k_attn_prep first
    const bool fused = p.nt == 1;
    if (!fused) {
        hipLaunchKernelGGL(k_attn_prep, dim3((unsigned) bt, p.nq + p.nkv), dim3(HD), 0, st, a);
        stage_mark(st);
    }
    const int nr = (p.nt * grp + 15) / 16;  // 16-row blocks of the multi-token query matrix
    if (fused) {
        if (grp == 8) hipLaunchKernelGGL((k_attn_split<8, true>), sg, sb, 0, st, a);
        else if (grp == 12) hipLaunchKernelGGL((k_attn_split<12, true>), sg, sb, 0, st, a);
        else hipLaunchKernelGGL((k_attn_split<4, true>), sg, sb, 0, st, a);
    } else if (nr <= 8 && p.B <= 65535) {
        // rows in groups of NRW 16-row blocks (RW groups), KW key streams per group, at most 4 waves
        const int nrw = nr == 1 ? 1 : 2, rw = (nr + nrw - 1) / nrw, kw = std::max(1, WAVES / rw);
        const size_t lds = std::max((size_t) rw * nrw * 16 * HD * 4, (size_t) rw * kw * 16 * MT_OS * 4);
        const dim3 mg(p.nsplit, p.nkv, p.B), mb(rw * kw * 64);
        if (nrw == 1) hipLaunchKernelGGL((k_attn_split_mt<1, false>), mg, mb, lds, st, a, grp, rw, kw);
        else if (rw == 1) hipLaunchKernelGGL((k_attn_split_mt<2, false>), mg, mb, lds, st, a, grp, rw, kw);
        else hipLaunchKernelGGL((k_attn_split_mt<2, true>), mg, mb, lds, st, a, grp, rw, kw);
    } else {
        if (grp == 8) hipLaunchKernelGGL((k_attn_split<8, false>), sg, sb, 0, st, a);
        else if (grp == 12) hipLaunchKernelGGL((k_attn_split<12, false>), sg, sb, 0, st, a);
        else hipLaunchKernelGGL((k_attn_split<4, false>), sg, sb, 0, st, a);
    }
    stage_mark(st);
    hipLaunchKernelGGL(k_attn_combine, dim3(p.nq, (unsigned) bt), dim3(combine_waves(p.nsplit) * 64), 0, st, a);
    stage_mark(st);
    FN_CK(hipGetLastError());
    return 0;
}

size_t attn_qsa_work_bytes(int B, int nq, int nt, int hd, int nsplit, int max_ctx, int top) {
    return attn_work_bytes(B, nq, nt, hd, nsplit) + qsa_work_bytes(B, nt, max_ctx, top);
}

int attn_qsa_launch(const AttnDecode &p, const QsaIndexer &ix, hipStream_t st) {
    if (p.B != ix.B || p.nt != ix.nt || p.max_ctx != ix.max_ctx || p.pos != ix.pos)
        FN_FAIL("attn_qsa: the attention and indexer shapes disagree");
    if (p.B < 1 || p.nt < 1 || p.nq < 1 || p.nkv < 1) FN_FAIL("attn: B, nt, nq and nkv must be >= 1");
    if (p.hd != HD) FN_FAIL("attn: only head_dim 256 is built");
    if (p.nq % p.nkv) FN_FAIL("attn: nq must be a multiple of nkv");
    if (p.nrot < 0 || p.nrot > std::min(HD, MAXROT) || (p.nrot & 1)) FN_FAIL("attn: nrot must be even and <= 128");
    if (p.nsplit < 1) FN_FAIL("attn: nsplit must be >= 1");
    if (!p.pos || !p.qg || !p.k || !p.v || !p.wq || !p.wk || !p.Kc || !p.Vc || !p.work || !p.og)
        FN_FAIL("attn: null pointer");
    const size_t aw = attn_work_bytes(p.B, p.nq, p.nt, p.hd, p.nsplit);
    if (p.work_bytes < attn_qsa_work_bytes(p.B, p.nq, p.nt, p.hd, p.nsplit, p.max_ctx, ix.top))
        FN_FAIL("attn_qsa: workspace too small");
    const int grp = p.nq / p.nkv;
    if (grp != 4 && grp != 8 && grp != 12) FN_FAIL("attn: query heads per kv head must be 4, 8 or 12");
    const int32_t *keys = nullptr, *nkeys = nullptr;
    float *iwork = reinterpret_cast<float *>(reinterpret_cast<char *>(p.work) + (aw + 255) / 256 * 256);
    if (qsa_select_launch(ix, iwork, p.work_bytes - (aw + 255) / 256 * 256, &keys, &nkeys, st)) return -1;
    AttnArgs a{};
    a.B = p.B; a.nq = p.nq; a.nkv = p.nkv; a.nt = p.nt; a.max_ctx = p.max_ctx; a.nsplit = p.nsplit;
    a.nrot = p.nrot; a.eps = p.eps; a.pos = p.pos; a.qg = p.qg; a.knew = p.k; a.vnew = p.v; a.wq = p.wq;
    a.wk = p.wk; a.Kc = p.Kc; a.Vc = p.Vc; a.og = p.og;
    a.keys = keys; a.nkeys = nkeys; a.kstride = ix.top * 4 + 4;
    if (p.status) a.status = p.status;
    else if (status_word(&a.status)) return -1;
    const size_t bt = (size_t) p.B * p.nt;
    a.Q = p.work;
    a.part_o = a.Q + bt * p.nq * HD;
    a.part_ml = a.part_o + bt * p.nq * p.nsplit * HD;
    for (int i = 0; i < p.nrot / 2; ++i)
        a.inv_freq[i] = (float) (1.0 / std::pow((double) p.theta, (double) (2 * i) / p.nrot));
    const dim3 sg(p.nsplit, p.nkv, (unsigned) bt), sb(WAVES * 64);
    if (p.nt == 1) {  // q norm + RoPE and the K/V append folded into the split kernel
        if (grp == 8) hipLaunchKernelGGL((k_attn_split<8, true, true>), sg, sb, 0, st, a);
        else if (grp == 12) hipLaunchKernelGGL((k_attn_split<12, true, true>), sg, sb, 0, st, a);
        else hipLaunchKernelGGL((k_attn_split<4, true, true>), sg, sb, 0, st, a);
    } else {
        hipLaunchKernelGGL(k_attn_prep, dim3((unsigned) bt, p.nq + p.nkv), dim3(HD), 0, st, a);
        stage_mark(st);
        if (grp == 8) hipLaunchKernelGGL((k_attn_split<8, false, true>), sg, sb, 0, st, a);
        else if (grp == 12) hipLaunchKernelGGL((k_attn_split<12, false, true>), sg, sb, 0, st, a);
        else hipLaunchKernelGGL((k_attn_split<4, false, true>), sg, sb, 0, st, a);
    }
    stage_mark(st);
    hipLaunchKernelGGL(k_attn_combine, dim3(p.nq, (unsigned) bt), dim3(combine_waves(p.nsplit) * 64), 0, st, a);
    stage_mark(st);
    FN_CK(hipGetLastError());
    return 0;
}

int advance_launch(int32_t *pos, int B, int nt, hipStream_t st) {
    if (!pos || B < 1) FN_FAIL("advance: bad arguments");
    hipLaunchKernelGGL(k_advance, dim3((B + 255) / 256), dim3(256), 0, st, pos, B, nt);
    FN_CK(hipGetLastError());
    return 0;
}

int advance_by_launch(int32_t *pos, const int32_t *kr, int B, hipStream_t st) {
    if (!pos || !kr || B < 1) FN_FAIL("advance_by: bad arguments");
    hipLaunchKernelGGL(k_advance_by, dim3((B + 255) / 256), dim3(256), 0, st, pos, kr, B);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

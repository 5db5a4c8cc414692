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
//   * K and V are read with the nontemporal hint and in batches of 16 loads per lane, so every wave keeps
//     16 KiB in flight (the first version waited on each V row and spent ~40 HBM latencies per tile).
//   * Each wave runs its own online softmax (running max per head via DPP/permlane wave max); the four waves
//     merge in LDS and write one (m, l, o[hd]) partial per query head per split.
//   * The combine kernel merges the splits with the log-sum-exp identity and applies o / L * sigmoid(gate).
// Device cache layouts (max_ctx a multiple of 64):
//   Kc: [B][nkv][max_ctx / 64][hd / 4][64][4]   Vc: [B][nkv][max_ctx][hd]
#include "gdn.h"

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
    if (P < 0 || P >= a.max_ctx) return;  // outside the cache: the host checks positions; never write past it
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
// Each wave walks its tiles; per tile the K reads go out in batches of 16 x 16 bytes per lane and the V rows in
// batches of 16 coalesced 1 KiB rows, so a wave keeps 16 KiB of loads in flight instead of waiting on each one.
template <int GRP> __global__ void __launch_bounds__(WAVES * 64) k_attn_split(const AttnArgs a) {
    constexpr int NB = GRP > 8 ? 8 : 16;            // loads in flight per lane per batch
    // LDS: q of the group and the per-wave tile probabilities while walking; the per-wave partials for the
    // merge afterwards (same bytes)
    constexpr int WALK = HD / 4 * GRP * 16 + WAVES * TILE * GRP * 4, MERGE = WAVES * GRP * HD * 4;
    __shared__ __align__(16) unsigned char smem[WALK > MERGE ? WALK : MERGE];
    __shared__ float mm[WAVES][GRP], ml[WAVES][GRP];
    float4 *qs = reinterpret_cast<float4 *>(smem);                                  // [HD/4][GRP]
    float *pb = reinterpret_cast<float *>(smem + HD / 4 * GRP * 16);                // [WAVES][TILE][GRP]
    float4 *mo = reinterpret_cast<float4 *>(smem);                                  // [WAVES][GRP][HD/4]

    const int sp = blockIdx.x, g = blockIdx.y, bt = blockIdx.z, b = bt / a.nt, t = bt - b * a.nt;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nk = min(a.pos[b] + t + 1, a.max_ctx);  // keys 0 .. nk-1 are visible
    const int ntiles = (nk + TILE - 1) / TILE;
    const int per = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tile0 = sp * per, tile1 = min(tile0 + per, ntiles);
    const float scale = rsqrtf((float) HD);  // 1/16 at HD = 256 (faie2fn.cu:1646)

    const float4 *Qg = reinterpret_cast<const float4 *>(a.Q + ((size_t) bt * a.nkv + g) * HD * GRP);
    for (int i = threadIdx.x; i < HD / 4 * GRP; i += WAVES * 64) qs[i] = Qg[i];
    __syncthreads();
    const float *Kbase = a.Kc + ((size_t) b * a.nkv + g) * a.max_ctx * HD;
    const float4 *Vbase = reinterpret_cast<const float4 *>(a.Vc + ((size_t) b * a.nkv + g) * a.max_ctx * HD);
    float *pw = pb + wave * TILE * GRP;

    float m[GRP], l[GRP];
    float4 o[GRP];
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
        o[hh] = f4(0.0f);
    }

    for (int tile = tile0 + wave; tile < tile1; tile += WAVES) {
        const int key0 = tile * TILE;
        const bool valid = key0 + lane < nk;
        // scores: lane = key; K read as 16-byte chunks of the key-tiled layout (coalesced 1 KiB per wave load),
        // q as LDS broadcasts
        const float4 *Kt = reinterpret_cast<const float4 *>(Kbase + (size_t) tile * TILE * HD);
        float s[GRP];
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) s[hh] = 0.0f;
        for (int cb = 0; cb < HD / 4; cb += NB) {
            float4 kf[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) kf[u] = ld_nt(&Kt[(cb + u) * TILE + lane]);
#pragma unroll
            for (int u = 0; u < NB; ++u) {
#pragma unroll
                for (int hh = 0; hh < GRP; ++hh) {
                    const float4 qv = qs[(cb + u) * GRP + hh];
                    s[hh] = fmaf(qv.x, kf[u].x, s[hh]);
                    s[hh] = fmaf(qv.y, kf[u].y, s[hh]);
                    s[hh] = fmaf(qv.z, kf[u].z, s[hh]);
                    s[hh] = fmaf(qv.w, kf[u].w, s[hh]);
                }
            }
        }
        // online softmax update (faie2fn.cu:1648-1663), one running max per head per wave
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
            const float sc = valid ? s[hh] * scale : -INFINITY;
            const float mn = fmaxf(m[hh], wave_max(sc));  // finite: the tile holds >= 1 visible key
            const float corr = expf(m[hh] - mn);           // 0 while m is -inf
            const float pr = valid ? expf(sc - mn) : 0.0f;
            l[hh] = fmaf(l[hh], corr, pr);
            o[hh].x *= corr; o[hh].y *= corr; o[hh].z *= corr; o[hh].w *= corr;
            m[hh] = mn;
            pw[lane * GRP + hh] = pr;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // p.V: lane = 4 output dims, one coalesced V row per key.  Rows past the last visible key are clamped to
        // it (finite data, probability 0) so a batch never branches per key.
        const int nj = min(TILE, nk - key0);
        for (int jb = 0; jb < nj; jb += NB) {
            float4 vf[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int row = min(key0 + jb + u, nk - 1);
                vf[u] = ld_nt(&Vbase[(size_t) row * (HD / 4) + lane]);
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const float *pj = pw + (jb + u) * GRP;
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
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // merge the waves (the walk's LDS is reused for the per-wave partials)
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        const float lw = wave_sum(l[hh]);
        if (lane == 0) {
            mm[wave][hh] = m[hh];
            ml[wave][hh] = lw;
        }
        mo[(wave * GRP + hh) * (HD / 4) + lane] = o[hh];
    }
    __syncthreads();
    const int d = threadIdx.x;  // WAVES * 64 == HD
    const float *mof = reinterpret_cast<const float *>(mo);
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, mm[w][hh]);
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float e = expf(mm[w][hh] - M);  // 0 for an idle wave
                L = fmaf(e, ml[w][hh], L);
                O = fmaf(e, mof[(w * GRP + hh) * HD + d], O);
            }
        }
        const size_t pi = ((size_t) bt * a.nq + g * GRP + hh) * a.nsplit + sp;
        a.part_o[pi * HD + d] = O;
        if (d == 0) {
            a.part_ml[pi * 2] = M;
            a.part_ml[pi * 2 + 1] = L;
        }
    }
}

// merge splits + sigmoid output gate (faie2fn.cu:1670-1690).  grid (nq, B nt), CW * 64 threads.
// Pass 1: the global max M over the splits' maxima.  Pass 2: wave w takes splits w, w + CW, ...; lane l owns dims
// 4l..4l+3 (one coalesced 1 KiB row per split) with NB rows in flight; the waves' sums meet in LDS.
constexpr int CW = 16;
__global__ void __launch_bounds__(CW * 64) k_attn_combine(const AttnArgs a) {
    constexpr int NB = 8;
    __shared__ float red[CW];
    __shared__ float4 acc[CW][HD / 4];
    __shared__ float lsum[CW];
    const int h = blockIdx.x, bt = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int ns = a.nsplit;
    const size_t base = ((size_t) bt * a.nq + h) * ns;
    const float *ml = a.part_ml + base * 2;
    float M = -INFINITY;
    for (int s = tid; s < ns; s += CW * 64) M = fmaxf(M, ml[2 * s]);
    M = wave_max(M);
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int w = 1; w < CW; ++w) M = fmaxf(M, red[w]);
    const float4 *po = reinterpret_cast<const float4 *>(a.part_o + base * HD);
    float4 O = f4(0.0f);
    float L = 0.0f;
    for (int s0 = wave; s0 < ns; s0 += CW * NB) {
        float4 v[NB];
        float w[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int s = min(s0 + CW * u, ns - 1);
            v[u] = ld_nt(&po[(size_t) s * (HD / 4) + lane]);
            const float m = ml[2 * s];
            // splits without keys (m = -inf) and the clamped repeats past the end weigh 0
            w[u] = (s0 + CW * u < ns && m != -INFINITY) ? expf(m - M) : 0.0f;
            L = fmaf(w[u], w[u] != 0.0f ? ml[2 * s + 1] : 0.0f, L);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            O.x = fmaf(w[u], v[u].x, O.x);
            O.y = fmaf(w[u], v[u].y, O.y);
            O.z = fmaf(w[u], v[u].z, O.z);
            O.w = fmaf(w[u], v[u].w, O.w);
        }
    }
    acc[wave][lane] = O;
    if (lane == 0) lsum[wave] = L;
    __syncthreads();
    if (tid < HD) {
        const float *af = reinterpret_cast<const float *>(acc);
        float Lt = 0.0f, Ot = 0.0f;
#pragma unroll
        for (int w = 0; w < CW; ++w) {
            Lt += lsum[w];
            Ot += af[w * HD + tid];
        }
        const float gate = a.qg[(((size_t) bt * a.nq + h) * 2 + 1) * HD + tid];
        a.og[((size_t) bt * a.nq + h) * HD + tid] = (Ot / Lt) * sigmoidf_(gate);
    }
}

__global__ void k_advance(int32_t *pos, int B, int nt) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) pos[b] += nt;
}

}  // namespace

size_t attn_work_bytes(int B, int nq, int nt, int hd, int nsplit) {
    const size_t bt = (size_t) B * nt;
    const size_t q = bt * nq * hd, po = bt * nq * nsplit * hd, pm = bt * nq * nsplit * 2;
    return (q + po + pm) * sizeof(float) + 256;
}

int attn_pick_nsplit(int B, int nkv, int nt, int ctx) {
    const int tiles = std::max(1, (ctx + TILE - 1) / TILE);
    const int most = std::max(1, (tiles + WAVES - 1) / WAVES);  // at least one tile per wave
    const long groups = std::max(1L, (long) B * nt * nkv);
    const int want = (int) std::max(1L, (1024 + groups - 1) / groups);
    return std::min(want, most);
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
    const size_t bt = (size_t) p.B * p.nt;
    a.Q = p.work;
    a.part_o = a.Q + bt * p.nq * HD;
    a.part_ml = a.part_o + bt * p.nq * p.nsplit * HD;
    // inv_freq[i] = (float)(1 / theta^(2i/nrot)) computed in double, as the reference (faie2fn.cu:2573-2576)
    for (int i = 0; i < p.nrot / 2; ++i)
        a.inv_freq[i] = (float) (1.0 / std::pow((double) p.theta, (double) (2 * i) / p.nrot));
    if (bt > 65535u * 65535u) FN_FAIL("attn: batch too large");
    hipLaunchKernelGGL(k_attn_prep, dim3((unsigned) bt, p.nq + p.nkv), dim3(HD), 0, st, a);
    switch (grp) {
        case 8: hipLaunchKernelGGL(k_attn_split<8>, dim3(p.nsplit, p.nkv, (unsigned) bt), dim3(WAVES * 64), 0, st, a); break;
        case 12: hipLaunchKernelGGL(k_attn_split<12>, dim3(p.nsplit, p.nkv, (unsigned) bt), dim3(WAVES * 64), 0, st, a); break;
        case 4: hipLaunchKernelGGL(k_attn_split<4>, dim3(p.nsplit, p.nkv, (unsigned) bt), dim3(WAVES * 64), 0, st, a); break;
        default: FN_FAIL("attn: query heads per kv head must be 4, 8 or 12");
    }
    hipLaunchKernelGGL(k_attn_combine, dim3(p.nq, (unsigned) bt), dim3(CW * 64), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

int advance_launch(int32_t *pos, int B, int nt, hipStream_t st) {
    if (!pos || B < 1) FN_FAIL("advance: bad arguments");
    hipLaunchKernelGGL(k_advance, dim3((B + 255) / 256), dim3(256), 0, st, pos, B, nt);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

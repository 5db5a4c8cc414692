// Model engine: fn_load reads a FAIE2-FlashNext GGUF and places it on one GPU; fn_forward runs nt <= 8 tokens of one
// sequence through the whole model and returns logits and the argmax token.
//
// The reference's model forward (engine/faie2fn.cu:1937-2031 Engine, 2370-2490 layer_forward / enqueue / forward,
// 2524-2696 fn_load) on its two GPUs, rebuilt on one MI355X: every layer on device 0, one stream, one hipGraph per
// token count.  Per layer (faie2fn.cu:2370-2420):
//   hyper-connection read  hn = RMSNorm_s(h) (per stream), lr = W_down+inject . hn, t = silu(lr / HC),
//                          a = W_up . t, x = (1/HC) sum_s sigmoid(a_s) hn_s, inj_s = 2 sigmoid(lr_inject,s / HC)
//                          (faie2fn.cu:1246-1273, 860-888, 2350-2359)
//   mixer                  DeltaNet: GEMV qkv / z / alpha-beta, the fused DeltaNet block, GEMV ssm_out;
//                          attention: GEMV q / k / v / indexer, QSA sparse attention, GEMV o
//   hyper-connection write h_s += y * inj_s, then hn = RMSNorm_s(h) for the next read (faie2fn.cu:1281-1327)
//   hyper-connection read  (FFN)
//   MoE                    router + shared-gate GEMV; the routed experts' SwiGLU rows, whose kernel also does the
//                          softmax top-k routing and the shared expert's SwiGLU (faie2fn.cu:1747-1798); down rows,
//                          the shared expert's down GEMV
//   hyper-connection write with y = sum_k w_k down_k + sigmoid(shared gate) shared down (faie2fn.cu:1298-1318)
// then the final hyper-connection read (no inject), the LM head GEMV and the argmax (lowest index on ties,
// faie2fn.cu:1910-1934).  The layers listed in <arch>.ple.layers first add the per-layer n-gram embedding
// (faie2fn.cu:1805-1896, 2373-2381): the bigram and trigram contexts of each position hash into rows of a table of
// IQ4_NL rows (per_layer_token_embd, 27 GB in the reference model's second shard, kept here in HBM where the
// reference maps it from pinned host memory); key and value GEMVs of the gathered row, a per-stream signed-sqrt
// gate, and a dilated causal conv (kernel 4, dilation 3) of the gated value feed the residual streams.  Shapes come
// from the GGUF metadata (the reference fixes them at build time and asserts them at load, faie2fn.cu:2532-2535); the
// kernels fix head_dim 256, DeltaNet head dim 128, the indexer's 4 x 128 and blocks of 4 keys.
#include "engine.h"
#include "gguf.h"
#include "model.h"
#include "qsa.h"
#include "quant.h"

#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

namespace fn {

namespace {

constexpr int MAXT = 8;                      // tokens per forward (faie2fn.cu:67)
constexpr int HDK = 256, DSK = 128;          // attention head dim, DeltaNet head dim (built sizes)
constexpr int IXH = 4, IXD = 128, IXR = 4;   // indexer heads, head dim, keys per block (built sizes)
constexpr int RING = 16;                     // conv ring slots (>= MAXT + 3, a power of two)
constexpr int PLE_HIST = 9;                  // PLE conv history: (kernel 4 - 1) x dilation 3 (faie2fn.cu:66)
constexpr int PLE_MAXH = 64;                 // n-gram heads the hashing kernel takes
constexpr int HC_KS = 4;                     // split of the hyper-connection down product along its rows
constexpr int UPMIX_U = 8;                   // 8-value chunks per lane of the fused up-and-mix kernel (HCR <= 512)
constexpr int UPMIX_HC = 8;                  // streams the fused up-and-mix kernel takes (HC <= 8)
constexpr int UPMIX_ROWS = 64;               // rows of the up weight per workgroup of the fused up-and-mix kernel

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// sum over a workgroup of nw waves (wave sums, then wave 0 adds the nw partials in wave order); every thread returns
// the sum.  red: nw floats of LDS.  Call from uniform control flow.
__device__ __forceinline__ float block_sum(float v, float *red, int nw) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

// RMSNorm of each of the HC streams: out[t][s D + c] = h * rsqrt(mean_c h^2 + eps) * w[s D + c] (faie2fn.cu:1226-1239).
// grid (nt, HC), 256 threads.  The sum of squares has the order of k_hc_add's and of the fused write + norm + down
// kernel's (thread tid: float4 tid, tid + 256, ... in order, sumsq4 each; then the wave sums in wave order), so
// every path gives the same bits.
__global__ void __launch_bounds__(256) k_groupnorm(const float *__restrict__ h, const float *__restrict__ w, int D,
                                                    float eps, float *__restrict__ out) {
    __shared__ float red[4];
    const size_t base = ((size_t) blockIdx.x * gridDim.y + blockIdx.y) * D;
    const float4 *h4 = reinterpret_cast<const float4 *>(h + base);
    float ss = 0.0f;
    for (int c = threadIdx.x; c < D / 4; c += 256) ss += sumsq4(h4[c]);
    const float r = rsqrtf(block_sum(ss, red, 4) / D + eps);
    const float4 *w4 = reinterpret_cast<const float4 *>(w + (size_t) blockIdx.y * D);
    float4 *o4 = reinterpret_cast<float4 *>(out + base);
    for (int c = threadIdx.x; c < D / 4; c += 256) {
        const float4 v = h4[c], wv = w4[c];
        o4[c] = make_float4(v.x * r * wv.x, v.y * r * wv.y, v.z * r * wv.z, v.w * r * wv.w);
    }
}

// sum of the ks split-K partials of the down (+ inject) product, in split order: part[k][t][r], ldr values a token
__device__ __forceinline__ float lr_sum(const float *__restrict__ part, int ks, int nt, int ldr, int t, int r) {
    float v = part[(size_t) t * ldr + r];
    for (int k = 1; k < ks; ++k) v += part[((size_t) k * nt + t) * ldr + r];
    return v;
}

// t[t][r] = silu(lr[t][r] / HC) for r < HCR (faie2fn.cu:1266-1273), lr the sum of the ks partials; the inject
// logits stay in the partials.  grid nt, 256 threads
__global__ void k_hc_lowrank(const float *__restrict__ lr, int ks, int nt, int ldr, int HCR, int HC,
                             float *__restrict__ t320) {
    const int t = blockIdx.x;
    for (int r = threadIdx.x; r < HCR; r += blockDim.x)
        t320[(size_t) t * HCR + r] = silu(lr_sum(lr, ks, nt, ldr, t, r) * (1.0f / HC));
}

// x[t][c] = (sum_s sigmoid(a[t][s D + c]) hn[t][s D + c]) / HC (streams in order), and, with inject logits,
// inj[t][s] = 2 sigmoid(lr[t][HCR + s] / HC) (faie2fn.cu:873-888).  grid (nt, ceil(D / 256)), 256 threads
__global__ void k_hc_mix(const float *__restrict__ a, const float *__restrict__ hn, int D, int HC,
                         const float *__restrict__ lr, int ks, int nt, int ldr, int HCR, float *__restrict__ x,
                         float *__restrict__ inj) {
    const int t = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x;
    if (c < D) {
        float s = 0.0f;
        for (int k = 0; k < HC; ++k) {
            const size_t i = (size_t) t * HC * D + (size_t) k * D + c;
            s += sigm(a[i]) * hn[i];
        }
        x[(size_t) t * D + c] = s / HC;
    }
    if (inj && blockIdx.y == 0 && (int) threadIdx.x < HC)
        inj[t * HC + threadIdx.x] = 2.0f * sigm(lr_sum(lr, ks, nt, ldr, t, HCR + threadIdx.x) / HC);
}

// The up product and the mix in one pass, for a BF16 up weight U [HC D][HCR] (the reference model's): the
// low-rank activation tt[t][r] = silu(lr[t][r] / HC) goes to the LDS, each row of U is summed by 8 lanes (lane li
// takes the 8-value chunks li, li + 8, ... in order, then a 3-step xor tree), and the workgroup's UPMIX_ROWS rows
// are the HC streams of UPMIX_ROWS / HC columns, so it finishes x for them:
// x[t][c] = (sum_s sigmoid(U[s D + c] . tt[t]) hn[t][s D + c]) / HC, streams in order; workgroup 0 also writes
// inj.  Replaces k_hc_lowrank + the up GEMV + k_hc_mix (faie2fn.cu:1266-1273, 873-888).
// grid ceil(D HC / UPMIX_ROWS), 8 UPMIX_ROWS threads, LDS nt HCR + 8 UPMIX_ROWS floats
__global__ void __launch_bounds__(UPMIX_ROWS * 8)
    k_hc_upmix(const uint8_t *__restrict__ U, size_t urs, const float *__restrict__ lr, int ks, int nt, int ldr,
               int HCR, int HC, int D, const float *__restrict__ hn, float *__restrict__ x, float *__restrict__ inj) {
    extern __shared__ float sm[];
    float *tt = sm, *as = sm + nt * HCR;  // tt [nt][HCR], as [nt][UPMIX_ROWS]
    const int tid = threadIdx.x, cpb = UPMIX_ROWS / HC, c0 = blockIdx.x * cpb;
    const int ri = tid >> 3, li = tid & 7, cc = ri / HC, s = ri - cc * HC, c = c0 + cc;
    const int nq = HCR / 8;
    // the lane's weight chunks li + 8 u, u < UPMIX_U, requested first: they do not depend on the activation
    const bool live = c < D;
    uint4 wq[UPMIX_U];
    if (live) {
        const uint4 *row = reinterpret_cast<const uint4 *>(U + ((size_t) s * D + c) * urs);
#pragma unroll
        for (int u = 0; u < UPMIX_U; ++u) wq[u] = row[min(li + 8 * u, nq - 1)];
    }
    // the mix's normalised streams, requested now as well (thread tid < cpb nt finishes column c0 + tid % cpb of
    // token tid / cpb)
    float hv[UPMIX_HC];
    const int mt = tid / cpb, mc = c0 + (tid - mt * cpb);
    const bool mixer = tid < cpb * nt && mc < D;
#pragma unroll
    for (int k = 0; k < UPMIX_HC; ++k)
        hv[k] = mixer && k < HC ? hn[(size_t) mt * HC * D + (size_t) k * D + mc] : 0.0f;
    for (int i = tid; i < nt * HCR; i += UPMIX_ROWS * 8) {
        const int t = i / HCR, r = i - t * HCR;
        tt[i] = silu(lr_sum(lr, ks, nt, ldr, t, r) * (1.0f / HC));
    }
    __syncthreads();
    float acc[MAXT];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) acc[t] = 0.0f;
    if (live) {
#pragma unroll
        for (int u = 0; u < UPMIX_U; ++u) {
            const int j = li + 8 * u;
            if (j >= nq) break;
            const uint4 w = wq[u];
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
            float wf[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wf[2 * e] = __uint_as_float(wv[e] << 16);
                wf[2 * e + 1] = __uint_as_float(wv[e] & 0xFFFF0000u);
            }
#pragma unroll
            for (int t = 0; t < MAXT; ++t) {
                if (t < nt) {
                    const float4 x0 = *reinterpret_cast<const float4 *>(tt + t * HCR + 8 * j);
                    const float4 x1 = *reinterpret_cast<const float4 *>(tt + t * HCR + 8 * j + 4);
                    float a = acc[t];
                    a = __builtin_fmaf(wf[0], x0.x, a);
                    a = __builtin_fmaf(wf[1], x0.y, a);
                    a = __builtin_fmaf(wf[2], x0.z, a);
                    a = __builtin_fmaf(wf[3], x0.w, a);
                    a = __builtin_fmaf(wf[4], x1.x, a);
                    a = __builtin_fmaf(wf[5], x1.y, a);
                    a = __builtin_fmaf(wf[6], x1.z, a);
                    a = __builtin_fmaf(wf[7], x1.w, a);
                    acc[t] = a;
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
        if (t < nt) {
            // the 8 lanes of a row: quad sums by DPP quad_perm (xor 1, xor 2), then lane 0 of the row adds lane 4's
            // (row_ror by n reads lane l - n of the 16-lane DPP row, so ror 12 reads l + 4: lane 0 gets lane 4,
            // lane 8 gets lane 12, each from its own 8-lane row)
            float v = acc[t];
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf,
                                                                       false));
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf,
                                                                       false));
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x12C, 0xf, 0xf,
                                                                       false));
            if (li == 0) as[t * UPMIX_ROWS + ri] = v;
        }
    }
    __syncthreads();
    if (mixer) {
        const int cx = mc - c0;
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < UPMIX_HC; ++k)
            if (k < HC) sum += sigm(as[mt * UPMIX_ROWS + cx * HC + k]) * hv[k];
        x[(size_t) mt * D + mc] = sum / HC;
    }
    if (inj && blockIdx.x == 0 && tid < nt * HC) {
        const int t = tid / HC, k = tid - t * HC;
        inj[t * HC + k] = 2.0f * sigm(lr_sum(lr, ks, nt, ldr, t, HCR + k) / HC);
    }
}

// hyper-connection write (faie2fn.cu:1281-1327): h[t][s][c] += yv[c] * inj[t][s], where yv = y, or for the MoE
// yv = sum_k wsel[t][k] dpart[t NEU + k][c] + sigmoid(rsg[t][NE]) y[t][c]; then (norm non-null)
// hn[t][s][c] = RMSNorm of the new stream s (the sum of squares in k_groupnorm's order).  grid (nt, HC), 256
// threads
__global__ void __launch_bounds__(256) k_hc_add(float *__restrict__ h, const float *__restrict__ y,
                                                 const float *__restrict__ inj, int D, int HC,
                                                 const float *__restrict__ dpart, const float *__restrict__ wsel,
                                                 int NEU, const float *__restrict__ rsg, int NE,
                                                 const float *__restrict__ norm, float eps, float *__restrict__ hn) {
    __shared__ float red[4];
    const int t = blockIdx.x, s = blockIdx.y, D4 = D / 4;
    float4 *hp = reinterpret_cast<float4 *>(h + ((size_t) t * HC + s) * D);
    const float4 *y4 = reinterpret_cast<const float4 *>(y + (size_t) t * D);
    const float is = inj[t * HC + s];
    const float sg = dpart ? sigm(rsg[(size_t) t * (NE + 1) + NE]) : 0.0f;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < D4; c += blockDim.x) {
        float4 yv = y4[c];
        if (dpart) {
            float4 m = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 *dp = reinterpret_cast<const float4 *>(dpart + (size_t) t * NEU * D) + c;
            for (int k = 0; k < NEU; ++k) {
                const float wk = wsel[t * NEU + k];
                const float4 d = dp[(size_t) k * D4];
                m.x += wk * d.x;
                m.y += wk * d.y;
                m.z += wk * d.z;
                m.w += wk * d.w;
            }
            yv = make_float4(m.x + sg * yv.x, m.y + sg * yv.y, m.z + sg * yv.z, m.w + sg * yv.w);
        }
        const float4 v = add_scaled(hp[c], yv, is);
        hp[c] = v;
        ss += sumsq4(v);
    }
    if (!norm) return;  // (uniform)
    const float r = rsqrtf(block_sum(ss, red, blockDim.x >> 6) / D + eps);
    float4 *op = reinterpret_cast<float4 *>(hn + ((size_t) t * HC + s) * D);
    const float4 *w4 = reinterpret_cast<const float4 *>(norm + (size_t) s * D);
    for (int c = threadIdx.x; c < D4; c += blockDim.x) {
        const float4 v = hp[c], w = w4[c];
        op[c] = make_float4(v.x * r * w.x, v.y * r * w.y, v.z * r * w.z, v.w * r * w.w);
    }
}

// routing for calls of several tokens (one call of one token routes inside the experts' gate/up kernel; both use
// route_pick, so the picks and weights are the same bits) and the shared expert's SwiGLU sha[t][r] = silu(shg) shu.
// grid nt, 256 threads (wave 0 routes, the other waves do the SwiGLU)
__global__ void __launch_bounds__(256) k_route(const float *__restrict__ rsg, int NE, int NEU,
                                               const float *__restrict__ shg, const float *__restrict__ shu, int FFS,
                                               int32_t *__restrict__ sel, float *__restrict__ wsel,
                                               float *__restrict__ sha) {
    const int t = blockIdx.x, tid = threadIdx.x;
    if (tid >= 64) {
        for (int r = tid - 64; r < FFS; r += 192) {
            const float g = shg[(size_t) t * FFS + r];
            sha[(size_t) t * FFS + r] = g / (1.0f + expf(-g)) * shu[(size_t) t * FFS + r];
        }
        return;
    }
    route_pick(rsg + (size_t) t * (NE + 1), NE, NEU, 0, sel + t * NEU, wsel + t * NEU);
}

// argmax of each token's logits, lowest index on ties (faie2fn.cu:1910-1934), in two passes: AM_CH chunks per
// token each leave their (value, index) (index V when no logit in the chunk beats -inf), then one wave merges them
constexpr int AM_CH = 128;
// grid (nt, AM_CH), 256 threads
__global__ void __launch_bounds__(256) k_argmax_part(const float *__restrict__ logits, int V, float *__restrict__ pv,
                                                     int32_t *__restrict__ pi) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int t = blockIdx.x, ch = blockIdx.y, per = (V + AM_CH - 1) / AM_CH;
    const int lo = ch * per, hi = min(V, lo + per);
    const float *l = logits + (size_t) t * V;
    float v = -INFINITY;
    int idx = V;
    for (int i = lo + threadIdx.x; i < hi; i += 256)
        if (l[i] > v) {
            v = l[i];
            idx = i;
        }
    wave_argmax(v, idx);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[w] = v;
        bi[w] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k) vi_max(v, idx, bv[k], bi[k]);
        pv[t * AM_CH + ch] = v;
        pi[t * AM_CH + ch] = idx;
    }
}

// grid nt, 64 threads
__global__ void k_argmax_merge(const float *__restrict__ pv, const int32_t *__restrict__ pi, int V,
                               int32_t *__restrict__ out) {
    const int t = blockIdx.x;
    float v = -INFINITY;
    int idx = V;
    for (int k = threadIdx.x; k < AM_CH; k += 64) vi_max(v, idx, pv[t * AM_CH + k], pi[t * AM_CH + k]);
    wave_argmax(v, idx);
    if (threadIdx.x == 0) out[t] = idx == V ? 0 : idx;
}

// tok_all[pos + t] = ids[t]: the token history the n-gram hashing reads (faie2fn.cu:1899-1903).  1 block
__global__ void k_store_tokens(const int32_t *__restrict__ ids, int32_t *__restrict__ tok_all,
                               const int32_t *__restrict__ pos, int nt, int max_ctx) {
    const int t = threadIdx.x, p = *pos + t;
    if (t < nt && p >= 0 && p < max_ctx) tok_all[p] = ids[t];
}

struct PleHash {
    unsigned long long mult[3], size[PLE_MAXH], off[PLE_MAXH];
};

// table rows of the n-gram heads of position pos + t (faie2fn.cu:1810-1823): head hd hashes the bigram (token,
// previous) and, for the second half of the heads, the trigram; contexts do not reach back across an EOS.
// grid nt, 64 threads
__global__ void k_ple_ids(const int32_t *__restrict__ tok_all, const int32_t *__restrict__ pos, int nheads, int eos,
                          const PleHash hsh, int32_t *__restrict__ rows) {
    const int t = blockIdx.x, hd = threadIdx.x;
    if (hd >= nheads) return;
    const int p = *pos + t;
    // ids widen to 64 bits with their sign, products wrap modulo 2^64 (the reference's unsigned long long arithmetic)
    const unsigned long long t0 = (unsigned long long) (long long) tok_all[p];
    const int p1 = p >= 1 ? tok_all[p - 1] : eos;
    const int p2 = (p >= 2 && p1 != eos) ? tok_all[p - 2] : eos;
    unsigned long long mixed = (t0 * hsh.mult[0]) ^ ((unsigned long long) (long long) p1 * hsh.mult[1]);
    if (hd >= nheads / 2) mixed ^= (unsigned long long) (long long) p2 * hsh.mult[2];
    rows[t * nheads + hd] = (int32_t) (mixed % hsh.size[hd] + hsh.off[hd]);
}

// per stream s (faie2fn.cu:1843-1875): gate = <RMSNorm(key_s) wk, RMSNorm(h_s) wq> / sqrt(D), signed square root
// (magnitude floored at 1e-6); gv = sigmoid(gate) * val; gvn = RMSNorm(gv) wc.  One thread per 4 columns, every
// input requested at the start.  grid (nt, HC), min(1024, D / 4 rounded up to 64) threads
__global__ void __launch_bounds__(1024) k_ple_gate(const float *__restrict__ key, const float *__restrict__ val,
                                                   const float *__restrict__ h, const float *__restrict__ wk,
                                                   const float *__restrict__ wq, const float *__restrict__ wc, int D,
                                                   float eps, float *__restrict__ gv, float *__restrict__ gvn) {
    __shared__ float red[16];
    const int t = blockIdx.x, s = blockIdx.y, HC = gridDim.y, D4 = D / 4, nw = blockDim.x >> 6;
    const size_t base = ((size_t) t * HC + s) * D;
    const float4 *kt = reinterpret_cast<const float4 *>(key + base), *ht = reinterpret_cast<const float4 *>(h + base);
    const float4 *vt = reinterpret_cast<const float4 *>(val + (size_t) t * D);
    const float4 *wk4 = reinterpret_cast<const float4 *>(wk + (size_t) s * D);
    const float4 *wq4 = reinterpret_cast<const float4 *>(wq + (size_t) s * D);
    const float4 *wc4 = reinterpret_cast<const float4 *>(wc + (size_t) s * D);
    float4 *gv4 = reinterpret_cast<float4 *>(gv + base), *gvn4 = reinterpret_cast<float4 *>(gvn + base);
    float sk = 0.0f, sq = 0.0f;
    for (int c = threadIdx.x; c < D4; c += blockDim.x) {
        const float4 k = kt[c], x = ht[c];
        sk += k.x * k.x + k.y * k.y + k.z * k.z + k.w * k.w;
        sq += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    }
    sk = block_sum(sk, red, nw);
    sq = block_sum(sq, red, nw);
    const float rk = rsqrtf(sk / D + eps), rq = rsqrtf(sq / D + eps);
    float dot = 0.0f;
    for (int c = threadIdx.x; c < D4; c += blockDim.x) {
        const float4 k = kt[c], x = ht[c], a = wk4[c], b = wq4[c];
        dot += (k.x * rk * a.x) * (x.x * rq * b.x) + (k.y * rk * a.y) * (x.y * rq * b.y) +
               (k.z * rk * a.z) * (x.z * rq * b.z) + (k.w * rk * a.w) * (x.w * rq * b.w);
    }
    dot = block_sum(dot, red, nw);
    float gate = dot / sqrtf((float) D);
    gate = gate == 0.0f ? 0.0f : copysignf(sqrtf(fmaxf(fabsf(gate), 1e-6f)), gate);
    const float sg = sigm(gate);
    float sv = 0.0f;
    for (int c = threadIdx.x; c < D4; c += blockDim.x) {
        const float4 v = vt[c];
        const float4 x = make_float4(sg * v.x, sg * v.y, sg * v.z, sg * v.w);
        gv4[c] = x;
        sv += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    }
    sv = block_sum(sv, red, nw);
    const float rv = rsqrtf(sv / D + eps);
    for (int c = threadIdx.x; c < D4; c += blockDim.x) {
        const float4 x = gv4[c], w = wc4[c];
        gvn4[c] = make_float4(x.x * rv * w.x, x.y * rv * w.y, x.z * rv * w.z, x.w * rv * w.w);
    }
}

// dilated causal depthwise conv (kernel 4, dilation 3) over gvn with its history, SiLU, then h += gv + conv; the
// history keeps the last 9 gvn of every channel (faie2fn.cu:1878-1896).  grid ceil(n / 256), 256 threads
__global__ void k_ple_conv(float *__restrict__ h, const float *__restrict__ gv, const float *__restrict__ gvn,
                           float *__restrict__ hist, const float *__restrict__ w, int n, int nt) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    float x[PLE_HIST + MAXT];
#pragma unroll
    for (int i = 0; i < PLE_HIST; ++i) x[i] = hist[(size_t) i * n + c];
    for (int t = 0; t < nt; ++t) x[PLE_HIST + t] = gvn[(size_t) t * n + c];
    const float w0 = w[c * 4 + 0], w1 = w[c * 4 + 1], w2 = w[c * 4 + 2], w3 = w[c * 4 + 3];
    for (int t = 0; t < nt; ++t) {
        const int i = PLE_HIST + t;
        const float sv = w0 * x[i - 9] + w1 * x[i - 6] + w2 * x[i - 3] + w3 * x[i];
        h[(size_t) t * n + c] += gv[(size_t) t * n + c] + silu(sv);
    }
    for (int i = 0; i < PLE_HIST; ++i) hist[(size_t) i * n + c] = x[nt + i];
}

// ------------------------------------------------------------------------------------------------------------

struct QW {
    QLayout L;
    uint8_t *p = nullptr;
};

struct MLayer {
    bool attn = false;
    float *hca_norm = nullptr, *hcf_norm = nullptr;
    QW hca_dinj, hca_up, hcf_dinj, hcf_up;
    // DeltaNet
    QW qkv, z, ab, ssm_out;
    float *conv_w = nullptr, *dt = nullptr, *ssm_a = nullptr, *ssm_norm = nullptr, *S = nullptr, *ring = nullptr;
    // attention
    QW q, k, v, o, ixqk;
    float *qn = nullptr, *kn = nullptr, *ixqn = nullptr, *ixkn = nullptr;
    float *Kc = nullptr, *Vc = nullptr, *IKc = nullptr, *BKc = nullptr;
    // FFN
    QW rsg, sh_gate, sh_up, sh_down, eg, eu, ed;
    // per-layer n-gram embedding
    bool ple = false;
    QW ple_key, ple_val;
    float *ple_nk = nullptr, *ple_nq = nullptr, *ple_nc = nullptr, *ple_conv = nullptr, *ple_hist = nullptr;
};

struct Model {
    ModelDims d;
    int max_ctx = 0, nsplit = 1;
    Gguf g, g2;  // the model, and the optional second shard (the n-gram table)
    QW ple_table;
    PleHash hsh{};
    int32_t *tok_all = nullptr, *ple_rows = nullptr;
    float *ple_emb = nullptr, *ple_k = nullptr, *ple_v = nullptr, *ple_gv = nullptr, *ple_gvn = nullptr;
    std::vector<MLayer> L;
    QW tok, head, out_down, out_up;
    float *out_norm = nullptr;
    // activations, MAXT tokens
    // h: the residual streams; h2: the other buffer of the pair a fused write moves them to
    float *h = nullptr, *h2 = nullptr, *hb[2] = {}, *hn = nullptr, *lr = nullptr, *t320 = nullptr, *a = nullptr;
    float *x = nullptr, *inj = nullptr;
    float *qkv = nullptr, *zz = nullptr, *abv = nullptr, *on = nullptr, *qg = nullptr, *kk = nullptr, *vv = nullptr;
    float *iqk = nullptr, *og = nullptr, *y = nullptr, *rsgv = nullptr, *shg = nullptr, *shu = nullptr, *sha = nullptr;
    float *shd = nullptr, *act = nullptr, *dpart = nullptr, *wsel = nullptr, *logits = nullptr, *work = nullptr;
    float *amv = nullptr;
    int32_t *ids = nullptr, *sel = nullptr, *pos = nullptr, *am = nullptr, *ami = nullptr;
    size_t work_bytes = 0;
    hipStream_t st = nullptr;
    // pinned host staging of one call's token ids, argmax ids and the status word (an asynchronous copy from or to
    // pageable memory is a blocking one), and the status word's device address
    int32_t *h_ids = nullptr, *h_am = nullptr;
    unsigned *h_status = nullptr, *status = nullptr;
    void *host = nullptr;
    hipGraphExec_t graph[MAXT + 1] = {};
    bool use_graphs = true;
    float *dbg = nullptr;  // host [NL][nt][HC D] when set
    int n_past = 0;
    double last_ms = 0;
    std::vector<void *> allocs;
    size_t bytes = 0;

    ~Model() {
        if (st) (void) hipStreamSynchronize(st);
        for (auto &ge : graph)
            if (ge) (void) hipGraphExecDestroy(ge);
        for (void *p : allocs) (void) hipFree(p);
        if (host) (void) hipHostFree(host);
        if (st) (void) hipStreamDestroy(st);
    }
    template <typename T> int alloc(T **p, size_t n) {
        const size_t nb = std::max<size_t>(n * sizeof(T), 16);
        const hipError_t e = hipMalloc((void **) p, nb);
        if (e != hipSuccess) {
            *p = nullptr;
            FN_FAIL("load: hipMalloc(" + std::to_string(nb) + " B) -> " + hipGetErrorString(e));
        }
        allocs.push_back((void *) *p);
        bytes += nb;
        FN_CK(hipMemset(*p, 0, nb));
        return 0;
    }
};

std::unique_ptr<Model> g_model;

// ---- load ----

int need(const Model &m, const std::string &name, const GTensor **t) {
    *t = m.g.find(name);
    if (!*t && m.g2.base) *t = m.g2.find(name);
    if (!*t) FN_FAIL("load: tensor " + name + " missing");
    return 0;
}

// shape of a 2-D weight (ggml order: ne[0] = columns) or a 3-D expert stack (ne[2] experts of ne[1] rows)
int check_shape(const std::string &name, const GTensor *t, uint64_t cols, uint64_t rows, uint64_t n3 = 1) {
    if (t->ne[0] != cols || t->ne[1] * t->ne[2] * t->ne[3] != rows * n3 || (n3 > 1 && t->ne[2] != n3))
        FN_FAIL("load: tensor " + name + " has shape [" + std::to_string(t->ne[0]) + ", " + std::to_string(t->ne[1]) +
                ", " + std::to_string(t->ne[2]) + "], expected " + std::to_string(cols) + " columns x " +
                std::to_string(rows * n3) + " rows");
    return 0;
}

// an F32 vector of n values to device memory
int load_f32(Model &m, const std::string &name, size_t n, float **out) {
    const GTensor *t;
    if (need(m, name, &t)) return -1;
    if (t->type != 0 && t->type != 1) FN_FAIL("load: tensor " + name + " must be F32 or F16");
    if ((size_t) (t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]) != n)
        FN_FAIL("load: tensor " + name + " has " + std::to_string(t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]) +
                " values, expected " + std::to_string(n));
    if (m.alloc(out, n)) return -1;
    if (t->type == 0) {
        FN_CK(hipMemcpy(*out, t->data, n * 4, hipMemcpyHostToDevice));
        return 0;
    }
    std::vector<float> hf(n);  // F16 -> F32 exactly (the reference's load_f32, faie2fn.cu:2173-2184)
    const uint16_t *hb = reinterpret_cast<const uint16_t *>(t->data);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t b = hb[i], sgn = (b >> 15) & 1, e = (b >> 10) & 31, f = b & 1023;
        const float v = e == 0    ? std::ldexp((float) f, -24)
                        : e == 31 ? (f ? NAN : INFINITY)
                                  : std::ldexp((float) (1024 + f), (int) e - 25);
        hf[i] = sgn ? -v : v;
    }
    FN_CK(hipMemcpy(*out, hf.data(), n * 4, hipMemcpyHostToDevice));
    return 0;
}

// GGUF rows (one tensor, or several of one type stacked row-wise) -> packed device weight of rows x cols
int load_qw(Model &m, const std::vector<std::string> &names, const std::vector<uint64_t> &rows, uint64_t cols,
            QW &w, uint64_t n3 = 1) {
    uint32_t type = 0;
    uint64_t total = 0, raw = 0;
    std::vector<const GTensor *> ts;
    for (size_t i = 0; i < names.size(); ++i) {
        const GTensor *t;
        if (need(m, names[i], &t) || check_shape(names[i], t, cols, rows[i], n3)) return -1;
        if (i && t->type != type) FN_FAIL("load: tensors " + names[0] + " and " + names[i] + " differ in type");
        type = t->type;
        total += rows[i] * n3;
        raw += t->nbytes;
        ts.push_back(t);
    }
    if (total > 0x7fffffffu) FN_FAIL("load: tensor " + names[0] + " has too many rows");
    if (!qlayout(type, (int) total, (int) cols, w.L)) return -1;  // fn_error says which type / shape
    uint8_t *stage = nullptr;
    FN_CK(hipMalloc((void **) &stage, raw));
    size_t off = 0;
    hipError_t e = hipSuccess;
    for (const GTensor *t : ts) {
        if (e == hipSuccess) e = hipMemcpy(stage + off, t->data, t->nbytes, hipMemcpyHostToDevice);
        off += t->nbytes;
    }
    int rc = e == hipSuccess ? 0 : -1;
    if (rc) set_error("load: upload of " + names[0] + " -> " + hipGetErrorString(e));
    if (!rc) rc = m.alloc(&w.p, w.L.bytes);
    if (!rc) rc = quant_pack_launch(w.L, stage, w.p, nullptr);
    const hipError_t es = hipDeviceSynchronize();
    (void) hipFree(stage);
    if (!rc && es != hipSuccess) FN_FAIL(std::string("load: pack -> ") + hipGetErrorString(es));
    return rc;
}

int load_qw1(Model &m, const std::string &name, uint64_t rows, uint64_t cols, QW &w, uint64_t n3 = 1) {
    return load_qw(m, {name}, {rows}, cols, w, n3);
}

int read_dims(const Gguf &g, ModelDims &d) {
    auto it = g.strs.find("general.architecture");
    if (it == g.strs.end()) FN_FAIL("load: general.architecture missing");
    const std::string a = it->second + ".";
    auto num = [&](const char *k, double dflt = -1) { return g.num(a + k, dflt); };
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
    auto arr = [&](const char *k) {
        auto it2 = g.iarrays.find(a + k);
        return it2 == g.iarrays.end() ? std::vector<int64_t>{} : it2->second;
    };
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
        if (d.ple_heads < 2 || d.ple_heads > PLE_MAXH || d.ple_hd < 32 || d.ple_hd % 32 ||
            d.ple_heads * d.ple_hd != d.D)
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

// the per-layer n-gram embedding: the hashed table (packed whole into HBM), each PLE layer's key / value weights,
// norms and conv, the hash constants, and the buffers of MAXT tokens (faie2fn.cu:2598-2603, 2661-2687)
int load_ple(Model &m) {
    const ModelDims &d = m.d;
    const uint64_t D = d.D, HCD = (uint64_t) d.HC * d.D;
    const GTensor *t;
    if (need(m, "per_layer_token_embd.weight", &t)) return -1;
    if (t->nd != 2 || t->ne[0] != (uint64_t) d.ple_hd)
        FN_FAIL("load: per_layer_token_embd.weight must be [" + std::to_string(d.ple_hd) + "] x rows");
    int64_t need_rows = 0;
    for (int i = 0; i < d.ple_heads; ++i) need_rows = std::max(need_rows, d.ple_off[i] + d.ple_size[i]);
    if ((int64_t) t->ne[1] < need_rows)
        FN_FAIL("load: per_layer_token_embd.weight has " + std::to_string(t->ne[1]) + " rows, the n-gram heads reach " +
                std::to_string(need_rows));
    if (load_qw1(m, "per_layer_token_embd.weight", t->ne[1], d.ple_hd, m.ple_table)) return -1;
    for (int il : d.ple) {
        MLayer &L = m.L[il];
        L.ple = true;
        const std::string p = "blk." + std::to_string(il) + ".";
        if (load_qw1(m, p + "ple_key.weight", HCD, D, L.ple_key) ||
            load_qw1(m, p + "ple_value.weight", D, D, L.ple_val) ||
            load_f32(m, p + "ple_norm_key.weight", HCD, &L.ple_nk) ||
            load_f32(m, p + "ple_norm_query.weight", HCD, &L.ple_nq) ||
            load_f32(m, p + "ple_norm_conv.weight", HCD, &L.ple_nc) ||
            load_f32(m, p + "ple_conv1d.weight", HCD * 4, &L.ple_conv) ||
            m.alloc(&L.ple_hist, (size_t) PLE_HIST * HCD))
            return -1;
    }
    for (int i = 0; i < 3; ++i) m.hsh.mult[i] = (unsigned long long) d.ple_mult[i];
    for (int i = 0; i < d.ple_heads; ++i) {
        m.hsh.size[i] = (unsigned long long) d.ple_size[i];
        m.hsh.off[i] = (unsigned long long) d.ple_off[i];
    }
    const size_t T = MAXT;
    return m.alloc(&m.ple_rows, T * d.ple_heads) || m.alloc(&m.ple_emb, T * D) || m.alloc(&m.ple_k, T * HCD) ||
                   m.alloc(&m.ple_v, T * D) || m.alloc(&m.ple_gv, T * HCD) || m.alloc(&m.ple_gvn, T * HCD)
               ? -1
               : 0;
}

int load_model(Model &m, int max_ctx_req) {
    const ModelDims &d = m.d;
    const uint64_t D = d.D, HCD = (uint64_t) d.HC * d.D;
    m.max_ctx = (std::max(max_ctx_req, 1) + 255) / 256 * 256;
    FN_CK(hipSetDevice(0));
    FN_CK(hipStreamCreateWithFlags(&m.st, hipStreamNonBlocking));
    // the status word's address, looked up now rather than under a graph capture
    if (status_word(&m.status)) return -1;
    FN_CK(hipHostMalloc(&m.host, 2 * MAXT * sizeof(int32_t) + 64, hipHostMallocDefault));
    m.h_ids = static_cast<int32_t *>(m.host);
    m.h_am = m.h_ids + MAXT;
    m.h_status = reinterpret_cast<unsigned *>(m.h_am + MAXT);
    if (load_qw1(m, "token_embd.weight", d.VOCAB, D, m.tok) || load_qw1(m, "output.weight", d.VOCAB, D, m.head) ||
        load_f32(m, "output_hc_norm.weight", HCD, &m.out_norm) ||
        load_qw1(m, "output_hc_down.weight", d.HCR, HCD, m.out_down) ||
        load_qw1(m, "output_hc_up.weight", HCD, d.HCR, m.out_up))
        return -1;
    m.L.resize(d.NL);
    for (int il = 0; il < d.NL; ++il) {
        MLayer &L = m.L[il];
        L.attn = d.attn_every > 0 && (il + 1) % d.attn_every == 0;
        const std::string p = "blk." + std::to_string(il) + ".";
        if (load_f32(m, p + "hc_attn_norm.weight", HCD, &L.hca_norm) ||
            load_f32(m, p + "hc_ffn_norm.weight", HCD, &L.hcf_norm) ||
            load_qw(m, {p + "hc_attn_down.weight", p + "hc_attn_inject.weight"}, {(uint64_t) d.HCR, (uint64_t) d.HC},
                    HCD, L.hca_dinj) ||
            load_qw1(m, p + "hc_attn_up.weight", HCD, d.HCR, L.hca_up) ||
            load_qw(m, {p + "hc_ffn_down.weight", p + "hc_ffn_inject.weight"}, {(uint64_t) d.HCR, (uint64_t) d.HC},
                    HCD, L.hcf_dinj) ||
            load_qw1(m, p + "hc_ffn_up.weight", HCD, d.HCR, L.hcf_up))
            return -1;
        if (!L.attn) {
            if (load_qw1(m, p + "attn_qkv.weight", d.CONVCH, D, L.qkv) ||
                load_qw1(m, p + "attn_gate.weight", d.DINNER, D, L.z) ||
                load_qw(m, {p + "ssm_alpha.weight", p + "ssm_beta.weight"}, {(uint64_t) d.NVH, (uint64_t) d.NVH}, D,
                        L.ab) ||
                load_qw1(m, p + "ssm_out.weight", D, d.DINNER, L.ssm_out) ||
                load_f32(m, p + "ssm_conv1d.weight", (size_t) d.CONVCH * 4, &L.conv_w) ||
                load_f32(m, p + "ssm_dt.bias", d.NVH, &L.dt) || load_f32(m, p + "ssm_a", d.NVH, &L.ssm_a) ||
                load_f32(m, p + "ssm_norm.weight", d.DS, &L.ssm_norm) ||
                m.alloc(&L.S, (size_t) d.NVH * DSK * DSK) || m.alloc(&L.ring, (size_t) RING * d.CONVCH))
                return -1;
        } else {
            const size_t cache = (size_t) d.NKV * m.max_ctx * HDK;
            if (load_qw1(m, p + "attn_q.weight", (uint64_t) d.NH * 2 * HDK, D, L.q) ||
                load_qw1(m, p + "attn_k.weight", (uint64_t) d.NKV * HDK, D, L.k) ||
                load_qw1(m, p + "attn_v.weight", (uint64_t) d.NKV * HDK, D, L.v) ||
                load_qw1(m, p + "attn_output.weight", D, (uint64_t) d.NH * HDK, L.o) ||
                load_qw(m, {p + "indexer.q_proj.weight", p + "indexer.k_proj.weight"},
                        {(uint64_t) IXH * IXD, (uint64_t) IXD}, D, L.ixqk) ||
                load_f32(m, p + "attn_q_norm.weight", HDK, &L.qn) ||
                load_f32(m, p + "attn_k_norm.weight", HDK, &L.kn) ||
                load_f32(m, p + "indexer.q_norm.weight", IXD, &L.ixqn) ||
                load_f32(m, p + "indexer.k_norm.weight", IXD, &L.ixkn) || m.alloc(&L.Kc, cache) ||
                m.alloc(&L.Vc, cache) || m.alloc(&L.IKc, (size_t) m.max_ctx * IXD) ||
                m.alloc(&L.BKc, (size_t) m.max_ctx / IXR * IXD))
                return -1;
        }
        if (load_qw(m, {p + "ffn_gate_inp.weight", p + "ffn_gate_inp_shexp.weight"}, {(uint64_t) d.NE, 1}, D, L.rsg) ||
            load_qw1(m, p + "ffn_gate_shexp.weight", d.FFS, D, L.sh_gate) ||
            load_qw1(m, p + "ffn_up_shexp.weight", d.FFS, D, L.sh_up) ||
            load_qw1(m, p + "ffn_down_shexp.weight", D, d.FFS, L.sh_down) ||
            load_qw1(m, p + "ffn_gate_exps.weight", d.FFE, D, L.eg, d.NE) ||
            load_qw1(m, p + "ffn_up_exps.weight", d.FFE, D, L.eu, d.NE) ||
            load_qw1(m, p + "ffn_down_exps.weight", D, d.FFE, L.ed, d.NE))
            return -1;
        if (L.eg.L.type != L.eu.L.type) FN_FAIL("load: " + p + " gate and up experts differ in type");
    }
    if (d.ple_layers && load_ple(m)) return -1;
    // activations for MAXT tokens
    const size_t T = MAXT;
    const int ldr = d.HCR + d.HC;
    m.nsplit = attn_pick_nsplit(1, d.NKV, MAXT, 4 * d.top + 4);
    for (int nt = 1; nt <= MAXT; ++nt)
        m.work_bytes = std::max(m.work_bytes, attn_qsa_work_bytes(1, d.NH, nt, HDK, m.nsplit, m.max_ctx, d.top) + 256);
    if (m.alloc(&m.hb[0], T * HCD) || m.alloc(&m.hb[1], T * HCD) || m.alloc(&m.hn, T * HCD) ||
        m.alloc(&m.lr, (size_t) std::max(HC_KS, d.HC) * T * ldr) ||
        m.alloc(&m.amv, T * AM_CH) || m.alloc(&m.ami, T * AM_CH) ||
        m.alloc(&m.t320, T * d.HCR) || m.alloc(&m.a, T * HCD) || m.alloc(&m.x, T * D) || m.alloc(&m.inj, T * d.HC) ||
        m.alloc(&m.qkv, T * d.CONVCH) || m.alloc(&m.zz, T * d.DINNER) || m.alloc(&m.abv, T * 2 * d.NVH) ||
        m.alloc(&m.on, T * d.DINNER) || m.alloc(&m.qg, T * d.NH * 2 * HDK) || m.alloc(&m.kk, T * d.NKV * HDK) ||
        m.alloc(&m.vv, T * d.NKV * HDK) || m.alloc(&m.iqk, T * (IXH * IXD + IXD)) || m.alloc(&m.og, T * d.NH * HDK) ||
        m.alloc(&m.y, T * D) || m.alloc(&m.rsgv, T * (d.NE + 1)) || m.alloc(&m.shg, T * d.FFS) ||
        m.alloc(&m.shu, T * d.FFS) || m.alloc(&m.sha, T * d.FFS) || m.alloc(&m.shd, T * D) ||
        m.alloc(&m.act, T * d.NEU * d.FFE) || m.alloc(&m.dpart, T * d.NEU * D) || m.alloc(&m.wsel, T * d.NEU) ||
        m.alloc(&m.logits, T * d.VOCAB) || m.alloc(&m.work, m.work_bytes / 4 + 1) || m.alloc(&m.ids, T) ||
        m.alloc(&m.sel, T * d.NEU) || m.alloc(&m.pos, 1) || m.alloc(&m.am, T) || m.alloc(&m.tok_all, m.max_ctx))
        return -1;
    FN_CK(hipDeviceSynchronize());
    return 0;
}

// ---- forward ----

int gemv(const QW &w, const float *x, int nt, float *y, hipStream_t st) {
    return gemv_launch(w.L, w.p, x, nt, y, nullptr, 0, st);
}

// the rest of a hyper-connection read once the down (+ inject) product's ks partials are in m.lr: with a BF16 up
// weight (the reference model's) the low-rank SiLU, the up product and the mix are one kernel, else three; into
// m.x and (with inject rows) m.inj
int hc_up(Model &m, const QW &dinj, const QW &up, int nt, int ks) {
    const ModelDims &d = m.d;
    const bool inj = dinj.L.rows > d.HCR;
    const int ldr = dinj.L.rows;
    if (up.L.type == QT_BF16 && UPMIX_ROWS % d.HC == 0 && d.HC <= UPMIX_HC && d.HCR % 8 == 0 &&
        d.HCR <= 64 * UPMIX_U) {
        const int cpb = UPMIX_ROWS / d.HC;
        const size_t lds = ((size_t) nt * d.HCR + 8 * UPMIX_ROWS) * 4;
        hipLaunchKernelGGL(k_hc_upmix, dim3((d.D + cpb - 1) / cpb), dim3(UPMIX_ROWS * 8), lds, m.st, up.p + up.L.off[0],
                           up.L.rs[0], m.lr, ks, nt, ldr, d.HCR, d.HC, d.D, m.hn, m.x, inj ? m.inj : nullptr);
        FN_CK(hipGetLastError());
        return 0;
    }
    hipLaunchKernelGGL(k_hc_lowrank, dim3(nt), dim3(256), 0, m.st, m.lr, ks, nt, ldr, d.HCR, d.HC, m.t320);
    if (gemv(up, m.t320, nt, m.a, m.st)) return -1;
    hipLaunchKernelGGL(k_hc_mix, dim3(nt, (d.D + 255) / 256), dim3(256), 0, m.st, m.a, m.hn, d.D, d.HC, m.lr, ks, nt,
                       ldr, d.HCR, m.x, inj ? m.inj : nullptr);
    FN_CK(hipGetLastError());
    return 0;
}

// One hyper-connection stage: with y, the write of y into the streams (y[t] inj[t][s] into stream s, inj the
// previous read's inject weights) ahead of the read; then the read: each stream's RMSNorm with weight norm into
// m.hn, the down (+ inject) product (a few hundred rows of HC D columns, split by stream, its consumers summing the
// partials) and hc_up.  With a BF16 down weight (the reference model's) the write, the norm and the down product
// are one kernel for a one-token call, and the streams move to the other buffer of the pair; else k_hc_add (or
// k_groupnorm without y) and the split down GEMV (faster for several tokens: the fused kernel's every workgroup
// would norm all of them).  Both give the same bits: the same sums of squares in the same order, and the split
// GEMV sums each row with 64 lanes as the fused kernel does.  dpart: y is the shared expert's part of an MoE output whose routed rows wait in m.dpart
// (expert formats without the MoE output kernel).
int hc_stage(Model &m, const float *y, bool dpart, const float *norm, const QW &dinj, const QW &up, int nt) {
    const ModelDims &d = m.d;
    if (!dpart && nt == 1 && hc_down_supported(dinj.L, d.D, d.HC)) {
        if (hc_down_launch(m.h, y, m.inj, norm, d.D, d.HC, d.eps, dinj.L, dinj.p, nt, y ? m.h2 : nullptr, m.hn, m.lr,
                           m.st))
            return -1;
        if (y) std::swap(m.h, m.h2);
        return hc_up(m, dinj, up, nt, d.HC);
    }
    if (y)
        hipLaunchKernelGGL(k_hc_add, dim3(nt, d.HC), dim3(256), 0, m.st, m.h, y, m.inj, d.D, d.HC,
                           dpart ? m.dpart : nullptr, m.wsel, d.NEU, m.rsgv, d.NE, norm, d.eps, m.hn);
    else
        hipLaunchKernelGGL(k_groupnorm, dim3(nt, d.HC), dim3(256), 0, m.st, m.h, norm, d.D, d.eps, m.hn);
    FN_CK(hipGetLastError());
    int ks = 1;
    if (gemv_split_launch(dinj.L, dinj.p, m.hn, nt, HC_KS, m.lr, &ks, m.st)) return -1;
    return hc_up(m, dinj, up, nt, ks);
}

unsigned hc_add_threads(int D) { return (unsigned) std::min(1024, (D / 4 + 63) / 64 * 64); }

int mixer(Model &m, MLayer &L, int nt) {
    const ModelDims &d = m.d;
    if (!L.attn) {
        const GemvPart g[3] = {{&L.qkv.L, L.qkv.p, m.qkv}, {&L.z.L, L.z.p, m.zz}, {&L.ab.L, L.ab.p, m.abv}};
        if (gemv_group_launch(g, 3, m.x, nt, m.st)) return -1;
        GdnBlock p{1, d.NKH, d.NVH, DSK, DSK, 0, 0, nt, RING, d.eps, m.pos, m.qkv, L.conv_w, L.ring, m.abv, L.dt,
                   L.ssm_a, L.S, m.zz, L.ssm_norm, m.on};
        if (gdn_block_launch(p, m.st)) return -1;
        return gemv(L.ssm_out, m.on, nt, m.y, m.st);
    }
    const GemvPart g[4] = {{&L.q.L, L.q.p, m.qg}, {&L.k.L, L.k.p, m.kk}, {&L.v.L, L.v.p, m.vv},
                           {&L.ixqk.L, L.ixqk.p, m.iqk}};
    if (gemv_group_launch(g, 4, m.x, nt, m.st)) return -1;
    AttnDecode p{1, d.NH, d.NKV, HDK, d.NROT, nt, m.max_ctx, m.nsplit, d.theta, d.eps, m.pos, m.qg, m.kk, m.vv, L.qn,
                 L.kn, L.Kc, L.Vc, m.work, m.work_bytes, m.og};
    QsaIndexer ix{1, nt, m.max_ctx, d.top, d.NROT, d.theta, d.eps, m.pos, m.iqk, L.ixqn, L.ixkn, L.IKc, L.BKc};
    if (attn_qsa_launch(p, ix, m.st)) return -1;
    return gemv(L.o, m.og, nt, m.y, m.st);
}

// the FFN of x into m.shd: the MoE output when *whole, else the shared expert's part (the routed rows in m.dpart)
int ffn(Model &m, MLayer &L, int nt, bool *whole) {
    const ModelDims &d = m.d;
    const GemvPart g[3] = {{&L.rsg.L, L.rsg.p, m.rsgv}, {&L.sh_gate.L, L.sh_gate.p, m.shg},
                           {&L.sh_up.L, L.sh_up.p, m.shu}};
    if (gemv_group_launch(g, 3, m.x, nt, m.st)) return -1;
    // routing (softmax top-k of the router logits, faie2fn.cu:1747-1798): for one token inside the experts' gate/up
    // kernel, which then also writes the picks, their weights and the shared expert's SwiGLU (one kernel fewer); for
    // several tokens in its own kernel (each of their gate/up workgroups would route again)
    if (nt > 1) {
        hipLaunchKernelGGL(k_route, dim3(nt), dim3(256), 0, m.st, m.rsgv, d.NE, d.NEU, m.shg, m.shu, d.FFS, m.sel,
                           m.wsel, m.sha);
        FN_CK(hipGetLastError());
    }
    RouteIn rt;
    rt.rsg = m.rsgv;
    rt.NE = d.NE;
    rt.NEU = d.NEU;
    rt.FFS = d.FFS;
    rt.sel = m.sel;
    rt.wsel = m.wsel;
    rt.shg = m.shg;
    rt.shu = m.shu;
    rt.sha = m.sha;
    const int np = nt * d.NEU;
    if (swiglu_launch(L.eg.L, L.eg.p, L.eu.L, L.eu.p, d.FFE, m.sel, np, d.NEU, m.x, m.act, m.st,
                      nt > 1 ? nullptr : &rt))
        return -1;
    // the experts' down rows, the shared expert's down row and their weighted sum in one kernel where it is built
    // for the formats (the reference model's are), else the rows, a GEMV, and the sum inside the stream write
    const bool fused = moe_down_supported(L.ed.L, L.sh_down.L, d.D, d.NEU);
    if (fused) {
        if (moe_down_launch(L.ed.L, L.ed.p, L.sh_down.L, L.sh_down.p, d.D, m.sel, m.wsel, d.NEU, m.act, m.sha, m.rsgv,
                            d.NE, nt, m.shd, m.st))
            return -1;
    } else if (gemv(L.sh_down, m.sha, nt, m.shd, m.st) ||
               rows_launch(L.ed.L, L.ed.p, d.D, m.sel, np, 1, m.act, m.dpart, m.st)) {
        return -1;
    }
    *whole = fused;
    return 0;
}

// the n-gram embedding of a PLE layer added to the residual streams m.h (faie2fn.cu:2374-2381)
int ple(Model &m, MLayer &L, int nt) {
    const ModelDims &d = m.d;
    const int HCD = d.HC * d.D;
    hipLaunchKernelGGL(k_ple_ids, dim3(nt), dim3(64), 0, m.st, m.tok_all, m.pos, d.ple_heads, d.ple_eos, m.hsh,
                       m.ple_rows);
    FN_CK(hipGetLastError());
    // ple_emb[t][hd * ple_hd + c] = table[row(t, hd)][c]: the gather is the embedding lookup of nt * heads rows
    if (embed_launch(m.ple_table.L, m.ple_table.p, m.ple_rows, nt * d.ple_heads, 1, m.ple_emb, m.st) ||
        gemv(L.ple_key, m.ple_emb, nt, m.ple_k, m.st) || gemv(L.ple_val, m.ple_emb, nt, m.ple_v, m.st))
        return -1;
    hipLaunchKernelGGL(k_ple_gate, dim3(nt, d.HC), dim3(hc_add_threads(d.D)), 0, m.st, m.ple_k, m.ple_v, m.h,
                       L.ple_nk, L.ple_nq, L.ple_nc, d.D, d.eps, m.ple_gv, m.ple_gvn);
    hipLaunchKernelGGL(k_ple_conv, dim3((HCD + 255) / 256), dim3(256), 0, m.st, m.h, m.ple_gv, m.ple_gvn, L.ple_hist,
                       L.ple_conv, HCD, nt);
    FN_CK(hipGetLastError());
    return 0;
}

int enqueue(Model &m, int nt) {
    const ModelDims &d = m.d;
    const size_t HCD = (size_t) d.HC * d.D;
    if (d.ple_layers) {
        hipLaunchKernelGGL(k_store_tokens, dim3(1), dim3(MAXT), 0, m.st, m.ids, m.tok_all, m.pos, nt, m.max_ctx);
        FN_CK(hipGetLastError());
    }
    m.h = m.hb[0];  // every call (and every captured graph) starts from the same buffer of the pair
    m.h2 = m.hb[1];
    if (embed_launch(m.tok.L, m.tok.p, m.ids, nt, d.HC, m.h, m.st)) return -1;
    // the FFN output of a layer is written into the streams by the next stage (its write and the next read's norm
    // and down product are one kernel); pend is that output, pend_dp whether its routed rows wait in m.dpart
    const float *pend = nullptr;
    bool pend_dp = false;
    const auto dbg_copy = [&](int il) -> int {
        if (m.dbg)
            FN_CK(hipMemcpyAsync(m.dbg + (size_t) il * nt * HCD, m.h, (size_t) nt * HCD * 4, hipMemcpyDeviceToHost,
                                 m.st));
        return 0;
    };
    for (int il = 0; il < d.NL; ++il) {
        MLayer &L = m.L[il];
        if (L.ple) {
            // the n-gram embedding reads and writes the streams themselves: the pending write goes first, alone
            if (pend) {
                hipLaunchKernelGGL(k_hc_add, dim3(nt, d.HC), dim3(256), 0, m.st, m.h, pend, m.inj,
                                   d.D, d.HC, pend_dp ? m.dpart : nullptr, m.wsel, d.NEU, m.rsgv, d.NE, nullptr,
                                   d.eps, m.hn);
                FN_CK(hipGetLastError());
                pend = nullptr;
            }
            if ((il > 0 && dbg_copy(il - 1)) || ple(m, L, nt) ||
                hc_stage(m, nullptr, false, L.hca_norm, L.hca_dinj, L.hca_up, nt))
                return -1;
        } else if (hc_stage(m, pend, pend_dp, L.hca_norm, L.hca_dinj, L.hca_up, nt) || (il > 0 && dbg_copy(il - 1))) {
            return -1;
        }
        bool whole = true;
        if (mixer(m, L, nt) || hc_stage(m, m.y, false, L.hcf_norm, L.hcf_dinj, L.hcf_up, nt) ||
            ffn(m, L, nt, &whole))
            return -1;
        pend = m.shd;
        pend_dp = !whole;
    }
    if (hc_stage(m, pend, pend_dp, m.out_norm, m.out_down, m.out_up, nt) || dbg_copy(d.NL - 1)) return -1;
    if (gemv(m.head, m.x, nt, m.logits, m.st)) return -1;
    hipLaunchKernelGGL(k_argmax_part, dim3(nt, AM_CH), dim3(256), 0, m.st, m.logits, d.VOCAB, m.amv, m.ami);
    hipLaunchKernelGGL(k_argmax_merge, dim3(nt), dim3(64), 0, m.st, m.amv, m.ami, d.VOCAB, m.am);
    FN_CK(hipGetLastError());
    return advance_launch(m.pos, 1, nt, m.st);
}

int capture(Model &m, int nt) {
    FN_CK(hipStreamBeginCapture(m.st, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue(m, nt);
    hipGraph_t g = nullptr;
    const hipError_t ec = hipStreamEndCapture(m.st, &g);
    if (rc) {
        if (g) (void) hipGraphDestroy(g);
        return -1;
    }
    FN_CK(ec);
    const hipError_t ei = hipGraphInstantiate(&m.graph[nt], g, nullptr, nullptr, 0);
    (void) hipGraphDestroy(g);
    FN_CK(ei);
    return 0;
}

int drop_graphs(Model &m) {
    FN_CK(hipStreamSynchronize(m.st));
    for (auto &ge : m.graph)
        if (ge) {
            FN_CK(hipGraphExecDestroy(ge));
            ge = nullptr;
        }
    return 0;
}

}  // namespace

int model_load(const char *shard1, const char *shard2, int max_ctx) {
    g_model.reset();
    auto m = std::make_unique<Model>();
    if (gguf_open(m->g, shard1) || read_dims(m->g, m->d)) return -1;
    // the second shard (the reference model keeps the n-gram table there): its tensors join the first's
    if (shard2 && *shard2 && std::string(shard2) != shard1 && gguf_open(m->g2, shard2)) return -1;
    path_free();
    if (load_model(*m, max_ctx)) return -1;
    g_model = std::move(m);
    return 0;
}

int model_forward(const int32_t *tokens, int nt, float *logits, int32_t *argmax) {
    if (!g_model) FN_FAIL("not loaded");
    Model &m = *g_model;
    if (nt < 1 || nt > MAXT) FN_FAIL("nt out of range");
    if (!tokens) FN_FAIL("forward: null tokens");
    if (m.n_past + nt > m.max_ctx) FN_FAIL("context full");
    for (int t = 0; t < nt; ++t)
        if (tokens[t] < 0 || tokens[t] >= m.d.VOCAB) FN_FAIL("forward: token id outside the vocabulary");
    const auto t0 = std::chrono::steady_clock::now();
    std::memcpy(m.h_ids, tokens, (size_t) nt * 4);
    FN_CK(hipMemcpyAsync(m.ids, m.h_ids, (size_t) nt * 4, hipMemcpyHostToDevice, m.st));
    const bool graphs = m.use_graphs && !m.dbg;
    if (graphs) {
        if (!m.graph[nt] && capture(m, nt)) return -1;
        FN_CK(hipGraphLaunch(m.graph[nt], m.st));
    } else if (enqueue(m, nt)) {
        return -1;
    }
    if (logits)
        FN_CK(hipMemcpyAsync(logits, m.logits, (size_t) nt * m.d.VOCAB * 4, hipMemcpyDeviceToHost, m.st));
    FN_CK(hipMemcpyAsync(m.h_am, m.am, (size_t) nt * 4, hipMemcpyDeviceToHost, m.st));
    FN_CK(hipMemcpyAsync(m.h_status, m.status, sizeof(unsigned), hipMemcpyDeviceToHost, m.st));
    FN_CK(hipStreamSynchronize(m.st));
    if (const unsigned bits = *m.h_status) {
        unsigned cleared = 0;
        if (status_read(&cleared, true)) return -1;
        FN_FAIL("forward: a kernel recorded misuse (status bits " + std::to_string(bits) + ")");
    }
    if (argmax) std::memcpy(argmax, m.h_am, (size_t) nt * 4);
    m.n_past += nt;
    m.last_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return 0;
}

int model_debug_layers(float *out) {
    if (!g_model) FN_FAIL("not loaded");
    g_model->dbg = out;
    return 0;
}

int model_reset() {
    if (!g_model) FN_FAIL("not loaded");
    Model &m = *g_model;
    FN_CK(hipStreamSynchronize(m.st));
    for (MLayer &L : m.L)
        if (!L.attn) {
            FN_CK(hipMemset(L.S, 0, (size_t) m.d.NVH * DSK * DSK * 4));
            FN_CK(hipMemset(L.ring, 0, (size_t) RING * m.d.CONVCH * 4));
        }
    for (MLayer &L : m.L)
        if (L.ple) FN_CK(hipMemset(L.ple_hist, 0, (size_t) PLE_HIST * m.d.HC * m.d.D * 4));
    FN_CK(hipMemset(m.pos, 0, 4));
    FN_CK(hipDeviceSynchronize());
    m.n_past = 0;
    return 0;
}

int model_use_graphs(int on) {
    if (!g_model) FN_FAIL("not loaded");
    if (drop_graphs(*g_model)) return -1;
    g_model->use_graphs = on != 0;
    return 0;
}

bool model_loaded() { return (bool) g_model; }
void model_free() { g_model.reset(); }
int model_n_past() { return g_model ? g_model->n_past : -1; }
double model_dev_gb() { return g_model ? g_model->bytes / 1e9 : -1; }
double model_last_ms() { return g_model ? g_model->last_ms : -1; }
int model_layers() { return g_model ? g_model->d.NL : -1; }
int model_dims(ModelDims *d) {
    if (!g_model) FN_FAIL("not loaded");
    *d = g_model->d;
    return 0;
}

int model_inspect(const char *path, ModelDims *d) {
    Gguf g;
    if (gguf_open(g, path) || read_dims(g, *d)) return -1;
    return 0;
}

}  // namespace fn

// Model engine: fn_load places a FAIE2-FlashNext GGUF on one GPU (model_load.hip); fn_forward runs nt <= 8 tokens of
// one sequence through the whole model and returns logits and the argmax token.
//
// The reference model's forward (engine/faie2fn.cu:2370-2490) on its two GPUs, rebuilt on one MI355X: every layer
// on device 0, one stream, one hipGraph per token count, weights and state in per-layer arenas addressed by slot
// (model_impl.h).  Per layer (the reference's order, faie2fn.cu:2370-2420):
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
// faie2fn.cu:1910-1934).  The layers listed in <arch>.ple.layers first add the per-layer n-gram embedding (the
// reference model's, faie2fn.cu:2373-2381): the table rows the bigram and trigram contexts of each position hash to
// (decoded with the hash in one kernel, the context read from a ring of recent token ids), their key and value
// GEMVs, and per stream a signed-sqrt gate and a dilated causal conv (kernel 4, dilation 3) over a ring of earlier
// conv inputs (ngram.hip).  The n-gram table (IQ4_NL rows, 27 GB in the reference model's second shard) is kept in
// HBM where the reference maps it from pinned host memory.  Shapes come from the GGUF metadata; the kernels fix
// head_dim 256, DeltaNet head dim 128, the indexer's 4 x 128 and blocks of 4 keys.
#include "engine.h"
#include "model_impl.h"
#include "qsa.h"

#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

namespace fn {

namespace {

constexpr int UPMIX_U = 8;       // 8-value chunks per lane of the fused up-and-mix kernel (HCR <= 512)
constexpr int UPMIX_HC = 8;      // streams the fused up-and-mix kernel takes (HC <= 8)
constexpr int UPMIX_ROWS = 64;   // rows of the up weight per workgroup of the fused up-and-mix kernel

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
    // Requests in the order their values are needed (a value waits for everything requested before it: vmcnt
    // counts loads in issue order), each unconditional with clamped indices so that all issue before the first
    // wait: the low-rank partials of the thread's first activation entry (ks <= UPMIX_HC of them), then the lane's
    // weight chunks li + 8 u, u < UPMIX_U, then the mix's normalised streams (thread tid < cpb nt finishes column
    // c0 + tid % cpb of token tid / cpb).
    const int i0 = min(tid, nt * HCR - 1), t0 = i0 / HCR, rr0 = i0 - t0 * HCR;
    float lp[UPMIX_HC];
#pragma unroll
    for (int k = 0; k < UPMIX_HC; ++k) lp[k] = lr[((size_t) min(k, ks - 1) * nt + t0) * ldr + rr0];
    __builtin_amdgcn_sched_barrier(0);
    const bool live = c < D;
    uint4 wq[UPMIX_U];
    {
        const uint4 *row = reinterpret_cast<const uint4 *>(U + ((size_t) s * D + min(c, D - 1)) * urs);
#pragma unroll
        for (int u = 0; u < UPMIX_U; ++u) wq[u] = row[min(li + 8 * u, nq - 1)];
    }
    float hv[UPMIX_HC];
    const int mt = tid / cpb, mc = c0 + (tid - mt * cpb);
    const bool mixer = tid < cpb * nt && mc < D;
    {
        const float *hm = hn + (size_t) min(mt, nt - 1) * HC * D + min(mc, D - 1);
#pragma unroll
        for (int k = 0; k < UPMIX_HC; ++k) hv[k] = hm[(size_t) min(k, HC - 1) * D];
    }
    __builtin_amdgcn_sched_barrier(0);
    // the activation: silu of the partials' sum in split order (lr_sum's), the first entry from the registers.
    // Unconditional (a thread past the entries writes the last entry's value to it again), so that the compiler
    // does not move the partials' loads under a branch, behind the weight chunks.
    {
        float v = lp[0];
#pragma unroll
        for (int k = 1; k < UPMIX_HC; ++k)
            if (k < ks) v += lp[k];
        tt[i0] = silu(v * (1.0f / HC));
    }
    for (int i = tid + UPMIX_ROWS * 8; i < nt * HCR; i += UPMIX_ROWS * 8) {
        const int t = i / HCR, r = i - t * HCR;
        tt[i] = silu(lr_sum(lr, ks, nt, ldr, t, r) * (1.0f / HC));
    }
    lds_barrier();  // (the exchange is through the LDS alone; the weight chunks stay in flight)
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

// grid nt, 64 threads.  The forward's last kernel: it also moves the sequence position on by nt (one launch fewer
// than a separate advance; nothing after it in the forward reads the position)
__global__ void k_argmax_merge(const float *__restrict__ pv, const int32_t *__restrict__ pi, int V,
                               int32_t *__restrict__ out, int32_t *__restrict__ pos) {
    const int t = blockIdx.x;
    float v = -INFINITY;
    int idx = V;
    for (int k = threadIdx.x; k < AM_CH; k += 64) vi_max(v, idx, pv[t * AM_CH + k], pi[t * AM_CH + k]);
    wave_argmax(v, idx);
    if (threadIdx.x == 0) out[t] = idx == V ? 0 : idx;
    if (t == 0 && threadIdx.x == 0) pos[0] += (int) gridDim.x;
}

// ---- forward ----

// the model's GEMVs take the plan of the shape alone (no split-K: the forward holds no work buffer for one, whatever
// the sweep override asks)
int gemv(const QW &w, const float *x, int nt, float *y, hipStream_t st) {
    return gemv_launch(w.L, w.p, x, nt, y, nullptr, 0, st, 1);
}

// the rest of a hyper-connection read once the down (+ inject) product's ks partials are in m.a.lr: with a BF16 up
// weight (the reference model's) the low-rank SiLU, the up product and the mix are one kernel, else three; into
// m.a.x and (with inject rows) m.a.inj
int hc_up(Model &m, const QW &dinj, const QW &up, int nt, int ks) {
    const ModelDims &d = m.d;
    Acts &a = m.a;
    const bool inj = dinj.L.rows > d.HCR;
    const int ldr = dinj.L.rows;
    if (up.L.type == QT_BF16 && UPMIX_ROWS % d.HC == 0 && d.HC <= UPMIX_HC && ks <= UPMIX_HC && d.HCR % 8 == 0 &&
        d.HCR <= 64 * UPMIX_U) {
        const int cpb = UPMIX_ROWS / d.HC;
        const size_t lds = ((size_t) nt * d.HCR + 8 * UPMIX_ROWS) * 4;
        hipLaunchKernelGGL(k_hc_upmix, dim3((d.D + cpb - 1) / cpb), dim3(UPMIX_ROWS * 8), lds, m.st, up.p + up.L.off[0],
                           up.L.rs[0], a.lr, ks, nt, ldr, d.HCR, d.HC, d.D, a.hn, a.x, inj ? a.inj : nullptr);
        FN_CK(hipGetLastError());
        return 0;
    }
    hipLaunchKernelGGL(k_hc_lowrank, dim3(nt), dim3(256), 0, m.st, a.lr, ks, nt, ldr, d.HCR, d.HC, a.t320);
    if (gemv(up, a.t320, nt, a.a, m.st)) return -1;
    hipLaunchKernelGGL(k_hc_mix, dim3(nt, (d.D + 255) / 256), dim3(256), 0, m.st, a.a, a.hn, d.D, d.HC, a.lr, ks, nt,
                       ldr, d.HCR, a.x, inj ? a.inj : nullptr);
    FN_CK(hipGetLastError());
    return 0;
}

// One hyper-connection stage: with y, the write of y into the streams (y[t] inj[t][s] into stream s, inj the
// previous read's inject weights) ahead of the read; then the read: each stream's RMSNorm with weight norm into
// m.a.hn, the down (+ inject) product (a few hundred rows of HC D columns, split by stream, its consumers summing the
// partials) and hc_up.  With a BF16 down weight (the reference model's) the write, the norm and the down product
// are one kernel for a one-token call, and the streams move to the other buffer of the pair; else k_hc_add (or
// k_groupnorm without y) and the split down GEMV (faster for several tokens: the fused kernel's every workgroup
// would norm all of them).  Both give the same bits: the same sums of squares in the same order, and the split
// GEMV sums each row with 64 lanes as the fused kernel does.  dpart: y is the shared expert's part of an MoE output
// whose routed rows wait in m.a.dpart (expert formats without the MoE output kernel).
int hc_stage(Model &m, const float *y, bool dpart, const float *norm, const QW &dinj, const QW &up, int nt) {
    const ModelDims &d = m.d;
    Acts &a = m.a;
    if (!dpart && nt == 1 && hc_down_supported(dinj.L, d.D, d.HC)) {
        if (hc_down_launch(m.h, y, a.inj, norm, d.D, d.HC, d.eps, dinj.L, dinj.p, nt, y ? m.h2 : nullptr, a.hn, a.lr,
                           m.st))
            return -1;
        if (y) std::swap(m.h, m.h2);
        return hc_up(m, dinj, up, nt, d.HC);
    }
    if (y)
        hipLaunchKernelGGL(k_hc_add, dim3(nt, d.HC), dim3(256), 0, m.st, m.h, y, a.inj, d.D, d.HC,
                           dpart ? a.dpart : nullptr, a.wsel, d.NEU, a.rsgv, d.NE, norm, d.eps, a.hn);
    else
        hipLaunchKernelGGL(k_groupnorm, dim3(nt, d.HC), dim3(256), 0, m.st, m.h, norm, d.D, d.eps, a.hn);
    FN_CK(hipGetLastError());
    int ks = 1;
    if (gemv_split_launch(dinj.L, dinj.p, a.hn, nt, HC_KS, a.lr, &ks, m.st)) return -1;
    return hc_up(m, dinj, up, nt, ks);
}

int mixer(Model &m, const Layer &L, int nt) {
    const ModelDims &d = m.d;
    Acts &a = m.a;
    if (!L.attn()) {
        const QW in = L.q(DN_IN), zp = L.q(DN_ZPROJ), ab = L.q(DN_AB);
        const GemvPart g[3] = {{&in.L, in.p, a.qkv}, {&zp.L, zp.p, a.zz}, {&ab.L, ab.p, a.abv}};
        if (gemv_group_launch(g, 3, a.x, nt, m.st)) return -1;
        GdnBlock p{1, d.NKH, d.NVH, DSK, DSK, 0, 0, nt, RING, d.eps, a.pos, a.qkv, L.f(DN_CONVW), L.f(DN_RING), a.abv,
                   L.f(DN_DT), L.f(DN_A), L.f(DN_STATE), a.zz, L.f(DN_NORMW), a.on};
        if (gdn_block_launch(p, m.st)) return -1;
        return gemv(L.q(DN_OUT), a.on, nt, a.y, m.st);
    }
    const QW qg = L.q(AT_QG), k = L.q(AT_K), v = L.q(AT_V), ix = L.q(AT_IX);
    const GemvPart g[4] = {{&qg.L, qg.p, a.qg}, {&k.L, k.p, a.kk}, {&v.L, v.p, a.vv}, {&ix.L, ix.p, a.iqk}};
    if (gemv_group_launch(g, 4, a.x, nt, m.st)) return -1;
    AttnDecode p{1, d.NH, d.NKV, HDK, d.NROT, nt, m.max_ctx, m.nsplit, d.theta, d.eps, a.pos, a.qg, a.kk, a.vv,
                 L.f(AT_QNORM), L.f(AT_KNORM), L.f(AT_KCACHE), L.f(AT_VCACHE), a.work, m.work_bytes, a.og,
                 a.status};
    QsaIndexer qix{1, nt, m.max_ctx, d.top, d.NROT, d.theta, d.eps, a.pos, a.iqk, L.f(AT_IXQNORM), L.f(AT_IXKNORM),
                   L.f(AT_IXKEYS), L.f(AT_IXBLOCKS), a.status};
    if (attn_qsa_launch(p, qix, m.st)) return -1;
    return gemv(L.q(AT_O), a.og, nt, a.y, m.st);
}

// the FFN of x into m.a.shd: the MoE output when *whole, else the shared expert's part (the routed rows in m.a.dpart)
int ffn(Model &m, const Layer &L, int nt, bool *whole) {
    const ModelDims &d = m.d;
    Acts &a = m.a;
    const QW rt = L.q(FF_ROUTER), sg = L.q(FF_SH_GATE), su = L.q(FF_SH_UP);
    const GemvPart g[3] = {{&rt.L, rt.p, a.rsgv}, {&sg.L, sg.p, a.shg}, {&su.L, su.p, a.shu}};
    if (gemv_group_launch(g, 3, a.x, nt, m.st)) return -1;
    // routing (softmax top-k of the router logits, faie2fn.cu:1747-1798): for one token inside the experts' gate/up
    // kernel, which then also writes the picks, their weights and the shared expert's SwiGLU (one kernel fewer); for
    // several tokens in its own kernel (each of their gate/up workgroups would route again)
    if (nt > 1) {
        hipLaunchKernelGGL(k_route, dim3(nt), dim3(256), 0, m.st, a.rsgv, d.NE, d.NEU, a.shg, a.shu, d.FFS, a.sel,
                           a.wsel, a.sha);
        FN_CK(hipGetLastError());
    }
    RouteIn route;
    route.rsg = a.rsgv;
    route.NE = d.NE;
    route.NEU = d.NEU;
    route.FFS = d.FFS;
    route.sel = a.sel;
    route.wsel = a.wsel;
    route.shg = a.shg;
    route.shu = a.shu;
    route.sha = a.sha;
    const int np = nt * d.NEU;
    const QW xg = L.q(FF_X_GATE), xu = L.q(FF_X_UP), xd = L.q(FF_X_DOWN), sd = L.q(FF_SH_DOWN);
    if (swiglu_launch(xg.L, xg.p, xu.L, xu.p, d.FFE, a.sel, np, d.NEU, a.x, a.act, m.st, nt > 1 ? nullptr : &route))
        return -1;
    // the experts' down rows, the shared expert's down row and their weighted sum in one kernel where it is built
    // for the formats (the reference model's are), else the rows, a GEMV, and the sum inside the stream write
    const bool fused = moe_down_supported(xd.L, sd.L, d.D, d.NEU);
    if (fused) {
        if (moe_down_launch(xd.L, xd.p, sd.L, sd.p, d.D, a.sel, a.wsel, d.NEU, a.act, a.sha, a.rsgv, d.NE, nt, a.shd,
                            m.st))
            return -1;
    } else if (gemv(sd, a.sha, nt, a.shd, m.st) || rows_launch(xd.L, xd.p, d.D, a.sel, np, 1, a.act, a.dpart, m.st)) {
        return -1;
    }
    *whole = fused;
    return 0;
}

// the n-gram embedding of a layer added to the residual streams m.h (the reference's order, faie2fn.cu:2374-2381):
// the table rows the call's n-gram contexts hash to, their key and value projections, then each stream's gate and
// dilated conv
int ngram(Model &m, const Layer &L, int nt) {
    const ModelDims &d = m.d;
    Acts &a = m.a;
    NgramGather ng;
    ng.ids = a.ids;
    ng.pos = a.pos;
    ng.ring = a.ng_tok;
    ng.ring_mask = NG_RING - 1;
    ng.tab = a.ng_tab;
    ng.heads = d.ple_heads;
    ng.eos = d.ple_eos;
    const QW tab = m.top.q(NG_TABLE), kw = L.q(NG_KEY), vw = L.q(NG_VAL);
    if (ngram_gather_launch(tab.L, tab.p, ng, nt, a.ng_emb, m.st)) return -1;
    const GemvPart g[2] = {{&kw.L, kw.p, a.ng_key}, {&vw.L, vw.p, a.ng_val}};
    if (gemv_group_launch(g, 2, a.ng_emb, nt, m.st)) return -1;
    NgramCall c;
    c.nt = nt;
    c.HC = d.HC;
    c.D = d.D;
    c.eps = d.eps;
    c.pos = a.pos;
    return ngram_inject_launch(c, a.ng_key, a.ng_val, m.h, L, m.st);
}

int enqueue(Model &m, int nt) {
    const ModelDims &d = m.d;
    Acts &a = m.a;
    const size_t HCD = (size_t) d.HC * d.D;
    m.h = a.hb[0];  // every call (and every captured graph) starts from the same buffer of the pair
    m.h2 = a.hb[1];
    const QW tok = m.top.q(TOK_EMBED);
    if (embed_launch(tok.L, tok.p, a.ids, nt, d.HC, m.h, m.st)) return -1;
    // the FFN output of a layer is written into the streams by the next stage (its write and the next read's norm
    // and down product are one kernel); pend is that output, pend_dp whether its routed rows wait in m.a.dpart
    const float *pend = nullptr;
    bool pend_dp = false;
    const auto dbg_copy = [&](int il) -> int {
        if (m.dbg)
            FN_CK(hipMemcpyAsync(m.dbg + (size_t) il * nt * HCD, m.h, (size_t) nt * HCD * 4, hipMemcpyDeviceToHost,
                                 m.st));
        return 0;
    };
    for (int il = 0; il < d.NL; ++il) {
        const Layer &L = m.layers[il];
        if (L.ngram()) {
            // the n-gram embedding reads and writes the streams themselves: the pending write goes first, alone
            if (pend) {
                hipLaunchKernelGGL(k_hc_add, dim3(nt, d.HC), dim3(256), 0, m.st, m.h, pend, a.inj, d.D, d.HC,
                                   pend_dp ? a.dpart : nullptr, a.wsel, d.NEU, a.rsgv, d.NE, nullptr, d.eps, a.hn);
                FN_CK(hipGetLastError());
                pend = nullptr;
            }
            if ((il > 0 && dbg_copy(il - 1)) || ngram(m, L, nt) ||
                hc_stage(m, nullptr, false, L.f(R0_NORM), L.q(R0_DOWN), L.q(R0_UP), nt))
                return -1;
        } else if (hc_stage(m, pend, pend_dp, L.f(R0_NORM), L.q(R0_DOWN), L.q(R0_UP), nt) ||
                   (il > 0 && dbg_copy(il - 1))) {
            return -1;
        }
        bool whole = true;
        if (mixer(m, L, nt) || hc_stage(m, a.y, false, L.f(R1_NORM), L.q(R1_DOWN), L.q(R1_UP), nt) ||
            ffn(m, L, nt, &whole))
            return -1;
        pend = a.shd;
        pend_dp = !whole;
    }
    if (hc_stage(m, pend, pend_dp, m.top.f(FIN_NORM), m.top.q(FIN_DOWN), m.top.q(FIN_UP), nt) || dbg_copy(d.NL - 1))
        return -1;
    if (gemv(m.top.q(LM_HEAD), a.x, nt, a.logits, m.st)) return -1;
    hipLaunchKernelGGL(k_argmax_part, dim3(nt, AM_CH), dim3(256), 0, m.st, a.logits, d.VOCAB, a.amv, a.ami);
    hipLaunchKernelGGL(k_argmax_merge, dim3(nt), dim3(64), 0, m.st, a.amv, a.ami, d.VOCAB, a.am, a.pos);
    FN_CK(hipGetLastError());
    return 0;
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

std::unique_ptr<Model> g_model;

// zero what a sequence accumulates: DeltaNet state and conv rings, K / V and indexer caches need no clearing (a
// position is written before it is read), n-gram conv input and token rings, and the position
int clear_sequence(Model &m) {
    FN_CK(hipStreamSynchronize(m.st));
    for (const Layer &L : m.layers)
        for (Slot s : {DN_STATE, DN_RING, NG_HIST})
            if (L.has(s)) FN_CK(hipMemsetAsync(L.f(s), 0, L.piece[s].bytes, m.st));
    if (m.a.ng_tok) FN_CK(hipMemsetAsync(m.a.ng_tok, 0, NG_RING * 4, m.st));
    FN_CK(hipMemsetAsync(m.a.pos, 0, 4, m.st));
    FN_CK(hipStreamSynchronize(m.st));
    m.n_past = 0;
    m.failed = false;
    return 0;
}

}  // namespace

Model::~Model() {
    if (st) (void) hipStreamSynchronize(st);
    for (auto &ge : graph)
        if (ge) (void) hipGraphExecDestroy(ge);
    for (void *p : allocs) (void) hipFree(p);
    if (host) (void) hipHostFree(host);
    if (st) (void) hipStreamDestroy(st);
}

int model_load(const char *shard1, const char *shard2, int max_ctx) {
    g_model.reset();
    auto m = std::make_unique<Model>();
    // the mappings live only while loading: every weight is copied to the device, the shapes to m->d
    Gguf g, g2;
    if (gguf_open(g, shard1) || read_dims(g, m->d)) return -1;
    // the second shard (the reference model keeps the n-gram table there): its tensors join the first's
    if (shard2 && *shard2 && std::string(shard2) != shard1 && gguf_open(g2, shard2)) return -1;
    m->max_ctx = (std::max(max_ctx, 1) + 255) / 256 * 256;
    if (plan_weights(*m, g, g2)) return -1;
    path_free();
    FN_CK(hipSetDevice(0));
    FN_CK(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
    FN_CK(hipHostMalloc(&m->host, IO_WORDS * sizeof(int32_t), hipHostMallocDefault));
    m->h_io = static_cast<int32_t *>(m->host);
    if (commit_weights(*m)) return -1;
    g_model = std::move(m);
    return 0;
}

int model_forward(const int32_t *tokens, int nt, float *logits, int32_t *argmax) {
    if (!g_model) FN_FAIL("not loaded");
    Model &m = *g_model;
    if (m.failed) FN_FAIL("forward: an earlier call failed on the device; fn_reset starts a new sequence");
    if (nt < 1 || nt > MAXT) FN_FAIL("nt out of range");
    if (!tokens) FN_FAIL("forward: null tokens");
    if (m.n_past + nt > m.max_ctx) FN_FAIL("context full");
    for (int t = 0; t < nt; ++t)
        if (tokens[t] < 0 || tokens[t] >= m.d.VOCAB) FN_FAIL("forward: token id outside the vocabulary");
    const auto t0 = std::chrono::steady_clock::now();
    // the call's ids and a cleared status word in, one copy; the status word and the argmax ids out, one copy
    std::memcpy(m.h_io, tokens, (size_t) nt * 4);
    m.h_io[MAXT] = 0;
    FN_CK(hipMemcpyAsync(m.a.io, m.h_io, (MAXT + 1) * sizeof(int32_t), hipMemcpyHostToDevice, m.st));
    const bool graphs = m.use_graphs && !m.dbg;
    if (graphs) {
        if (!m.graph[nt] && capture(m, nt)) return -1;
        FN_CK(hipGraphLaunch(m.graph[nt], m.st));
    } else if (enqueue(m, nt)) {
        return -1;
    }
    if (logits)
        FN_CK(hipMemcpyAsync(logits, m.a.logits, (size_t) nt * m.d.VOCAB * 4, hipMemcpyDeviceToHost, m.st));
    FN_CK(hipMemcpyAsync(m.h_io + MAXT, m.a.io + MAXT, (size_t) (nt + 1) * 4, hipMemcpyDeviceToHost, m.st));
    FN_CK(hipStreamSynchronize(m.st));
    if (const unsigned bits = (unsigned) m.h_io[MAXT]) {
        // the device advanced its position and wrote state for tokens the host does not count: refuse further
        // calls until fn_reset
        m.failed = true;
        FN_FAIL("forward: a kernel recorded misuse (status bits " + std::to_string(bits) + "); fn_reset to continue");
    }
    if (argmax) std::memcpy(argmax, m.h_io + MAXT + 1, (size_t) nt * 4);
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
    return clear_sequence(*g_model);
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

// QSA indexer for gfx950: the sparse-attention selection the reference runs once a query has more than `top`
// complete blocks of 4 keys (engine/faie2fn.cu:1480-1607).  Four kernels:
//   k_ix_prep    indexer q heads: RMSNorm + RoPE (as the attention q); raw index key appended; the 4-key blocks this
//                call completes get their block key rope(rmsnorm(mean of 4 raw keys) * wkn) at the block start
//   k_ix_blocks  the same block keys over a range of blocks (prefill / rebuilding a cache)
//   k_ix_score   score(block j) = sum over the 4 heads of relu(q_h . BK_j) / sqrt(128); lane = block over a
//                block-tiled key store, so each wave load is one coalesced 1 KiB row of 64 blocks
//   k_ix_select  the top `top` blocks by score, ties at the threshold kept lowest index first, by a 4-pass radix
//                select on the score bits in LDS histograms (the reference binary-searches 32 bit-passes); it emits
//                the sorted list of visible keys (kept blocks, then the incomplete tail) that the attention split
//                kernel gathers from.  A query with <= top complete blocks gets the dense list 0..pos.
// Device layouts: IKc [B][max_ctx][128]; BKc [B][max_ctx/4/64][32][64][4] (64 blocks x 128 dims per tile; max_ctx a
// multiple of 256).
#include "qsa.h"

#include <algorithm>
#include <cmath>

namespace fn {

namespace {

constexpr int IXH = 4, IXD = 128, IXR = 4, BT = 64;  // heads, head dim, keys per block, blocks per tile
constexpr int MAXROT = 128;

struct IxArgs {
    int B, nt, max_ctx, top, nrot;
    float eps;
    const int32_t *pos;
    const float *iqk, *wqn, *wkn;
    float *IKc, *BKc;
    float *Qix;      // [B nt][IXH][IXD]
    float *scores;   // [B nt][max_ctx / IXR]
    int32_t *keys;   // [B nt][top * IXR + IXR]
    int32_t *nkeys;  // [B nt]
    int j0, j1;      // block range of k_ix_blocks
    float inv_freq[MAXROT / 2];
};

__device__ __forceinline__ size_t bk_index(int max_ctx, int b, int j, int d) {
    const size_t tile = (size_t) b * (max_ctx / IXR / BT) + j / BT;
    return ((tile * (IXD / 4) + d / 4) * BT + (j % BT)) * 4 + (d % 4);
}

// RMSNorm * w then RoPE at position P of one 128-long row held two dims per lane (dims 2l, 2l+1); buf is this
// wave's 128-float LDS row.  Returns the lane's two outputs.
__device__ __forceinline__ float2 norm_rope_row(float2 x, const float *w, float *buf, int lane, int P, int nrot,
                                                const float *inv, float eps) {
    const float ss = wave_sum(x.x * x.x + x.y * x.y);
    const float r = rsqrtf(ss / IXD + eps);
    float2 y = make_float2(x.x * r * w[2 * lane], x.y * r * w[2 * lane + 1]);
    buf[2 * lane] = y.x;
    buf[2 * lane + 1] = y.y;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int half = nrot / 2;
    float out[2] = {y.x, y.y};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int d = 2 * lane + e;
        if (d < nrot) {
            const int i = d < half ? d : d - half;
            const float x0 = buf[i], x1 = buf[i + half];
            const float ang = (float) P * inv[i];  // fp32 angle (faie2fn.cu:1440)
            const float cs = cosf(ang), sn = sinf(ang);
            out[e] = d < half ? x0 * cs - x1 * sn : x1 * cs + x0 * sn;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return make_float2(out[0], out[1]);
}

// block key j of sequence b from its four raw keys (one wave, two dims per lane)
__device__ __forceinline__ void block_key(const IxArgs &a, int b, int j, float *buf, int lane) {
    const float *k = a.IKc + ((size_t) b * a.max_ctx + (size_t) j * IXR) * IXD;
    float2 x = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int e = 0; e < IXR; ++e) {
        const float2 v = reinterpret_cast<const float2 *>(k + e * IXD)[lane];
        x.x += v.x;
        x.y += v.y;
    }
    x.x /= IXR;
    x.y /= IXR;
    const float2 y = norm_rope_row(x, a.wkn, buf, lane, j * IXR, a.nrot, a.inv_freq, a.eps);
    a.BKc[bk_index(a.max_ctx, b, j, 2 * lane)] = y.x;
    a.BKc[bk_index(a.max_ctx, b, j, 2 * lane + 1)] = y.y;
}

// grid B, 256 threads (wave h = indexer head h)
__global__ void __launch_bounds__(256) k_ix_prep(const IxArgs a) {
    __shared__ float buf[4][IXD];
    const int b = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int pos = a.pos[b];
    for (int t = 0; t < a.nt; ++t) {
        const int P = pos + t;
        if (P < 0 || P >= a.max_ctx) break;  // past the cache: nothing to append (the host checks positions)
        const size_t bt = (size_t) b * a.nt + t;
        const float *row = a.iqk + bt * (IXH * IXD + IXD);
        const float2 x = reinterpret_cast<const float2 *>(row + wave * IXD)[lane];
        const float2 y = norm_rope_row(x, a.wqn, buf[wave], lane, P, a.nrot, a.inv_freq, a.eps);
        reinterpret_cast<float2 *>(a.Qix + (bt * IXH + wave) * IXD)[lane] = y;
        if (wave == 0)
            reinterpret_cast<float2 *>(a.IKc + ((size_t) b * a.max_ctx + P) * IXD)[lane] =
                reinterpret_cast<const float2 *>(row + IXH * IXD)[lane];
    }
    __syncthreads();  // the raw keys written above are read back below
    const int end = min(pos + a.nt, a.max_ctx);
    for (int j = pos / IXR + wave; j < end / IXR; j += 4) block_key(a, b, j, buf[wave], lane);
}

// grid (B, ceil((j1 - j0) / 4)), 256 threads: block keys of blocks [j0, j1) of every sequence
__global__ void __launch_bounds__(256) k_ix_blocks(const IxArgs a) {
    __shared__ float buf[4][IXD];
    const int b = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = a.j0 + blockIdx.y * 4 + wave;
    if (j < a.j1) block_key(a, b, j, buf[wave], lane);
}

// grid (B nt, G), 256 threads; wave-strided over tiles of 64 blocks, lane = block
__global__ void __launch_bounds__(256) k_ix_score(const IxArgs a) {
    __shared__ float4 qs[IXD / 4][IXH];
    const int bt = blockIdx.x, b = bt / a.nt, t = bt - b * a.nt;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nb = min(a.pos[b] + t + 1, a.max_ctx) / IXR;
    if (nb <= a.top) return;  // dense: nothing to select
    for (int i = threadIdx.x; i < IXH * IXD / 4; i += 256) {
        const int h = i / (IXD / 4), c = i % (IXD / 4);
        qs[c][h] = reinterpret_cast<const float4 *>(a.Qix + ((size_t) bt * IXH + h) * IXD)[c];
    }
    __syncthreads();
    const float inv = 1.0f / sqrtf((float) IXD);
    const int ntiles = (nb + BT - 1) / BT;
    const float4 *Bb = reinterpret_cast<const float4 *>(a.BKc) + (size_t) b * (a.max_ctx / IXR / BT) * (IXD / 4) * BT;
    for (int tile = blockIdx.y * 4 + wave; tile < ntiles; tile += gridDim.y * 4) {
        const float4 *Bt = Bb + (size_t) tile * (IXD / 4) * BT;
        float s[IXH] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int cb = 0; cb < IXD / 4; cb += 16) {
            float4 kf[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) kf[u] = ld_nt(&Bt[(cb + u) * BT + lane]);
#pragma unroll
            for (int u = 0; u < 16; ++u)
#pragma unroll
                for (int h = 0; h < IXH; ++h) {
                    const float4 q = qs[cb + u][h];
                    s[h] = fmaf(q.x, kf[u].x, s[h]);
                    s[h] = fmaf(q.y, kf[u].y, s[h]);
                    s[h] = fmaf(q.z, kf[u].z, s[h]);
                    s[h] = fmaf(q.w, kf[u].w, s[h]);
                }
        }
        const int j = tile * BT + lane;
        float r = 0.0f;
#pragma unroll
        for (int h = 0; h < IXH; ++h) r += fmaxf(s[h], 0.0f);
        if (j < nb) a.scores[(size_t) bt * (a.max_ctx / IXR) + j] = r * inv;
    }
}

// exclusive prefix count of `flag` over the 1024 threads (index order) and the total, through LDS
__device__ __forceinline__ int block_excl_count(bool flag, int *wsum, int &total) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned long long m = __ballot(flag);
    const int before_in_wave = __popcll(m & ((1ull << lane) - 1ull));
    __syncthreads();
    if (lane == 0) wsum[wave] = __popcll(m);
    __syncthreads();
    int before = before_in_wave, tot = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int c = wsum[w];
        before += w < wave ? c : 0;
        tot += c;
    }
    total = tot;
    return before;
}

// grid B nt, 1024 threads
__global__ void __launch_bounds__(1024) k_ix_select(const IxArgs a) {
    __shared__ int hist[256];
    __shared__ int wsum[16];
    __shared__ unsigned sh_prefix;
    __shared__ int sh_need;
    const int bt = blockIdx.x, b = bt / a.nt, t = bt - b * a.nt, tid = threadIdx.x;
    const int P = min(a.pos[b] + t, a.max_ctx - 1);
    const int nb = (P + 1) / IXR;
    int32_t *keys = a.keys + (size_t) bt * (a.top * IXR + IXR);
    if (nb <= a.top) {  // dense: every key 0..P
        for (int k = tid; k <= P; k += 1024) keys[k] = k;
        if (tid == 0) a.nkeys[bt] = P + 1;
        return;
    }
    const unsigned *s = reinterpret_cast<const unsigned *>(a.scores + (size_t) bt * (a.max_ctx / IXR));
    // radix select, most significant byte first: the bits of the top-th largest score (scores are >= 0, so their
    // bits order like the values) and how many of the entries equal to it are kept
    unsigned prefix = 0, pmask = 0;
    int need = a.top;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += 1024) hist[i] = 0;
        __syncthreads();
        for (int j = tid; j < nb; j += 1024) {
            const unsigned u = s[j];
            if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1);
        }
        __syncthreads();
        if (tid < 64) {  // wave 0: digit where the count from the top reaches `need`
            const int l = tid;  // lane l holds digits 255-4l .. 252-4l (descending)
            int c[4], sum = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                c[e] = hist[255 - 4 * l - e];
                sum += c[e];
            }
            // inclusive scan of the lane sums over the wave (descending digit order)
            int incl = sum;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int v = __shfl_up(incl, off);
                if (l >= off) incl += v;
            }
            const int excl = incl - sum;
            const bool here = excl < need && incl >= need;
            const unsigned long long m = __ballot(here);
            const int owner = __ffsll((long long) m) - 1;
            if (l == owner) {
                int acc = excl, d = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (acc + c[e] >= need) {
                        d = 255 - 4 * l - e;
                        break;
                    }
                    acc += c[e];
                }
                sh_prefix = prefix | ((unsigned) d << shift);
                sh_need = need - acc;  // entries still to take among those with this digit
            }
        }
        __syncthreads();
        prefix = sh_prefix;
        need = sh_need;
        pmask |= 255u << shift;
        __syncthreads();
    }
    const unsigned thr = prefix;  // `need` entries equal to thr are kept, lowest index first
    // emit the kept blocks in index order: block j's keys 4j..4j+3 at list slot 4 * (kept blocks before j)
    int base_kept = 0, base_eq = 0;
    for (int j0 = 0; j0 < nb; j0 += 1024) {
        const int j = j0 + tid;
        const unsigned u = j < nb ? s[j] : 0u;
        const bool eq = j < nb && u == thr;
        int eq_total;
        const int eq_before = block_excl_count(eq, wsum, eq_total);
        const bool keep = j < nb && (u > thr || (eq && base_eq + eq_before < need));
        int kept_total;
        const int kept_before = block_excl_count(keep, wsum, kept_total);
        if (keep) {
            const int slot = (base_kept + kept_before) * IXR;
#pragma unroll
            for (int e = 0; e < IXR; ++e) keys[slot + e] = j * IXR + e;
        }
        base_kept += kept_total;
        base_eq += eq_total;
    }
    // the incomplete tail block is always visible (faie2fn.cu:1630)
    const int tail0 = nb * IXR;
    if (tid <= P - tail0) keys[a.top * IXR + tid] = tail0 + tid;
    if (tid == 0) a.nkeys[bt] = a.top * IXR + (P + 1 - tail0);
}

IxArgs make_args(const QsaIndexer &p) {
    IxArgs a{};
    a.B = p.B; a.nt = p.nt; a.max_ctx = p.max_ctx; a.top = p.top; a.nrot = p.nrot; a.eps = p.eps; a.pos = p.pos;
    a.iqk = p.iqk; a.wqn = p.wqn; a.wkn = p.wkn; a.IKc = p.IKc; a.BKc = p.BKc;
    for (int i = 0; i < p.nrot / 2; ++i)
        a.inv_freq[i] = (float) (1.0 / std::pow((double) p.theta, (double) (2 * i) / p.nrot));
    return a;
}

int check(const QsaIndexer &p) {
    if (p.B < 1 || p.nt < 1) FN_FAIL("qsa: B and nt must be >= 1");
    if (p.max_ctx < 256 || p.max_ctx % 256) FN_FAIL("qsa: max_ctx must be a positive multiple of 256");
    if (p.nrot < 0 || p.nrot > MAXROT || p.nrot % 4) FN_FAIL("qsa: nrot must be a multiple of 4, at most 128");
    if (p.top < 1 || p.top * IXR + IXR > 65536) FN_FAIL("qsa: top must be in [1, 16383]");
    return 0;
}

}  // namespace

size_t qsa_work_bytes(int B, int nt, int max_ctx, int top) {
    const size_t bt = (size_t) B * nt;
    return (bt * IXH * IXD + bt * (max_ctx / IXR)) * 4 + (bt * ((size_t) top * IXR + IXR) + bt) * 4 + 256;
}

int qsa_select_launch(const QsaIndexer &p, float *work, size_t work_bytes, const int32_t **keys, const int32_t **nkeys,
                      hipStream_t st) {
    if (check(p)) return -1;
    if (!p.pos || !p.iqk || !p.wqn || !p.wkn || !p.IKc || !p.BKc || !work) FN_FAIL("qsa: null pointer");
    if (work_bytes < qsa_work_bytes(p.B, p.nt, p.max_ctx, p.top)) FN_FAIL("qsa: workspace too small");
    IxArgs a = make_args(p);
    const size_t bt = (size_t) p.B * p.nt;
    a.Qix = work;
    a.scores = a.Qix + bt * IXH * IXD;
    a.keys = reinterpret_cast<int32_t *>(a.scores + bt * (p.max_ctx / IXR));
    a.nkeys = a.keys + bt * ((size_t) p.top * IXR + IXR);
    *keys = a.keys;
    *nkeys = a.nkeys;
    const int tiles = p.max_ctx / IXR / BT;
    const int G = std::max(1, std::min(128, (tiles + 3) / 4));
    hipLaunchKernelGGL(k_ix_prep, dim3(p.B), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_ix_score, dim3((unsigned) bt, G), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_ix_select, dim3((unsigned) bt), dim3(1024), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

int qsa_blocks_launch(const QsaIndexer &p, int j0, int j1, hipStream_t st) {
    if (check(p)) return -1;
    if (!p.IKc || !p.BKc || !p.wkn) FN_FAIL("qsa: null pointer");
    if (j0 < 0 || j1 > p.max_ctx / IXR || j0 > j1) FN_FAIL("qsa: block range outside the cache");
    if (j1 == j0) return 0;
    IxArgs a = make_args(p);
    a.j0 = j0;
    a.j1 = j1;
    hipLaunchKernelGGL(k_ix_blocks, dim3(p.B, (j1 - j0 + 3) / 4), dim3(256), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

// QSA indexer for gfx950: the sparse-attention selection the reference runs once a query has more than `top`
// complete blocks of 4 keys (engine/faie2fn.cu:1480-1607).  Four kernels:
//   k_ix_prep    indexer q heads: RMSNorm + RoPE (as the attention q); raw index key appended; the 4-key blocks this
//                call completes get their block key rope(rmsnorm(mean of 4 raw keys) * wkn) at the block start
//   k_ix_blocks  the same block keys over a range of blocks (prefill / rebuilding a cache)
//   k_ix_score   score(block j) = sum over the 4 heads of relu(q_h . BK_j) / sqrt(128); lane = block over a
//                block-tiled key store, so each wave load is one coalesced 1 KiB row of 64 blocks.  For one-token
//                calls k_ix_prep's work runs inside it (k_ix_score<true>), one dependent launch fewer
//   k_ix_select  the top `top` blocks by score, ties at the threshold kept lowest index first, by a 3-pass radix
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
    unsigned *status;  // per-device status word (FN_STATUS_POS)
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
        if (P < 0 || P >= a.max_ctx) {  // past the cache: nothing to append; the status word says so
            if (threadIdx.x == 0) atomicOr(a.status, FN_STATUS_POS);
            break;
        }
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

// grid (B nt, G), 256 threads.  Workgroup y takes tiles y, y + G, ... of 64 blocks; lane = block, and wave w loads
// dims 32w .. 32w+31 of the tile (8 coalesced 1 KiB rows), so one tile is 4 waves' loads in flight at once.  The
// four waves' partial head dots meet in LDS; wave 0 applies the relu per head and stores the tile's 64 scores.
// PREP (one-token calls, nt = 1): k_ix_prep's work rides in this launch.  Every workgroup of a query normalises and
// ropes the 4 index q heads itself (wave h = head h, as k_ix_prep), with its first tile's loads already in flight;
// workgroup 0 appends the raw index key; when the new key completes block jn, the workgroup owning jn's tile
// (y = (jn / 64) % G) builds the block key from the 3 cached raw keys and the new one (the same arithmetic as
// block_key), stores it, and scores block jn from its own copy: no workgroup reads a block key this launch writes.
// Both happen before the dense test, so a dense query's caches are kept up to date.  Same bits as k_ix_prep followed
// by the plain kernel.
template <bool PREP>
__global__ void __launch_bounds__(256) k_ix_score(const IxArgs a) {
    constexpr int CW = IXD / 4 / 4;  // float4 chunks per wave
    __shared__ float4 qs[IXD / 4][IXH];
    __shared__ float part[2][4][IXH][BT];
    __shared__ float buf[PREP ? 4 : 1][IXD];  // PREP: the waves' RoPE rows; row 0 then holds the new block key
    const int bt = blockIdx.x, b = bt / a.nt, t = bt - b * a.nt;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int P = a.pos[b] + t;
    const int nb = min(P + 1, a.max_ctx) / IXR;
    const int ntiles = (nb + BT - 1) / BT;
    int tile = blockIdx.y;
    const bool live = nb > a.top && tile < ntiles;  // sparse query, and this workgroup has tiles
    // PREP: the head's query row, the new raw key and the 3 cached raw keys of the block the new key would complete
    // requested first (unconditional, clamped), so that the query's norm and RoPE wait for them and not for the tile
    float2 x, nk, rk[IXR - 1];
    if constexpr (PREP) {
        const float *row = a.iqk + (size_t) bt * (IXH * IXD + IXD);
        x = reinterpret_cast<const float2 *>(row + wave * IXD)[lane];
        nk = reinterpret_cast<const float2 *>(row + IXH * IXD)[lane];
        const int pc = min(max(P, 0), a.max_ctx - 1);
        const float *k = a.IKc + ((size_t) b * a.max_ctx + (size_t) (pc / IXR) * IXR) * IXD;
#pragma unroll
        for (int e = 0; e < IXR - 1; ++e) rk[e] = reinterpret_cast<const float2 *>(k + e * IXD)[lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    const float4 *Bb = reinterpret_cast<const float4 *>(a.BKc) +
                       ((size_t) b * (a.max_ctx / IXR / BT) * (IXD / 4) + wave * CW) * BT + lane;
    float4 kf[CW];
    if (live) {
#pragma unroll
        for (int c = 0; c < CW; ++c) kf[c] = ld_nt(&Bb[((size_t) tile * (IXD / 4) + c) * BT]);
    }
    int jn = -1;  // PREP: the block this call's key completes, when this workgroup builds it
    if constexpr (PREP) {
        const bool valid = P >= 0 && P < a.max_ctx;
        if (!valid) {  // past the cache: nothing to append; the status word says so
            if (blockIdx.y == 0 && threadIdx.x == 0) atomicOr(a.status, FN_STATUS_POS);
        } else {
            if (blockIdx.y == 0 && wave == 0)
                reinterpret_cast<float2 *>(a.IKc + ((size_t) b * a.max_ctx + P) * IXD)[lane] = nk;
            if ((P + 1) % IXR == 0 && (P / IXR / BT) % (int) gridDim.y == (int) blockIdx.y) jn = P / IXR;
        }
        const float2 y = norm_rope_row(x, a.wqn, buf[wave], lane, P, a.nrot, a.inv_freq, a.eps);
        float *qf = reinterpret_cast<float *>(qs);
        qf[((2 * lane / 4) * IXH + wave) * 4 + (2 * lane) % 4] = y.x;
        qf[((2 * lane / 4) * IXH + wave) * 4 + (2 * lane) % 4 + 1] = y.y;
        if (jn >= 0 && wave == 0) {  // (uniform in the wave)
            // block_key's sum: the 4 raw keys in order, the last one the new key (its cached copy's bits)
            float2 sm = make_float2(0.0f, 0.0f);
#pragma unroll
            for (int e = 0; e < IXR; ++e) {
                const float2 v = e < IXR - 1 ? rk[e] : nk;
                sm.x += v.x;
                sm.y += v.y;
            }
            sm.x /= IXR;
            sm.y /= IXR;
            const float2 bk = norm_rope_row(sm, a.wkn, buf[0], lane, jn * IXR, a.nrot, a.inv_freq, a.eps);
            a.BKc[bk_index(a.max_ctx, b, jn, 2 * lane)] = bk.x;
            a.BKc[bk_index(a.max_ctx, b, jn, 2 * lane + 1)] = bk.y;
            buf[0][2 * lane] = bk.x;
            buf[0][2 * lane + 1] = bk.y;
        }
    }
    if (!live) return;  // (after the appends: a dense query's caches still grow)
    if constexpr (!PREP) {
        for (int i = threadIdx.x; i < IXH * IXD / 4; i += 256) {
            const int h = i / (IXD / 4), c = i % (IXD / 4);
            qs[c][h] = reinterpret_cast<const float4 *>(a.Qix + ((size_t) bt * IXH + h) * IXD)[c];
        }
    }
    __syncthreads();
    const float inv = 1.0f / sqrtf((float) IXD);
    float *out = a.scores + (size_t) bt * (a.max_ctx / IXR);
    for (int it = 0; tile < ntiles; tile += gridDim.y, ++it) {
        if (PREP && jn >= 0 && tile == jn / BT && lane == jn % BT) {  // block jn from this workgroup's own copy
#pragma unroll
            for (int c = 0; c < CW; ++c)
                kf[c] = reinterpret_cast<const float4 *>(buf[0])[wave * CW + c];
        }
        float s[IXH] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int h = 0; h < IXH; ++h) {
                const float4 q = qs[wave * CW + c][h];
                s[h] = fmaf(q.x, kf[c].x, s[h]);
                s[h] = fmaf(q.y, kf[c].y, s[h]);
                s[h] = fmaf(q.z, kf[c].z, s[h]);
                s[h] = fmaf(q.w, kf[c].w, s[h]);
            }
        const int next = tile + gridDim.y;
        if (next < ntiles) {
#pragma unroll
            for (int c = 0; c < CW; ++c) kf[c] = ld_nt(&Bb[((size_t) next * (IXD / 4) + c) * BT]);
        }
        float (*pt)[IXH][BT] = part[it & 1];  // alternating buffers: one barrier per tile
#pragma unroll
        for (int h = 0; h < IXH; ++h) pt[wave][h][lane] = s[h];
        __syncthreads();
        if (wave == 0) {
            float r = 0.0f;
#pragma unroll
            for (int h = 0; h < IXH; ++h) r += fmaxf(pt[0][h][lane] + pt[1][h][lane] + pt[2][h][lane] + pt[3][h][lane], 0.0f);
            const int j = tile * BT + lane;
            if (j < nb) out[j] = r * inv;
        }
    }
}

// exclusive prefix sums of x and y over the 1024 threads in thread order, and their totals (wsum: 32 ints of LDS);
// the wave scans are DPP (a shuffle-based scan, an LDS-crossbar permute per step, took ~1.8 us of this kernel)
__device__ __forceinline__ int2 block_excl_scan2(int x, int y, int2 *wsum, int2 &total) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ix = wave_incl_scan(x), iy = wave_incl_scan(y);
    __syncthreads();  // wsum free
    if (lane == 63) wsum[wave] = make_int2(ix, iy);
    __syncthreads();
    int2 before = make_int2(ix - x, iy - y), tot = make_int2(0, 0);
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int2 c = wsum[w];
        if (w < wave) {
            before.x += c.x;
            before.y += c.y;
        }
        tot.x += c.x;
        tot.y += c.y;
    }
    total = tot;
    return before;
}

// grid B nt, 1024 threads.  Thread t owns the contiguous blocks t*per .. t*per+per-1, per = ceil(nb / 1024) rounded
// up to a multiple of 4 so that they load as float4; with PER > 0 the scores stay in registers (nb <= 1024 PER), with
// PER == 0 every pass re-reads them (L2-resident).  Scores are >= +0, so their bits order like the values.
// With the scores in registers (PER > 0) the selection first tries one pass: a 16384-bin LDS histogram of bits
// [30:17] (the exponent and 6 mantissa bits, bins 1/64 of an octave wide), one block scan (descending) for the bin
// where the count from the top reaches `top`; every block above that bin is kept, and the bin's own blocks (a few
// dozen for the scores of real queries) are ranked exactly among themselves in the LDS (higher score first, equal
// scores lower index first) and the first `need` of them kept.  A bin of more than 1024 blocks (mass ties) falls
// through to the radix select: 11-bit digits [30:20], [19:9] and 9-bit [8:0], each pass a 2048-bin LDS histogram of
// the entries that match the digits fixed so far, then a block scan for the digit at which the count from the top
// reaches `need`.  Its histogram has 8 copies, by lane % 8, in different banks: lanes of one atomic instruction that
// share a digit mostly hit different words.
template <int PER>
__global__ void __launch_bounds__(1024) k_ix_select(const IxArgs a) {
    constexpr int NBIN = 2048, NC = 8, HS = NBIN + 1, MAXPER = PER > 0 ? PER : 4;
    __shared__ int hist[NC * HS];
    __shared__ int2 wsum[16];
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
    // this row of scores is max_ctx / 4 long, a multiple of 64: a float4 that starts below nb stays inside it
    const unsigned *s = reinterpret_cast<const unsigned *>(a.scores + (size_t) bt * (a.max_ctx / IXR));
    const int per = ((nb + 1023) / 1024 + 3) & ~3, j0 = min(tid * per, nb), jn = min(j0 + per, nb);
    unsigned v[MAXPER];
    if (PER > 0) {
        // every float4 requested before the first is used: unconditional loads (a float4 past the thread's run reads
        // the row's first one instead; every use below checks j < jn), so that none sits under a branch with a wait
#pragma unroll
        for (int i = 0; i < MAXPER; i += 4) {
            const uint4 u = *reinterpret_cast<const uint4 *>(s + (j0 + i < jn ? j0 + i : 0));
            v[i] = u.x; v[i + 1] = u.y; v[i + 2] = u.z; v[i + 3] = u.w;
        }
    }
    // the incomplete tail block is always visible (faie2fn.cu:1630)
    const auto tail = [&]() {
        const int tail0 = nb * IXR;
        if (tid <= P - tail0) keys[a.top * IXR + tid] = tail0 + tid;
        if (tid == 0) a.nkeys[bt] = a.top * IXR + (P + 1 - tail0);
    };
    int4 *kv = reinterpret_cast<int4 *>(keys);
    if constexpr (PER > 0) {
        constexpr int FS = 17, NF = 1 << (31 - FS), BPT = NF / 1024, CMAX = 1024;
        static_assert(NF <= NC * HS, "the one-pass histogram shares the radix histogram's LDS");
        static_assert(PER <= 32, "a thread's kept blocks are one 32-bit mask");
        __shared__ uint2 cand[CMAX];               // (score bits, block) of the threshold bin
        __shared__ unsigned kept[PER * 1024 / 32];  // bitmap of the threshold bin's kept blocks
        __shared__ int sh_bin, sh_bneed, sh_bcnt, sh_slot;
        int4 *h4 = reinterpret_cast<int4 *>(hist);
        for (int i = tid; i < NF / 4; i += 1024) h4[i] = make_int4(0, 0, 0, 0);
        for (int i = tid; i < PER * 32; i += 1024) kept[i] = 0u;
        if (tid == 0) sh_slot = 0;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (j0 + i < jn) atomicAdd(&hist[v[i] >> FS], 1);
        __syncthreads();
        // thread t holds bins NF - BPT (t + 1) .. NF - 1 - BPT t: the scan in thread order runs over them descending
        const int lo = NF - BPT * (tid + 1);
        int c[BPT], sum = 0;
#pragma unroll
        for (int q = 0; q < BPT / 4; ++q) {
            const int4 h = h4[lo / 4 + q];
            c[4 * q] = h.x; c[4 * q + 1] = h.y; c[4 * q + 2] = h.z; c[4 * q + 3] = h.w;
        }
#pragma unroll
        for (int k = 0; k < BPT; ++k) sum += c[k];
        int2 tot;
        const int excl = block_excl_scan2(sum, 0, wsum, tot).x;
        if (excl < a.top && excl + sum >= a.top) {  // exactly one thread: counts >= 0, total = nb > top
            int run = excl;
#pragma unroll
            for (int k = BPT - 1; k >= 0; --k) {
                if (run < a.top && run + c[k] >= a.top) {
                    sh_bin = lo + k;
                    sh_bneed = a.top - run;  // blocks still to take from this bin
                    sh_bcnt = c[k];
                }
                run += c[k];
            }
        }
        __syncthreads();
        const unsigned bin = (unsigned) sh_bin;
        const int bneed = sh_bneed, bcnt = sh_bcnt;
        if (bcnt <= CMAX) {  // (uniform)
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (j0 + i < jn && (v[i] >> FS) == bin) cand[atomicAdd(&sh_slot, 1)] = make_uint2(v[i], (unsigned) (j0 + i));
            __syncthreads();
            if (bcnt <= 64) {  // (uniform) one wave, the other candidates read across lanes
                if (tid < 64) {
                    const uint2 me = tid < bcnt ? cand[tid] : make_uint2(0u, 0u);
                    int rank = 0;
                    for (int k = 0; k < bcnt; ++k) {
                        const unsigned ox = (unsigned) __builtin_amdgcn_readlane((int) me.x, k);
                        const unsigned oj = (unsigned) __builtin_amdgcn_readlane((int) me.y, k);
                        rank += ox > me.x || (ox == me.x && oj < me.y);
                    }
                    if (tid < bcnt && rank < bneed) atomicOr(&kept[me.y >> 5], 1u << (me.y & 31));
                }
            } else if (tid < bcnt) {
                const uint2 me = cand[tid];
                int rank = 0;
                for (int k = 0; k < bcnt; ++k) {
                    const uint2 o = cand[k];
                    rank += o.x > me.x || (o.x == me.x && o.y < me.y);
                }
                if (rank < bneed) atomicOr(&kept[me.y >> 5], 1u << (me.y & 31));
            }
            __syncthreads();
            // every block above the bin, and the bin's kept ones (the thread's run spans at most two bitmap words,
            // read once), as a bit mask; then one scan gives each thread its list slot
            const int w0 = j0 >> 5;
            const unsigned kw0 = kept[w0], kw1 = w0 + 1 < PER * 32 ? kept[w0 + 1] : 0u;
            unsigned keep = 0u;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int j = j0 + i;
                const unsigned d = v[i] >> FS, kw = (j >> 5) == w0 ? kw0 : kw1;
                keep |= (unsigned) (j < jn && (d > bin || (d == bin && ((kw >> (j & 31)) & 1u)))) << i;
            }
            int slot = block_excl_scan2(__builtin_popcount(keep), 0, wsum, tot).x;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int j = j0 + i;
                if ((keep >> i) & 1u) kv[slot++] = make_int4(j * IXR, j * IXR + 1, j * IXR + 2, j * IXR + 3);
            }
            tail();
            return;
        }
        __syncthreads();  // the radix passes reuse the histogram's LDS
    }
    int *hl = hist + (tid & (NC - 1)) * HS;
    unsigned prefix = 0, pmask = 0;
    int need = a.top;
    constexpr int SHIFT[3] = {20, 9, 0};
#pragma unroll
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = SHIFT[pass];
        for (int i = tid; i < NC * HS; i += 1024) hist[i] = 0;
        __syncthreads();
        if (PER > 0) {
#pragma unroll
            for (int i = 0; i < MAXPER; ++i)
                if (j0 + i < jn && (v[i] & pmask) == prefix) atomicAdd(&hl[(v[i] >> shift) & (NBIN - 1)], 1);
        } else {
            for (int j = j0; j < jn; ++j) {
                const unsigned u = s[j];
                if ((u & pmask) == prefix) atomicAdd(&hl[(u >> shift) & (NBIN - 1)], 1);
            }
        }
        __syncthreads();
        // thread t holds digits 2047-2t and 2046-2t: the scan in thread order runs over the digits descending
        int c0 = 0, c1 = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            c0 += hist[c * HS + NBIN - 1 - 2 * tid];
            c1 += hist[c * HS + NBIN - 2 - 2 * tid];
        }
        int2 tot;
        const int excl = block_excl_scan2(c0 + c1, 0, wsum, tot).x;
        if (excl < need && excl + c0 + c1 >= need) {  // exactly one thread: counts are >= 0 and the total >= need
            const bool first = excl + c0 >= need;
            const unsigned d = first ? NBIN - 1 - 2 * tid : NBIN - 2 - 2 * tid;
            sh_prefix = prefix | (d << shift);
            sh_need = need - (first ? excl : excl + c0);  // entries still to take among those with this digit
        }
        __syncthreads();
        prefix = sh_prefix;
        need = sh_need;
        pmask |= (pass == 2 ? 511u : 2047u) << shift;
    }
    const unsigned thr = prefix;  // every entry above thr is kept, and the first `need` entries equal to it
    // this thread's entries above / equal, then one scan gives each thread its list slot and its equal-rank
    int gt = 0, eq = 0;
    if (PER > 0) {
#pragma unroll
        for (int i = 0; i < MAXPER; ++i)
            if (j0 + i < jn) {
                gt += v[i] > thr;
                eq += v[i] == thr;
            }
    } else {
        for (int j = j0; j < jn; ++j) {
            const unsigned u = s[j];
            gt += u > thr;
            eq += u == thr;
        }
    }
    int2 tot;
    const int2 before = block_excl_scan2(gt, eq, wsum, tot);
    int slot = before.x + min(before.y, need), eq_rank = before.y;
    auto emit = [&](int j, unsigned u) {
        const bool keep = u > thr || (u == thr && eq_rank < need);
        eq_rank += u == thr;
        if (keep) kv[slot++] = make_int4(j * IXR, j * IXR + 1, j * IXR + 2, j * IXR + 3);
    };
    if (PER > 0) {
#pragma unroll
        for (int i = 0; i < MAXPER; ++i)
            if (j0 + i < jn) emit(j0 + i, v[i]);
    } else {
        for (int j = j0; j < jn; ++j) emit(j, s[j]);
    }
    tail();
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
    if (p.status) a.status = p.status;
    else if (status_word(&a.status)) return -1;
    const size_t bt = (size_t) p.B * p.nt;
    a.Qix = work;
    a.scores = a.Qix + bt * IXH * IXD;
    a.keys = reinterpret_cast<int32_t *>(a.scores + bt * (p.max_ctx / IXR));
    a.nkeys = a.keys + bt * ((size_t) p.top * IXR + IXR);
    *keys = a.keys;
    *nkeys = a.nkeys;
    // about 1024 workgroups of scoring over all queries, at most one per tile
    const int tiles = p.max_ctx / IXR / BT;
    const int G = (int) std::max<size_t>(1, std::min<size_t>(tiles, (1024 + bt - 1) / bt));
    const int nbmax = p.max_ctx / IXR;
    if (p.nt == 1) {  // the prep inside the scoring launch
        hipLaunchKernelGGL(k_ix_score<true>, dim3((unsigned) bt, G), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(k_ix_prep, dim3(p.B), dim3(256), 0, st, a);
        stage_mark(st);
        hipLaunchKernelGGL(k_ix_score<false>, dim3((unsigned) bt, G), dim3(256), 0, st, a);
    }
    stage_mark(st);
    if (nbmax <= 1024 * 8)
        hipLaunchKernelGGL(k_ix_select<8>, dim3((unsigned) bt), dim3(1024), 0, st, a);
    else if (nbmax <= 1024 * 32)
        hipLaunchKernelGGL(k_ix_select<32>, dim3((unsigned) bt), dim3(1024), 0, st, a);
    else
        hipLaunchKernelGGL(k_ix_select<0>, dim3((unsigned) bt), dim3(1024), 0, st, a);
    stage_mark(st);
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

// The per-layer n-gram embedding's injection into the residual streams (the reference's gate and dilated conv,
// engine/faie2fn.cu:1843-1896, with its 9-deep shifted history; the math is the reference model's, the kernel is
// this engine's own: one workgroup per stream over the call's tokens, the conv input kept in a ring indexed by
// position).
#include "model_impl.h"

namespace fn {

namespace {

struct InjectArgs {
    int nt, D, HC;
    float eps;
    const int32_t *pos;
    const float *key, *val, *wk, *wq, *wc, *conv;
    float *h, *ring;
};

__device__ __forceinline__ float sq4(float4 v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }
__device__ __forceinline__ float4 mul4(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float silu1(float x) { return x / (1.0f + expf(-x)); }

// sums over the workgroup of two values at once (wave sums, then the waves' partials in wave order); red: 2 x 16
// floats of LDS, used alternately by consecutive calls so that one barrier per call suffices
__device__ __forceinline__ void wg_sum2(float &a, float &b, float *red, int nw) {
    a = wave_sum(a);
    b = wave_sum(b);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[w] = a;
        red[16 + w] = b;
    }
    __syncthreads();
    float sa = 0.0f, sb = 0.0f;
    for (int i = 0; i < nw; ++i) {
        sa += red[i];
        sb += red[16 + i];
    }
    a = sa;
    b = sb;
}

// For stream s = blockIdx.x and each token t in order, at position p = *pos + t:
//   gate = <RMSNorm(key_s) wk_s, RMSNorm(h_s) wq_s> / sqrt(D), taken as a signed square root (magnitude >= 1e-6)
//   g = sigmoid(gate) val;  u = RMSNorm(g) wc_s, stored in the ring at slot p mod NG_RING
//   h_s += g + silu(w0 u(p - 9) + w1 u(p - 6) + w2 u(p - 3) + w3 u(p))          (u of negative positions = 0)
// A thread owns the same float4 of channels for every token, so the ring entries it reads are its own earlier
// writes or an earlier call's; the only barriers are the reductions'.  grid HC, min(1024, D/4 rounded up to 64)
// threads
__global__ void __launch_bounds__(1024) k_ngram_inject(InjectArgs a) {
    __shared__ float red[3][32];
    const int s = blockIdx.x, D4 = a.D / 4, nw = blockDim.x >> 6, HCD = a.HC * a.D;
    const int p0 = *a.pos;
    const float4 *wk = reinterpret_cast<const float4 *>(a.wk + (size_t) s * a.D);
    const float4 *wq = reinterpret_cast<const float4 *>(a.wq + (size_t) s * a.D);
    const float4 *wc = reinterpret_cast<const float4 *>(a.wc + (size_t) s * a.D);
    const float4 *cw = reinterpret_cast<const float4 *>(a.conv) + (size_t) s * a.D;  // [channel][4 taps]
    int r = 0;
    for (int t = 0; t < a.nt; ++t) {
        const int p = p0 + t;
        const float4 *kt = reinterpret_cast<const float4 *>(a.key + ((size_t) t * a.HC + s) * a.D);
        float4 *ht = reinterpret_cast<float4 *>(a.h + ((size_t) t * a.HC + s) * a.D);
        const float4 *vt = reinterpret_cast<const float4 *>(a.val + (size_t) t * a.D);
        float sk = 0.0f, sh = 0.0f;
        for (int c = threadIdx.x; c < D4; c += blockDim.x) {
            sk += sq4(kt[c]);
            sh += sq4(ht[c]);
        }
        wg_sum2(sk, sh, red[r], nw);
        r = (r + 1) % 3;
        const float rk = rsqrtf(sk / a.D + a.eps), rh = rsqrtf(sh / a.D + a.eps);
        float dot = 0.0f, dummy = 0.0f;
        for (int c = threadIdx.x; c < D4; c += blockDim.x) {
            const float4 kn = mul4(mul4(kt[c], rk), wk[c]), hn = mul4(mul4(ht[c], rh), wq[c]);
            dot += kn.x * hn.x + kn.y * hn.y + kn.z * hn.z + kn.w * hn.w;
        }
        wg_sum2(dot, dummy, red[r], nw);
        r = (r + 1) % 3;
        float gate = dot / sqrtf((float) a.D);
        if (gate != 0.0f) gate = copysignf(sqrtf(fmaxf(fabsf(gate), 1e-6f)), gate);
        const float sg = 1.0f / (1.0f + expf(-gate));
        float sv = 0.0f;
        for (int c = threadIdx.x; c < D4; c += blockDim.x) sv += sq4(mul4(vt[c], sg));
        wg_sum2(sv, dummy, red[r], nw);
        r = (r + 1) % 3;
        const float rv = rsqrtf(sv / a.D + a.eps);
        const size_t slot = (size_t) (p & (NG_RING - 1)) * HCD + (size_t) s * a.D;
        const size_t s3 = (size_t) ((p - 3) & (NG_RING - 1)) * HCD + (size_t) s * a.D;
        const size_t s6 = (size_t) ((p - 6) & (NG_RING - 1)) * HCD + (size_t) s * a.D;
        const size_t s9 = (size_t) ((p - 9) & (NG_RING - 1)) * HCD + (size_t) s * a.D;
        for (int c = threadIdx.x; c < D4; c += blockDim.x) {
            const float4 g = mul4(vt[c], sg), u = mul4(mul4(g, rv), wc[c]);
            reinterpret_cast<float4 *>(a.ring + slot)[c] = u;
            const float4 u3 = p >= 3 ? reinterpret_cast<const float4 *>(a.ring + s3)[c] : make_float4(0, 0, 0, 0);
            const float4 u6 = p >= 6 ? reinterpret_cast<const float4 *>(a.ring + s6)[c] : make_float4(0, 0, 0, 0);
            const float4 u9 = p >= 9 ? reinterpret_cast<const float4 *>(a.ring + s9)[c] : make_float4(0, 0, 0, 0);
            const float uu[4] = {u.x, u.y, u.z, u.w}, v3[4] = {u3.x, u3.y, u3.z, u3.w};
            const float v6[4] = {u6.x, u6.y, u6.z, u6.w}, v9[4] = {u9.x, u9.y, u9.z, u9.w};
            const float gg[4] = {g.x, g.y, g.z, g.w};
            float add[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 w = cw[4 * c + j];
                const float conv = w.x * v9[j] + w.y * v6[j] + w.z * v3[j] + w.w * uu[j];
                add[j] = gg[j] + silu1(conv);
            }
            const float4 hv = ht[c];
            ht[c] = make_float4(hv.x + add[0], hv.y + add[1], hv.z + add[2], hv.w + add[3]);
        }
    }
}

}  // namespace

int ngram_inject_launch(const NgramCall &c, const float *key, const float *val, float *h, const Layer &L,
                        hipStream_t st) {
    if (c.nt < 1 || c.nt > MAXT || c.D < 4 || c.D % 4 || c.HC < 1 || !c.pos || !key || !val || !h)
        FN_FAIL("ngram: bad arguments");
    InjectArgs a{c.nt, c.D, c.HC, c.eps, c.pos, key, val, L.f(NG_KNORM), L.f(NG_QNORM), L.f(NG_CNORM),
                 L.f(NG_CONVW), h, L.f(NG_HIST)};
    const unsigned threads = (unsigned) std::min(1024, (c.D / 4 + 63) / 64 * 64);
    hipLaunchKernelGGL(k_ngram_inject, dim3((unsigned) c.HC), dim3(threads), 0, st, a);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace fn

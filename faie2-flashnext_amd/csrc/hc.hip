// The hyper-connection write, the next read's per-stream RMSNorm and the read's down (+ inject) product in one
// kernel, for BF16 down weights (the reference model's): the reference runs the write (faie2fn.cu:1281-1327), the
// norm (:1226-1239) and the down GEMV (:1254-1265) as separate steps; here the first two ride in every workgroup of
// the third, so the model forward saves one launch per read.
#include "quant_impl.cuh"

namespace fn {

namespace {

constexpr int HC_RW = 1;          // rows of the down weight a wave sums (one: 4 rows a workgroup, the most workgroups)
constexpr int HC_DR = 4 * HC_RW;  // rows a workgroup sums
constexpr int HC_CH = 4;  // float4s of a stream a thread takes (D <= 4096)

// grid (ceil(R / HC_DR), HC), 256 threads; stream k = blockIdx.y.  Every workgroup of stream k computes, for t < NT,
//   v[t][c] = h[t][k][c] + y[t][c] inj[t][k]  (v = h without y),  hn[t][k][c] = v rsqrt(mean_c v^2 + eps) w[k D + c]
// with the same arithmetic (so the same bits), keeps hn in the LDS in the GEMV's x layout, and workgroup (0, k)
// writes v to hout (when y is given) and hn to hn.  Then its rows: part[k][t][r] = W[r][k D, k D + D) . hn[t][k],
// 64 lanes a row (lane l sums groups l, l + 64, ... in order, then the wave sum).  Token t's arithmetic does not
// depend on NT.
template <int NT>
__global__ void __launch_bounds__(256) k_hc_down(const float *__restrict__ h, const float *__restrict__ y,
                                                 const float *__restrict__ inj, const float *__restrict__ w, int D,
                                                 int HC, float eps, PP W, int R, float *__restrict__ hout,
                                                 float *__restrict__ hn, float *__restrict__ part) {
    extern __shared__ float4 xs[];  // [G][xs_stride(NT)]
    __shared__ float red[NT][4];
    constexpr int NWB = Q<QT_BF16>::NW, GPL = 2;  // groups per lane per row (G <= 128)
    constexpr bool PRE = NT <= 2;  // the streams of every token requested up front (8 float4 registers a token)
    const int k = blockIdx.y, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, G = D / 32, D4 = D / 4;
    const bool writer = blockIdx.x == 0;
    // Requests in the order their values are needed, since a value waits for everything requested before it (vmcnt
    // counts loads in issue order): the streams (h, and y when given; the y slot reads h again without one, unused)
    // and the norm weight, then the wave's rows' weight words, which only the dot product after the norm uses.
    // Every load is unconditional (indices clamped), so that all of them issue before the first wait.
    float4 hv[PRE ? NT : 1][HC_CH], yv[PRE ? NT : 1][HC_CH];
    if constexpr (PRE) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 *h4 = reinterpret_cast<const float4 *>(h + ((size_t) t * HC + k) * D);
            const float4 *y4 = reinterpret_cast<const float4 *>(y ? y + (size_t) t * D : h);
#pragma unroll
            for (int j = 0; j < HC_CH; ++j) {
                const int c = min(tid + 256 * j, D4 - 1);
                hv[t][j] = h4[c];
                yv[t][j] = y4[c];
            }
        }
    }
    // the norm weight of the thread's float4s (tid, tid + 256, ... < D / 4; at most HC_CH of them)
    const float4 *w4 = reinterpret_cast<const float4 *>(w + (size_t) k * D);
    float4 wc[HC_CH];
#pragma unroll
    for (int j = 0; j < HC_CH; ++j) wc[j] = w4[min(tid + 256 * j, D4 - 1)];
    uint32_t wr[HC_RW][GPL][NWB];
    const int r0 = blockIdx.x * HC_DR + wv * HC_RW;
#pragma unroll
    for (int j = 0; j < HC_RW; ++j) {
        RP rp = row_planes(W, min(r0 + j, R - 1));
        rp.b0 += (size_t) k * D * 2;  // stream k's columns
#pragma unroll
        for (int u = 0; u < GPL; ++u) Q<QT_BF16>::load(rp, min(lane + 64 * u, G - 1), wr[j][u]);
    }
    // v and its sum of squares, the thread's float4s in order for each token
    float ss[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float4 *h4 = reinterpret_cast<const float4 *>(h + ((size_t) t * HC + k) * D);
        const float4 *y4 = y ? reinterpret_cast<const float4 *>(y + (size_t) t * D) : nullptr;
        const float is = y ? inj[t * HC + k] : 0.0f;
        ss[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < HC_CH; ++j) {
            const int c = tid + 256 * j;
            if (c < D4) {
                float4 v;
                if constexpr (PRE) v = hv[t][j];
                else v = h4[c];
                if (y) {
                    if constexpr (PRE) v = add_scaled(v, yv[t][j], is);
                    else v = add_scaled(v, y4[c], is);
                    if (writer) reinterpret_cast<float4 *>(hout + ((size_t) t * HC + k) * D)[c] = v;
                }
                ss[t] += sumsq4(v);
                xs[(c >> 3) * xs_stride(NT) + t * 8 + (c & 7)] = v;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) ss[t] = wave_sum(ss[t]);
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) red[t][wv] = ss[t];
    }
    // LDS-only barriers: the waves exchange through the LDS alone, and the weight words stay in flight across them
    lds_barrier();
    // hn = v r w, in place in the LDS (each thread rescales the float4s it wrote)
    float r[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float sum = 0.0f;  // the wave partials in wave order, as block_sum adds them
#pragma unroll
        for (int i = 0; i < 4; ++i) sum += red[t][i];
        r[t] = rsqrtf(sum / D + eps);
    }
#pragma unroll
    for (int j = 0; j < HC_CH; ++j) {
        const int c = tid + 256 * j;
        if (c >= D4) break;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float4 *px = xs + (c >> 3) * xs_stride(NT) + t * 8 + (c & 7);
            const float4 v = *px, wj = wc[j];
            const float4 o = make_float4(v.x * r[t] * wj.x, v.y * r[t] * wj.y, v.z * r[t] * wj.z, v.w * r[t] * wj.w);
            *px = o;
            if (writer) reinterpret_cast<float4 *>(hn + ((size_t) t * HC + k) * D)[c] = o;
        }
    }
    lds_barrier();
    const NoTab T;
#pragma unroll
    for (int j = 0; j < HC_RW; ++j) {
        const int r = r0 + j;
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int u = 0; u < GPL; ++u) {
            const int g = lane + 64 * u;
            if (g < G) accumulate<QT_BF16, NT>(wr[j][u], g, xs + g * xs_stride(NT), acc, T);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = wave_sum(acc[t]);
        if (lane == 0 && r < R) {
#pragma unroll
            for (int t = 0; t < NT; ++t) part[((size_t) k * NT + t) * R + r] = acc[t];
        }
    }
}

template <int NT>
int hc_down_nt(const float *h, const float *y, const float *inj, const float *w, int D, int HC, float eps,
               const QLayout &L, const uint8_t *packed, float *hout, float *hn, float *part, hipStream_t st) {
    const size_t lds = (size_t) (D / 32) * xs_stride(NT) * sizeof(float4);
    hipLaunchKernelGGL(k_hc_down<NT>, dim3((unsigned) ((L.rows + HC_DR - 1) / HC_DR), (unsigned) HC), dim3(256), lds,
                       st, h, y, inj, w, D, HC, eps, planes(L, packed), L.rows, hout, hn, part);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace

bool hc_down_supported(const QLayout &L, int D, int HC) {
    return L.type == QT_BF16 && D % 32 == 0 && D / 4 <= 256 * HC_CH && L.cols == D * HC &&
           (size_t) (D / 32) * xs_stride(MAXNT) * sizeof(float4) <= (size_t) kLdsPerCu;
}

int hc_down_launch(const float *h, const float *y, const float *inj, const float *w, int D, int HC, float eps,
                   const QLayout &L, const uint8_t *packed, int nt, float *hout, float *hn, float *part,
                   hipStream_t st) {
    if (!hc_down_supported(L, D, HC)) FN_FAIL("hc down: not built for this weight");
    if (!h || !w || !packed || !hn || !part || (y && (!inj || !hout))) FN_FAIL("hc down: null pointer");
    switch (nt) {
        case 1: return hc_down_nt<1>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 2: return hc_down_nt<2>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 3: return hc_down_nt<3>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 4: return hc_down_nt<4>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 5: return hc_down_nt<5>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 6: return hc_down_nt<6>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 7: return hc_down_nt<7>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        case 8: return hc_down_nt<8>(h, y, inj, w, D, HC, eps, L, packed, hout, hn, part, st);
        default: FN_FAIL("hc down: nt must be 1..8");
    }
}

}  // namespace fn

// The MoE output kernel (quant_impl.cuh, k_moe_down) for every expert format, with the shared expert's down
// weight in Q8_0 (the reference model's, flashnext/inspect_fn.txt).  The reference runs the routed experts' down
// rows, the shared expert's down GEMV and the weighted sum as separate steps (engine/faie2fn.cu:2293-2348).
#include "quant_impl.cuh"

namespace fn {

namespace {

// The MoE output of each token, the routed experts' down rows and the shared expert's in one pass:
//   y[t][r] = fma(sigmoid(rsg[t][NE]), Ws[r] . sha[t], m),  m = sum over k in order of fma(wsel[t][k], d_k, m),
//   d_k = We[sel[t][k] R + r] . act[t NEU + k].
// Every dot product has the arithmetic of k_rows (16 lanes per row, lane li sums groups li, li + 16, ... in order,
// then the 16-lane sum) and the sums run in item order (expert k < NEU, then the shared expert), so both kernels
// below give the same bits.  G <= 16 MOE_GPL (rows of at most 1024 values).  256 threads.
constexpr int MOE_GPL = 2;  // groups per lane per row: G <= 16 MOE_GPL

// One-token calls: a workgroup takes 4 rows and its 4 waves split the items (item i to wave i % 4; lanes
// 16 q .. 16 q + 15 of a wave take row q), four times the workgroups of the 16-row kernel.  A pass requests the
// weight words of up to MOE_IPW items per wave and stages their x rows (act or sha) into the LDS (9 float4 per
// group); the dot products go to the LDS and one lane per row sums them.  grid (ceil(R / 4), nt).
constexpr int MOE_IPW = 4;  // items a wave holds in registers in one pass

template <uint32_t TY, uint32_t TS>
__global__ void __launch_bounds__(256) k_moe_down4(PP Pe, PP Ps, int R, int nexp, int G, int cols,
                                                   const int32_t *__restrict__ sel, const float *__restrict__ wsel,
                                                   int NEU, const float *__restrict__ act,
                                                   const float *__restrict__ sha, const float *__restrict__ rsg,
                                                   int NE, float *__restrict__ y) {
    extern __shared__ float4 xs[];  // [NEU + 1][G][9], then (floats) the dot products [NEU + 1][4] and factors
    constexpr int NW = Q<TY>::NW, NWS = Q<TS>::NW;
    // (the wave index made visibly uniform: the items' expert ids are then scalar loads, which do not wait behind the
    // weight words already requested the way a vector load would)
    const int t = blockIdx.y, tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63,
              li = lane & 15, q = lane >> 4;
    const int r = blockIdx.x * 4 + q, rr = min(r, R - 1), NI = NEU + 1, G8 = G * 8;
    float *dsum = reinterpret_cast<float *>(xs + (size_t) NI * G * 9), *wl = dsum + NI * 4;
    const int32_t *es = sel + (size_t) t * NEU;
    // the sums' factors, staged now so that the final sums read only the LDS: wl[k] = wsel[t][k], wl[NEU] = sigmoid
    // of the shared expert's gate logit
    for (int k = tid; k < NI; k += 256)
        wl[k] = k < NEU ? wsel[(size_t) t * NEU + k] : sigmoidf_(rsg[(size_t) t * (NE + 1) + NE]);
    for (int p0 = 0; p0 < NI; p0 += 4 * MOE_IPW) {  // (the same count in every wave)
        const int i0 = p0 + w;
        // the pass's x rows (items p0 .. p0 + 4 MOE_IPW - 1), by the whole workgroup: requested first
        const int ni = min(NI - p0, 4 * MOE_IPW), nx = ni * G8;
        const auto xsrc = [&](int e) {
            const int i = p0 + e / G8, j = e - (i - p0) * G8;
            return reinterpret_cast<const float4 *>(i < NEU ? act + ((size_t) t * NEU + i) * cols
                                                            : sha + (size_t) t * cols)[j];
        };
        const auto xdst = [&](int e, float4 v) {
            const int i = p0 + e / G8, j = e - (i - p0) * G8;
            xs[(i * G + (j >> 3)) * 9 + (j & 7)] = v;
        };
        LdsStage<8> xst;
        xst.load(nx, 0, tid, 256, xsrc);
        uint32_t we[MOE_IPW][MOE_GPL][NW], ws[MOE_GPL][NWS];
        const bool has_s = (NEU - i0) % 4 == 0 && NEU >= i0 && NEU < i0 + 4 * MOE_IPW;  // the shared item is ours
        // weight words of the wave's items i0 + 4 j (groups li + 16 u, clamped to valid addresses).  Every load is
        // issued, unconditionally: a slot past the experts re-requests the wave's last expert row (already on its
        // way, so no new traffic), and every wave requests the shared row.  (Loads under a branch were merged into
        // the array after the branch by register copies, each waiting for the load: one round trip per item.)
        const int ilast = w < NEU ? w + 4 * ((NEU - 1 - w) / 4) : 0;
#pragma unroll
        for (int j = 0; j < MOE_IPW; ++j) {
            const int i = i0 + 4 * j, ie = i < NEU ? i : ilast;
            const RP rp = row_planes(Pe, min(max(es[ie], 0), nexp - 1) * R + rr);
#pragma unroll
            for (int u = 0; u < MOE_GPL; ++u) Q<TY>::load(rp, min(li + 16 * u, G - 1), we[j][u]);
        }
        {
            const RP rp = row_planes(Ps, rr);
#pragma unroll
            for (int u = 0; u < MOE_GPL; ++u) Q<TS>::load(rp, min(li + 16 * u, G - 1), ws[u]);
        }
        if (p0 == 0) {
            tab_fill<TY>(tid, 256);
            tab_fill<TS>(tid, 256);
        }
        // the pass's x rows (items p0 .. p0 + 4 MOE_IPW - 1) -> LDS, by the whole workgroup
        xst.store(nx, 0, tid, 256, xdst);
        stage_rest<8>(nx, tid, 256, xsrc, xdst);
        __syncthreads();
        const TabT<TY> T;
#pragma unroll
        for (int j = 0; j < MOE_IPW; ++j) {
            const int i = i0 + 4 * j;
            if (i < NEU) {
                float d = 0.0f;
#pragma unroll
                for (int u = 0; u < MOE_GPL; ++u) {
                    const int g = li + 16 * u;
                    if (g < G) accumulate<TY, 1>(we[j][u], g, xs + (i * G + g) * 9, &d, T);
                }
                d = row_sum(d);
                if (li == 0) dsum[i * 4 + q] = d;
            }
        }
        if (has_s) {
            const TabT<TS> TSt;
            float d = 0.0f;
#pragma unroll
            for (int u = 0; u < MOE_GPL; ++u) {
                const int g = li + 16 * u;
                if (g < G) accumulate<TS, 1>(ws[u], g, xs + (NEU * G + g) * 9, &d, TSt);
            }
            d = row_sum(d);
            if (li == 0) dsum[NEU * 4 + q] = d;
        }
    }
    __syncthreads();
    if (tid < 4 && blockIdx.x * 4 + tid < R) {
        float m = 0.0f;
        for (int k = 0; k < NEU; ++k) m = __builtin_fmaf(wl[k], dsum[k * 4 + tid], m);
        y[(size_t) t * R + blockIdx.x * 4 + tid] = __builtin_fmaf(wl[NEU], dsum[NEU * 4 + tid], m);
    }
}

// Several tokens: a workgroup takes 16 rows of one token, wave w rows 4 w .. 4 w + 3 and every item, so the x rows
// are staged once for 16 rows.  The experts' weight words are requested KC at a time, the next KC while the
// current ones are summed, and the shared expert's with the first.  grid (ceil(R / 16), nt).
template <uint32_t TY> constexpr int moe_kc() { return Q<TY>::NW <= 5 ? 4 : (Q<TY>::NW <= 10 ? 2 : 1); }

template <uint32_t TY, uint32_t TS>
__global__ void __launch_bounds__(256) k_moe_down16(PP Pe, PP Ps, int R, int nexp, int G, int cols,
                                                    const int32_t *__restrict__ sel, const float *__restrict__ wsel,
                                                    int NEU, const float *__restrict__ act,
                                                    const float *__restrict__ sha, const float *__restrict__ rsg,
                                                    int NE, float *__restrict__ y) {
    extern __shared__ float4 xs[];  // [NEU + 1][G][9]
    constexpr int NW = Q<TY>::NW, NWS = Q<TS>::NW, KC = moe_kc<TY>();
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, li = lane & 15;
    const int r = blockIdx.x * 16 + (tid >> 6) * 4 + (lane >> 4), rr = min(r, R - 1);
    const int32_t *es = sel + (size_t) t * NEU;
    uint32_t wa[KC][MOE_GPL][NW], wb[KC][MOE_GPL][NW], ws[MOE_GPL][NWS];
    // experts [k0, k0 + KC) of the token, row rr, groups li + 16 u (clamped: valid addresses, values unused)
    const auto load = [&](int k0, uint32_t (&w)[KC][MOE_GPL][NW]) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int e = min(max(es[min(k0 + j, NEU - 1)], 0), nexp - 1);
            const RP rp = row_planes(Pe, e * R + rr);
#pragma unroll
            for (int u = 0; u < MOE_GPL; ++u) Q<TY>::load(rp, min(li + 16 * u, G - 1), w[j][u]);
        }
    };
    // the token's x rows requested first, then the weight words
    const int G8 = G * 8, nx = (NEU + 1) * G8;
    const auto xsrc = [&](int i) {
        const int k = i / G8, j = i - k * G8;
        return reinterpret_cast<const float4 *>(k < NEU ? act + ((size_t) t * NEU + k) * cols
                                                        : sha + (size_t) t * cols)[j];
    };
    const auto xdst = [&](int i, float4 v) {
        const int k = i / G8, j = i - k * G8;
        xs[(k * G + (j >> 3)) * 9 + (j & 7)] = v;
    };
    LdsStage<8> xst;
    xst.load(nx, 0, tid, 256, xsrc);
    load(0, wa);
    {
        const RP rp = row_planes(Ps, rr);
#pragma unroll
        for (int u = 0; u < MOE_GPL; ++u) Q<TS>::load(rp, min(li + 16 * u, G - 1), ws[u]);
    }
    if (KC < NEU) load(KC, wb);
    xst.store(nx, 0, tid, 256, xdst);
    stage_rest<8>(nx, tid, 256, xsrc, xdst);
    tab_fill<TY>(tid, 256);
    tab_fill<TS>(tid, 256);
    __syncthreads();
    const TabT<TY> T;
    float m = 0.0f;
    // the KC experts of w, starting at k0, onto m in order
    const auto sum = [&](int k0, const uint32_t (&w)[KC][MOE_GPL][NW]) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int k = k0 + j;
            if (k >= NEU) break;  // (uniform)
            float d = 0.0f;
#pragma unroll
            for (int u = 0; u < MOE_GPL; ++u) {
                const int g = li + 16 * u;
                if (g < G) accumulate<TY, 1>(w[j][u], g, xs + (k * G + g) * 9, &d, T);
            }
            d = row_sum(d);
            m = __builtin_fmaf(wsel[(size_t) t * NEU + k], d, m);
        }
    };
    for (int k0 = 0; k0 < NEU; k0 += 2 * KC) {
        sum(k0, wa);
        if (k0 + 2 * KC < NEU) load(k0 + 2 * KC, wa);
        if (k0 + KC >= NEU) break;
        sum(k0 + KC, wb);
        if (k0 + 3 * KC < NEU) load(k0 + 3 * KC, wb);
    }
    const TabT<TS> TSt;
    float d = 0.0f;
#pragma unroll
    for (int u = 0; u < MOE_GPL; ++u) {
        const int g = li + 16 * u;
        if (g < G) accumulate<TS, 1>(ws[u], g, xs + (NEU * G + g) * 9, &d, TSt);
    }
    d = row_sum(d);
    if (li == 0 && r < R)
        y[(size_t) t * R + r] = __builtin_fmaf(sigmoidf_(rsg[(size_t) t * (NE + 1) + NE]), d, m);
}

// the kernel forced by moe_down_override: 0 automatic, 1 the 16-row kernel, 4 the 4-row kernel
int g_moe_down_waves = 0;

template <uint32_t TY, uint32_t TS>
int moe_down_t(const QLayout &Le, const PP &Pe, const QLayout &Ls, const PP &Ps, int R, const int32_t *sel,
               const float *wsel, int NEU, const float *act, const float *sha, const float *rsg, int NE, int nt,
               float *y, hipStream_t st) {
    const int G = Le.cols / 32;
    const size_t xl = (size_t) (NEU + 1) * G * 9 * sizeof(float4);
    if (g_moe_down_waves == 4 || (g_moe_down_waves == 0 && nt == 1))
        hipLaunchKernelGGL((k_moe_down4<TY, TS>), dim3((unsigned) ((R + 3) / 4), (unsigned) nt), dim3(256),
                           xl + (size_t) (NEU + 1) * 5 * sizeof(float), st, Pe, Ps, R, Le.rows / R, G, Le.cols, sel,
                           wsel, NEU, act, sha, rsg, NE, y);
    else
        hipLaunchKernelGGL((k_moe_down16<TY, TS>), dim3((unsigned) ((R + 15) / 16), (unsigned) nt), dim3(256), xl,
                           st, Pe, Ps, R, Le.rows / R, G, Le.cols, sel, wsel, NEU, act, sha, rsg, NE, y);
    FN_CK(hipGetLastError());
    return 0;
}

}  // namespace

void moe_down_override(int waves_per_row) {
    g_moe_down_waves = waves_per_row < 0 ? 0 : (waves_per_row == 1 ? 1 : (waves_per_row > 1 ? 4 : g_moe_down_waves));
}

bool moe_down_supported(const QLayout &Le, const QLayout &Ls, int R, int NEU) {
    const int G = Le.cols / 32;
    if (Ls.type != QT_Q8_0 || Ls.cols != Le.cols || Ls.rows != R || G < 1 || G > 16 * MOE_GPL) return false;
    // the x rows of a token's NEU + 1 items, their dot products and factors in the LDS beside a grid format's tables
    const size_t lds = (size_t) (NEU + 1) * G * 9 * sizeof(float4) + (size_t) (NEU + 1) * 5 * sizeof(float) +
                       (size_t) tab_lds<QT_IQ2_S>();  // (the largest codebook and sign masks of any format)
    if (NEU < 1 || NEU > 64 || lds > (size_t) kLdsPerCu) return false;
    switch (Le.type) {
        case QT_BF16: case QT_Q8_0: case QT_IQ4_NL: case QT_IQ4_XS: case QT_IQ3_S: case QT_IQ2_XXS: case QT_IQ2_XS:
        case QT_IQ2_S: case QT_IQ3_XXS: case QT_Q2_0: case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: return true;
        default: return false;
    }
}

int moe_down_launch(const QLayout &Le, const uint8_t *pe, const QLayout &Ls, const uint8_t *ps, int R,
                    const int32_t *sel, const float *wsel, int NEU, const float *act, const float *sha, const float *rsg,
                    int NE, int nt, float *y, hipStream_t st) {
    if (!moe_down_supported(Le, Ls, R, NEU)) FN_FAIL("moe down: formats or shapes not built");
    if (!pe || !ps || !sel || !wsel || !act || !sha || !rsg || !y || nt < 1 || NEU < 1 || NEU > 64 || R < 1 ||
        Le.rows % R)
        FN_FAIL("moe down: bad arguments");
    if (((uintptr_t) act | (uintptr_t) sha) % 16) FN_FAIL("moe down: act and sha must be 16-byte aligned");
    const PP Pe = planes(Le, pe), Ps = planes(Ls, ps);
#define FN_MOE(T)                                                                                                    \
    case T: return moe_down_t<T, QT_Q8_0>(Le, Pe, Ls, Ps, R, sel, wsel, NEU, act, sha, rsg, NE, nt, y, st);
    switch (Le.type) {
        FN_MOE(QT_BF16)
        FN_MOE(QT_Q8_0)
        FN_MOE(QT_IQ4_NL)
        FN_MOE(QT_IQ4_XS)
        FN_MOE(QT_IQ3_S)
        FN_MOE(QT_IQ2_XXS)
        FN_MOE(QT_IQ2_XS)
        FN_MOE(QT_IQ2_S)
        FN_MOE(QT_IQ3_XXS)
        FN_MOE(QT_Q2_0)
        FN_MOE(QT_Q4_K)
        FN_MOE(QT_Q5_K)
        FN_MOE(QT_Q6_K)
        default: FN_FAIL("moe down: unsupported type");
    }
#undef FN_MOE
}

}  // namespace fn

// Grouped GEMV instantiations: the format sets of the model's projections that read one activation row
// (quant_impl.cuh, k_gemv_grp).  The reference runs these as separate GEMVs (engine/faie2fn.cu:2385-2404,
// 2416-2424); here they share one launch and one staging of x per workgroup.
#include "quant_impl.cuh"

namespace fn {

namespace {

// the format sets built as one launch, each in the order its parts take the kernel's slots
//   {IQ4_XS, IQ3_S, BF16}: DeltaNet qkv / z / alpha-beta (z in IQ3_S), FFN shared gate / shared up / router
//   {IQ4_XS, Q6_K, BF16}: DeltaNet qkv / z / alpha-beta (z in Q6_K)
//   {IQ4_XS, IQ4_XS, Q6_K, BF16}: attention q / k / v / indexer q-and-k
constexpr int kKinds = 3;
constexpr uint32_t kKind[kKinds][4] = {{QT_IQ4_XS, QT_IQ3_S, QT_BF16, 0},
                                       {QT_IQ4_XS, QT_Q6_K, QT_BF16, 0},
                                       {QT_IQ4_XS, QT_IQ4_XS, QT_Q6_K, QT_BF16}};
constexpr int kKindN[kKinds] = {3, 3, 4};

int launch_kind(int k, const QLayout *const *L, const PP *P, float *const *y, const float *x, int nt, int lpr,
                hipStream_t st) {
    switch (k) {
        case 0: return gemv_grp<QT_IQ4_XS, QT_IQ3_S, QT_BF16>(L, P, y, x, nt, lpr, st);
        case 1: return gemv_grp<QT_IQ4_XS, QT_Q6_K, QT_BF16>(L, P, y, x, nt, lpr, st);
        default: return gemv_grp<QT_IQ4_XS, QT_IQ4_XS, QT_Q6_K, QT_BF16>(L, P, y, x, nt, lpr, st);
    }
}

}  // namespace

int gemv_group_launch(const GemvPart *parts, int n, const float *x, int nt, hipStream_t st) {
    if (n < 1 || n > 4 || !parts || !x) FN_FAIL("gemv group: 1 to 4 parts and x");
    if (nt < 1 || nt > MAXNT) FN_FAIL("gemv: nt must be 1..8");
    for (int i = 0; i < n; ++i) {
        const GemvPart &g = parts[i];
        if (!g.L || !g.packed || !g.y) FN_FAIL("gemv group: null part");
        if (g.L->cols != parts[0].L->cols) FN_FAIL("gemv group: parts differ in cols");
        if (!gemv_planes_fit(*g.L)) FN_FAIL("gemv: a plane of the packed weight exceeds 4 GiB");
    }
    // a matching format set: every slot takes the first unused part of its format
    int kind = -1, slot_of[4] = {0, 0, 0, 0};
    for (int k = 0; k < kKinds && kind < 0; ++k) {
        if (kKindN[k] != n) continue;
        bool used[4] = {false, false, false, false}, ok = true;
        for (int s = 0; s < n && ok; ++s) {
            ok = false;
            for (int i = 0; i < n; ++i)
                if (!used[i] && parts[i].L->type == kKind[k][s]) {
                    used[i] = ok = true;
                    slot_of[s] = i;
                    break;
                }
        }
        if (ok) kind = k;
    }
    // x of MAXNT tokens in the LDS beside the codebooks (IQ3_S: its grid and the sign masks, 4 KiB): sized for the
    // largest call, so that whether the parts share a launch never depends on nt (token t of an nt-token call keeps
    // the bits of a one-token call); the separate launches take no split-K, like the grouped one
    // (and the half sums of x when a part's format has a minimum: Q6_K in kinds 1 and 2)
    bool fac = false;
    for (int s = 0; kind >= 0 && s < kKindN[kind]; ++s)
        fac = fac || kKind[kind][s] == QT_Q4_K || kKind[kind][s] == QT_Q5_K || kKind[kind][s] == QT_Q6_K;
    const size_t xlds = (size_t) (parts[0].L->cols / 32) *
                        (xs_stride(MAXNT) * sizeof(float4) + (fac ? MAXNT * 2 * sizeof(float) : 0));
    if (kind < 0 || xlds + (size_t) tab_lds<QT_IQ3_S>() > (size_t) kLdsPerCu) {
        for (int i = 0; i < n; ++i)
            if (gemv_launch(*parts[i].L, parts[i].packed, x, nt, parts[i].y, nullptr, 0, st, 1)) return -1;
        return 0;
    }
    // lanes per row: the fewest any part's own plan takes, at least 32 (the group is built for 32 and 64)
    int lpr = 64;
    const QLayout *L[4];
    PP P[4];
    float *y[4];
    for (int s = 0; s < n; ++s) {
        const GemvPart &g = parts[slot_of[s]];
        lpr = std::min(lpr, std::max(32, gemv_plan(*g.L).lpr));
        L[s] = g.L;
        P[s] = planes(*g.L, g.packed);
        y[s] = g.y;
    }
    if ((uintptr_t) x % 16) FN_FAIL("gemv: weight and x must be 16-byte aligned");
    for (int s = 0; s < n; ++s)
        if ((uintptr_t) parts[s].packed % 16) FN_FAIL("gemv: weight and x must be 16-byte aligned");
    return launch_kind(kind, L, P, y, x, nt, lpr, st);
}

}  // namespace fn

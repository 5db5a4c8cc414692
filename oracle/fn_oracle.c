/*
 * fn_oracle.c -- float64 CPU restatement of the FAIE2-FlashNext decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels of libfaie2fn.so: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The product path never calls it and has no
 * CPU fallback.
 *
 * Every function restates the arithmetic of the reference CUDA engine (engine/faie2fn.cu) in float64 on the same
 * fp32 inputs; the citations name the reference lines each step follows.  Two conventions are kept on purpose
 * because they change results beyond 1e-5:
 *   - the RoPE angle is the fp32 product (float) pos * inv_freq_f32 (faie2fn.cu:1440, 2573-2576); only cos/sin
 *     of that fp32 angle are evaluated in float64;
 *   - the softplus in the decay gate switches to the identity above 20 (faie2fn.cu:1409).
 *
 * Layouts (all C-contiguous, batch-major; b = sequence, t = token of this call, C = 2*nkh*dk + nvh*dv):
 *   qkv [B][nt][C] channel order [q: kh*dk+i][k: nkh*dk + kh*dk+i][v: 2*nkh*dk + h*dv+j]  (faie2fn.cu:1377)
 *   conv_w [C][4] oldest tap first (faie2fn.cu:1383, 1392-1395)
 *   conv_state [B][3][C] raw inputs of the three previous tokens, oldest first
 *   ab [B][nt][2*nvh] alpha rows 0..nvh-1, beta rows nvh..2nvh-1 (faie2fn.cu:1407-1408)
 *   S [B][nvh][dk][dv] row = key index i, column = value index j (faie2fn.cu:1386-1388)
 *   z, out [B][nt][nvh*dv]
 *   attention: qg [B][nt][nq][2][hd] (query then gate per head, faie2fn.cu:1463, 1686),
 *   k/v new rows [B][nt][nkv][hd], cache rows [B][max_ctx][nkv][hd] (faie2fn.cu:1461, 1477), og [B][nt][nq][hd].
 *
 * Head maps: head_map 0 = tiled, value head h reads key head h % nkh (faie2fn.cu:10-11, 1374);
 *            head_map 1 = grouped, key head h / (nvh / nkh) (the layout of HF Qwen3-Next checkpoints).
 * Gate activation of the gated RMSNorm: 0 = sigmoid (faie2fn.cu:1363, 1424), 1 = silu.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

static int g_threads = 0;

EXPORT void orc_set_threads(int n) { g_threads = n; }

EXPORT int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int nthreads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

static double silu_d(double x) { return x / (1.0 + exp(-x)); }         /* faie2fn.cu:301 */
static double sigm_d(double x) { return 1.0 / (1.0 + exp(-x)); }       /* faie2fn.cu:309 */

static int key_head(int h, int nkh, int nvh, int head_map) {
    return head_map == 0 ? h % nkh : h / (nvh / nkh);
}

/* log-decay of value head h from its alpha logit: ssm_a * softplus(a + dt_bias), softplus = identity above 20
 * (faie2fn.cu:1408-1410). */
static double gdn_log_decay(double a, double dtb, double ssm_a) {
    const double x = a + dtb;
    const double sp = x > 20.0 ? x : log1p(exp(x));
    return sp * ssm_a;
}

/* Delta rule on one value head for one token (faie2fn.cu:1411-1421), in float64:
 *   kv_j = sum_i S_ij k_i (old S); delta_j = beta (v_j - gamma kv_j); S_ij <- gamma S_ij + k_i delta_j;
 *   o_j = sum_i S_ij q_i / sqrt(dk) over the updated S. */
static void delta_rule(int dk, int dv, double *S, const double *q, const double *k, const double *v, double beta,
                       double gamma, double *o) {
    double *kv = (double *) malloc(sizeof(double) * (size_t) dv);
    for (int j = 0; j < dv; ++j) kv[j] = 0.0;
    for (int i = 0; i < dk; ++i)
        for (int j = 0; j < dv; ++j) kv[j] += S[(size_t) i * dv + j] * k[i];
    for (int j = 0; j < dv; ++j) {
        const double delta = (v[j] - gamma * kv[j]) * beta;
        kv[j] = delta;
    }
    for (int j = 0; j < dv; ++j) o[j] = 0.0;
    for (int i = 0; i < dk; ++i)
        for (int j = 0; j < dv; ++j) {
            double *s = &S[(size_t) i * dv + j];
            *s = gamma * *s + k[i] * kv[j];
            o[j] += *s * q[i];
        }
    const double scale = 1.0 / sqrt((double) dk);  /* GDN_SCALE, faie2fn.cu:1352 */
    for (int j = 0; j < dv; ++j) o[j] *= scale;
    free(kv);
}

/* DeltaNet core (the state part of k_gdn, faie2fn.cu:1407-1421) on already normalized q, k and given beta and
 * log-decay g: gamma = exp(g).  q,k [B][nt][nkh][dk]; v [B][nt][nvh][dv]; beta,g [B][nt][nvh]; S in/out;
 * o [B][nt][nvh][dv]. */
EXPORT void orc_gdn_core(int B, int nkh, int nvh, int dk, int dv, int head_map, int nt, const float *q,
                         const float *k, const float *v, const float *beta, const float *g, double *S, double *o) {
    const int nt_ = nthreads();
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt_)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < nvh; ++h) {
            const int kh = key_head(h, nkh, nvh, head_map);
            double *qd = (double *) malloc(sizeof(double) * (size_t) (2 * dk + dv));
            double *kd = qd + dk, *vd = kd + dk;
            double *Sh = S + ((size_t) b * nvh + h) * dk * dv;
            for (int t = 0; t < nt; ++t) {
                const size_t bt = (size_t) b * nt + t;
                for (int i = 0; i < dk; ++i) {
                    qd[i] = q[(bt * nkh + kh) * dk + i];
                    kd[i] = k[(bt * nkh + kh) * dk + i];
                }
                for (int j = 0; j < dv; ++j) vd[j] = v[(bt * nvh + h) * dv + j];
                const double bt_ = beta[bt * nvh + h], gm = exp((double) g[bt * nvh + h]);
                delta_rule(dk, dv, Sh, qd, kd, vd, bt_, gm, o + (bt * nvh + h) * dv);
            }
            free(qd);
        }
}

/* Fused DeltaNet block, k_gdn (faie2fn.cu:1366-1431) for B sequences:
 *   conv: x^ = silu(w0 x[t-3] + w1 x[t-2] + w2 x[t-1] + w3 x[t]) per channel, state advanced (:1392-1398)
 *   l2norm q, k: x * rsqrt(sum x^2 + 1e-6) (:1399-1402)
 *   beta = sigmoid(b), gamma = exp(ssm_a * softplus(a + dt_bias)) (:1407-1410)
 *   delta rule + readout (:1411-1421)
 *   gated RMSNorm: on = o * rsqrt(mean o^2 + eps) * w * act(z) (:1422-1424). */
EXPORT void orc_gdn_block(int B, int nkh, int nvh, int dk, int dv, int head_map, int gate_act, int nt,
                          const float *qkv, const float *conv_w, double *conv_state, const float *ab,
                          const float *dt_bias, const float *ssm_a, double *S, const float *z,
                          const float *norm_w, double eps, double *out) {
    const int C = 2 * nkh * dk + nvh * dv;
    const int nt_ = nthreads();
    double *xh = (double *) malloc(sizeof(double) * (size_t) B * C);   /* conv + silu outputs of one token */
    for (int t = 0; t < nt; ++t) {
#pragma omp parallel for schedule(static) num_threads(nt_)
        for (int b = 0; b < B; ++b) {
            const float *x = qkv + ((size_t) b * nt + t) * C;
            double *st = conv_state + (size_t) b * 3 * C;
            double *xb = xh + (size_t) b * C;
            for (int c = 0; c < C; ++c) {
                const float *w = conv_w + (size_t) c * 4;
                const double acc = (double) w[0] * st[c] + (double) w[1] * st[C + c] + (double) w[2] * st[2 * C + c] +
                                   (double) w[3] * (double) x[c];
                xb[c] = silu_d(acc);
                st[c] = st[C + c];
                st[C + c] = st[2 * C + c];
                st[2 * C + c] = (double) x[c];
            }
            /* l2norm of the q and k vectors of every key head */
            for (int kh = 0; kh < nkh; ++kh)
                for (int part = 0; part < 2; ++part) {
                    double *p = xb + part * nkh * dk + kh * dk;
                    double ss = 0.0;
                    for (int i = 0; i < dk; ++i) ss += p[i] * p[i];
                    const double r = 1.0 / sqrt(ss + 1e-6);
                    for (int i = 0; i < dk; ++i) p[i] *= r;
                }
        }
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt_)
        for (int b = 0; b < B; ++b)
            for (int h = 0; h < nvh; ++h) {
                const int kh = key_head(h, nkh, nvh, head_map);
                const double *xb = xh + (size_t) b * C;
                const double *qd = xb + kh * dk, *kd = xb + nkh * dk + kh * dk, *vd = xb + 2 * nkh * dk + h * dv;
                const size_t bt = (size_t) b * nt + t;
                const float *abt = ab + bt * 2 * nvh;
                const double beta = sigm_d((double) abt[nvh + h]);
                const double gamma = exp(gdn_log_decay((double) abt[h], (double) dt_bias[h], (double) ssm_a[h]));
                double *Sh = S + ((size_t) b * nvh + h) * dk * dv;
                double *o = out + bt * nvh * dv + (size_t) h * dv;
                delta_rule(dk, dv, Sh, qd, kd, vd, beta, gamma, o);
                double ss = 0.0;
                for (int j = 0; j < dv; ++j) ss += o[j] * o[j];
                const double r = 1.0 / sqrt(ss / dv + eps);
                const float *zz = z + bt * nvh * dv + (size_t) h * dv;
                for (int j = 0; j < dv; ++j) {
                    const double gz = gate_act == 0 ? sigm_d((double) zz[j]) : silu_d((double) zz[j]);
                    o[j] = o[j] * r * (double) norm_w[j] * gz;
                }
            }
    }
    free(xh);
}

/* inv_freq[i] = (float)(1 / theta^(2i/nrot)), computed in double and rounded to fp32 (faie2fn.cu:2573-2576). */
EXPORT void orc_rope_inv_freq(int nrot, double theta, float *inv) {
    for (int i = 0; i < nrot / 2; ++i) inv[i] = (float) (1.0 / pow(theta, (double) (2 * i) / nrot));
}

/* RMSNorm x * rsqrt(mean x^2 + eps) * w, then RoPE on dims < nrot with pairs (i, i + nrot/2) at position pos
 * (faie2fn.cu:1438-1445, 1466-1474).  x fp32 in, y float64 out. */
static void norm_rope(int hd, int nrot, const float *inv, double eps, int pos, const float *x, const float *w,
                      double *y) {
    double ss = 0.0;
    for (int d = 0; d < hd; ++d) ss += (double) x[d] * (double) x[d];
    const double r = 1.0 / sqrt(ss / hd + eps);
    for (int d = 0; d < hd; ++d) y[d] = (double) x[d] * r * (double) w[d];
    for (int i = 0; i < nrot / 2; ++i) {
        const float ang = (float) pos * inv[i];  /* fp32 angle, as the reference */
        const double cs = cos((double) ang), sn = sin((double) ang);
        const double a = y[i], b = y[i + nrot / 2];
        y[i] = a * cs - b * sn;
        y[i + nrot / 2] = b * cs + a * sn;
    }
}

/* GQA decode attention for nt new tokens of B sequences (k_qk_norm_rope + k_attn_split + k_attn_combine,
 * faie2fn.cu:1451-1478, 1612-1690, with the indexer mask null = dense):
 *   Q = rope(rmsnorm(q) * wq), K_new = rope(rmsnorm(k) * wk), V_new = v, appended at positions pos[b] + t;
 *   token t of sequence b attends keys 0 .. pos[b] + t (cache rows < pos[b] from Kc/Vc, the rest new);
 *   q head h uses kv head h / (nq / nkv) (faie2fn.cu:1621); score = q.k / sqrt(hd) (:1646);
 *   og = softmax-weighted V * sigmoid(gate) (:1686-1689).
 * Kc, Vc [B][max_ctx][nkv][hd] fp32 are read for rows < pos[b] only.  Outputs: knew_o/vnew_o [B][nt][nkv][hd]
 * (the appended rows), og [B][nt][nq][hd]. */
EXPORT void orc_attn_masked(int B, int nq, int nkv, int hd, int nrot, double theta, double eps, int nt, const int *pos,
                            const float *qg, const float *knew, const float *vnew, const float *wq, const float *wk,
                            int max_ctx, const float *Kc, const float *Vc, const uint8_t *mask, int mstride, int ixr,
                            int top, double *knew_o, double *vnew_o, double *og) {
    float *inv = (float *) malloc(sizeof(float) * (size_t) (nrot / 2 + 1));
    orc_rope_inv_freq(nrot, theta, inv);
    const int grp = nq / nkv;
    const double scale = 1.0 / sqrt((double) hd);
    const int nt_ = nthreads();
    /* new K/V rows */
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < nt; ++t)
            for (int g = 0; g < nkv; ++g) {
                const size_t i = (((size_t) b * nt + t) * nkv + g) * hd;
                norm_rope(hd, nrot, inv, eps, pos[b] + t, knew + i, wk, knew_o + i);
                for (int d = 0; d < hd; ++d) vnew_o[i + d] = (double) vnew[i + d];
            }
#pragma omp parallel for collapse(3) schedule(dynamic) num_threads(nt_)
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < nt; ++t)
            for (int h = 0; h < nq; ++h) {
                const int g = h / grp, p = pos[b] + t, nk = p + 1;
                double *qd = (double *) malloc(sizeof(double) * (size_t) hd * 2);
                double *acc = qd + hd;
                double *sc = (double *) malloc(sizeof(double) * (size_t) nk);
                const float *qrow = qg + (((size_t) b * nt + t) * nq + h) * 2 * hd;
                norm_rope(hd, nrot, inv, eps, p, qrow, wq, qd);
                /* with a block mask (QSA, faie2fn.cu:1628-1636): when the token has more than `top` complete blocks,
                 * a key is visible iff its block is kept or it lies in the incomplete tail */
                const int nb = (p + 1) / (ixr > 0 ? ixr : 1);
                const int sel = mask != NULL && nb > top;
                const uint8_t *mt = mask ? mask + ((size_t) b * nt + t) * mstride : NULL;
                double mx = -INFINITY;
                for (int key = 0; key < nk; ++key) {
                    if (sel && key / ixr < nb && !mt[key / ixr]) {
                        sc[key] = -INFINITY;
                        continue;
                    }
                    double s = 0.0;
                    if (key < pos[b]) {
                        const float *kr = Kc + (((size_t) b * max_ctx + key) * nkv + g) * hd;
                        for (int d = 0; d < hd; ++d) s += qd[d] * (double) kr[d];
                    } else {
                        const double *kr = knew_o + (((size_t) b * nt + (key - pos[b])) * nkv + g) * hd;
                        for (int d = 0; d < hd; ++d) s += qd[d] * kr[d];
                    }
                    sc[key] = s * scale;
                    if (sc[key] > mx) mx = sc[key];
                }
                double l = 0.0;
                for (int d = 0; d < hd; ++d) acc[d] = 0.0;
                for (int key = 0; key < nk; ++key) {
                    if (sc[key] == -INFINITY) continue;
                    const double e = exp(sc[key] - mx);
                    l += e;
                    if (key < pos[b]) {
                        const float *vr = Vc + (((size_t) b * max_ctx + key) * nkv + g) * hd;
                        for (int d = 0; d < hd; ++d) acc[d] += e * (double) vr[d];
                    } else {
                        const double *vr = vnew_o + (((size_t) b * nt + (key - pos[b])) * nkv + g) * hd;
                        for (int d = 0; d < hd; ++d) acc[d] += e * vr[d];
                    }
                }
                double *out = og + (((size_t) b * nt + t) * nq + h) * hd;
                const float *gate = qrow + hd;
                for (int d = 0; d < hd; ++d) out[d] = acc[d] / l * sigm_d((double) gate[d]);
                free(sc);
                free(qd);
            }
    free(inv);
}

EXPORT void orc_attn(int B, int nq, int nkv, int hd, int nrot, double theta, double eps, int nt, const int *pos,
                     const float *qg, const float *knew, const float *vnew, const float *wq, const float *wk,
                     int max_ctx, const float *Kc, const float *Vc, double *knew_o, double *vnew_o, double *og) {
    orc_attn_masked(B, nq, nkv, hd, nrot, theta, eps, nt, pos, qg, knew, vnew, wq, wk, max_ctx, Kc, Vc, NULL, 0, 1, 0,
                    knew_o, vnew_o, og);
}

/* ---------------------------------------------------------------------------------------------------------------
 * QSA indexer (faie2fn.cu:1480-1607): ixh query heads and one raw key of ixd dims per token, keys compressed into
 * blocks of ixr consecutive positions, the top `top` blocks by score kept per query. */

/* RMSNorm + RoPE of a row given in float64 (the block-key path averages fp32 raw keys first) */
static void norm_rope_d(int d_, int nrot, const float *inv, double eps, int pos, const double *x, const float *w,
                        double *y) {
    double ss = 0.0;
    for (int d = 0; d < d_; ++d) ss += x[d] * x[d];
    const double r = 1.0 / sqrt(ss / d_ + eps);
    for (int d = 0; d < d_; ++d) y[d] = x[d] * r * (double) w[d];
    for (int i = 0; i < nrot / 2; ++i) {
        const float ang = (float) pos * inv[i];
        const double cs = cos((double) ang), sn = sin((double) ang);
        const double a = y[i], b = y[i + nrot / 2];
        y[i] = a * cs - b * sn;
        y[i + nrot / 2] = b * cs + a * sn;
    }
}

/* k_ix_qk + k_ix_blocks (faie2fn.cu:1482-1530) for nt new tokens of B sequences.
 *   iqk [B][nt][ixh*ixd + ixd]: the indexer's query heads, then the raw index key;
 *   Qix out [B][nt][ixh][ixd] = rope(rmsnorm(q_h) * wqn) at position pos[b] + t;
 *   IKc [B][max_ctx][ixd] fp32 in/out: the raw key of token t stored at row pos[b] + t;
 *   BKc [B][max_ctx/ixr][ixd] float64 in/out: every block completed by this call, j in [pos/ixr, (pos+nt)/ixr),
 *   gets rope(rmsnorm(mean of its ixr raw keys) * wkn) at position ixr*j. */
EXPORT void orc_ix_prep(int B, int nt, int ixh, int ixd, int ixr, int nrot, double theta, double eps, int max_ctx,
                        const int *pos, const float *iqk, const float *wqn, const float *wkn, double *Qix, float *IKc,
                        double *BKc) {
    float *inv = (float *) malloc(sizeof(float) * (size_t) (nrot / 2 + 1));
    orc_rope_inv_freq(nrot, theta, inv);
    double *x = (double *) malloc(sizeof(double) * (size_t) ixd);
    const int row = ixh * ixd + ixd, maxb = max_ctx / ixr;
    for (int b = 0; b < B; ++b) {
        for (int t = 0; t < nt; ++t) {
            const float *r = iqk + ((size_t) b * nt + t) * row;
            const int P = pos[b] + t;
            for (int h = 0; h < ixh; ++h) {
                for (int d = 0; d < ixd; ++d) x[d] = (double) r[h * ixd + d];
                norm_rope_d(ixd, nrot, inv, eps, P, x, wqn, Qix + (((size_t) b * nt + t) * ixh + h) * ixd);
            }
            memcpy(IKc + ((size_t) b * max_ctx + P) * ixd, r + ixh * ixd, sizeof(float) * (size_t) ixd);
        }
        for (int j = pos[b] / ixr; j < (pos[b] + nt) / ixr; ++j) {
            for (int d = 0; d < ixd; ++d) {
                double m = 0.0;
                for (int e = 0; e < ixr; ++e) m += (double) IKc[((size_t) b * max_ctx + (size_t) j * ixr + e) * ixd + d];
                x[d] = m / ixr;
            }
            norm_rope_d(ixd, nrot, inv, eps, j * ixr, x, wkn, BKc + ((size_t) b * maxb + j) * ixd);
        }
    }
    free(x);
    free(inv);
}

/* block keys of blocks [j0, j1) of every sequence from the raw keys (k_ix_blocks over a range) */
EXPORT void orc_ix_blocks(int B, int ixd, int ixr, int nrot, double theta, double eps, int max_ctx, int j0, int j1,
                          const float *IKc, const float *wkn, double *BKc) {
    float *inv = (float *) malloc(sizeof(float) * (size_t) (nrot / 2 + 1));
    orc_rope_inv_freq(nrot, theta, inv);
    double *x = (double *) malloc(sizeof(double) * (size_t) ixd);
    const int maxb = max_ctx / ixr;
    for (int b = 0; b < B; ++b)
        for (int j = j0; j < j1; ++j) {
            for (int d = 0; d < ixd; ++d) {
                double m = 0.0;
                for (int e = 0; e < ixr; ++e) m += (double) IKc[((size_t) b * max_ctx + (size_t) j * ixr + e) * ixd + d];
                x[d] = m / ixr;
            }
            norm_rope_d(ixd, nrot, inv, eps, j * ixr, x, wkn, BKc + ((size_t) b * maxb + j) * ixd);
        }
    free(x);
    free(inv);
}

/* k_ix_score (faie2fn.cu:1534-1555): scores[b][t][j] = sum_h relu(Qix[b][t][h] . BKc[b][j]) / sqrt(ixd) for the
 * nb = (pos + t + 1) / ixr complete blocks of token t (entries past nb are left as they are). */
EXPORT void orc_ix_score(int B, int nt, int ixh, int ixd, int ixr, int max_ctx, const int *pos, const double *Qix,
                         const double *BKc, double *scores) {
    const int maxb = max_ctx / ixr;
    const int nt_ = nthreads();
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt_)
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < nt; ++t) {
            const int nb = (pos[b] + t + 1) / ixr;
            for (int j = 0; j < nb; ++j) {
                const double *k = BKc + ((size_t) b * maxb + j) * ixd;
                double s = 0.0;
                for (int h = 0; h < ixh; ++h) {
                    const double *q = Qix + (((size_t) b * nt + t) * ixh + h) * ixd;
                    double p = 0.0;
                    for (int d = 0; d < ixd; ++d) p += q[d] * k[d];
                    s += p > 0.0 ? p : 0.0;
                }
                scores[((size_t) b * nt + t) * maxb + j] = s / sqrt((double) ixd);
            }
        }
}

/*
 * quant_oracle.c -- CPU restatement of the GGUF weight decode and the GEMV of the projections around the path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the dequant / GEMV kernels of libfaie2fn.so: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The product path never calls it.
 *
 * The reference decodes weights with ggml's arithmetic (engine/faie2fn.cu:343-689, "ggml-quants.c arithmetic",
 * :345) and gates its GPU decode bit for bit against gguf-py (flashnext/test_fn_quants.py:30-37, dequant error
 * exactly 0; GEMV within 1e-5 of float64 on the decoded weights).  Neither ggml nor gguf-py is in this image, so
 * this file restates ggml's dequantize_row_* (ggml/src/ggml-quants.c, the published block formats of GGUF) loop by
 * loop, on the same block byte layouts the reference's DQ<T> decoders read (faie2fn.cu:441-655):
 *   - every product ggml forms in float is formed here in float, in ggml's order, so that each value is the float
 *     ggml returns: for Q4_K / Q5_K the product d1 * q is exact and the one rounding is in "- m1" (fmaf is that
 *     single rounding); for Q6_K (d * sc) is exact and the rounding is in "* q"; for IQ4_XS (d * (ls - 32)) is
 *     exact and the rounding is in "* level".
 *   - fp16 scales are decoded from their bits (sign, 5-bit exponent, 10-bit fraction; subnormals, inf, NaN) with
 *     ldexp, exactly; bf16 is its bits in the high half of a float.
 * The GEMV oracle is the float64 dot product of those float values with x.
 *
 * Block layouts (bytes), values per block in brackets:
 *   BF16 [1]     2: bf16 bits
 *   Q8_0 [32]    34: d f16 | qs int8[32]
 *   IQ4_NL [32]  18: d f16 | qs[16] (byte j: low nibble -> value j, high nibble -> value j + 16)
 *   IQ4_XS [256] 136: d f16 | scales_h u16 | scales_l[4] | qs[128] (16 bytes per group of 32, IQ4_NL order)
 *   Q4_K [256]   144: d f16 | dmin f16 | scales[12] | qs[128]
 *   Q5_K [256]   176: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
 *   Q6_K [256]   210: ql[128] | qh[64] | scales int8[16] | d f16
 *   IQ3_S [256]  110: d f16 | qs[64] | qh[8] | signs[32] | scales[4] (a 4-bit scale per group of 32; each group is
 *                8 grid points of 4 magnitudes from the format's 512-point codebook, 9-bit index = qs byte + one qh
 *                bit, signs one bit per value; ggml dequantize_row_iq3_s, reference DQ<T_IQ3_S> faie2fn.cu:565-583)
 *   IQ2_XXS [256] 66: d f16 | qs u16[32] (per group of 32: 4 grid bytes, then a word of 4 x 7-bit sign indices and
 *                a 4-bit scale in bits 28-31; faie2fn.cu:495-509)
 *   IQ2_XS [256] 74: d f16 | qs u16[32] (9-bit grid index, 7-bit sign index) | scales[8] (two 4-bit scales per group,
 *                one per half; :511-527)
 *   IQ2_S [256]  82: d f16 | qs[32] grid low bytes | signs[32] | qh[8] (2 high index bits per 8 values) | scales[8]
 *                (:529-546)
 *   IQ3_XXS [256] 98: d f16 | qs[64] grid bytes | scales_and_signs u32[8] (4 x 7-bit sign indices, 4-bit scale in bits
 *                28-31; :548-563)
 *   Q2_0 [64]    18: d f16 | qs[16] (2-bit codes, value v in bits 2 (v % 4) of byte v / 4): y = d * (q - 1) (the
 *                reference fork's type 42, :470-485)
 * The IQ2 / IQ3_XXS sign indices select a sign byte ksign(i) = i | parity(i) << 7 (GGUF's ksigns_iq2xs), bit j negating
 * value j of a run of 8.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* the IQ3_S codebook (GGUF iq3s_grid; the same data file the GPU decode includes) */
static const uint32_t IQ3S_GRID[512] = {
#include "../faie2-flashnext_amd/csrc/iq3s_grid.inc"
};

/* the IQ2 / IQ3_XXS codebooks (GGUF iq2xxs_grid, iq2xs_grid, iq2s_grid as low-word / high-word pairs; iq3xxs_grid) */
static const uint32_t IQ2XXS_GRID[512] = {
#include "../faie2-flashnext_amd/csrc/iq2xxs_grid.inc"
};
static const uint32_t IQ2XS_GRID[1024] = {
#include "../faie2-flashnext_amd/csrc/iq2xs_grid.inc"
};
static const uint32_t IQ2S_GRID[2048] = {
#include "../faie2-flashnext_amd/csrc/iq2s_grid.inc"
};
static const uint32_t IQ3XXS_GRID[256] = {
#include "../faie2-flashnext_amd/csrc/iq3xxs_grid.inc"
};

/* the sign byte of a 7-bit sign index: the index with its parity as bit 7 (an even count of negated values) */
static unsigned ksign(unsigned i) { return i | (unsigned) (__builtin_popcount(i) & 1) << 7; }

/* magnitude j (0..7) of entry e of a codebook of 8-byte entries stored as two words */
static float mag8(const uint32_t *grid, unsigned e, int j) {
    return (float) ((grid[2 * e + (j >> 2)] >> (8 * (j & 3))) & 255);
}

/* the 16 levels of the IQ4 formats (GGUF kvalues_iq4nl) */
static const int8_t IQ4_LEVELS[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

EXPORT float orc_f16_to_f32(uint16_t h) {
    const int sign = h >> 15, e = (h >> 10) & 0x1F, f = h & 0x3FF;
    float v;
    if (e == 0) v = ldexpf((float) f, -24);                 /* subnormal (and zero) */
    else if (e == 31) v = f ? NAN : INFINITY;
    else v = ldexpf((float) (1024 + f), e - 25);            /* (1 + f / 1024) * 2^(e - 15) */
    return sign ? -v : v;
}

static float f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t) (p[0] | p[1] << 8)); }

/* ggml get_scale_min_k4 (faie2fn.cu:432-440): 6-bit scale and min of group j from the 12 packed bytes */
static void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* values per block and bytes per block; 0 for a type this oracle does not decode */
EXPORT int orc_qblock(uint32_t type, int *qk, int *bytes) {
    switch (type) {
        case 30: *qk = 1; *bytes = 2; return 1;
        case 8: *qk = 32; *bytes = 34; return 1;
        case 20: *qk = 32; *bytes = 18; return 1;
        case 23: *qk = 256; *bytes = 136; return 1;
        case 12: *qk = 256; *bytes = 144; return 1;
        case 13: *qk = 256; *bytes = 176; return 1;
        case 14: *qk = 256; *bytes = 210; return 1;
        case 21: *qk = 256; *bytes = 110; return 1;
        case 16: *qk = 256; *bytes = 66; return 1;
        case 17: *qk = 256; *bytes = 74; return 1;
        case 22: *qk = 256; *bytes = 82; return 1;
        case 18: *qk = 256; *bytes = 98; return 1;
        case 42: *qk = 64; *bytes = 18; return 1;
        default: return 0;
    }
}

/* one GGUF row of `cols` values -> y[cols] */
static void dq_row(uint32_t type, const uint8_t *r, int cols, float *y) {
    switch (type) {
        case 30: /* BF16 */
            for (int j = 0; j < cols; ++j) {
                const uint32_t bits = (uint32_t) (r[2 * j] | r[2 * j + 1] << 8) << 16;
                memcpy(&y[j], &bits, 4);
            }
            break;
        case 8: /* Q8_0: y = d * q */
            for (int b = 0; b < cols / 32; ++b, r += 34, y += 32) {
                const float d = f16(r);
                for (int j = 0; j < 32; ++j) y[j] = d * (float) (int8_t) r[2 + j];
            }
            break;
        case 20: /* IQ4_NL: y = d * level */
            for (int b = 0; b < cols / 32; ++b, r += 18, y += 32) {
                const float d = f16(r);
                const uint8_t *qs = r + 2;
                for (int j = 0; j < 16; ++j) {
                    y[j] = d * (float) IQ4_LEVELS[qs[j] & 0xF];
                    y[j + 16] = d * (float) IQ4_LEVELS[qs[j] >> 4];
                }
            }
            break;
        case 23: /* IQ4_XS: dl = d * (ls - 32), y = dl * level */
            for (int b = 0; b < cols / 256; ++b, r += 136) {
                const float d = f16(r);
                const int sh = r[2] | r[3] << 8;
                const uint8_t *sl = r + 4, *qs = r + 8;
                for (int ib = 0; ib < 8; ++ib, y += 32, qs += 16) {
                    const int ls = ((sl[ib / 2] >> 4 * (ib % 2)) & 0xF) | (((sh >> 2 * ib) & 3) << 4);
                    const float dl = d * (float) (ls - 32);
                    for (int j = 0; j < 16; ++j) {
                        y[j] = dl * (float) IQ4_LEVELS[qs[j] & 0xF];
                        y[j + 16] = dl * (float) IQ4_LEVELS[qs[j] >> 4];
                    }
                }
            }
            break;
        case 12: /* Q4_K: y = d*sc * q - dmin*m */
            for (int b = 0; b < cols / 256; ++b, r += 144) {
                const float d = f16(r), dmin = f16(r + 2);
                const uint8_t *sc = r + 4, *q = r + 16;
                for (int p = 0; p < 4; ++p, q += 32) {
                    int s1, m1, s2, m2;
                    scale_min_k4(2 * p, sc, &s1, &m1);
                    scale_min_k4(2 * p + 1, sc, &s2, &m2);
                    const float d1 = d * (float) s1, n1 = dmin * (float) m1;
                    const float d2 = d * (float) s2, n2 = dmin * (float) m2;
                    for (int l = 0; l < 32; ++l) *y++ = fmaf(d1, (float) (q[l] & 0xF), -n1);
                    for (int l = 0; l < 32; ++l) *y++ = fmaf(d2, (float) (q[l] >> 4), -n2);
                }
            }
            break;
        case 13: /* Q5_K: Q4_K with a fifth bit from qh */
            for (int b = 0; b < cols / 256; ++b, r += 176) {
                const float d = f16(r), dmin = f16(r + 2);
                const uint8_t *sc = r + 4, *qh = r + 16, *ql = r + 48;
                for (int p = 0; p < 4; ++p, ql += 32) {
                    int s1, m1, s2, m2;
                    scale_min_k4(2 * p, sc, &s1, &m1);
                    scale_min_k4(2 * p + 1, sc, &s2, &m2);
                    const float d1 = d * (float) s1, n1 = dmin * (float) m1;
                    const float d2 = d * (float) s2, n2 = dmin * (float) m2;
                    const int u1 = 1 << (2 * p), u2 = 2 << (2 * p);
                    for (int l = 0; l < 32; ++l) *y++ = fmaf(d1, (float) ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)), -n1);
                    for (int l = 0; l < 32; ++l) *y++ = fmaf(d2, (float) ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)), -n2);
                }
            }
            break;
        case 21: /* IQ3_S: db = d * (1 + 2 * scale), y = db * grid * sign, ggml's order of the products */
            for (int b = 0; b < cols / 256; ++b, r += 110) {
                const float d = f16(r);
                const uint8_t *qs = r + 2, *qh = r + 66, *signs = r + 74, *scales = r + 106;
                for (int ib = 0; ib < 8; ++ib, y += 32) {
                    const float db = d * (float) (1 + 2 * ((scales[ib / 2] >> (4 * (ib % 2))) & 0xF));
                    for (int l = 0; l < 4; ++l) {
                        const uint32_t g1 = IQ3S_GRID[qs[8 * ib + 2 * l] | ((qh[ib] << (8 - 2 * l)) & 256)];
                        const uint32_t g2 = IQ3S_GRID[qs[8 * ib + 2 * l + 1] | ((qh[ib] << (7 - 2 * l)) & 256)];
                        const uint8_t sg = signs[4 * ib + l];
                        for (int j = 0; j < 4; ++j) {
                            y[8 * l + j] = db * (float) ((g1 >> (8 * j)) & 255) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                            y[8 * l + 4 + j] = db * (float) ((g2 >> (8 * j)) & 255) * ((sg >> (j + 4)) & 1 ? -1.0f : 1.0f);
                        }
                    }
                }
            }
            break;
        case 16: /* IQ2_XXS: db = d * (0.5 + s) * 0.25, y = db * grid * sign */
            for (int b = 0; b < cols / 256; ++b, r += 66) {
                const float d = f16(r);
                for (int ib = 0; ib < 8; ++ib) {
                    const uint8_t *q = r + 2 + 8 * ib;
                    const uint32_t a1 = (uint32_t) q[4] | (uint32_t) q[5] << 8 | (uint32_t) q[6] << 16 | (uint32_t) q[7] << 24;
                    const float db = d * (0.5f + (float) (a1 >> 28)) * 0.25f;
                    for (int l = 0; l < 4; ++l, y += 8) {
                        const unsigned sg = ksign((a1 >> (7 * l)) & 127);
                        for (int j = 0; j < 8; ++j) y[j] = db * mag8(IQ2XXS_GRID, q[l], j) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
            break;
        case 17: /* IQ2_XS: db = d * (0.5 + s_half) * 0.25 */
            for (int b = 0; b < cols / 256; ++b, r += 74) {
                const float d = f16(r);
                const uint8_t *sc = r + 66;
                for (int ib = 0; ib < 8; ++ib) {
                    const float db0 = d * (0.5f + (float) (sc[ib] & 0xF)) * 0.25f;
                    const float db1 = d * (0.5f + (float) (sc[ib] >> 4)) * 0.25f;
                    for (int l = 0; l < 4; ++l, y += 8) {
                        const unsigned q = (unsigned) r[2 + 2 * (4 * ib + l)] | (unsigned) r[3 + 2 * (4 * ib + l)] << 8;
                        const unsigned sg = ksign(q >> 9);
                        for (int j = 0; j < 8; ++j)
                            y[j] = (l < 2 ? db0 : db1) * mag8(IQ2XS_GRID, q & 511, j) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
            break;
        case 22: /* IQ2_S: 10-bit grid index (qs byte + 2 bits of qh), a full sign byte per 8 values */
            for (int b = 0; b < cols / 256; ++b, r += 82) {
                const float d = f16(r);
                const uint8_t *qs = r + 2, *signs = r + 34, *qh = r + 66, *sc = r + 74;
                for (int ib = 0; ib < 8; ++ib) {
                    const float db0 = d * (0.5f + (float) (sc[ib] & 0xF)) * 0.25f;
                    const float db1 = d * (0.5f + (float) (sc[ib] >> 4)) * 0.25f;
                    for (int l = 0; l < 4; ++l, y += 8) {
                        const unsigned e = qs[4 * ib + l] | ((qh[ib] << (8 - 2 * l)) & 0x300);
                        const unsigned sg = signs[4 * ib + l];
                        for (int j = 0; j < 8; ++j)
                            y[j] = (l < 2 ? db0 : db1) * mag8(IQ2S_GRID, e, j) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
            break;
        case 18: /* IQ3_XXS: db = d * (0.5 + s) * 0.5, 4-magnitude grid points in pairs */
            for (int b = 0; b < cols / 256; ++b, r += 98) {
                const float d = f16(r);
                const uint8_t *qs = r + 2, *ss = r + 66;
                for (int ib = 0; ib < 8; ++ib) {
                    const uint32_t aux = (uint32_t) ss[4 * ib] | (uint32_t) ss[4 * ib + 1] << 8 |
                                         (uint32_t) ss[4 * ib + 2] << 16 | (uint32_t) ss[4 * ib + 3] << 24;
                    const float db = d * (0.5f + (float) (aux >> 28)) * 0.5f;
                    for (int l = 0; l < 4; ++l, y += 8) {
                        const unsigned sg = ksign((aux >> (7 * l)) & 127);
                        const uint32_t g1 = IQ3XXS_GRID[qs[8 * ib + 2 * l]], g2 = IQ3XXS_GRID[qs[8 * ib + 2 * l + 1]];
                        for (int j = 0; j < 4; ++j) {
                            y[j] = db * (float) ((g1 >> (8 * j)) & 255) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                            y[j + 4] = db * (float) ((g2 >> (8 * j)) & 255) * ((sg >> (j + 4)) & 1 ? -1.0f : 1.0f);
                        }
                    }
                }
            }
            break;
        case 42: /* Q2_0: y = d * (q - 1) */
            for (int b = 0; b < cols / 64; ++b, r += 18, y += 64) {
                const float d = f16(r);
                for (int v = 0; v < 64; ++v) y[v] = d * (float) ((int) ((r[2 + v / 4] >> (2 * (v % 4))) & 3) - 1);
            }
            break;
        case 14: /* Q6_K: y = d * sc * (q - 32) */
            for (int b = 0; b < cols / 256; ++b, r += 210) {
                const float d = f16(r + 208);
                const uint8_t *ql = r, *qh = r + 128;
                const int8_t *sc = (const int8_t *) (r + 192);
                for (int n = 0; n < 2; ++n, ql += 64, qh += 32, sc += 8, y += 128)
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                        const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l] = d * (float) sc[is] * (float) q1;
                        y[l + 32] = d * (float) sc[is + 2] * (float) q2;
                        y[l + 64] = d * (float) sc[is + 4] * (float) q3;
                        y[l + 96] = d * (float) sc[is + 6] * (float) q4;
                    }
            }
            break;
    }
}

/* rows GGUF rows of `cols` values -> out [rows][cols]; -1 for an unsupported type or shape */
EXPORT int orc_dequant(uint32_t type, const uint8_t *W, int rows, int cols, float *out) {
    int qk, bb;
    if (!orc_qblock(type, &qk, &bb) || cols % qk || rows < 1) return -1;
    const size_t rb = (size_t) cols / qk * bb;
    for (int r = 0; r < rows; ++r) dq_row(type, W + (size_t) r * rb, cols, out + (size_t) r * cols);
    return 0;
}

/* y [nt][rows] = sum_c W[r][c] x[t][c] in float64 over the decoded float weights */
EXPORT int orc_gemv(uint32_t type, const uint8_t *W, int rows, int cols, const float *x, int nt, double *y) {
    int qk, bb;
    if (!orc_qblock(type, &qk, &bb) || cols % qk || rows < 1) return -1;
    const size_t rb = (size_t) cols / qk * bb;
    float *w = (float *) malloc(sizeof(float) * (size_t) cols);
    for (int r = 0; r < rows; ++r) {
        dq_row(type, W + (size_t) r * rb, cols, w);
        for (int t = 0; t < nt; ++t) {
            double s = 0.0;
            const float *xt = x + (size_t) t * cols;
            for (int c = 0; c < cols; ++c) s += (double) w[c] * (double) xt[c];
            y[(size_t) t * rows + r] = s;
        }
    }
    free(w);
    return 0;
}

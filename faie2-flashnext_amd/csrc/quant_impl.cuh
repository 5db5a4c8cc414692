// Templates of the GGUF weight formats and their kernels (decode, dequant, GEMV, embedding rows, expert rows), shared
// by quant.hip (layouts, plans, dispatch) and the quant_t*.hip units that instantiate them per group of formats (one
// unit per group, so the formats compile in parallel).  Everything here has internal linkage: each unit gets its own
// copies of the kernels and lookup tables it uses.
#pragma once

#include "quant.h"

#include <algorithm>
#include <type_traits>

namespace fn {

// GEMV plan overrides (quant.hip): split-K, lanes per row, kernel, resident waves per CU, persistent grid
extern int g_ov_ks, g_ov_lpr, g_ov_kernel, g_ov_wpc, g_persist;

namespace {

constexpr int MAXNT = 8;

// ------------------------------------------------------------------------------------------------------------
// the IQ4 codebook (the GGUF format's 16 non-uniform levels), and its signed bytes packed four to a word for
// byte-permute lookups: word k holds entries 4k..4k+3, entry 4k in the low byte

constexpr int kIq4Levels[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

constexpr uint32_t pack4(int k) {
    return (uint32_t) (uint8_t) kIq4Levels[4 * k] | (uint32_t) (uint8_t) kIq4Levels[4 * k + 1] << 8 |
           (uint32_t) (uint8_t) kIq4Levels[4 * k + 2] << 16 | (uint32_t) (uint8_t) kIq4Levels[4 * k + 3] << 24;
}
constexpr uint32_t KV0 = pack4(0), KV1 = pack4(1), KV2 = pack4(2), KV3 = pack4(3);
static_assert(KV0 == 0xBFAD9881u && KV3 == 0x71594535u, "IQ4 level packing");

// the lookup state of the formats that decode without a table
struct NoTab {};

// The IQ4 levels (IQ4_NL, IQ4_XS) as 16 floats in LDS, copied once per workgroup (tab_fill): a value's lookup is one
// LDS read at its index's byte offset, with no conversion after it.  The 16 words sit in 16 distinct banks, so the
// lanes of a read never conflict (equal indices are broadcast).  (Before: three v_perm_b32 lookups in the signed
// level bytes held in registers, two shifts, two and-ors per four values, then a signed-byte conversion each.)
__device__ __forceinline__ float *iq4_lds() {
    __shared__ float lev[16];
    return lev;
}
struct Iq4LdsTab {
    const float *lev;
    __device__ __forceinline__ Iq4LdsTab() : lev(iq4_lds()) {}
    // the level of the index held at byte offset off (4 x index) of the table
    __device__ __forceinline__ float at(uint32_t off) const {
        return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(lev) + off);
    }
};
template <uint32_t TY> constexpr bool iq4_fmt() { return TY == QT_IQ4_NL || TY == QT_IQ4_XS; }
// byte K of x, zero-extended, in one instruction (the compiler splits a constant-mask field extract into a shift and
// an and; bytes 1 and 2 go through v_bfe_u32 as written)
template <int K> __device__ __forceinline__ uint32_t byte_of(uint32_t x) {
    if constexpr (K == 0) return x & 0xFFu;
    else if constexpr (K == 3) return x >> 24;
    else {
        uint32_t r;
        asm("v_bfe_u32 %0, %1, %2, 8" : "=v"(r) : "v"(x), "i"(8 * K));
        return r;
    }
}

// Codebooks of the grid formats (GGUF's iq3s_grid, iq3xxs_grid, iq2xxs_grid, iq2xs_grid, iq2s_grid; 8-byte entries as
// low-word / high-word pairs).  A lane's decode looks up 8 grid points per group at data-dependent indices, so the
// kernels that read these formats copy their codebook into LDS once per workgroup (tab_fill, before their first
// barrier) and gather from there.
__device__ const uint32_t kIq3sGrid[512] = {
#include "iq3s_grid.inc"
};
__device__ const uint32_t kIq3xxsGrid[256] = {
#include "iq3xxs_grid.inc"
};
__device__ const uint32_t kIq2xxsGrid[512] = {
#include "iq2xxs_grid.inc"
};
__device__ const uint32_t kIq2xsGrid[1024] = {
#include "iq2xs_grid.inc"
};
__device__ const uint32_t kIq2sGrid[2048] = {
#include "iq2s_grid.inc"
};

template <uint32_t TY> struct GridOf { static constexpr int words = 0; };
template <> struct GridOf<QT_IQ3_S> { static constexpr int words = 512; };
template <> struct GridOf<QT_IQ3_XXS> { static constexpr int words = 256; };
template <> struct GridOf<QT_IQ2_XXS> { static constexpr int words = 512; };
template <> struct GridOf<QT_IQ2_XS> { static constexpr int words = 1024; };
template <> struct GridOf<QT_IQ2_S> { static constexpr int words = 2048; };

template <uint32_t TY> __device__ __forceinline__ const uint32_t *grid_src() {
    if constexpr (TY == QT_IQ3_S) return kIq3sGrid;
    else if constexpr (TY == QT_IQ3_XXS) return kIq3xxsGrid;
    else if constexpr (TY == QT_IQ2_XXS) return kIq2xxsGrid;
    else if constexpr (TY == QT_IQ2_XS) return kIq2xsGrid;
    else return kIq2sGrid;
}

template <uint32_t TY> __device__ __forceinline__ uint32_t *grid_lds() {
    __shared__ uint32_t grid[GridOf<TY>::words];
    return grid;
}

// Byte masks of a sign byte: entry s is two words whose byte j is 0xFF where bit j (first word) or bit 4 + j
// (second word) of s is set.  The grid formats' magnitudes are bytes 1..127, so a word of four of them takes its
// signs as (g ^ m) + (m & 0x01010101): every flagged byte negated in two's complement with no carry between bytes,
// ready for the signed-byte conversion (two operations per four values instead of a bit test and an or per value).
constexpr uint32_t sign_mask4(uint32_t s) {
    return (s & 1u ? 0xFFu : 0u) | (s & 2u ? 0xFF00u : 0u) | (s & 4u ? 0xFF0000u : 0u) | (s & 8u ? 0xFF000000u : 0u);
}
struct SignTab {
    uint32_t w[512];
    constexpr SignTab() : w() {
        for (uint32_t s = 0; s < 256; ++s) {
            w[2 * s] = sign_mask4(s & 15u);
            w[2 * s + 1] = sign_mask4(s >> 4);
        }
    }
};
__device__ const SignTab kSignTab{};
static_assert(SignTab().w[2 * 0x81] == 0xFFu && SignTab().w[2 * 0x81 + 1] == 0xFF000000u, "sign byte masks");
__device__ __forceinline__ uint32_t *sign_lds() {
    __shared__ uint32_t sgn[512];
    return sgn;
}
__device__ __forceinline__ uint32_t neg_bytes(uint32_t g, uint32_t m) { return (g ^ m) + (m & 0x01010101u); }

template <uint32_t TY> struct GridTab {
    const uint32_t *grid, *sgn;
    __device__ __forceinline__ GridTab() : grid(grid_lds<TY>()), sgn(sign_lds()) {}
};

// per-format lookup state held by a decoding lane: the IQ4 levels or the grid codebook in LDS (none for the other
// formats)
template <uint32_t TY, bool G = (GridOf<TY>::words > 0)> struct TabOf {
    using type = typename std::conditional<iq4_fmt<TY>(), Iq4LdsTab, NoTab>::type;
};
template <uint32_t TY> struct TabOf<TY, true> { using type = GridTab<TY>; };
template <uint32_t TY> using TabT = typename TabOf<TY>::type;

// LDS the format's table takes in a GEMV / dequant workgroup, and its fill by the workgroup's nth threads (the
// caller's next barrier publishes it)
template <uint32_t TY> constexpr int tab_lds() {
    return GridOf<TY>::words > 0 ? GridOf<TY>::words * 4 + 2048 : (iq4_fmt<TY>() ? 64 : 0);
}
template <uint32_t TY> __device__ __forceinline__ void tab_fill(int tid, int nth) {
    if constexpr (iq4_fmt<TY>()) {
        if (tid < 16) {
            const uint32_t kw = tid < 4 ? KV0 : (tid < 8 ? KV1 : (tid < 12 ? KV2 : KV3));
            iq4_lds()[tid] = (float) (int8_t) (kw >> (8 * (tid & 3)));
        }
    } else if constexpr (GridOf<TY>::words > 0) {
        uint32_t *g = grid_lds<TY>(), *sg = sign_lds();
        const uint32_t *src = grid_src<TY>();
        for (int i = tid; i < GridOf<TY>::words; i += nth) g[i] = src[i];
        for (int i = tid; i < 512; i += nth) sg[i] = kSignTab.w[i];
    }
}

// the sign byte of a 7-bit sign index of the IQ2 / IQ3_XXS formats: the index with its parity as bit 7 (an even
// count of negated values; GGUF's ksigns_iq2xs)
__device__ __forceinline__ uint32_t ksign(uint32_t i) { return i | (uint32_t) (__builtin_popcount(i) & 1) << 7; }

__device__ __forceinline__ float sbyte(uint32_t w, int k) { return (float) ((int32_t) (w << (24 - 8 * k)) >> 24); }
__device__ __forceinline__ float h2f(uint32_t bits) {
    return (float) __builtin_bit_cast(_Float16, (unsigned short) (bits & 0xFFFFu));
}
// byte k (0..11) of the 12 bytes w0 w1 w2
__device__ __forceinline__ uint32_t byte12(uint32_t w0, uint32_t w1, uint32_t w2, int k) {
    const uint32_t w = k < 4 ? w0 : (k < 8 ? w1 : w2);
    return (w >> (8 * (k & 3))) & 0xFFu;
}

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void ld16(const uint8_t *p, uint32_t *w) {
    const v4u v = *reinterpret_cast<const v4u *>(p);
    w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
}
__device__ __forceinline__ void ld8(const uint8_t *p, uint32_t *w) {
    const v2u v = *reinterpret_cast<const v2u *>(p);
    w[0] = v.x, w[1] = v.y;
}
__device__ __forceinline__ uint32_t ld2(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

// planes of a packed weight as the kernels see them
struct PP {
    const uint8_t *p0, *p1, *p2;
    size_t rs0, rs1, rs2;
};

// the three planes of one row
struct RP {
    const uint8_t *b0, *b1, *b2;
};
__device__ __forceinline__ RP row_planes(const PP &P, int row) {
    return RP{P.p0 + (size_t) row * P.rs0, P.p1 + (size_t) row * P.rs1, P.p2 + (size_t) row * P.rs2};
}
// The same for the GEMV's weight loads: a plane is its base (wave-uniform, in SGPRs) and the row's 32-bit byte
// offset, so that a load's address is the base plus one 32-bit VGPR (the load's scalar-base form) instead of a
// 64-bit multiply-add per plane per batch.  Needs planes under 4 GiB (gemv_launch checks).
struct Plane32 {
    const uint8_t *base;
    uint32_t off;
    __device__ __forceinline__ const uint8_t *operator+(uint32_t x) const { return base + (off + x); }
};
struct RP32 {
    Plane32 b0, b1, b2;
};
__device__ __forceinline__ RP32 row_planes32(const PP &P, int row) {
    const uint32_t r = (uint32_t) row;
    return RP32{{P.p0, r * (uint32_t) P.rs0}, {P.p1, r * (uint32_t) P.rs1}, {P.p2, r * (uint32_t) P.rs2}};
}

// one decoded group: GGUF value j = fl(s[j / 16] * q[j] - m[j / 16])
struct Grp {
    float q[32];
    float s[2], m[2];
};

template <uint32_t TY> struct Q;

// groups a GEMV lane keeps in flight per batch for a format of nw raw words per group (two batches live at once)
constexpr int prefetch_groups(int nw) { return nw <= 8 ? 4 : (nw <= 12 ? 2 : 1); }

// BF16: a group is 32 consecutive values (64 bytes); q holds the values themselves, s = 1
template <> struct Q<QT_BF16> {
    static constexpr int NW = 16;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const uint8_t *p = R.b0 + 64 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) ld16(p + 16 * i, w + 4 * i);
    }
    __device__ static void unpack(const uint32_t *w, int, Grp &o, const NoTab &T) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            o.q[2 * i] = __uint_as_float(w[i] << 16);
            o.q[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
        o.s[0] = o.s[1] = 1.0f;
        o.m[0] = o.m[1] = 0.0f;
    }
};

// Q8_0: 32 int8 quants, one fp16 scale (ggml: y = d * q)
template <> struct Q<QT_Q8_0> {
    static constexpr int NW = 9;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const uint8_t *q = R.b0 + 32 * g;
        ld16(q, w);
        ld16(q + 16, w + 4);
        w[8] = ld2(R.b1 + 2 * g);
    }
    __device__ static void unpack(const uint32_t *w, int, Grp &o, const NoTab &T) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) o.q[4 * i + k] = sbyte(w[i], k);
        o.s[0] = o.s[1] = h2f(w[8]);
        o.m[0] = o.m[1] = 0.0f;
    }
};

// IQ4_NL: 16 bytes of nibble indices (byte b: low nibble = value b, high nibble = value b + 16), fp16 scale
// (ggml: y = d * level)
template <> struct Q<QT_IQ4_NL> {
    static constexpr int NW = 5;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        ld16(R.b0 + 16 * g, w);
        w[4] = ld2(R.b1 + 2 * g);
    }
    __device__ static void levels(const uint32_t *w, Grp &o, const Iq4LdsTab &T) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // 4 x the index of each value in its byte (low nibbles, then high): a byte is the table offset
            const uint32_t lo = (w[i] << 2) & 0x3C3C3C3Cu, hi = (w[i] >> 2) & 0x3C3C3C3Cu;
            o.q[4 * i] = T.at(byte_of<0>(lo));
            o.q[4 * i + 1] = T.at(byte_of<1>(lo));
            o.q[4 * i + 2] = T.at(byte_of<2>(lo));
            o.q[4 * i + 3] = T.at(byte_of<3>(lo));
            o.q[16 + 4 * i] = T.at(byte_of<0>(hi));
            o.q[16 + 4 * i + 1] = T.at(byte_of<1>(hi));
            o.q[16 + 4 * i + 2] = T.at(byte_of<2>(hi));
            o.q[16 + 4 * i + 3] = T.at(byte_of<3>(hi));
        }
    }
    __device__ static void unpack(const uint32_t *w, int, Grp &o, const Iq4LdsTab &T) {
        levels(w, o, T);
        o.s[0] = o.s[1] = h2f(w[4]);
        o.m[0] = o.m[1] = 0.0f;
    }
};

// IQ4_XS: super-blocks of 256 (d fp16, scales_h u16, scales_l[4], qs[128]); group ib has a 6-bit scale ls and
// the IQ4_NL nibble layout (ggml: dl = d * (ls - 32), y = dl * level)
template <> struct Q<QT_IQ4_XS> {
    static constexpr int NW = 6;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        ld16(R.b0 + 16 * g, w);  // super-block g / 8 at 128 (g / 8), group g % 8 at 16 (g % 8) inside it
        ld8(R.b1 + 8 * (g >> 3), w + 4);
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const Iq4LdsTab &T) {
        const int ib = g & 7;
        Q<QT_IQ4_NL>::levels(w, o, T);
        const uint32_t sl = (w[5] >> (8 * (ib >> 1))) >> (4 * (ib & 1)) & 0xFu;
        const uint32_t sh = (w[4] >> (16 + 2 * ib)) & 3u;
        const float dl = h2f(w[4]) * (float) ((int) (sl | sh << 4) - 32);
        o.s[0] = o.s[1] = dl;
        o.m[0] = o.m[1] = 0.0f;
    }
};

// 6-bit scale and min of group ib from the 12 packed scale bytes of Q4_K / Q5_K (ggml get_scale_min_k4)
__device__ __forceinline__ void scale_min_k(const uint32_t *h, int ib, float &sc, float &mn) {
    const uint32_t b_ib = byte12(h[0], h[1], h[2], ib), b_4 = byte12(h[0], h[1], h[2], ib + 4);
    if (ib < 4) {
        sc = (float) (b_ib & 63u);
        mn = (float) (b_4 & 63u);
    } else {
        const uint32_t b_m4 = byte12(h[0], h[1], h[2], ib - 4);
        sc = (float) ((b_4 & 0xFu) | (b_m4 >> 6) << 4);
        mn = (float) ((b_4 >> 4) | (b_ib >> 6) << 4);
    }
}

// Q4_K: super-blocks of 256 (d, dmin fp16, 12 scale bytes, qs[128]); group ib reads the low (even ib) or high
// (odd ib) nibbles of qs[32 (ib/2) .. +31] (ggml: y = d*sc * q - dmin*m)
template <> struct Q<QT_Q4_K> {
    static constexpr int NW = 12;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = true;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const uint8_t *q = R.b0 + 16 * (g & ~1);  // the 32 bytes of groups 2k and 2k + 1
        ld16(q, w);
        ld16(q + 16, w + 4);
        ld16(R.b1 + 16 * (g >> 3), w + 8);
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const NoTab &T) {
        const int ib = g & 7, sh = 4 * (ib & 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = (w[i] >> sh) & 0x0F0F0F0Fu;  // the group's 4 nibbles of word i, one per byte
#pragma unroll
            for (int k = 0; k < 4; ++k) o.q[4 * i + k] = (float) ((q >> (8 * k)) & 0xFFu);
        }
        float sc, mn;
        scale_min_k(w + 9, ib, sc, mn);
        o.s[0] = o.s[1] = h2f(w[8]) * sc;
        o.m[0] = o.m[1] = h2f(w[8] >> 16) * mn;
    }
};

// Q5_K: Q4_K plus a fifth bit per value: bit ib of qh[j] (ggml: q = nibble + 16 * bit)
template <> struct Q<QT_Q5_K> {
    static constexpr int NW = 20;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = true;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const uint8_t *q = R.b0 + 16 * (g & ~1);
        ld16(q, w);
        ld16(q + 16, w + 4);
        const uint8_t *h = R.b1 + 32 * (g >> 3);
        ld16(h, w + 8);
        ld16(h + 16, w + 12);
        ld16(R.b2 + 16 * (g >> 3), w + 16);
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const NoTab &T) {
        const int ib = g & 7, sh = 4 * (ib & 1);
        const uint32_t rot = (uint32_t) (ib + 28) & 31u;  // a right rotation by ib - 4 takes bit 8k + ib to 8k + 4
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // 4 values per 32-bit operation: the nibbles, then bit ib of each qh byte moved to bit 4 of its byte
            const uint32_t hb = __builtin_amdgcn_alignbit(w[8 + i], w[8 + i], rot);
            const uint32_t q = (hb & 0x10101010u) | ((w[i] >> sh) & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 4; ++k) o.q[4 * i + k] = (float) ((q >> (8 * k)) & 0xFFu);
        }
        float sc, mn;
        scale_min_k(w + 17, ib, sc, mn);
        o.s[0] = o.s[1] = h2f(w[16]) * sc;
        o.m[0] = o.m[1] = h2f(w[16] >> 16) * mn;
    }
};

// Q6_K: super-blocks of 256 (ql[128], qh[64], int8 scales[16], d fp16).  Value 128 n + 32 qu + l (n < 2, qu < 4,
// l < 32): low 4 bits from nibble (qu >> 1) of ql[64 n + 32 (qu & 1) + l], high 2 bits from bits 2 qu of
// qh[32 n + l], scale scales[8 n + 2 qu + l / 16] (ggml: y = d * sc * (q - 32)).  Decoded as q with the minimum
// m = 32 s, so that the GEMV takes the factored form s (q.x) - 32 s (sum x) like the other formats with a minimum;
// the GGUF value itself is s (q - 32) (gguf_value).
template <> struct Q<QT_Q6_K> {
    static constexpr int NW = 18;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = true;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const int ib = g & 7, n = ib >> 2, qu = ib & 3, sb = g >> 3;
        const uint8_t *l = R.b0 + 128 * sb + 64 * n + 32 * (qu & 1);
        ld16(l, w);
        ld16(l + 16, w + 4);
        const uint8_t *h = R.b1 + 64 * sb + 32 * n;
        ld16(h, w + 8);
        ld16(h + 16, w + 12);
        const uint8_t *t = R.b2 + 18 * sb;
        w[16] = ld2(t + 8 * n + 2 * qu);
        w[17] = ld2(t + 16);
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const NoTab &T) {
        const int qu = g & 3, lsh = 4 * (qu >> 1);
        const uint32_t rot = (uint32_t) (2 * qu + 28) & 31u;  // a right rotation by 2 qu - 4: bits 8k + 2qu, + 1 to 8k + 4, 5
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // 4 six-bit codes per 32-bit operation (low nibble, then 2 high bits at bits 4-5 of each byte)
            const uint32_t hb = __builtin_amdgcn_alignbit(w[8 + i], w[8 + i], rot);
            const uint32_t q = (hb & 0x30303030u) | ((w[i] >> lsh) & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 4; ++k) o.q[4 * i + k] = (float) ((q >> (8 * k)) & 0xFFu);
        }
        const float d = h2f(w[17]);
        o.s[0] = d * sbyte(w[16], 0);
        o.s[1] = d * sbyte(w[16], 1);
        o.m[0] = 32.0f * o.s[0];
        o.m[1] = 32.0f * o.s[1];
    }
};

// IQ3_S: super-blocks of 256 (d fp16, qs[64], qh[8], signs[32], scales[4]); packed as plane 0 = qs, plane 1 = qh,
// signs and scales (44 bytes), plane 2 = d.  Group ib: db = d * (1 + 2 * (4-bit scale ib)); its 32 values are 8 grid
// points of 4 magnitudes, point 2l (2l + 1) at index qs[8 ib + 2l (+1)] | bit 2l (2l + 1) of qh[ib] << 8, value
// 8l + j negated by bit j of signs[4 ib + l] (ggml: y = db * grid[j] * sign)
template <> struct Q<QT_IQ3_S> {
    static constexpr int NW = 6;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const int ib = g & 7;
        ld8(R.b0 + 8 * g, w);                                 // qs of the group
        const uint8_t *h = R.b1 + 44 * (g >> 3);
        w[2] = *reinterpret_cast<const uint32_t *>(h + (ib & 4));   // the qh word holding byte ib
        w[3] = *reinterpret_cast<const uint32_t *>(h + 8 + 4 * ib); // 32 sign bits
        w[4] = *reinterpret_cast<const uint32_t *>(h + 40);         // the 4 scale bytes
        w[5] = ld2(R.b2 + 2 * (g >> 3));
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const GridTab<QT_IQ3_S> &T) {
        const int ib = g & 7;
        const uint32_t qh = (w[2] >> (8 * (ib & 3))) & 0xFFu;
        const uint32_t sc = (w[4] >> (8 * (ib >> 1) + 4 * (ib & 1))) & 0xFu;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t qq = l < 2 ? w[0] : w[1];
            const int s = 16 * (l & 1);
            const uint32_t sb = (w[3] >> (8 * l)) & 255u;  // the signs of values 8 l .. 8 l + 7
            const uint32_t g1 = neg_bytes(T.grid[((qq >> s) & 255u) | ((qh << (8 - 2 * l)) & 256u)], T.sgn[2 * sb]);
            const uint32_t g2 =
                neg_bytes(T.grid[((qq >> (s + 8)) & 255u) | ((qh << (7 - 2 * l)) & 256u)], T.sgn[2 * sb + 1]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                o.q[8 * l + j] = sbyte(g1, j);
                o.q[8 * l + 4 + j] = sbyte(g2, j);
            }
        }
        o.s[0] = o.s[1] = h2f(w[5]) * (float) (1 + 2 * (int) sc);
        o.m[0] = o.m[1] = 0.0f;
    }
};

// 8 magnitudes of an 8-byte grid entry e (two words at 2e) with the signs of sign byte sg into q[8l .. 8l + 7]
template <uint32_t TY>
__device__ __forceinline__ void grid8(float *q, const GridTab<TY> &T, uint32_t e, uint32_t sg) {
    const uint32_t g0 = neg_bytes(T.grid[2 * e], T.sgn[2 * sg]), g1 = neg_bytes(T.grid[2 * e + 1], T.sgn[2 * sg + 1]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        q[j] = sbyte(g0, j);
        q[4 + j] = sbyte(g1, j);
    }
}

// IQ2_XXS: super-blocks of 256 (d fp16, qs u16[32]); packed as plane 0 = qs, plane 1 = d.  Group ib: 4 grid bytes
// (8-magnitude points from {8, 25, 43}) and a word of 4 seven-bit sign indices with a 4-bit scale s in bits 28-31;
// db = d (0.5 + s) / 4 (ggml: y = db * grid[j] * sign; every product exact)
template <> struct Q<QT_IQ2_XXS> {
    static constexpr int NW = 3;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        ld8(R.b0 + 8 * g, w);
        w[2] = ld2(R.b1 + 2 * (g >> 3));
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const GridTab<QT_IQ2_XXS> &T) {
#pragma unroll
        for (int l = 0; l < 4; ++l) grid8(o.q + 8 * l, T, (w[0] >> (8 * l)) & 255u, ksign((w[1] >> (7 * l)) & 127u));
        o.s[0] = o.s[1] = h2f(w[2]) * (0.5f + (float) (w[1] >> 28)) * 0.25f;
        o.m[0] = o.m[1] = 0.0f;
    }
};

// IQ2_XS: super-blocks of 256 (d, qs u16[32], scales[8]); packed as plane 0 = qs, plane 1 = scales, plane 2 = d.
// Group ib: 4 codes of a 9-bit grid index (512 points) and a 7-bit sign index; scale nibbles of scales[ib] for its
// first and second 16 values
template <> struct Q<QT_IQ2_XS> {
    static constexpr int NW = 4;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const int ib = g & 7;
        ld8(R.b0 + 8 * g, w);
        w[2] = *reinterpret_cast<const uint32_t *>(R.b1 + 8 * (g >> 3) + (ib & 4));
        w[3] = ld2(R.b2 + 2 * (g >> 3));
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const GridTab<QT_IQ2_XS> &T) {
        const int ib = g & 7;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t c = (w[l >> 1] >> (16 * (l & 1))) & 0xFFFFu;
            grid8(o.q + 8 * l, T, c & 511u, ksign(c >> 9));
        }
        const uint32_t sc = (w[2] >> (8 * (ib & 3))) & 0xFFu;
        const float d = h2f(w[3]);
        o.s[0] = d * (0.5f + (float) (sc & 15u)) * 0.25f;
        o.s[1] = d * (0.5f + (float) (sc >> 4)) * 0.25f;
        o.m[0] = o.m[1] = 0.0f;
    }
};

// IQ2_S: super-blocks of 256 (d, qs[32] grid low bytes, signs[32], qh[8], scales[8]); packed as plane 0 = qs + signs,
// plane 1 = qh + scales, plane 2 = d.  Group ib: grid index qs[4 ib + l] | bits 2l, 2l + 1 of qh[ib] << 8 (1024
// points), a full sign byte per 8 values, two scale nibbles
template <> struct Q<QT_IQ2_S> {
    static constexpr int NW = 5;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const int ib = g & 7;
        const uint8_t *a = R.b0 + 64 * (g >> 3), *h = R.b1 + 16 * (g >> 3);
        w[0] = *reinterpret_cast<const uint32_t *>(a + 4 * ib);
        w[1] = *reinterpret_cast<const uint32_t *>(a + 32 + 4 * ib);
        w[2] = *reinterpret_cast<const uint32_t *>(h + (ib & 4));
        w[3] = *reinterpret_cast<const uint32_t *>(h + 8 + (ib & 4));
        w[4] = ld2(R.b2 + 2 * (g >> 3));
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const GridTab<QT_IQ2_S> &T) {
        const int ib = g & 7;
        const uint32_t qh = (w[2] >> (8 * (ib & 3))) & 0xFFu, sc = (w[3] >> (8 * (ib & 3))) & 0xFFu;
#pragma unroll
        for (int l = 0; l < 4; ++l)
            grid8(o.q + 8 * l, T, ((w[0] >> (8 * l)) & 255u) | ((qh << (8 - 2 * l)) & 0x300u), (w[1] >> (8 * l)) & 255u);
        const float d = h2f(w[4]);
        o.s[0] = d * (0.5f + (float) (sc & 15u)) * 0.25f;
        o.s[1] = d * (0.5f + (float) (sc >> 4)) * 0.25f;
        o.m[0] = o.m[1] = 0.0f;
    }
};

// IQ3_XXS: super-blocks of 256 (d, qs[64] grid bytes, scales_and_signs u32[8]); packed as plane 0 = qs + the words,
// plane 1 = d.  Group ib: 8 grid bytes (4-magnitude points, 256 of them) and a word of 4 sign indices with a 4-bit
// scale; db = d (0.5 + s) / 2
template <> struct Q<QT_IQ3_XXS> {
    static constexpr int NW = 4;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        const int ib = g & 7;
        const uint8_t *a = R.b0 + 96 * (g >> 3);
        ld8(a + 8 * ib, w);
        w[2] = *reinterpret_cast<const uint32_t *>(a + 64 + 4 * ib);
        w[3] = ld2(R.b1 + 2 * (g >> 3));
    }
    __device__ static void unpack(const uint32_t *w, int g, Grp &o, const GridTab<QT_IQ3_XXS> &T) {
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t qq = w[l >> 1], s = 16 * (l & 1), sg = ksign((w[2] >> (7 * l)) & 127u);
            const uint32_t g1 = neg_bytes(T.grid[(qq >> s) & 255u], T.sgn[2 * sg]);
            const uint32_t g2 = neg_bytes(T.grid[(qq >> (s + 8)) & 255u], T.sgn[2 * sg + 1]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                o.q[8 * l + j] = sbyte(g1, j);
                o.q[8 * l + 4 + j] = sbyte(g2, j);
            }
        }
        o.s[0] = o.s[1] = h2f(w[3]) * (0.5f + (float) (w[2] >> 28)) * 0.5f;
        o.m[0] = o.m[1] = 0.0f;
    }
};

// Q2_0 (the reference fork's type 42): blocks of 64 (d fp16, 16 bytes of 2-bit codes, value v at bits 2 (v % 4) of
// byte v / 4); packed as plane 0 = codes, plane 1 = d; y = d * (q - 1)
template <> struct Q<QT_Q2_0> {
    static constexpr int NW = 3;
    static constexpr int U = prefetch_groups(NW);
    static constexpr bool MIN = false;
    template <class R_> __device__ static void load(const R_ &R, int g, uint32_t *w) {
        ld8(R.b0 + 8 * g, w);
        w[2] = ld2(R.b1 + 2 * (g >> 1));
    }
    __device__ static void unpack(const uint32_t *w, int, Grp &o, const NoTab &T) {
#pragma unroll
        for (int v = 0; v < 32; ++v) o.q[v] = (float) ((int) ((w[v >> 4] >> (2 * (v & 15))) & 3u) - 1);
        o.s[0] = o.s[1] = h2f(w[2]);
        o.m[0] = o.m[1] = 0.0f;
    }
};

// the GGUF value of code q (a decoded group's entry) in half h, rounded once as ggml's dequantisers round it:
// fl(s q - m), or for Q6_K, whose minimum is 32 s, fl(s (q - 32)) (the same value, and the sign of a zero kept)
template <uint32_t TY> __device__ __forceinline__ float gguf_value(const Grp &o, int h, float q) {
    if constexpr (TY == QT_BF16) return q;
    else if constexpr (TY == QT_Q6_K) return o.s[h] * (q - 32.0f);
    else return __builtin_fmaf(o.s[h], q, -o.m[h]);
}

template <uint32_t TY> __device__ __forceinline__ void decode(const PP &P, int row, int g, Grp &o) {
    uint32_t w[Q<TY>::NW];
    const TabT<TY> T;
    Q<TY>::load(row_planes(P, row), g, w);
    Q<TY>::unpack(w, g, o, T);
}

// ------------------------------------------------------------------------------------------------------------
// kernels

// planes -> float rows, one thread per (row, group of 32), the GGUF value fl(s * q - m) rounded once
template <uint32_t TY> __global__ void k_dequant(PP P, int rows, int G, int cols, float *__restrict__ out) {
    if constexpr (tab_lds<TY>() > 0) {
        tab_fill<TY>(threadIdx.x, blockDim.x);
        __syncthreads();
    }
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) rows * G) return;
    const int row = (int) (i / G), g = (int) (i % G);
    Grp o;
    decode<TY>(P, row, g, o);
    float4 *dst = reinterpret_cast<float4 *>(out + (size_t) row * cols + (size_t) g * 32);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int h = c >> 2;
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float q = o.q[4 * c + k];
            v[k] = gguf_value<TY>(o, h, q);
        }
        dst[c] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// sum over the LPR lanes of a row (16: one DPP row, 32: half a wave, 64: the wave); every lane of the row gets it
template <int LPR> __device__ __forceinline__ float lane_row_sum(float v) {
    if constexpr (LPR == 16) return row_sum(v);
    else if constexpr (LPR == 32) return half_sum(v);
    else return wave_sum(v);
}

// one group's contribution to the NT accumulators; xg points at the group's x in LDS: float4 c of token t at
// xg[t * 8 + c] (offsets known at compile time).  The arithmetic (and its order) does not depend on NT: token t of
// an NT-token call gets the bits a one-token call gets.
// FAC (formats with a minimum, Q4_K / Q5_K): sum_j (s q_j - m) x_j is taken as s (sum_j q_j x_j) - m (sum_j x_j),
// with the half-group sums of x from xsm[2 t + h] (x_half_sums), which every row of the call shares: the dequantised
// value is never formed, one multiply-add per value fewer.  Without FAC each value is dequantised to fl(s q - m)
// first (the GGUF value, as k_dequant writes it).
template <uint32_t TY, int NT, bool FAC = false>
__device__ __forceinline__ void accumulate(const uint32_t *w, int g, const float4 *xg, float *acc,
                                           const TabT<TY> &T, const float *xsm = nullptr) {
    Grp o;
    Q<TY>::unpack(w, g, o, T);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if constexpr (Q<TY>::MIN && !FAC) {
            float wv[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) wv[j] = gguf_value<TY>(o, h, o.q[16 * h + j]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float a = acc[t];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 xv = xg[t * 8 + 4 * h + c];
                    a = __builtin_fmaf(wv[4 * c], xv.x, a);
                    a = __builtin_fmaf(wv[4 * c + 1], xv.y, a);
                    a = __builtin_fmaf(wv[4 * c + 2], xv.z, a);
                    a = __builtin_fmaf(wv[4 * c + 3], xv.w, a);
                }
                acc[t] = a;
            }
        } else if constexpr (Q<TY>::MIN) {
            // one chain per half and token: s (q . x) - m (sum x), three operations a token beyond the products
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float d = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 xv = xg[t * 8 + 4 * h + c];
                    d = __builtin_fmaf(o.q[16 * h + 4 * c], xv.x, d);
                    d = __builtin_fmaf(o.q[16 * h + 4 * c + 1], xv.y, d);
                    d = __builtin_fmaf(o.q[16 * h + 4 * c + 2], xv.z, d);
                    d = __builtin_fmaf(o.q[16 * h + 4 * c + 3], xv.w, d);
                }
                acc[t] = __builtin_fmaf(-o.m[h], xsm[2 * t + h], __builtin_fmaf(o.s[h], d, acc[t]));
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 xv = xg[t * 8 + 4 * h + c];
                    d0 = __builtin_fmaf(o.q[16 * h + 4 * c], xv.x, d0);
                    d1 = __builtin_fmaf(o.q[16 * h + 4 * c + 1], xv.y, d1);
                    d0 = __builtin_fmaf(o.q[16 * h + 4 * c + 2], xv.z, d0);
                    d1 = __builtin_fmaf(o.q[16 * h + 4 * c + 3], xv.w, d1);
                }
                acc[t] = __builtin_fmaf(o.s[h], d0 + d1, acc[t]);
            }
        }
    }
}


// x of tokens [0, NT) and groups [c0, c0 + nch) -> LDS, group-major: float4 c of token t of group c0 + gr at
// xs[gr * xs_stride(NT) + t * 8 + c].  The stride is odd (in float4), so the lanes of a row, which read consecutive
// groups, hit distinct bank quads, and every read's offset inside a group is an immediate.  One pass moves XB float4
// per thread; its loads are clamped to the last element, so the pass's array stays in registers.
constexpr int xs_stride(int nt) { return nt * 8 + 1; }

// formats whose GEMV takes the factored minimum (accumulate<FAC>) and so stages the half-group sums of x
template <uint32_t TY> constexpr bool gemv_fac() { return Q<TY>::MIN; }
// LDS bytes per group of x in the GEMV kernels: the x float4s (xs_stride(nt) of them) and, for gemv_fac formats,
// the nt x 2 half-group sums
template <uint32_t TY> constexpr int xs_group_bytes(int nt) {
    return (nt * 8 + 1) * (int) sizeof(float4) + (gemv_fac<TY>() ? nt * 2 * (int) sizeof(float) : 0);
}

// the half-group sums of the staged x (groups [0, nch) of the LDS layout below): xsm[(gr NT + t) 2 + h] = the 16
// values x[t][32 gr + 16 h + j], j = 0..15, added in order, so that every launch shape and token count gets the
// same sums.  nth threads; the caller publishes them with a barrier.
template <int NT>
__device__ __forceinline__ void x_half_sums(const float4 *xs, int nch, float *xsm, int tid, int nth) {
    for (int i = tid; i < nch * NT * 2; i += nth) {
        const int h = i & 1, tg = i >> 1, gr = tg / NT, t = tg - gr * NT;
        const float4 *p = xs + gr * xs_stride(NT) + t * 8 + 4 * h;
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 v = p[c];
            s += v.x;
            s += v.y;
            s += v.z;
            s += v.w;
        }
        xsm[i] = s;
    }
}

typedef float f4v __attribute__((ext_vector_type(4)));

// The x of a pass is held as native 4-float vectors: a float4 (a struct) loaded and stored unchanged becomes a
// 16-byte global-to-LDS memcpy, which the compiler places (load and store) at the store, behind the weight loads
// requested in between, so that the store waited for them all (vmcnt counts loads in issue order).
template <int NT, int XB> struct XPass {
    f4v r[XB];
    __device__ __forceinline__ void load(const float *__restrict__ x, int cols, int c0, int nch, int e0, int tid,
                                         int nth) {
        const int nx = NT * 8 * nch;
#pragma unroll
        for (int k = 0; k < XB; ++k) {
            const int e = min(e0 + tid + nth * k, nx - 1), tg = e >> 3, t = tg / nch, gr = tg - t * nch;
            r[k] = *reinterpret_cast<const f4v *>(x + (size_t) t * cols + (size_t) (c0 + gr) * 32 + 4 * (e & 7));
        }
    }
    // stores clamped like the loads (a lane past the end writes the last element's value to its place again), so
    // that the loads and stores of a pass sit in one basic block
    __device__ __forceinline__ void store(float4 *xs, int nch, int e0, int tid, int nth) const {
        const int nx = NT * 8 * nch;
#pragma unroll
        for (int k = 0; k < XB; ++k) {
            const int e = min(e0 + tid + nth * k, nx - 1), tg = e >> 3, t = tg / nch, gr = tg - t * nch;
            *reinterpret_cast<f4v *>(xs + gr * xs_stride(NT) + t * 8 + (e & 7)) = r[k];
        }
    }
};

// the passes of x after the first (x of many tokens): loaded and stored here, before the caller requests weights
template <int NT, int XB>
__device__ __forceinline__ void stage_x_rest(const float *__restrict__ x, int cols, int c0, int nch, float4 *xs,
                                             int tid) {
    for (int e0 = 512 * XB; e0 < NT * 8 * nch; e0 += 512 * XB) {
        XPass<NT, XB> q;
        q.load(x, cols, c0, nch, e0, tid, 512);
        q.store(xs, nch, e0, tid, 512);
    }
}

// batch j of row-set s over the groups [c0, c1): groups c0 + li + LPR (U j + u), u < U, of row s RPW + lane / LPR.
// Row and group are clamped into the weight: a lane past the last row or group loads a valid address whose value
// it never uses.
template <uint32_t TY, int LPR>
__device__ __forceinline__ void load_batch(const PP &P, int rows, int s, int j, int lane, int c0, int c1,
                                           uint32_t (&w)[Q<TY>::U][Q<TY>::NW]) {
    constexpr int U = Q<TY>::U;
    const RP32 R = row_planes32(P, min(s * (64 / LPR) + lane / LPR, rows - 1));
    const int gb = c0 + lane % LPR + LPR * U * j;
#pragma unroll
    for (int u = 0; u < U; ++u) Q<TY>::load(R, min(gb + LPR * u, c1 - 1), w[u]);
}

template <uint32_t TY, int NT, int LPR>
__device__ __forceinline__ void acc_batch(const uint32_t (&w)[Q<TY>::U][Q<TY>::NW], int j, int lane, int c0, int c1,
                                          const float4 *xs, const float *xsm, float *acc, const TabT<TY> &T) {
    constexpr int U = Q<TY>::U;
    const int gb = c0 + lane % LPR + LPR * U * j;
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (gb + LPR * u < c1) {
            const int gr = gb + LPR * u - c0;
            if constexpr (gemv_fac<TY>())
                accumulate<TY, NT, true>(w[u], gb + LPR * u, xs + gr * xs_stride(NT), acc, T, xsm + gr * NT * 2);
            else
                accumulate<TY, NT>(w[u], gb + LPR * u, xs + gr * xs_stride(NT), acc, T);
        }
}

// end of a row-set: the row sums (every lane of a row gets them) stored by the row's first lane; accumulators reset
template <int NT, int LPR>
__device__ __forceinline__ void flush_rows(int s, int lane, int rows, float *acc, float *__restrict__ out) {
    const int row = s * (64 / LPR) + lane / LPR;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = lane_row_sum<LPR>(acc[t]);
    if (lane % LPR == 0 && row < rows) {
#pragma unroll
        for (int t = 0; t < NT; ++t) out[(size_t) t * rows + row] = acc[t];
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
}

// GEMV of one split (blockIdx.y) of the groups: [g0, g1), g0 = blockIdx.y * gps.  A wave works on row-sets of
// 64 / LPR rows, LPR lanes per row; lane li of a row sums its groups li, li + LPR, ... in ascending order into one
// accumulator per token, then the row's LPR lanes are summed.  That arithmetic is the same in both kernels below,
// for every launch shape and token count, so token t of an nt-token call gets the bits of a one-token call on x[t].
//
// k_gemv, for a split whose x fits the LDS: the workgroup stages x once, then each wave walks its own row-sets
// s = global wave id, + waves in the grid, ..., in batches of U groups per lane, with the next batch's loads (the
// next row-set's, at the end of one) in flight while it sums the current one.  The host sizes the grid to the
// workgroups resident at once, so no workgroup waits for another to finish.  Two walks, picked by the host from the
// batches per wave (same bits):

// short walk (a wave has a few batches): a batch is loaded only when the wave has it.  The compiler's wait counts
// then merge the paths with and without the load and wait as if nothing newer were in flight, which costs nothing
// at this depth and saves the surplus loads of the deep walk
template <uint32_t TY, int NT, int LPR>
__device__ __forceinline__ void gemv_walk_short(const PP &P, int rows, int g0, int g1, int ng, int NS, int nws,
                                                int NB, const float *__restrict__ x, int cols,
                                                float *__restrict__ out, float4 *xs, float *xsm, int blk) {
    constexpr int NW = Q<TY>::NW, U = Q<TY>::U, XB = NT <= 2 ? 4 : 8;
    const int tid = threadIdx.x, lane = tid & 63;
    // the wave's batches in order: (s, j), then (s1, j1) = next(s, j), ...; wave-uniform, so the row reductions run
    // on whole waves
    int s = blk * 8 + __builtin_amdgcn_readfirstlane(tid >> 6), j = 0, s1, j1;
    const auto next = [NB, nws](int s_, int j_, int &sn, int &jn) {
        sn = j_ + 1 == NB ? s_ + nws : s_;
        jn = j_ + 1 == NB ? 0 : j_ + 1;
    };
    next(s, j, s1, j1);
    uint32_t wa[U][NW], wb[U][NW];
    // x [NT][cols] -> xs (the layout of XPass).  The first pass of x is requested before the first two weight
    // batches, so that its LDS writes wait for x alone (vmcnt counts loads in issue order); scheduling fences keep
    // the compiler from moving the weight loads ahead of it.  Further passes (x of many tokens) go before the
    // weight loads too, so that no path with a different count of loads in flight joins the walk.
    XPass<NT, XB> xp;
    xp.load(x, cols, g0, ng, 0, tid, 512);
    stage_x_rest<NT, XB>(x, cols, g0, ng, xs, tid);
    __builtin_amdgcn_sched_barrier(0);
    // unconditional (load_batch clamps the row: a wave past the last row-set loads a row it never sums), so that
    // this is one basic block with the x pass
    load_batch<TY, LPR>(P, rows, s, j, lane, g0, g1, wa);
    load_batch<TY, LPR>(P, rows, s1, j1, lane, g0, g1, wb);
    __builtin_amdgcn_sched_barrier(0);
    xp.store(xs, ng, 0, tid, 512);
    __syncthreads();
    if constexpr (gemv_fac<TY>()) {
        x_half_sums<NT>(xs, ng, xsm, tid, 512);
        lds_barrier();
    }
    const TabT<TY> T;  // (IQ4 formats) the level table, (grid formats) the codebook, both in LDS
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    // two batches in flight: while one is summed, the other (and then the one after it) is loading
    while (s < NS) {
        acc_batch<TY, NT, LPR>(wa, j, lane, g0, g1, xs, xsm, acc, T);
        if (j == NB - 1) flush_rows<NT, LPR>(s, lane, rows, acc, out);
        s = s1;
        j = j1;
        next(s, j, s1, j1);
        if (s >= NS) break;
        if (s1 < NS) load_batch<TY, LPR>(P, rows, s1, j1, lane, g0, g1, wa);
        acc_batch<TY, NT, LPR>(wb, j, lane, g0, g1, xs, xsm, acc, T);
        if (j == NB - 1) flush_rows<NT, LPR>(s, lane, rows, acc, out);
        s = s1;
        j = j1;
        next(s, j, s1, j1);
        if (s >= NS) break;
        if (s1 < NS) load_batch<TY, LPR>(P, rows, s1, j1, lane, g0, g1, wb);
    }
}

// deep walk (many batches per wave): a steady-state pipeline whose wait counts stay exact
template <uint32_t TY, int NT, int LPR>
__device__ __forceinline__ void gemv_walk_deep(const PP &P, int rows, int g0, int g1, int ng, int NS, int nws, int NB,
                                               const float *__restrict__ x, int cols, float *__restrict__ out,
                                               float4 *xs, float *xsm) {
    constexpr int NW = Q<TY>::NW, U = Q<TY>::U, XB = NT <= 2 ? 4 : 8;
    const int tid = threadIdx.x, lane = tid & 63;
    // The wave's batches: b = 0 .. n-1, batch b = groups batch b % NB of row-set w0 + (b / NB) * nws.  Everything
    // here is wave-uniform; readfirstlane makes that visible to the compiler, so the loops branch on scalars.
    const int w0 = blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = w0 < NS ? ((NS - 1 - w0) / nws + 1) * NB : 0;
    uint32_t wa[U][NW], wb[U][NW];
    const TabT<TY> T;  // (IQ4 formats) the level table, (grid formats) the codebook, both in LDS
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    // x [NT][cols] -> xs (the layout of XPass).  The first part of x is requested before the wave's first one or two
    // weight batches, so that its LDS writes wait for x alone.  A wave with one batch or none takes a short path
    // with no prefetch; every wave passes the one barrier either way.
    XPass<NT, XB> xp;
    {
        const int b1 = n > 1 ? 1 : 0;
        xp.load(x, cols, g0, ng, 0, tid, 512);
        stage_x_rest<NT, XB>(x, cols, g0, ng, xs, tid);
        __builtin_amdgcn_sched_barrier(0);  // (as in the short walk) x, then the weights, then x's LDS writes
        load_batch<TY, LPR>(P, rows, w0, 0, lane, g0, g1, wa);
        load_batch<TY, LPR>(P, rows, w0 + (b1 / NB) * nws, b1 % NB, lane, g0, g1, wb);
        __builtin_amdgcn_sched_barrier(0);
        xp.store(xs, ng, 0, tid, 512);
    }
    __syncthreads();
    if constexpr (gemv_fac<TY>()) {
        x_half_sums<NT>(xs, ng, xsm, tid, 512);
        lds_barrier();
    }
#define FN_GEMV_LOAD(W, B) load_batch<TY, LPR>(P, rows, w0 + ((B) / NB) * nws, (B) % NB, lane, g0, g1, W)
#define FN_GEMV_SUM(W, B)                                                                      \
    do {                                                                                       \
        acc_batch<TY, NT, LPR>(W, (B) % NB, lane, g0, g1, xs, xsm, acc, T);                    \
        if ((B) % NB == NB - 1) flush_rows<NT, LPR>(w0 + ((B) / NB) * nws, lane, rows, acc, out); \
    } while (0)
    // Steady state: two batches in flight while one is summed.  Every pass issues the same loads and the loop leaves
    // only at its test, so the compiler's wait counts stay exact (a path that skips a load makes them assume nothing
    // newer is in flight, and each wait would then drain the prefetched batch too).  The last two or three batches
    // go after the loop.
    int b = 0;
    for (; b + 3 < n; b += 2) {
        FN_GEMV_SUM(wa, b);
        FN_GEMV_LOAD(wa, b + 2);
        FN_GEMV_SUM(wb, b + 1);
        FN_GEMV_LOAD(wb, b + 3);
    }
    if (b < n) FN_GEMV_SUM(wa, b);
    if (b + 2 < n) FN_GEMV_LOAD(wa, b + 2);
    if (b + 1 < n) FN_GEMV_SUM(wb, b + 1);
    if (b + 2 < n) FN_GEMV_SUM(wa, b + 2);
#undef FN_GEMV_SUM
#undef FN_GEMV_LOAD
}

template <uint32_t TY, int NT, int LPR, bool DEEP>
__global__ void __launch_bounds__(512) k_gemv(PP P, int rows, int G, int gps, const float *__restrict__ x, int cols,
                                                float *__restrict__ out) {
    extern __shared__ float4 xs[];
    constexpr int U = Q<TY>::U, RPW = 64 / LPR;
    const int g0 = blockIdx.y * gps, g1 = min(G, g0 + gps), ng = g1 - g0;
    if (ng <= 0) return;  // (the plan gives every split a group; whole workgroup, before any barrier)
    const int NS = (rows + RPW - 1) / RPW, nws = gridDim.x * 8;
    const int NB = (ng + LPR * U - 1) / (LPR * U);
    out += (size_t) blockIdx.y * NT * rows;
    tab_fill<TY>(threadIdx.x, 512);  // published by the walk's barrier after the x staging
    float *xsm = reinterpret_cast<float *>(xs + gps * xs_stride(NT));  // (gemv_fac formats) the x sums, after x
    if constexpr (DEEP) gemv_walk_deep<TY, NT, LPR>(P, rows, g0, g1, ng, NS, nws, NB, x, cols, out, xs, xsm);
    else gemv_walk_short<TY, NT, LPR>(P, rows, g0, g1, ng, NS, nws, NB, x, cols, out, xs, xsm, blockIdx.x);
}

// k_gemv_c, for an x too large for the LDS: x goes through it in chunks of kc groups (a multiple of LPR, so a
// group's lane does not depend on the chunking); the workgroup's 8 waves take one row-set each and walk the chunks
// together.  Grid: one workgroup per 8 row-sets.
template <uint32_t TY, int NT, int LPR>
__global__ void __launch_bounds__(512) k_gemv_c(PP P, int rows, int G, int gps, int kc, const float *__restrict__ x,
                                                  int cols, float *__restrict__ out) {
    extern __shared__ float4 xs[];
    constexpr int NW = Q<TY>::NW, U = Q<TY>::U, RPW = 64 / LPR, XB = NT <= 2 ? 4 : 8;
    const int g0 = blockIdx.y * gps, g1 = min(G, g0 + gps);
    if (g1 <= g0) return;  // (the plan gives every split a group; whole workgroup, before any barrier)
    const int tid = threadIdx.x, lane = tid & 63;
    const int s = blockIdx.x * 8 + (tid >> 6);
    const bool live = s < (rows + RPW - 1) / RPW;  // wave-uniform
    out += (size_t) blockIdx.y * NT * rows;
    tab_fill<TY>(tid, 512);  // published by the chunk loop's first barrier
    float *xsm = reinterpret_cast<float *>(xs + kc * xs_stride(NT));  // (gemv_fac formats) the chunk's x sums
    const TabT<TY> T;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    uint32_t wa[U][NW], wb[U][NW];
    XPass<NT, XB> xp;
    for (int c0 = g0; c0 < g1; c0 += kc) {
        const int c1 = min(g1, c0 + kc), nch = c1 - c0, NB = (nch + LPR * U - 1) / (LPR * U);
        __syncthreads();  // every wave is done reading the previous chunk
        xp.load(x, cols, c0, nch, 0, tid, 512);
        stage_x_rest<NT, XB>(x, cols, c0, nch, xs, tid);
        __builtin_amdgcn_sched_barrier(0);  // (as in k_gemv's walks) x, then the weights, then x's LDS writes
        load_batch<TY, LPR>(P, rows, s, 0, lane, c0, c1, wa);  // (row clamped: a dead wave's loads go unused)
        __builtin_amdgcn_sched_barrier(0);
        xp.store(xs, nch, 0, tid, 512);
        __syncthreads();
        if constexpr (gemv_fac<TY>()) {
            x_half_sums<NT>(xs, nch, xsm, tid, 512);
            lds_barrier();
        }
        if (!live) continue;
        for (int j = 0; j < NB; j += 2) {
            if (j + 1 < NB) load_batch<TY, LPR>(P, rows, s, j + 1, lane, c0, c1, wb);
            acc_batch<TY, NT, LPR>(wa, j, lane, c0, c1, xs, xsm, acc, T);
            if (j + 1 >= NB) break;
            if (j + 2 < NB) load_batch<TY, LPR>(P, rows, s, j + 2, lane, c0, c1, wa);
            acc_batch<TY, NT, LPR>(wb, j + 1, lane, c0, c1, xs, xsm, acc, T);
        }
    }
    if (live) flush_rows<NT, LPR>(s, lane, rows, acc, out);
}


constexpr int kLdsPerCu = 160 * 1024;  // LDS of a CDNA4 CU (the most one workgroup can take)


inline PP planes(const QLayout &L, const uint8_t *packed) {
    PP P{packed + L.off[0], packed + L.off[1], packed + L.off[2], L.rs[0], L.rs[1], L.rs[2]};
    return P;
}

// One GEMV launch.  x of the split in the LDS at once when it fits the CU's 160 KB: k_gemv on a grid of the
// workgroups resident at once.  Else k_gemv_c with chunks of the largest multiple of LPR groups whose x fits 80 KB
// (two workgroups per CU), evened out.
template <uint32_t TY, int NT, int LPR>
int gemv_nt(const QLayout &L, const GemvPlan &pl, const PP &P, const float *x, float *out, hipStream_t st) {
    const int gps = (pl.ngroups + pl.ks - 1) / pl.ks, ns = (L.rows + 64 / LPR - 1) / (64 / LPR);
    int nwg = (ns + 7) / 8;
    constexpr int XS = xs_group_bytes<TY>(NT);  // LDS bytes per group of x (and its sums)
    constexpr int LDS = kLdsPerCu - tab_lds<TY>();            // what x may take beside the format's table
    if (gps <= LDS / XS && g_ov_kernel != 1) {
        static int by_regs = 0;  // workgroups per CU the registers allow (the deep walk's, the larger of the two)
        if (!by_regs) {
            int n = 0;
            FN_CK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv<TY, NT, LPR, true>, 512, 0));
            by_regs = std::max(1, n);
        }
        const size_t lds = (size_t) gps * XS;
        int per_cu = std::min(by_regs, std::max(1, (int) (kLdsPerCu / (lds + tab_lds<TY>()))));
        // one token through a tall weight (each wave would walk 32 or more batches): one workgroup per CU more than
        // fit at once (measured: the Q5_K LM head, 248320 x 2560, 143-156 -> 114-117 us; the launch shape never
        // changes the bits)
        {
            const int nb1 = (gps + LPR * Q<TY>::U - 1) / (LPR * Q<TY>::U);
            const int nwg1 = std::min(nwg, device_cus() * per_cu);
            if (NT == 1 && (ns + 8 * nwg1 - 1) / (8 * nwg1) * nb1 >= 32 &&
                (size_t) (per_cu + 1) * (lds + tab_lds<TY>()) <= (size_t) kLdsPerCu)
                ++per_cu;
        }
        if (g_ov_wpc) per_cu = std::max(1, g_ov_wpc / 8);
        if (g_persist) nwg = std::min(nwg, device_cus() * per_cu);
        // batches of the busiest wave; from 4 on the deep walk's exact waits pay for its surplus loads (measured)
        const int nb = (gps + LPR * Q<TY>::U - 1) / (LPR * Q<TY>::U), per_wave = (ns + 8 * nwg - 1) / (8 * nwg) * nb;
        const bool deep = g_ov_kernel == 3 || (g_ov_kernel != 4 && per_wave >= 4);
        const auto kern = deep ? k_gemv<TY, NT, LPR, true> : k_gemv<TY, NT, LPR, false>;
        hipLaunchKernelGGL(kern, dim3((unsigned) nwg, (unsigned) pl.ks), dim3(512), lds, st, P, L.rows, pl.ngroups,
                           gps, x, L.cols, out);
    } else {
        int kc = g_ov_kernel == 1 ? LPR : std::max(LPR, (kLdsPerCu / 2 - tab_lds<TY>()) / XS / LPR * LPR);
        const int nch = (gps + kc - 1) / kc;
        kc = std::min(kc, ((gps + nch - 1) / nch + LPR - 1) / LPR * LPR);
        const size_t lds = (size_t) kc * XS;
        hipLaunchKernelGGL((k_gemv_c<TY, NT, LPR>), dim3((unsigned) nwg, (unsigned) pl.ks), dim3(512), lds, st, P,
                           L.rows, pl.ngroups, gps, kc, x, L.cols, out);
    }
    FN_CK(hipGetLastError());
    return 0;
}

// Grouped GEMV: weights of different formats and the same cols over one x, in one launch.  Workgroups
// [0, nwg_0) walk part 0, the next nwg_1 part 1, and so on; each stages x itself and walks its part's row-sets
// (wave w of the part's workgroups: row-sets w, w + 8 nwg, ...) with the short walk, LPR lanes per row for every
// part.  A row's arithmetic is the GEMV's with that LPR, whatever the grid's split among the parts.
struct GPart {
    PP P;
    int rows, nwg;
    float *out;
};
template <int N> struct GParts {
    GPart p[N];
};

template <int NT, int LPR, int I, int N, uint32_t TY, uint32_t... R>
__device__ __forceinline__ void grp_walk(const GParts<N> &ps, int blk, int G, const float *__restrict__ x, int cols,
                                         float4 *xs) {
    if (blk < ps.p[I].nwg) {
        constexpr int U = Q<TY>::U, RPW = 64 / LPR;
        const GPart &p = ps.p[I];
        tab_fill<TY>(threadIdx.x, 512);  // published by the walk's barrier after the x staging
        // (gemv_fac formats) the x sums after the x groups; the launch sizes the LDS for them when a part needs them
        float *xsm = reinterpret_cast<float *>(xs + G * xs_stride(NT));
        gemv_walk_short<TY, NT, LPR>(p.P, p.rows, 0, G, G, (p.rows + RPW - 1) / RPW, p.nwg * 8,
                                     (G + LPR * U - 1) / (LPR * U), x, cols, p.out, xs, xsm, blk);
    } else if constexpr (sizeof...(R) > 0) {
        grp_walk<NT, LPR, I + 1, N, R...>(ps, blk - ps.p[I].nwg, G, x, cols, xs);
    }
}

template <int NT, int LPR, uint32_t... TS>
__global__ void __launch_bounds__(512) k_gemv_grp(GParts<sizeof...(TS)> ps, int G, const float *__restrict__ x,
                                                    int cols) {
    extern __shared__ float4 xs[];
    grp_walk<NT, LPR, 0, sizeof...(TS), TS...>(ps, blockIdx.x, G, x, cols, xs);
}

// parts in the order of TS; the caller has checked that x of NT tokens fits the LDS beside the formats' tables.
// The grid is the workgroups resident at once (or fewer: one row-set per wave at most), shared among the parts by
// their packed bytes, at least one workgroup each.
template <int NT, int LPR, uint32_t... TS>
int gemv_grp_nt(const QLayout *const *L, const PP *P, float *const *y, const float *x, hipStream_t st) {
    constexpr int N = sizeof...(TS), RPW = 64 / LPR;
    const int G = L[0]->cols / 32;
    constexpr bool FAC = (gemv_fac<TS>() || ...);
    const size_t lds = (size_t) G * (xs_stride(NT) * sizeof(float4) + (FAC ? NT * 2 * sizeof(float) : 0)),
                 tabs = (size_t) (tab_lds<TS>() + ...);
    static int by_regs = 0;
    if (!by_regs) {
        int n = 0;
        FN_CK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv_grp<NT, LPR, TS...>, 512, 0));
        by_regs = std::max(1, n);
    }
    const int per_cu = std::min(by_regs, std::max(1, (int) (kLdsPerCu / (lds + tabs))));
    const int budget = device_cus() * per_cu;
    GParts<N> ps;
    int need[N], sum_need = 0;
    double bytes = 0;
    for (int i = 0; i < N; ++i) {
        need[i] = ((L[i]->rows + RPW - 1) / RPW + 7) / 8;
        sum_need += need[i];
        bytes += (double) L[i]->bytes;
    }
    int nwg = 0;
    for (int i = 0; i < N; ++i) {
        int w = need[i];
        if (sum_need > budget) w = std::min(need[i], std::max(1, (int) (budget * (double) L[i]->bytes / bytes)));
        ps.p[i] = GPart{P[i], L[i]->rows, w, y[i]};
        nwg += w;
    }
    hipLaunchKernelGGL((k_gemv_grp<NT, LPR, TS...>), dim3((unsigned) nwg), dim3(512), lds, st, ps, G, x, L[0]->cols);
    FN_CK(hipGetLastError());
    return 0;
}

template <int LPR, uint32_t... TS>
int gemv_grp_l(const QLayout *const *L, const PP *P, float *const *y, const float *x, int nt, hipStream_t st) {
    switch (nt) {
        case 1: return gemv_grp_nt<1, LPR, TS...>(L, P, y, x, st);
        case 2: return gemv_grp_nt<2, LPR, TS...>(L, P, y, x, st);
        case 3: return gemv_grp_nt<3, LPR, TS...>(L, P, y, x, st);
        case 4: return gemv_grp_nt<4, LPR, TS...>(L, P, y, x, st);
        case 5: return gemv_grp_nt<5, LPR, TS...>(L, P, y, x, st);
        case 6: return gemv_grp_nt<6, LPR, TS...>(L, P, y, x, st);
        case 7: return gemv_grp_nt<7, LPR, TS...>(L, P, y, x, st);
        case 8: return gemv_grp_nt<8, LPR, TS...>(L, P, y, x, st);
        default: FN_FAIL("gemv: nt must be 1..8");
    }
}

template <uint32_t... TS>
int gemv_grp(const QLayout *const *L, const PP *P, float *const *y, const float *x, int nt, int lpr, hipStream_t st) {
    return lpr == 32 ? gemv_grp_l<32, TS...>(L, P, y, x, nt, st) : gemv_grp_l<64, TS...>(L, P, y, x, nt, st);
}

template <uint32_t TY, int LPR>
int gemv_tl(const QLayout &L, const GemvPlan &pl, const PP &P, const float *x, int nt, float *out, hipStream_t st) {
    switch (nt) {
        case 1: return gemv_nt<TY, 1, LPR>(L, pl, P, x, out, st);
        case 2: return gemv_nt<TY, 2, LPR>(L, pl, P, x, out, st);
        case 3: return gemv_nt<TY, 3, LPR>(L, pl, P, x, out, st);
        case 4: return gemv_nt<TY, 4, LPR>(L, pl, P, x, out, st);
        case 5: return gemv_nt<TY, 5, LPR>(L, pl, P, x, out, st);
        case 6: return gemv_nt<TY, 6, LPR>(L, pl, P, x, out, st);
        case 7: return gemv_nt<TY, 7, LPR>(L, pl, P, x, out, st);
        case 8: return gemv_nt<TY, 8, LPR>(L, pl, P, x, out, st);
        default: FN_FAIL("gemv: nt must be 1..8");
    }
}

template <uint32_t TY>
int gemv_t(const QLayout &L, const GemvPlan &pl, const PP &P, const float *x, int nt, float *out, hipStream_t st) {
    switch (pl.lpr) {
        case 16: return gemv_tl<TY, 16>(L, pl, P, x, nt, out, st);
        case 32: return gemv_tl<TY, 32>(L, pl, P, x, nt, out, st);
        default: return gemv_tl<TY, 64>(L, pl, P, x, nt, out, st);
    }
}

// ------------------------------------------------------------------------------------------------------------
// n float4 into the LDS with nth threads (thread tid takes elements tid, tid + nth, ...), in rounds of XR per thread:
// a round's loads are all issued (unconditionally, clamped to the last element) before any of its stores, so it costs
// one memory round trip -- a loop of load-then-store, or loads under a branch, waits for each load before the next.
// Loads complete in issue order, so a caller issues the first round's loads (load), then other loads the LDS rows
// are not waiting for, then the stores (store), then the further rounds (stage_rest, for n > XR nth).
// src(e) returns element e, dst(e, v) stores it.
template <int XR> struct LdsStage {
    float4 r[XR];
    template <typename Src> __device__ __forceinline__ void load(int n, int e0, int tid, int nth, const Src &src) {
#pragma unroll
        for (int k = 0; k < XR; ++k) r[k] = src(min(e0 + tid + nth * k, n - 1));
    }
    template <typename Dst>
    __device__ __forceinline__ void store(int n, int e0, int tid, int nth, const Dst &dst) const {
#pragma unroll
        for (int k = 0; k < XR; ++k) {
            const int e = e0 + tid + nth * k;
            if (e < n) dst(e, r[k]);
        }
    }
};
template <int XR, typename Src, typename Dst>
__device__ __forceinline__ void stage_rest(int n, int tid, int nth, const Src &src, const Dst &dst) {
    for (int e0 = nth * XR; e0 < n; e0 += nth * XR) {
        LdsStage<XR> st;
        st.load(n, e0, tid, nth, src);
        st.store(n, e0, tid, nth, dst);
    }
}

// rows selected on the device: the model's token embedding and routed experts

// embedding rows: out[t][k cols + c] = decoded W[ids[t]][c], for k < copies.  grid nt, 256 threads
template <uint32_t TY>
__global__ void __launch_bounds__(256) k_embed(PP P, int G, int cols, const int32_t *__restrict__ ids, int copies,
                                               float *__restrict__ out) {
    if constexpr (tab_lds<TY>() > 0) {
        tab_fill<TY>(threadIdx.x, blockDim.x);
        __syncthreads();
    }
    const int t = blockIdx.x, row = ids[t];
    for (int g = threadIdx.x; g < G; g += blockDim.x) {
        Grp o;
        decode<TY>(P, row, g, o);
        float4 v[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int h = c >> 2;
            float e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float q = o.q[4 * c + k];
                e[k] = gguf_value<TY>(o, h, q);
            }
            v[c] = make_float4(e[0], e[1], e[2], e[3]);
        }
        for (int k = 0; k < copies; ++k) {
            float4 *dst = reinterpret_cast<float4 *>(out + ((size_t) t * copies + k) * cols + (size_t) g * 32);
#pragma unroll
            for (int c = 0; c < 8; ++c) dst[c] = v[c];
        }
    }
}

// n-gram rows (NgramGather): workgroup t hashes the context of token t once per thread, then decodes its
// (head, group) items; the context's earlier positions come from the token ring and this call's own from ids, and
// thread 0 writes token t's ring slot, which no workgroup of the call reads.  grid nt, 256 threads
template <uint32_t TY>
__global__ void __launch_bounds__(256) k_ngram_rows(PP P, int G, int cols, NgramGather ng, float *__restrict__ out) {
    if constexpr (tab_lds<TY>() > 0) {
        tab_fill<TY>(threadIdx.x, blockDim.x);
        __syncthreads();
    }
    const int t = blockIdx.x, p0 = *ng.pos, p = p0 + t;
    long long c[3];
    c[0] = ng.ids[t];
    bool open = true;
#pragma unroll
    for (int k = 1; k < 3; ++k) {
        open = open && p - k >= 0;
        const int q = p - k;
        c[k] = open ? (q >= p0 ? ng.ids[q - p0] : ng.ring[q & ng.ring_mask]) : ng.eos;
        open = open && c[k] != ng.eos;
    }
    if (threadIdx.x == 0) ng.ring[p & ng.ring_mask] = ng.ids[t];
    const uint64_t *mult = ng.tab, *size = ng.tab + 3, *first = ng.tab + 3 + ng.heads;
    for (int i = threadIdx.x; i < ng.heads * G; i += blockDim.x) {
        const int hd = i / G, g = i - hd * G;
        uint64_t key = (uint64_t) c[0] * mult[0] ^ (uint64_t) c[1] * mult[1];
        if (2 * hd >= ng.heads) key ^= (uint64_t) c[2] * mult[2];
        const int row = (int) (first[hd] + key % size[hd]);
        Grp o;
        decode<TY>(P, row, g, o);
        float4 *dst = reinterpret_cast<float4 *>(out + ((size_t) t * ng.heads + hd) * cols + (size_t) g * 32);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            float e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float q = o.q[4 * v + k];
                e[k] = gguf_value<TY>(o, v >> 2, q);
            }
            dst[v] = make_float4(e[0], e[1], e[2], e[3]);
        }
    }
}

// row r of expert sel[p] (R rows per expert) against x[p / xdiv]: 16 lanes per row; lane li sums its groups li,
// li + 16, ... in order, then the 16 lanes are summed.  Plain rows: 4 rows per wave, 16 per workgroup.
// SWIGLU: the gate row of Wg and the up row of Wu, out = silu(g) * u; lanes 0-15 of each 32-lane half of a wave
// take the gate row and lanes 16-31 the up row (2 rows per wave, 8 per workgroup), and the up sum crosses over by a
// swizzle, so every lane decodes one weight.  grid (ceil(R / rows per workgroup), npairs), 256 threads.
// One memory round trip before the arithmetic: the lane's first ROWS_PRE groups of weight words, the x row (into
// LDS, group-major with an odd float4 stride so that a row's 16 lanes read distinct bank quads) and the format's
// codebook are all requested before the one barrier.  LDS: 9 float4 per group of x.
constexpr int ROWS_PRE = 5;
template <bool SWIGLU> constexpr int rows_per_wg() { return SWIGLU ? 8 : 16; }
template <uint32_t TY, bool SWIGLU>
__global__ void __launch_bounds__(256) k_rows(PP Pg, PP Pu, int R, int nexp, int G, int cols,
                                              const int32_t *__restrict__ sel, int xdiv, const float *__restrict__ x,
                                              float *__restrict__ out, RouteIn rt) {
    extern __shared__ float4 xs[];  // [G][9]
    __shared__ int e_sh;
    constexpr int NW = Q<TY>::NW;
    const int p = blockIdx.y, tid = threadIdx.x, lane = tid & 63, li = lane & 15;
    const bool up = SWIGLU && (lane & 16);  // (SWIGLU) this lane sums the up row
    const int r = SWIGLU ? blockIdx.x * 8 + (tid >> 6) * 2 + (lane >> 5)
                         : blockIdx.x * 16 + (tid >> 6) * 4 + (lane >> 4);
    const bool routed = SWIGLU && rt.rsg != nullptr;
    uint32_t w[ROWS_PRE][NW];
    RP rw;
    const auto load_pre = [&](int e) {  // an id outside the weight reads its last expert
        const int row = min(max(e, 0), nexp - 1) * R + min(r, R - 1);
        rw = row_planes(up ? Pu : Pg, row);
#pragma unroll
        for (int k = 0; k < ROWS_PRE; ++k) Q<TY>::load(rw, min(li + 16 * k, G - 1), w[k]);  // (clamped: valid address)
    };
    // x and the codebook into the LDS; a routed call leaves wave 0 out, so that its router logits, the first thing
    // it loads, wait behind nothing.  The x rows are requested before the weight words, whose arrival the LDS stores
    // then do not wait for.
    const int s0 = routed ? 64 : 0;
    const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t) (p / xdiv) * cols);
    const auto xsrc = [&](int i) { return xp[i]; };
    const auto xdst = [&](int i, float4 v) { xs[(i >> 3) * 9 + (i & 7)] = v; };
    LdsStage<4> xst;
    if (tid >= s0) xst.load(G * 8, 0, tid - s0, 256 - s0, xsrc);
    if (!routed) load_pre(sel ? sel[p] : 0);
    if (tid >= s0) {
        xst.store(G * 8, 0, tid - s0, 256 - s0, xdst);
        stage_rest<4>(G * 8, tid - s0, 256 - s0, xsrc, xdst);
        tab_fill<TY>(tid - s0, 256 - s0);
    }
    if (routed) {
        const int t = p / rt.NEU, k = p - t * rt.NEU;
        const bool writer = k == 0 && blockIdx.x == 0;
        if (tid < 64) {
            const int e = route_pick(rt.rsg + (size_t) t * (rt.NE + 1), rt.NE, writer ? rt.NEU : k + 1, k,
                                     writer ? rt.sel + t * rt.NEU : nullptr, writer ? rt.wsel + t * rt.NEU : nullptr);
            if (tid == 0) e_sh = e;
        } else if (writer) {
            for (int i = tid - 64; i < rt.FFS; i += 192) {
                const float g = rt.shg[(size_t) t * rt.FFS + i];
                rt.sha[(size_t) t * rt.FFS + i] = g / (1.0f + expf(-g)) * rt.shu[(size_t) t * rt.FFS + i];
            }
        }
    }
    __syncthreads();
    if (routed) load_pre(e_sh);
    const TabT<TY> T;
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < ROWS_PRE; ++k) {
        const int g = li + 16 * k;
        if (g < G) accumulate<TY, 1>(w[k], g, xs + 9 * g, &a, T);
    }
    for (int g = li + 16 * ROWS_PRE; g < G; g += 16) {  // rows longer than 80 groups
        uint32_t wn[NW];
        Q<TY>::load(rw, g, wn);
        accumulate<TY, 1>(wn, g, xs + 9 * g, &a, T);
    }
    a = row_sum(a);
    if constexpr (SWIGLU) {
        const float u = swz_xor16(a);  // the up row's sum, at the gate row's lanes
        if (!up && li == 0 && r < R) out[(size_t) p * R + r] = a / (1.0f + expf(-a)) * u;
    } else {
        if (li == 0 && r < R) out[(size_t) p * R + r] = a;
    }
}



template <uint32_t TY>
int embed_t(const QLayout &L, const PP &P, const int32_t *ids, int nt, int copies, float *out, hipStream_t st) {
    hipLaunchKernelGGL(k_embed<TY>, dim3((unsigned) nt), dim3(256), 0, st, P, L.cols / 32, L.cols, ids, copies, out);
    FN_CK(hipGetLastError());
    return 0;
}

template <uint32_t TY>
int ngram_t(const QLayout &L, const PP &P, const NgramGather &g, int nt, float *out, hipStream_t st) {
    hipLaunchKernelGGL(k_ngram_rows<TY>, dim3((unsigned) nt), dim3(256), 0, st, P, L.cols / 32, L.cols, g, out);
    FN_CK(hipGetLastError());
    return 0;
}

template <uint32_t TY, bool SW>
int rows_t(const QLayout &L, const PP &Pg, const PP &Pu, int R, const int32_t *sel, int npairs, int xdiv,
           const float *x, float *out, hipStream_t st, const RouteIn &rt) {
    const size_t lds = (size_t) (L.cols / 32) * 9 * sizeof(float4);
    if (lds + tab_lds<TY>() > (size_t) kLdsPerCu) FN_FAIL("rows: x row too long for the LDS");
    constexpr int RW = rows_per_wg<SW>();
    hipLaunchKernelGGL((k_rows<TY, SW>), dim3((unsigned) ((R + RW - 1) / RW), (unsigned) npairs), dim3(256), lds, st, Pg,
                       Pu, R, L.rows / R, L.cols / 32, L.cols, sel, xdiv, x, out, rt);
    FN_CK(hipGetLastError());
    return 0;
}


// the instantiations a unit provides for one format
struct QOps {
    int (*gemv)(const QLayout &, const GemvPlan &, const PP &, const float *, int, float *, hipStream_t);
    int (*dequant)(const QLayout &, const PP &, float *, hipStream_t);
    int (*embed)(const QLayout &, const PP &, const int32_t *, int, int, float *, hipStream_t);
    int (*ngram)(const QLayout &, const PP &, const NgramGather &, int, float *, hipStream_t);
    int (*rows)(const QLayout &, const PP &, const PP &, int, const int32_t *, int, int, const float *, float *,
                hipStream_t, const RouteIn &);
    int (*swiglu)(const QLayout &, const PP &, const PP &, int, const int32_t *, int, int, const float *, float *,
                  hipStream_t, const RouteIn &);
};

template <uint32_t TY> int dequant_t(const QLayout &L, const PP &P, float *out, hipStream_t st) {
    const int G = L.cols / 32;
    const size_t n = (size_t) L.rows * G;
    hipLaunchKernelGGL(k_dequant<TY>, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, P, L.rows, G, L.cols, out);
    FN_CK(hipGetLastError());
    return 0;
}

template <uint32_t TY> const QOps *qops_of() {
    static const QOps o{&gemv_t<TY>, &dequant_t<TY>, &embed_t<TY>, &ngram_t<TY>, &rows_t<TY, false>,
                        &rows_t<TY, true>};
    return &o;
}

}  // namespace

// per-unit lookups: the operations of a format instantiated in that unit, or null
const void *qops_group1(uint32_t type);
const void *qops_group2(uint32_t type);
const void *qops_group3(uint32_t type);
const void *qops_group4(uint32_t type);
const void *qops_group5(uint32_t type);

}  // namespace fn

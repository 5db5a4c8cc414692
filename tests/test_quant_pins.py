"""Pins of the GGUF weight decode in the oracle (CPU only).

The reference gates its GPU decode bit for bit against gguf-py (flashnext/test_fn_quants.py:30-37) on slices of the
real model; neither gguf-py, ggml nor the model is in this image, and the reference ships no fixture of decoded
weights.  The oracle's decode (oracle/quant_oracle.c) is therefore pinned by:

* the independent numpy twin (oracle/twin.py, gguf-py's vectorised structure) on random bytes of every format;
* blocks *packed* from chosen integer codes, scales and mins by the packers below, written from the field
  descriptions of each format in the opposite direction (codes -> bytes), and decoded back to the exact value
  s * q - m rounded once to float32 -- a transposed nibble, a wrong bit position, a swapped scale/min or a wrong
  group order in either direction fails it;
* library conversions: numpy's float16 -> float32 over all 65536 fp16 bit patterns, torch's bfloat16 -> float32;
* special blocks: all-zero, unit scales.
"""

import numpy as np
import pytest

import oracle
import oracle.twin as twin

RNG = np.random.default_rng(7)
TYPES = dict(Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14, IQ4_NL=20, IQ3_S=21, IQ4_XS=23, BF16=30, IQ2_XXS=16, IQ2_XS=17,
             IQ2_S=22, IQ3_XXS=18, Q2_0=42)
LEVELS = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def f16_bits(x):
    return int(np.float16(x).view(np.uint16))


def rand_f16_scale(rng, lo=-6, hi=2):
    """A random normal fp16 value (sign, exponent in [lo, hi), random fraction) as (bits, exact float)."""
    e = int(rng.integers(lo, hi))
    v = (1.0 + int(rng.integers(0, 1024)) / 1024.0) * 2.0 ** e * (1 if rng.random() < 0.5 else -1)
    return f16_bits(v), v


def random_finite(qtype, rows, cols, rng):
    """Random GGUF bytes of a format with every fp16 / bf16 field finite (exponent MSB cleared)."""
    qk, bb = oracle.qblock(qtype)
    raw = rng.integers(0, 256, size=rows * (cols // qk) * bb, dtype=np.uint8)
    blk = raw.reshape(-1, bb)
    hi_bytes = {30: [1], 8: [1], 20: [1], 21: [1], 23: [1], 12: [1, 3], 13: [1, 3], 14: [209], 16: [1], 17: [1], 22: [1],
                18: [1], 42: [1]}[qtype]
    for b in hi_bytes:
        blk[:, b] &= 0xBF
    return raw


# ---------------------------------------------------------------------------------------------------------
# packers: codes -> GGUF bytes, one block at a time


def pack_q8_0(d_bits, q):
    return np.concatenate([np.array([d_bits & 255, d_bits >> 8], np.uint8), np.asarray(q, np.int8).view(np.uint8)])


def pack_iq4_nl(d_bits, idx):
    idx = np.asarray(idx)
    qs = (idx[:16] | (idx[16:] << 4)).astype(np.uint8)
    return np.concatenate([np.array([d_bits & 255, d_bits >> 8], np.uint8), qs])


def pack_iq4_xs(d_bits, ls, idx):
    """ls [8] 6-bit group scales, idx [256] level indices."""
    sh, sl = 0, np.zeros(4, np.uint8)
    qs = np.zeros(128, np.uint8)
    for g in range(8):
        sl[g // 2] |= (ls[g] & 15) << (4 * (g % 2))
        sh |= (ls[g] >> 4) << (2 * g)
        gi = np.asarray(idx[32 * g:32 * g + 32])
        qs[16 * g:16 * g + 16] = gi[:16] | (gi[16:] << 4)
    head = np.array([d_bits & 255, d_bits >> 8, sh & 255, sh >> 8], np.uint8)
    return np.concatenate([head, sl, qs])


def pack_k_scales(sc, mn):
    """8 six-bit scales and mins -> the 12 bytes of a Q4_K / Q5_K super-block."""
    out = np.zeros(12, np.uint8)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return out


def pack_q4_k(d_bits, dm_bits, sc, mn, q):
    """q [256] 4-bit codes; group g = values 32 g .. 32 g + 31."""
    qs = np.zeros(128, np.uint8)
    for g in range(8):
        qs[32 * (g // 2):32 * (g // 2) + 32] |= (np.asarray(q[32 * g:32 * g + 32]) << (4 * (g % 2))).astype(np.uint8)
    head = np.array([d_bits & 255, d_bits >> 8, dm_bits & 255, dm_bits >> 8], np.uint8)
    return np.concatenate([head, pack_k_scales(sc, mn), qs])


def pack_q5_k(d_bits, dm_bits, sc, mn, q):
    """q [256] 5-bit codes."""
    q = np.asarray(q)
    qh = np.zeros(32, np.uint8)
    for g in range(8):
        qh |= ((q[32 * g:32 * g + 32] >> 4) << g).astype(np.uint8)
    b4 = pack_q4_k(d_bits, dm_bits, sc, mn, q & 15)
    return np.concatenate([b4[:16], qh, b4[16:]])


def pack_q6_k(d_bits, sc, c):
    """c [256] 6-bit codes (value = d * sc * (c - 32)), sc [16] int8."""
    ql, qh = np.zeros(128, np.uint8), np.zeros(64, np.uint8)
    for v in range(256):
        n, k, l = v // 128, (v % 128) // 32, v % 32
        ql[64 * n + 32 * (k & 1) + l] |= (c[v] & 15) << (4 * (k >> 1))
        qh[32 * n + l] |= (c[v] >> 4) << (2 * k)
    return np.concatenate([ql, qh, np.asarray(sc, np.int8).view(np.uint8),
                           np.array([d_bits & 255, d_bits >> 8], np.uint8)])


def pack_iq3_s(d_bits, sc, idx, neg):
    """sc [8] 4-bit group scales, idx [64] 9-bit codebook indices (grid point p = values 4p .. 4p + 3), neg [256] sign
    bits: the 110 bytes d | qs[64] | qh[8] | signs[32] | scales[4].  Point p of group ib = p // 8 is point
    k = p % 8 of the group: its low 8 index bits go to qs[p], the ninth to bit k of qh[ib]."""
    idx, neg = np.asarray(idx), np.asarray(neg)
    qs = (idx & 255).astype(np.uint8)
    qh = np.zeros(8, np.uint8)
    for p in range(64):
        qh[p // 8] |= (idx[p] >> 8) << (p % 8)
    signs = np.zeros(32, np.uint8)
    for v in range(256):
        signs[v // 8] |= neg[v] << (v % 8)
    scales = np.array([(sc[2 * i] & 15) | ((sc[2 * i + 1] & 15) << 4) for i in range(4)], np.uint8)
    return np.concatenate([np.array([d_bits & 255, d_bits >> 8], np.uint8), qs, qh, signs, scales])


def f32_once(x):
    """A float64 value that is exact, rounded once to float32."""
    return np.float32(x)


# ---------------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows,cols", [(3, 256), (7, 768), (1, 2560)])
def test_oracle_matches_numpy_twin(name, rows, cols):
    t = TYPES[name]
    raw = random_finite(t, rows, cols, RNG)
    a, b = oracle.dequant(t, raw, rows, cols), twin.dequant(t, raw, rows, cols)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_f16_decode_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    raw = random_finite(30, 4, 512, RNG)
    ref = torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16).float().numpy().reshape(4, 512)
    assert np.array_equal(oracle.dequant(30, raw, 4, 512).view(np.uint32), ref.view(np.uint32))


def test_q8_0_packed_codes():
    blocks, want = [], []
    for _ in range(8):
        db, d = rand_f16_scale(RNG)
        q = RNG.integers(-128, 128, size=32)
        blocks.append(pack_q8_0(db, q))
        want += [f32_once(d * v) for v in q]
    got = oracle.dequant(8, np.concatenate(blocks), 1, 256)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq4_nl_packed_codes():
    blocks, want = [], []
    for _ in range(8):
        db, d = rand_f16_scale(RNG)
        idx = RNG.integers(0, 16, size=32)
        blocks.append(pack_iq4_nl(db, idx))
        want += [f32_once(d * LEVELS[i]) for i in idx]
    got = oracle.dequant(20, np.concatenate(blocks), 1, 256)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq4_xs_packed_codes():
    blocks, want = [], []
    for _ in range(3):
        db, d = rand_f16_scale(RNG)
        ls = RNG.integers(0, 64, size=8)
        idx = RNG.integers(0, 16, size=256)
        blocks.append(pack_iq4_xs(db, ls, idx))
        for v in range(256):
            dl = np.float32(d * (int(ls[v // 32]) - 32))    # exact: 11 x 6 significant bits
            want.append(f32_once(float(dl) * LEVELS[idx[v]]))
    got = oracle.dequant(23, np.concatenate(blocks), 1, 768)[0]
    assert np.array_equal(got, np.array(want, np.float32))


@pytest.mark.parametrize("qtype", [12, 13])
def test_k_quants_packed_codes(qtype):
    blocks, want = [], []
    for _ in range(3):
        db, d = rand_f16_scale(RNG)
        mb, dm = rand_f16_scale(RNG)
        sc, mn = RNG.integers(0, 64, size=8), RNG.integers(0, 64, size=8)
        q = RNG.integers(0, 16 if qtype == 12 else 32, size=256)
        blocks.append((pack_q4_k if qtype == 12 else pack_q5_k)(db, mb, sc, mn, q))
        for v in range(256):
            g = v // 32
            want.append(f32_once(d * int(sc[g]) * int(q[v]) - dm * int(mn[g])))   # exact in float64, one rounding
    got = oracle.dequant(qtype, np.concatenate(blocks), 1, 768)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_q6_k_packed_codes():
    blocks, want = [], []
    for _ in range(3):
        db, d = rand_f16_scale(RNG)
        sc = RNG.integers(-128, 128, size=16)
        c = RNG.integers(0, 64, size=256)
        blocks.append(pack_q6_k(db, sc, c))
        for v in range(256):
            n, k, l = v // 128, (v % 128) // 32, v % 32
            ds = np.float32(d * int(sc[8 * n + 2 * k + l // 16]))  # exact: 11 x 8 significant bits
            want.append(f32_once(float(ds) * (int(c[v]) - 32)))
    got = oracle.dequant(14, np.concatenate(blocks), 1, 768)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq3_s_packed_codes():
    """IQ3_S blocks packed from chosen codebook indices (all 9 bits used), sign bits and scales decode to
    d * (1 + 2 sc) * magnitude * sign, each magnitude the byte j of its grid point (low byte first); the product
    d * (1 + 2 sc) is exact (11 x 5 significant bits), so each value is one rounding of an exact float64 product."""
    grid = twin.iq3s_grid()
    blocks, want = [], []
    for _ in range(3):
        db, d = rand_f16_scale(RNG)
        sc = RNG.integers(0, 16, size=8)
        idx = RNG.integers(0, 512, size=64)
        idx[:2] = [255, 256]            # both sides of the ninth bit
        neg = RNG.integers(0, 2, size=256)
        blocks.append(pack_iq3_s(db, sc, idx, neg))
        for v in range(256):
            mag = (int(grid[idx[v // 4]]) >> (8 * (v % 4))) & 255
            want.append(f32_once(d * (1 + 2 * int(sc[v // 32])) * mag * (-1 if neg[v] else 1)))
    got = oracle.dequant(21, np.concatenate(blocks), 1, 768)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq3_s_codebook():
    """The IQ3_S codebook data: 512 distinct points in ascending order, every magnitude an odd value 1..15 (3 bits
    of a 4-value lattice point); grid point 0 is (1, 1, 1, 1).  Where the reference tree is present (this container,
    not the GPU box), the values equal the ggml codebook the reference carries (engine/fn_tables.cuh:513, copied
    from ggml-common.h), read as text."""
    import os
    import re

    g = twin.iq3s_grid()
    assert g.shape == (512,) and np.all(np.diff(g.astype(np.int64)) > 0) and g[0] == 0x01010101
    mags = (g[:, None] >> (8 * np.arange(4, dtype=np.uint32))) & 255
    assert set(np.unique(mags).tolist()) <= set(range(1, 16, 2))
    ref = "/root/reference/engine/fn_tables.cuh"
    if not os.path.exists(ref):
        pytest.skip("reference tree not present (GPU box)")
    text = open(ref).read()
    i = text.index("iq3s_grid[512]")
    body = text[text.index("{", i) + 1:text.index("}", i)]
    want = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)], np.uint32)
    assert np.array_equal(g, want)


def ksign_bits(i):
    """sign bits of a 7-bit sign index: the index and, as bit 7, its parity (GGUF ksigns_iq2xs)"""
    b = i | ((bin(i).count("1") & 1) << 7)
    return [(b >> j) & 1 for j in range(8)]


def mags(name, per, e):
    w = twin.grid_words(name)
    words = per // 4
    return [(int(w[words * e + j // 4]) >> (8 * (j % 4))) & 255 for j in range(per)]


def test_iq2_xxs_packed_codes():
    """IQ2_XXS from chosen codes: per group 4 grid indices (bytes), 4 seven-bit sign indices and a 4-bit scale in one
    word; value = d (0.5 + s) / 4 x grid magnitude x sign (all products exact)."""
    blocks, want = [], []
    for _ in range(2):
        db_, d = rand_f16_scale(RNG)
        out = [db_ & 255, db_ >> 8]
        for ib in range(8):
            idx = RNG.integers(0, 256, size=4)
            sidx = RNG.integers(0, 128, size=4)
            sc = int(RNG.integers(0, 16))
            w = int(sidx[0]) | int(sidx[1]) << 7 | int(sidx[2]) << 14 | int(sidx[3]) << 21 | sc << 28
            out += [int(v) for v in idx] + [(w >> (8 * k)) & 255 for k in range(4)]
            dl = d * (0.5 + sc) * 0.25
            for l in range(4):
                m, sg = mags("iq2xxs_grid", 8, int(idx[l])), ksign_bits(int(sidx[l]))
                want += [f32_once(dl * m[j] * (-1 if sg[j] else 1)) for j in range(8)]
        blocks.append(np.array(out, np.uint8))
    got = oracle.dequant(16, np.concatenate(blocks), 1, 512)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq2_xs_packed_codes():
    """IQ2_XS: 16-bit codes of a 9-bit grid index and a 7-bit sign index, two 4-bit scales per group (first and
    second half)."""
    blocks, want = [], []
    for _ in range(2):
        db_, d = rand_f16_scale(RNG)
        qs, sc = [], []
        vals = []
        for ib in range(8):
            s0, s1 = int(RNG.integers(0, 16)), int(RNG.integers(0, 16))
            sc.append(s0 | s1 << 4)
            for l in range(4):
                e, si = int(RNG.integers(0, 512)), int(RNG.integers(0, 128))
                qs.append(e | si << 9)
                dl = d * (0.5 + (s0 if l < 2 else s1)) * 0.25
                m, sg = mags("iq2xs_grid", 8, e), ksign_bits(si)
                vals += [f32_once(dl * m[j] * (-1 if sg[j] else 1)) for j in range(8)]
        blocks.append(np.concatenate([np.array([db_ & 255, db_ >> 8], np.uint8),
                                      np.array(qs, np.uint16).view(np.uint8), np.array(sc, np.uint8)]))
        want += vals
    got = oracle.dequant(17, np.concatenate(blocks), 1, 512)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq2_s_packed_codes():
    """IQ2_S: a 10-bit grid index (byte of qs, two bits of qh[ib] at 2l), a full sign byte per 8 values, two 4-bit
    scales per group."""
    db_, d = rand_f16_scale(RNG)
    qs, signs, qh, sc, want = [], [], [], [], []
    for ib in range(8):
        s0, s1 = int(RNG.integers(0, 16)), int(RNG.integers(0, 16))
        sc.append(s0 | s1 << 4)
        h = 0
        for l in range(4):
            e, sb = int(RNG.integers(0, 1024)), int(RNG.integers(0, 256))
            qs.append(e & 255)
            h |= (e >> 8) << (2 * l)
            signs.append(sb)
            dl = d * (0.5 + (s0 if l < 2 else s1)) * 0.25
            m = mags("iq2s_grid", 8, e)
            want += [f32_once(dl * m[j] * (-1 if (sb >> j) & 1 else 1)) for j in range(8)]
        qh.append(h)
    blk = np.array([db_ & 255, db_ >> 8] + qs + signs + qh + sc, np.uint8)
    got = oracle.dequant(22, blk, 1, 256)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_iq3_xxs_packed_codes():
    """IQ3_XXS: per group 8 grid bytes (pairs of 4-magnitude points) and a word of 4 sign indices + a 4-bit scale;
    value = d (0.5 + s) / 2 x magnitude x sign."""
    db_, d = rand_f16_scale(RNG)
    qs, ss, want = [], [], []
    for ib in range(8):
        idx = [int(v) for v in RNG.integers(0, 256, size=8)]
        sidx = [int(v) for v in RNG.integers(0, 128, size=4)]
        s = int(RNG.integers(0, 16))
        qs += idx
        w = sidx[0] | sidx[1] << 7 | sidx[2] << 14 | sidx[3] << 21 | s << 28
        ss += [(w >> (8 * k)) & 255 for k in range(4)]
        dl = d * (0.5 + s) * 0.5
        for l in range(4):
            m = mags("iq3xxs_grid", 4, idx[2 * l]) + mags("iq3xxs_grid", 4, idx[2 * l + 1])
            sg = ksign_bits(sidx[l])
            want += [f32_once(dl * m[j] * (-1 if sg[j] else 1)) for j in range(8)]
    blk = np.array([db_ & 255, db_ >> 8] + qs + ss, np.uint8)
    got = oracle.dequant(18, blk, 1, 256)[0]
    assert np.array_equal(got, np.array(want, np.float32))


def test_q2_0_packed_codes():
    """Q2_0 (the reference fork's type 42, faie2fn.cu:470-485): value v of a 64-value block is d (q - 1) with q the
    2-bit code at bits 2 (v % 4) of byte v / 4."""
    blocks, want = [], []
    for _ in range(4):
        db_, d = rand_f16_scale(RNG)
        q = RNG.integers(0, 4, size=64)
        by = [int(q[4 * k] | q[4 * k + 1] << 2 | q[4 * k + 2] << 4 | q[4 * k + 3] << 6) for k in range(16)]
        blocks.append(np.array([db_ & 255, db_ >> 8] + by, np.uint8))
        want += [f32_once(d * (int(v) - 1)) for v in q]
    got = oracle.dequant(42, np.concatenate(blocks), 1, 256)[0]
    assert np.array_equal(got, np.array(want, np.float32))


@pytest.mark.parametrize("name,entries,per,levels", [("iq2xxs_grid", 256, 8, {8, 25, 43}),
                                                     ("iq2xs_grid", 512, 8, {8, 25, 43}),
                                                     ("iq2s_grid", 1024, 8, {8, 25, 43}),
                                                     ("iq3xxs_grid", 256, 4, {4, 12, 20, 28, 36, 44, 52, 62})])
def test_iq2_iq3xxs_codebooks(name, entries, per, levels):
    """The codebook data files: entry count, distinct entries in ascending order, magnitudes from the format's level
    set; where the reference tree is present, equal to the copy it carries (engine/fn_tables.cuh:21, 88, 219, 478)."""
    import os
    import re

    w = twin.grid_words(name).astype(np.uint64)
    vals = w if per == 4 else w[0::2] | (w[1::2] << np.uint64(32))
    assert len(vals) == entries and np.all(vals[1:] > vals[:-1])
    m = twin.grid_mags(name, per)
    assert set(np.unique(m).astype(int).tolist()) <= levels
    ref = "/root/reference/engine/fn_tables.cuh"
    if not os.path.exists(ref):
        pytest.skip("reference tree not present (GPU box)")
    text = open(ref).read()
    i = text.index(name + "[")
    body = text[text.index("{", i) + 1:text.index("}", i)]
    want = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)], np.uint64)
    assert np.array_equal(vals, want)


@pytest.mark.parametrize("name", list(TYPES))
def test_zero_block_decodes_to_zero(name):
    """All-zero bytes: every scale is +0, so every value is zero whatever the code's offset (IQ4 level -127, Q6_K
    code - 32, Q4_K/Q5_K min)."""
    t = TYPES[name]
    qk, bb = oracle.qblock(t)
    cols = max(qk, 256)
    assert np.all(oracle.dequant(t, np.zeros(cols // qk * bb, np.uint8), 1, cols) == 0)


def test_unit_scales_expose_codes():
    one = f16_bits(1.0)
    # Q8_0 with d = 1 returns the int8 codes themselves
    q = np.arange(-16, 16)
    assert np.array_equal(oracle.dequant(8, pack_q8_0(one, q), 1, 32)[0], q.astype(np.float32))
    # Q6_K with d = 1 and scales 1 returns code - 32 in value order
    c = RNG.integers(0, 64, size=256)
    got = oracle.dequant(14, pack_q6_k(one, np.ones(16, np.int64), c), 1, 256)[0]
    assert np.array_equal(got, (c - 32).astype(np.float32))
    # Q4_K with d = 1, scale 1, min 0 returns the 4-bit codes
    q4 = RNG.integers(0, 16, size=256)
    got = oracle.dequant(12, pack_q4_k(one, one, np.ones(8, np.int64), np.zeros(8, np.int64), q4), 1, 256)[0]
    assert np.array_equal(got, q4.astype(np.float32))


def test_gemv_oracle_is_float64_dot_of_decoded_rows():
    raw = random_finite(23, 9, 512, RNG)
    x = RNG.standard_normal((3, 512)).astype(np.float32)
    W = oracle.dequant(23, raw, 9, 512).astype(np.float64)
    ref = x.astype(np.float64) @ W.T
    assert np.allclose(oracle.gemv(23, raw, 9, 512, x), ref, rtol=1e-13, atol=1e-10)

"""GPU parity of the GGUF decode and the projection GEMV against the oracle.

The reference's quant gate (flashnext/test_fn_quants.py:30-37): the GPU decode equals the CPU decode exactly
(error 0), and the GEMV of 8 tokens is within 1e-5 (max|gpu - ref| / max|ref|) of float64 math on the decoded
weights.  Shapes are those of the projections on the path: the stacked DeltaNet input (qkv), its output (ssm_out),
the attention q / k / v / o projections and the alpha/beta rows, at the reference model's hidden size 2560 and at
the benchmark configs' 2048, plus ragged row counts.  Weights are random bytes with finite fp16 / bf16 scales (the reference's
real tensors are not in this image).

Every case prints what names it before the GPU call.
"""

import numpy as np
import pytest

import fn
import hiprt
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
TYPES = dict(Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14, IQ4_NL=20, IQ3_S=21, IQ4_XS=23, BF16=30, IQ2_XXS=16, IQ2_XS=17,
             IQ2_S=22, IQ3_XXS=18, Q2_0=42)
RNG = np.random.default_rng(31)


def _say(*a):
    print(*a, flush=True)


def random_finite(qtype, rows, cols, rng):
    qk, bb = oracle.qblock(qtype)
    raw = rng.integers(0, 256, size=rows * (cols // qk) * bb, dtype=np.uint8)
    blk = raw.reshape(-1, bb)
    for b in {30: [1], 8: [1], 20: [1], 21: [1], 23: [1], 12: [1, 3], 13: [1, 3], 14: [209], 16: [1], 17: [1], 22: [1],
              18: [1], 42: [1]}[qtype]:
        blk[:, b] &= 0xBF
    return raw


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows,cols", [(1, 256), (37, 768), (64, 2560)])
def test_dequant_bit_exact(fnlib, name, rows, cols):
    t = TYPES[name]
    _say(f"dequant {name} {rows}x{cols}")
    raw = random_finite(t, rows, cols, RNG)
    got = fnlib.dequant(t, raw, rows, cols)
    ref = oracle.dequant(t, raw, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# (type, rows, cols): the path's projections in the reference model (engine/faie2fn.cu:2386-2403;
# flashnext/inspect_fn.txt:77, 95-100, 132-137) and at the benchmark configs' hidden 2048
PATH_SHAPES = [
    ("IQ4_XS", 10240, 2560),   # attn_qkv (DeltaNet in)
    ("Q8_0", 2560, 6144),      # ssm_out / attn_output
    ("BF16", 96, 2560),        # ssm_alpha + ssm_beta rows
    ("Q6_K", 512, 2560),       # attn_v
    ("IQ4_XS", 512, 2560),     # attn_k
    ("Q6_K", 6144, 2560),      # attn_gate (z) of layer 1
    ("IQ3_S", 6144, 2560),     # attn_gate (z) of layer 0 (inspect_fn.txt:76)
    ("IQ2_XS", 640, 2560),     # one routed expert's gate / up rows (blk.0.ffn_gate_exps, inspect_fn.txt:80)
    ("IQ2_XXS", 640, 2560),    # blk.1.ffn_gate_exps
    ("IQ2_S", 640, 2560),
    ("IQ3_XXS", 640, 2560),
    ("Q2_0", 2560, 640),       # one routed expert's down rows (blk.1.ffn_down_exps)
    ("IQ4_XS", 8192, 2048),    # config 1/2 qkv: 8192 mixed channels from hidden 2048
    ("Q8_0", 2048, 4096),      # config 1/2 ssm_out
]


@pytest.mark.parametrize("name,rows,cols", PATH_SHAPES)
@pytest.mark.parametrize("nt", [1, 8])
def test_gemv_path_shapes(fnlib, name, rows, cols, nt):
    t = TYPES[name]
    _say(f"gemv {name} {rows}x{cols} nt={nt} plan={fnlib.gemv_plan(t, rows, cols)}")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    y = fnlib.gemv(t, raw, rows, cols, x)
    ref = oracle.gemv(t, raw, rows, cols, x)
    assert oracle.relerr(y, ref) <= TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows,nt", [(1, 1), (17, 3), (100, 5), (333, 8)])
def test_gemv_formats_ragged(fnlib, name, rows, nt):
    t = TYPES[name]
    cols = 768
    _say(f"gemv {name} {rows}x{cols} nt={nt}")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    y = fnlib.gemv(t, raw, rows, cols, x)
    ref = oracle.gemv(t, raw, rows, cols, x)
    assert oracle.relerr(y, ref) <= TOL
    # every row on its own is right too (no row of a partial tile is dropped or shifted)
    assert np.all(np.abs(y - ref) <= TOL * np.abs(ref).max())


@pytest.mark.parametrize("ks", [1, 2, 5, 80])
def test_gemv_split_k_invariance(fnlib, ks):
    t, rows, cols, nt = 23, 256, 2560, 4
    _say(f"gemv split-K ks={ks}")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    ref = oracle.gemv(t, raw, rows, cols, x)
    fnlib.gemv_override(ks)
    try:
        assert fnlib.gemv_plan(t, rows, cols)[2] == ks
        y = fnlib.gemv(t, raw, rows, cols, x)
    finally:
        fnlib.gemv_override(0)
    assert oracle.relerr(y, ref) <= TOL


# (type, rows, cols, nt): several batches per row-set (Q6_K / BF16 keep one group per lane in flight), ragged rows,
# row-sets beyond one per wave (rows large for the grid, and a grid sized for 8 waves per CU), x at the LDS limit,
# a short weight
STAGING_CASES = [
    ("IQ4_XS", 10240, 2560, 1),
    ("Q6_K", 6144, 2560, 3),
    ("Q8_0", 2560, 6144, 2),
    ("BF16", 333, 768, 8),
    ("Q5_K", 1000, 4096, 4),
    ("Q4_K", 40961, 512, 1),
    ("IQ4_NL", 3001, 2944, 8),
    ("Q8_0", 700, 4608, 8),     # 148 KB of x in LDS
    ("IQ4_XS", 130, 2560, 5),   # a short weight
    ("IQ3_S", 1000, 6144, 8),   # the codebook in LDS beside a chunked x
    ("IQ3_S", 2000, 2560, 2),
]


@pytest.mark.parametrize("name,rows,cols,nt", STAGING_CASES)
@pytest.mark.parametrize("wpc", [0, 8])
def test_gemv_chunked_x_matches_one_stage(fnlib, name, rows, cols, nt, wpc):
    """x staged in chunks of lpr groups (k_gemv_c, the path of an x too large for the LDS) and x staged once (k_gemv:
    persistent waves walking row-sets, grid sized for wpc waves per CU, with the deep and with the short walk) give
    the same bits: a row's groups are summed by the same lanes in the same order."""
    t = TYPES[name]
    _say(f"gemv chunked vs one-stage x {name} {rows}x{cols} nt={nt} waves/CU={wpc or 'auto'} "
         f"plan={fnlib.gemv_plan(t, rows, cols)}")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    try:
        fnlib.gemv_override(kernel=1)
        y1 = fnlib.gemv(t, raw, rows, cols, x)
        fnlib.gemv_override(kernel=3, waves_per_cu=wpc)
        y3 = fnlib.gemv(t, raw, rows, cols, x)
        fnlib.gemv_override(kernel=4, waves_per_cu=wpc)
        y4 = fnlib.gemv(t, raw, rows, cols, x)
    finally:
        fnlib.gemv_override(0)
    assert np.array_equal(y1, y3) and np.array_equal(y1, y4)
    assert oracle.relerr(y3, oracle.gemv(t, raw, rows, cols, x)) <= TOL


@pytest.mark.parametrize("name,rows,cols,nt", STAGING_CASES[:4])
def test_gemv_waves_switch_same_bits(fnlib, name, rows, cols, nt):
    """fn_gemv_waves(0) (one workgroup per row tile, the reference's non-persistent grid) and the default persistent
    grid give the same bits."""
    t = TYPES[name]
    _say(f"gemv waves switch {name} {rows}x{cols} nt={nt}")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    y1 = fnlib.gemv(t, raw, rows, cols, x)
    try:
        fnlib.d.fn_gemv_waves(0)
        assert fnlib.gemv_plan(t, rows, cols)[5] > 0
        y0 = fnlib.gemv(t, raw, rows, cols, x)
    finally:
        fnlib.d.fn_gemv_waves(1)
    assert np.array_equal(y0, y1)


@pytest.mark.parametrize("seed", range(16))
def test_gemv_random_shapes(fnlib, seed):
    """Seeded random format, rows (1 to 5000, ragged), columns (a multiple of the format's block, up to 8192: x
    larger than the LDS at high nt goes through the chunked kernel) and nt (1 to 8), against the oracle."""
    rng = np.random.default_rng(9100 + seed)
    name = str(rng.choice(list(TYPES)))
    t = TYPES[name]
    qk = oracle.qblock(t)[0]
    blk = max(qk, 32)
    rows = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 5001))]))
    cols = blk * int(rng.integers(1, 8192 // blk + 1))
    nt = int(rng.integers(1, 9))
    _say(f"gemv random seed={seed}: {name} {rows}x{cols} nt={nt} plan={fnlib.gemv_plan(t, rows, cols)}")
    raw = random_finite(t, rows, cols, rng)
    x = rng.standard_normal((nt, cols)).astype(np.float32)
    y = fnlib.gemv(t, raw, rows, cols, x)
    assert oracle.relerr(y, oracle.gemv(t, raw, rows, cols, x)) <= TOL


def test_gemv_tokens_independent(fnlib):
    """Token t of an nt-token call equals a one-token call on x[t] (the split order does not depend on nt)."""
    t, rows, cols = 8, 700, 2048
    _say("gemv nt=6 vs 6 x nt=1")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((6, cols)).astype(np.float32)
    y = fnlib.gemv(t, raw, rows, cols, x)
    for i in range(6):
        assert np.array_equal(y[i], fnlib.gemv(t, raw, rows, cols, x[i:i + 1])[0])


def test_device_entry_points(fnlib):
    """pack once, then dequant and GEMV on device buffers: the same values as the host hooks."""
    t, rows, cols, nt = 14, 300, 2560, 3
    _say("gemv device entry points Q6_K 300x2560 nt=3")
    raw = random_finite(t, rows, cols, RNG)
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    draw = hiprt.Buf.like(raw)
    packed = hiprt.Buf(fnlib.gemv_packed_bytes(t, rows, cols), np.uint8)
    wb = fnlib.gemv_work_bytes(t, rows, cols, nt)
    work = hiprt.Buf(max(wb, 16), np.uint8)
    dx, dy = hiprt.Buf.like(x), hiprt.Buf.empty((nt, rows))
    dW = hiprt.Buf.empty((rows, cols))
    fnlib.gemv_pack_dev(t, draw.ptr, rows, cols, packed.ptr)
    fnlib.dequant_dev(t, packed.ptr, rows, cols, dW.ptr)
    fnlib.gemv_dev(t, packed.ptr, rows, cols, dx.ptr, nt, dy.ptr, work.ptr, wb)
    hiprt.sync()
    W = dW.download((rows, cols))
    y = dy.download((nt, rows))
    assert np.array_equal(W.view(np.uint32), oracle.dequant(t, raw, rows, cols).view(np.uint32))
    assert np.array_equal(y, fnlib.gemv(t, raw, rows, cols, x))
    # a split-K plan needs its work buffer, and a short one is refused before any launch
    fnlib.gemv_override(2)
    try:
        wb2 = fnlib.gemv_work_bytes(t, rows, cols, nt)
        assert wb2 == 2 * nt * rows * 4
        with pytest.raises(RuntimeError, match="work buffer"):
            fnlib.gemv_dev(t, packed.ptr, rows, cols, dx.ptr, nt, dy.ptr, work.ptr, wb2 - 4)
    finally:
        fnlib.gemv_override(0)


def test_bench_gemv_runs(fnlib):
    _say("bench_gemv IQ4_XS 10240x2560 nt=1, 8 iters")
    ms = fnlib.bench_gemv(23, 10240, 2560, nt=1, iters=8)
    assert 0.0 < ms < 5.0



# Grouped launches (fn_gemv_group_dev): the model's projections that read one activation row, at the reference
# model's width (DeltaNet qkv / z / alpha-beta with z in either format, attention q / k / v / indexer, the FFN's
# router / shared gate / shared up), at the benchmark configs' 2048, at a small width, and a set that is not built
# (one launch per weight).
GROUPS = [
    ("deltanet, z IQ3_S", [("IQ4_XS", 10240), ("IQ3_S", 6144), ("BF16", 96)], 2560),
    ("deltanet, z Q6_K", [("IQ4_XS", 10240), ("Q6_K", 6144), ("BF16", 96)], 2560),
    ("attention", [("IQ4_XS", 12288), ("IQ4_XS", 512), ("Q6_K", 512), ("BF16", 640)], 2560),
    ("ffn", [("BF16", 513), ("IQ4_XS", 640), ("IQ3_S", 640)], 2560),
    ("width 2048", [("BF16", 64), ("IQ4_XS", 8192), ("Q6_K", 4096)], 2048),
    ("width 256", [("IQ4_XS", 40), ("IQ3_S", 24), ("BF16", 8)], 256),
    ("not built", [("Q8_0", 300), ("BF16", 77)], 2560),
]


def _group_run(fnlib, types, rows, raws, cols, x):
    nt = x.shape[0]
    packs = []
    for t, r, raw in zip(types, rows, raws):
        draw = hiprt.Buf.like(raw)
        p = hiprt.Buf(fnlib.gemv_packed_bytes(t, r, cols), np.uint8)
        fnlib.gemv_pack_dev(t, draw.ptr, r, cols, p.ptr)
        packs.append(p)
    dx = hiprt.Buf.like(x)
    ys = [hiprt.Buf.empty((nt, r)) for r in rows]
    fnlib.gemv_group_dev(types, rows, cols, [p.ptr for p in packs], dx.ptr, nt, [y.ptr for y in ys])
    hiprt.sync()
    return [y.download() for y in ys]


@pytest.mark.parametrize("name,parts,cols", GROUPS)
@pytest.mark.parametrize("nt", [1, 3, 8])
def test_gemv_group(fnlib, name, parts, cols, nt):
    """Every weight of a group within 1e-5 of float64 math; a weight whose own plan sums a row over as many lanes as
    the group (at least 32, the fewest of the parts' plans) gets its own GEMV's bits, and so does every weight of a
    set that is not built."""
    types = [TYPES[n] for n, _ in parts]
    rows = [r for _, r in parts]
    _say(f"gemv group {name}: {parts} cols={cols} nt={nt}")
    raws = [random_finite(t, r, cols, RNG) for t, r in zip(types, rows)]
    x = RNG.standard_normal((nt, cols)).astype(np.float32)
    ys = _group_run(fnlib, types, rows, raws, cols, x)
    lprs = [16 * fnlib.gemv_plan(t, r, cols)[1] for t, r in zip(types, rows)]
    glpr = min(max(32, v) for v in lprs)
    for t, r, raw, y, lpr in zip(types, rows, raws, ys, lprs):
        assert oracle.relerr(y, oracle.gemv(t, raw, r, cols, x)) <= TOL, (t, r)
        if lpr == glpr or name == "not built":
            assert np.array_equal(y, fnlib.gemv(t, raw, r, cols, x)), (t, r)


def test_gemv_group_tokens_independent(fnlib):
    """Token t of an 8-token grouped call equals a one-token grouped call on x[t]."""
    name, parts, cols = GROUPS[2]
    types = [TYPES[n] for n, _ in parts]
    rows = [r for _, r in parts]
    _say(f"gemv group {name}: nt=8 vs 8 x nt=1")
    raws = [random_finite(t, r, cols, RNG) for t, r in zip(types, rows)]
    x = RNG.standard_normal((8, cols)).astype(np.float32)
    ys = _group_run(fnlib, types, rows, raws, cols, x)
    for i in range(8):
        one = _group_run(fnlib, types, rows, raws, cols, x[i:i + 1])
        for y, y1 in zip(ys, one):
            assert np.array_equal(y[i], y1[0])


def test_gemv_group_path_independent_of_nt(fnlib):
    """At 5120 columns the x of 8 tokens does not fit the LDS beside the codebooks while the x of one token does;
    the path (grouped or one launch per weight) is chosen for the largest call, so a one-token call takes the same
    path as an 8-token one: every weight keeps its own GEMV's bits at nt 1 and 8, and token t of the 8-token call
    equals the one-token call on x[t]."""
    types = [TYPES["IQ4_XS"], TYPES["IQ3_S"], TYPES["BF16"]]
    rows, cols = [512, 256, 64], 5120
    _say(f"gemv group at cols={cols}: nt=8 vs nt=1, own-GEMV bits")
    raws = [random_finite(t, r, cols, RNG) for t, r in zip(types, rows)]
    x = RNG.standard_normal((8, cols)).astype(np.float32)
    ys = _group_run(fnlib, types, rows, raws, cols, x)
    for i in (0, 5):
        one = _group_run(fnlib, types, rows, raws, cols, x[i:i + 1])
        for t, r, raw, y, y1 in zip(types, rows, raws, ys, one):
            assert np.array_equal(y[i], y1[0]), (t, i)
            assert np.array_equal(y1, fnlib.gemv(t, raw, r, cols, x[i:i + 1])), (t, i)


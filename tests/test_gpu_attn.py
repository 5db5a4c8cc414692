"""GPU parity of the GQA decode kernels against the float64 oracle (normwise <= 1e-5 on og and appended K/V)."""

import numpy as np
import pytest

import fn_synth
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(*a):
    print(*a, flush=True)


def _check(fnlib, case, nsplit=0, nt_extra=None):
    Kc, Vc = case.Kc.copy(), case.Vc.copy()
    og = fnlib.attn(case.qg, case.k, case.v, case.wq, case.wk, Kc, Vc, case.pos, nsplit=nsplit)
    ref_og, ref_k, ref_v = oracle.attn(case.qg, case.k, case.v, case.wq, case.wk, case.Kc, case.Vc, case.pos)
    nt = case.qg.shape[1]
    got_k = np.stack([Kc[b, case.pos[b]:case.pos[b] + nt] for b in range(case.B)])
    got_v = np.stack([Vc[b, case.pos[b]:case.pos[b] + nt] for b in range(case.B)])
    e = (oracle.relerr(og, ref_og), oracle.relerr(got_k, ref_k), oracle.relerr(got_v, ref_v))
    assert max(e) <= TOL, e
    return og


@pytest.mark.parametrize("B,L", [(1, 4096), (2, 1000), (1, 64), (1, 1)])
def test_attn_config3(fnlib, B, L):
    _say(f"attn B={B} L={L}")
    _check(fnlib, fn_synth.AttnCase(B=B, L=L))


def test_attn_split_count_invariant(fnlib):
    """The result does not depend on how the keys are split (1, 3, 7, 16, 64 with some splits empty, automatic)."""
    _say("attn nsplit invariance L=3000")
    case = fn_synth.AttnCase(B=1, L=3000)
    outs = [_check(fnlib, case, nsplit=s) for s in (1, 3, 7, 16, 64, 0)]  # 64 > 47 tiles: empty splits
    for o in outs[1:]:
        assert oracle.relerr(o, outs[0]) <= 2e-6


def test_attn_ragged_batch(fnlib):
    """Sequences at different positions in one call."""
    _say("attn ragged B=4")
    case = fn_synth.AttnCase(B=4, L=700)
    case.pos = np.array([0, 63, 64, 699], np.int32)
    _check(fnlib, case)


def test_attn_multi_token(fnlib):
    """nt = 3 new tokens: token t attends the cache plus new tokens 0..t (causal)."""
    _say("attn nt=3")
    rng = np.random.default_rng(4)
    case = fn_synth.AttnCase(B=2, L=300, max_ctx=320)
    case.qg = rng.standard_normal((2, 3, 16, 2, 256)).astype(np.float32)
    case.k = rng.standard_normal((2, 3, 2, 256)).astype(np.float32)
    case.v = rng.standard_normal((2, 3, 2, 256)).astype(np.float32)
    case.pos = np.array([299, 17], np.int32)
    _check(fnlib, case)


def _mt_case(B, nq, nkv, nt, pos, max_ctx, seed):
    """nt new tokens per sequence at positions pos[b] .. pos[b] + nt - 1, cache rows below pos[b] filled."""
    rng = np.random.default_rng(seed)
    case = fn_synth.AttnCase(B=B, L=1, nq=nq, nkv=nkv, seed=seed, max_ctx=max_ctx)
    for b in range(B):
        case.Kc[b, :pos[b]] = rng.standard_normal((pos[b], nkv, 256), dtype=np.float32)
        case.Vc[b, :pos[b]] = rng.standard_normal((pos[b], nkv, 256), dtype=np.float32)
    case.qg = rng.standard_normal((B, nt, nq, 2, 256)).astype(np.float32)
    case.k = rng.standard_normal((B, nt, nkv, 256)).astype(np.float32)
    case.v = rng.standard_normal((B, nt, nkv, 256)).astype(np.float32)
    case.pos = np.array(pos, np.int32)
    return case


# (nq, nkv, nt, positions, max_ctx): R = nt * nq / nkv query rows per kv head in 16-row blocks -- 1 block (one row
# block per wave, two K/V blocks in flight), 2 (two per wave, half-block pipeline), 3 (two row groups, the second
# half padding), 4, 6 (three waves), 8 (four row groups, one key stream), 9 (above the matrix-core kernel's 8 blocks:
# the per-token kernel); positions 0 (the first token sees only itself), tile edges, the end of the cache
MT_SHAPES = [
    (16, 2, 2, [200, 0], 256),
    (8, 2, 3, [700], 768),
    (16, 2, 4, [1000, 63, 5], 1088),
    (24, 2, 4, [777, 60], 832),
    (16, 2, 8, [1500, 120], 1536),
    (24, 2, 8, [900], 960),
    (16, 2, 16, [640], 704),
    (16, 2, 17, [500], 576),
    (16, 2, 4, [1020], 1024),
    (32, 4, 4, [333, 64], 448),
]


@pytest.mark.parametrize("nq,nkv,nt,pos,max_ctx", MT_SHAPES)
def test_attn_multi_token_shapes(fnlib, nq, nkv, nt, pos, max_ctx):
    _say(f"attn multi-token nq={nq} nkv={nkv} nt={nt} pos={pos} max_ctx={max_ctx}")
    _check(fnlib, _mt_case(len(pos), nq, nkv, nt, pos, max_ctx, seed=nt * 100 + nq + pos[0]))


def test_attn_multi_token_split_invariant(fnlib):
    """nt = 4: the result does not depend on the split count (splits of odd and even 16-key block counts, splits
    past the last token's keys, splits that only the later tokens see into)."""
    _say("attn multi-token nsplit invariance L=3000 nt=4")
    case = _mt_case(2, 16, 2, 4, [2996, 1900], 3008, seed=77)
    outs = [_check(fnlib, case, nsplit=s) for s in (1, 3, 7, 16, 47, 64, 0)]
    for o in outs[1:]:
        assert oracle.relerr(o, outs[0]) <= 2e-6


@pytest.mark.parametrize("nq,nt", [(16, 4), (16, 2), (24, 8)])
def test_attn_multi_token_growing_scores(fnlib, nq, nt):
    """Scores that grow along the context (key scale 1 -> 21) and one outlier key 40x: the running max of every row
    moves many times mid-walk, so the multi-token kernel's rescale of o and l runs (it rescales once a block's max
    exceeds the row's reference by more than 8)."""
    _say(f"attn multi-token growing scores nq={nq} nt={nt}")
    L = 2000
    case = _mt_case(2, nq, 2, nt, [L - nt, 1234], 2048, seed=91 + nq + nt)
    ramp = (1.0 + 20.0 * np.arange(2048) / L).astype(np.float32)
    case.Kc *= ramp[None, :, None, None]
    case.Kc[0, 1500] *= 40.0
    _check(fnlib, case)


@pytest.mark.parametrize("seed", range(20))
def test_attn_random_shapes(fnlib, seed):
    """Seeded random shapes across both split kernels: 1, 2 or 4 kv heads, groups of 4, 8 or 12 query heads, 1 to 10
    new tokens (up to 120 query rows per kv head), 1 to 3 sequences at independent positions (0 and the end of the
    cache included), split counts from automatic to more splits than tiles."""
    rng = np.random.default_rng(7000 + seed)
    nkv = int(rng.choice([1, 2, 4]))
    grp = int(rng.choice([4, 8, 12]))
    nt = int(rng.integers(1, 11))
    B = int(rng.integers(1, 4))
    max_ctx = 64 * int(rng.integers(1, 24))
    if max_ctx < nt:
        max_ctx = 64
    choices = [0, max_ctx - nt] + [int(v) for v in rng.integers(0, max_ctx - nt + 1, size=3)]
    pos = [int(rng.choice(choices)) for _ in range(B)]
    nsplit = int(rng.choice([0, 1, 3, 7, 32]))
    _say(f"attn random seed={seed}: nq={nkv * grp} nkv={nkv} nt={nt} pos={pos} max_ctx={max_ctx} nsplit={nsplit}")
    _check(fnlib, _mt_case(B, nkv * grp, nkv, nt, pos, max_ctx, seed=seed), nsplit=nsplit)


def test_attn_reference_group_12(fnlib):
    """The reference model's own head shape: 24 query heads over 2 kv heads (faie2fn.cu:47-48)."""
    _say("attn nq=24 nkv=2")
    _check(fnlib, fn_synth.AttnCase(B=1, L=513, nq=24))


@pytest.mark.parametrize("B,L,nt,pick", [(1, 4096, 1, [0]), (1, 32768, 1, [0]), (1, 131072, 1, [0]),
                                         (16, 4096, 1, [0, 7, 15]), (16, 32768, 1, [0, 7, 15]),
                                         (16, 131072, 1, [0, 15]), (16, 32768, 4, [0, 15]), (1, 32768, 8, [0])])
def test_attn_full_size_device(fnlib, B, L, nt, pick):
    """Config 3 at every size it names (B = 1 and 16 at 4K, 32K and 128K) through the device entry point: caches
    filled in HBM, the oracle run on a subset of the sequences (they are independent), compared on og and the
    appended K/V rows.  nt > 1: the last nt
    positions are the new tokens (a verify step at full context)."""
    import fn
    import hiprt

    _say(f"attn full size B={B} L={L} nt={nt}, oracle on sequences {pick}")
    nq, nkv, hd = 16, 2, 256
    rng = np.random.default_rng(L + B)
    per_seq = nkv * L * hd
    K = hiprt.Buf.empty((B * per_seq,))
    V = hiprt.Buf.empty((B * per_seq,))
    fnlib.fill_normal_dev(K.ptr, B * per_seq, 11)
    fnlib.fill_normal_dev(V.ptr, B * per_seq, 12)
    qg = rng.standard_normal((B, nt, nq, 2, hd)).astype(np.float32)
    kn = rng.standard_normal((B, nt, nkv, hd)).astype(np.float32)
    vn = rng.standard_normal((B, nt, nkv, hd)).astype(np.float32)
    wq = rng.normal(1, 0.1, hd).astype(np.float32)
    wk = rng.normal(1, 0.1, hd).astype(np.float32)
    pos = np.full(B, L - nt, np.int32)
    d = {n: hiprt.Buf.like(x) for n, x in (("qg", qg), ("k", kn), ("v", vn), ("wq", wq), ("wk", wk), ("pos", pos))}
    nsplit = fnlib.attn_nsplit(B, nkv, nt, L)
    wb = fnlib.attn_work_bytes(B, nq, nt, nsplit)
    work = hiprt.Buf(wb)
    og = hiprt.Buf.empty((B, nt, nq, hd))
    fnlib.attn_dev(B, nq, nkv, nt, L, d["pos"].ptr, d["qg"].ptr, d["k"].ptr, d["v"].ptr, d["wq"].ptr, d["wk"].ptr,
                   K.ptr, V.ptr, nsplit, work.ptr, wb, og.ptr, None)
    hiprt.sync()
    got = og.download()
    for b in pick:
        Kd = hiprt.dtoh(K.ptr + b * per_seq * 4, (per_seq,))
        Vd = hiprt.dtoh(V.ptr + b * per_seq * 4, (per_seq,))
        Kr, Vr = fn.kv_from_device(Kd, Vd, 1, L, nkv, hd)
        ref_og, ref_k, ref_v = oracle.attn(qg[b:b + 1], kn[b:b + 1], vn[b:b + 1], wq, wk, Kr, Vr, pos[b:b + 1])
        e = (oracle.relerr(got[b:b + 1], ref_og), oracle.relerr(Kr[:, L - nt:L], ref_k),
             oracle.relerr(Vr[:, L - nt:L], ref_v))
        assert max(e) <= TOL, (b, e)
    for x in (K, V, work, og, *d.values()):
        x.free()


def test_attn_position_outside_cache_sets_status(fnlib):
    """fn_attn_dev with a new token at or past max_ctx: nothing is written past the cache, the result stays finite,
    and the per-device status word records FN_STATUS_POS until it is cleared (one-token and multi-token paths)."""
    import fn
    import hiprt

    B, nq, nkv, hd, max_ctx = 2, 16, 2, 256, 128
    _say("attn position outside the cache -> status word")
    fnlib.dev_status()  # start clean
    rng = np.random.default_rng(3)
    for nt, pos in ((1, [5, 128]), (3, [126, 7])):
        K = hiprt.Buf.like(rng.standard_normal(B * nkv * max_ctx * hd).astype(np.float32))
        V = hiprt.Buf.like(rng.standard_normal(B * nkv * max_ctx * hd).astype(np.float32))
        k0, v0 = K.download(), V.download()
        d = {n: hiprt.Buf.like(x) for n, x in (
            ("qg", rng.standard_normal((B, nt, nq, 2, hd)).astype(np.float32)),
            ("k", rng.standard_normal((B, nt, nkv, hd)).astype(np.float32)),
            ("v", rng.standard_normal((B, nt, nkv, hd)).astype(np.float32)),
            ("wq", np.ones(hd, np.float32)), ("wk", np.ones(hd, np.float32)), ("pos", np.array(pos, np.int32)))}
        nsplit = fnlib.attn_nsplit(B, nkv, nt, max_ctx)
        wb = fnlib.attn_work_bytes(B, nq, nt, nsplit)
        work, og = hiprt.Buf(wb), hiprt.Buf.empty((B, nt, nq, hd))
        fnlib.attn_dev(B, nq, nkv, nt, max_ctx, d["pos"].ptr, d["qg"].ptr, d["k"].ptr, d["v"].ptr, d["wq"].ptr,
                       d["wk"].ptr, K.ptr, V.ptr, nsplit, work.ptr, wb, og.ptr, None)
        assert fnlib.dev_status(clear=False) & fn.STATUS_POS
        assert fnlib.dev_status() & fn.STATUS_POS
        assert fnlib.dev_status() == 0
        assert np.isfinite(og.download()).all()
        # the other sequence's rows (inside the cache) were appended; nothing else changed size
        assert K.download().shape == k0.shape and V.download().shape == v0.shape
        for x in (K, V, work, og, *d.values()):
            x.free()

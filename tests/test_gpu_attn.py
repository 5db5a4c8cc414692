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


def test_attn_reference_group_12(fnlib):
    """The reference model's own head shape: 24 query heads over 2 kv heads (faie2fn.cu:47-48)."""
    _say("attn nq=24 nkv=2")
    _check(fnlib, fn_synth.AttnCase(B=1, L=513, nq=24))


@pytest.mark.parametrize("B,L,pick", [(16, 32768, [0, 7, 15]), (1, 131072, [0])])
def test_attn_full_size_device(fnlib, B, L, pick):
    """BASELINE config 3 at full size through the device entry point: caches filled in HBM, the oracle run on a
    subset of the sequences (they are independent), compared on og and the appended K/V row."""
    import fn
    import hiprt

    _say(f"attn full size B={B} L={L}, oracle on sequences {pick}")
    nq, nkv, hd = 16, 2, 256
    rng = np.random.default_rng(L + B)
    per_seq = nkv * L * hd
    K = hiprt.Buf.empty((B * per_seq,))
    V = hiprt.Buf.empty((B * per_seq,))
    fnlib.fill_normal_dev(K.ptr, B * per_seq, 11)
    fnlib.fill_normal_dev(V.ptr, B * per_seq, 12)
    qg = rng.standard_normal((B, 1, nq, 2, hd)).astype(np.float32)
    kn = rng.standard_normal((B, 1, nkv, hd)).astype(np.float32)
    vn = rng.standard_normal((B, 1, nkv, hd)).astype(np.float32)
    wq = rng.normal(1, 0.1, hd).astype(np.float32)
    wk = rng.normal(1, 0.1, hd).astype(np.float32)
    pos = np.full(B, L - 1, np.int32)
    d = {n: hiprt.Buf.like(x) for n, x in (("qg", qg), ("k", kn), ("v", vn), ("wq", wq), ("wk", wk), ("pos", pos))}
    nsplit = fnlib.attn_nsplit(B, nkv, 1, L)
    wb = fnlib.attn_work_bytes(B, nq, 1, nsplit)
    work = hiprt.Buf(wb)
    og = hiprt.Buf.empty((B, 1, nq, hd))
    fnlib.attn_dev(B, nq, nkv, 1, L, d["pos"].ptr, d["qg"].ptr, d["k"].ptr, d["v"].ptr, d["wq"].ptr, d["wk"].ptr, K.ptr,
                   V.ptr, nsplit, work.ptr, wb, og.ptr, None)
    hiprt.sync()
    got = og.download()
    for b in pick:
        Kd = hiprt.dtoh(K.ptr + b * per_seq * 4, (per_seq,))
        Vd = hiprt.dtoh(V.ptr + b * per_seq * 4, (per_seq,))
        Kr, Vr = fn.kv_from_device(Kd, Vd, 1, L, nkv, hd)
        ref_og, ref_k, ref_v = oracle.attn(qg[b:b + 1], kn[b:b + 1], vn[b:b + 1], wq, wk, Kr, Vr, pos[b:b + 1])
        e = (oracle.relerr(got[b:b + 1], ref_og), oracle.relerr(Kr[:, L - 1:L], ref_k), oracle.relerr(Vr[:, L - 1:L], ref_v))
        assert max(e) <= TOL, (b, e)
    for x in (K, V, work, og, *d.values()):
        x.free()

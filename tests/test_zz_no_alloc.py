"""fn_attn_noalloc_dev (workspace in a device array of the library) against fn_attn_dev (caller workspace): the same
kernels on the same inputs, so og and the appended K/V rows must agree bit for bit.  Two calls in a row, the second
with a smaller input, so the second runs over what the first left in the array; the first is also checked against
the float64 oracle on one sequence."""

import numpy as np
import pytest

import fn
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
NQ, NKV, HD = 16, 2, 256


def _say(*a):
    print(*a, flush=True)


def _run_pair(fnlib, B, L, nt, seed, check_oracle):
    import hiprt

    max_ctx = (L + 63) // 64 * 64
    _say(f"noalloc B={B} L={L} nt={nt} max_ctx={max_ctx}")
    rng = np.random.default_rng(seed)
    per_seq = NKV * max_ctx * HD
    K1, V1 = hiprt.Buf.empty((B * per_seq,)), hiprt.Buf.empty((B * per_seq,))
    fnlib.fill_normal_dev(K1.ptr, B * per_seq, seed)
    fnlib.fill_normal_dev(V1.ptr, B * per_seq, seed + 1)
    K2, V2 = hiprt.Buf.empty((B * per_seq,)), hiprt.Buf.empty((B * per_seq,))
    K2.copy_from(K1)
    V2.copy_from(V1)
    qg = rng.standard_normal((B, nt, NQ, 2, HD)).astype(np.float32)
    kn = rng.standard_normal((B, nt, NKV, HD)).astype(np.float32)
    vn = rng.standard_normal((B, nt, NKV, HD)).astype(np.float32)
    wq = rng.normal(1, 0.1, HD).astype(np.float32)
    wk = rng.normal(1, 0.1, HD).astype(np.float32)
    pos = np.array([L - nt - (b * 37) % (L - nt + 1) for b in range(B)], np.int32)  # ragged, the first at the end
    d = {n: hiprt.Buf.like(x) for n, x in (("qg", qg), ("k", kn), ("v", vn), ("wq", wq), ("wk", wk), ("pos", pos))}
    nsplit = fnlib.attn_nsplit(B, NKV, nt, L)
    wb = fnlib.attn_work_bytes(B, NQ, nt, nsplit)
    assert wb <= fn.NOALLOC_SCRATCH_BYTES
    work = hiprt.Buf(wb)
    og1, og2 = hiprt.Buf.empty((B, nt, NQ, HD)), hiprt.Buf.empty((B, nt, NQ, HD))
    fnlib.attn_dev(B, NQ, NKV, nt, max_ctx, d["pos"].ptr, d["qg"].ptr, d["k"].ptr, d["v"].ptr, d["wq"].ptr,
                   d["wk"].ptr, K1.ptr, V1.ptr, nsplit, work.ptr, wb, og1.ptr, None)
    fnlib.attn_noalloc_dev(B, NQ, NKV, nt, max_ctx, d["pos"].ptr, d["qg"].ptr, d["k"].ptr, d["v"].ptr, d["wq"].ptr,
                           d["wk"].ptr, K2.ptr, V2.ptr, nsplit, og2.ptr, None)
    hiprt.sync()
    a, b = og1.download(), og2.download()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "og differs from fn_attn_dev"
    for X, Y in ((K1, K2), (V1, V2)):
        assert np.array_equal(X.download().view(np.uint32), Y.download().view(np.uint32)), "cache differs"
    if check_oracle:
        Kd = hiprt.dtoh(K2.ptr, (per_seq,))
        Vd = hiprt.dtoh(V2.ptr, (per_seq,))
        Kr, Vr = fn.kv_from_device(Kd, Vd, 1, max_ctx, NKV, HD)
        # rows at and past pos[0] of the oracle's input are the new ones; its input cache is the filled one
        Kin, Vin = Kr.copy(), Vr.copy()
        ref_og, ref_k, ref_v = oracle.attn(qg[:1], kn[:1], vn[:1], wq, wk, Kin, Vin, pos[:1])
        p0 = int(pos[0])
        e = (oracle.relerr(b[:1], ref_og), oracle.relerr(Kr[:, p0:p0 + nt], ref_k),
             oracle.relerr(Vr[:, p0:p0 + nt], ref_v))
        assert max(e) <= TOL, e
    for x in (K1, V1, K2, V2, work, og1, og2, *d.values()):
        x.free()


def test_noalloc_matches_caller_workspace(fnlib):
    """A large call, then a smaller one over the array the first left behind, then a multi-token one."""
    _run_pair(fnlib, B=4, L=3000, nt=1, seed=5, check_oracle=True)
    _run_pair(fnlib, B=1, L=500, nt=1, seed=6, check_oracle=True)
    _run_pair(fnlib, B=2, L=1000, nt=4, seed=7, check_oracle=False)


def test_noalloc_rejects_oversize(fnlib):
    """Shapes whose workspace exceeds the array fail with an error before anything runs."""
    with pytest.raises(RuntimeError, match="workspace"):
        fnlib.attn_noalloc_dev(64, 16, 2, 8, 4096, None, None, None, None, None, None, None, None, 64, None)

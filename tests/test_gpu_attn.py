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

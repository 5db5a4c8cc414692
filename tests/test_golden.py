"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the float64
oracle): the oracle must still reproduce them (CPU), and the HIP path must match them (GPU, <= 1e-5 normwise)."""

import os

import numpy as np
import pytest

import fn_synth
import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLD, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _core_run(step_fn, steps, dtype=np.float32):
    gen = fn_synth.CoreSteps(B=1, seed=0)
    S = gen.S0.astype(dtype)
    o = [step_fn(gen.step(), S) for _ in range(steps)]
    return np.stack(o, 1), S


def _block_run(step_fn, steps, gate_act):
    lay = fn_synth.BlockLayer(B=1, config=1, layer=0)
    S, conv = lay.S0.copy(), lay.conv0.copy()
    out = [step_fn(lay, lay.step(), S, conv, gate_act) for _ in range(steps)]
    return np.stack(out, 1), S


def _check_state(S, g, tol):
    assert oracle.relerr(S[:, :, ::16, ::16], g["S_sample"]) <= tol
    assert oracle.relerr(S.astype(np.float64).sum(axis=(2, 3)), g["S_sum"]) <= tol * 10
    assert oracle.relerr((S.astype(np.float64) ** 2).sum(axis=(2, 3)), g["S_sumsq"]) <= tol


def test_oracle_reproduces_golden():
    g = load("gdn_core_c0.npz")
    o, S = _core_run(lambda x, S: oracle.gdn_core(*x, S)[:, 0], int(g["steps"]), np.float64)
    assert oracle.relerr(o, g["o"]) <= 1e-6
    _check_state(S, g, 1e-6)
    for name in ("gdn_block_c1_sigmoid.npz", "gdn_block_c1_silu.npz"):
        g = load(name)
        f = lambda lay, x, S, conv, ga: oracle.gdn_block(x[0], lay.conv_w, conv, x[1], lay.dt_bias, lay.ssm_a, S, x[2],
                                                         lay.norm_w, 16, 32, gate_act=ga)[:, 0]
        lay = fn_synth.BlockLayer(B=1, config=1, layer=0)
        S, conv = lay.S0.astype(np.float64), lay.conv0.astype(np.float64)
        out = np.stack([f(lay, lay.step(), S, conv, int(g["gate_act"])) for _ in range(int(g["steps"]))], 1)
        assert oracle.relerr(out, g["out"]) <= 1e-6
        _check_state(S, g, 1e-6)
    g = load("attn_c3_l512.npz")
    c = fn_synth.AttnCase(B=1, L=512)
    og, kr, vr = oracle.attn(c.qg, c.k, c.v, c.wq, c.wk, c.Kc, c.Vc, c.pos)
    assert oracle.relerr(og, g["og"]) <= 1e-6 and oracle.relerr(kr, g["k_row"]) <= 1e-6


@pytest.mark.gpu
def test_gpu_matches_golden(fnlib):
    print("golden fixtures vs GPU", flush=True)
    g = load("gdn_core_c0.npz")
    o, S = _core_run(lambda x, S: fnlib.gdn(*x, S)[:, 0], int(g["steps"]))
    assert oracle.relerr(o, g["o"]) <= 1e-5
    _check_state(S, g, 1e-5)
    for name in ("gdn_block_c1_sigmoid.npz", "gdn_block_c1_silu.npz"):
        g = load(name)
        f = lambda lay, x, S, conv, ga: fnlib.gdn_block(x[0], lay.conv_w, conv, x[1], lay.dt_bias, lay.ssm_a, S, x[2],
                                                        lay.norm_w, 16, 32, gate_act=ga)[:, 0]
        out, S = _block_run(f, int(g["steps"]), int(g["gate_act"]))
        assert oracle.relerr(out, g["out"]) <= 1e-5
        _check_state(S, g, 1e-5)
    g = load("attn_c3_l512.npz")
    c = fn_synth.AttnCase(B=1, L=512)
    Kc, Vc = c.Kc.copy(), c.Vc.copy()
    og = fnlib.attn(c.qg, c.k, c.v, c.wq, c.wk, Kc, Vc, c.pos)
    assert oracle.relerr(og, g["og"]) <= 1e-5
    assert oracle.relerr(Kc[:, 511:512], g["k_row"]) <= 1e-5

"""The committed golden fixtures:

* tests/golden/{gdn_core_c0, gdn_block_c1_*, attn_c3_l512}.npz, written by tests/golden/make_golden.py from the
  float64 oracle: regression pins: the oracle must still reproduce them (CPU), the HIP path must match them (GPU);
* tests/golden/*_hf.npz, written by tests/golden/make_golden_hf.py from an independent implementation (the
  transformers library's Qwen3-Next routines: torch_recurrent_gated_delta_rule, causal_conv1d_update, l2norm,
  Qwen3NextRMSNormGated): config 0 over all 64 steps and the config-1 block with the SiLU gate; the oracle (CPU)
  and the HIP path (GPU) must both match them.

Bar: <= 1e-5 normwise (the library computes the recurrence in float32)."""

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


def _core_hf_run(step_fn, g, dtype):
    gen = fn_synth.CoreSteps(B=1, seed=0)
    S = gen.S0.astype(dtype)
    o = [step_fn(gen.step(), S) for _ in range(int(g["steps"]))]
    return np.stack(o)[g["o_steps"]], S


def _block_hf_run(step_fn, g, dtype):
    lay = fn_synth.BlockLayer(B=1, config=1, layer=0)
    S, conv = lay.S0.astype(dtype), lay.conv0.astype(dtype)
    out = [step_fn(lay, lay.step(), S, conv) for _ in range(int(g["steps"]))]
    return np.stack(out)[g["out_steps"]], S, conv


def test_oracle_matches_library_fixtures():
    """The float64 oracle against the fixtures of the transformers Qwen3-Next routines (64 steps of config 0, 16
    steps of the SiLU-gated block): outputs, final state and conv state."""
    g = load("gdn_core_c0_hf.npz")
    o, S = _core_hf_run(lambda x, S: oracle.gdn_core(*x, S)[0, 0], g, np.float64)
    assert oracle.relerr(o, g["o"]) <= 1e-5
    _check_state(S, g, 1e-5)
    g = load("gdn_block_c1_silu_hf.npz")
    f = lambda lay, x, S, conv: oracle.gdn_block(x[0], lay.conv_w, conv, x[1], lay.dt_bias, lay.ssm_a, S, x[2],
                                                 lay.norm_w, 16, 32, gate_act=1)[0, 0]
    out, S, conv = _block_hf_run(f, g, np.float64)
    assert oracle.relerr(out, g["out"]) <= 1e-5
    _check_state(S, g, 1e-5)
    assert oracle.relerr(conv[0], g["conv"]) <= 1e-6


@pytest.mark.gpu
def test_gpu_matches_library_fixtures(fnlib):
    """The HIP path against the transformers fixtures: the core over config 0's 64 steps, the fused block with the
    SiLU gate over 16 steps (host-array hooks, state and conv state carried between calls)."""
    print("library (transformers Qwen3-Next) fixtures vs GPU", flush=True)
    g = load("gdn_core_c0_hf.npz")
    o, S = _core_hf_run(lambda x, S: fnlib.gdn(*x, S)[0, 0], g, np.float32)
    assert oracle.relerr(o, g["o"]) <= 1e-5
    _check_state(S, g, 1e-5)
    g = load("gdn_block_c1_silu_hf.npz")
    f = lambda lay, x, S, conv: fnlib.gdn_block(x[0], lay.conv_w, conv, x[1], lay.dt_bias, lay.ssm_a, S, x[2],
                                                lay.norm_w, 16, 32, gate_act=1)[0, 0]
    out, S, conv = _block_hf_run(f, g, np.float32)
    assert oracle.relerr(out, g["out"]) <= 1e-5
    _check_state(S, g, 1e-5)
    assert oracle.relerr(conv[0], g["conv"]) <= 1e-6


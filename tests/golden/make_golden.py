"""Writes the golden fixtures of this directory from the float64 C oracle (oracle/fn_oracle.c) on the seeded inputs
of faie2-flashnext_amd/fn_synth.py.  The reference ships no vectors for this path (its oracle, flashnext/ref_fn.py,
needs a transformers build and a GGUF model that are not available), so these pin the oracle against regressions
and give the GPU tests stored expected values.  Inputs are not stored: the fixtures name the generator and seed.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "faie2-flashnext_amd")]

import fn_synth  # noqa: E402
import oracle  # noqa: E402

CORE_STEPS, BLOCK_STEPS = 6, 4


def core_c0():
    gen = fn_synth.CoreSteps(B=1, seed=0)
    S = gen.S0.astype(np.float64)
    o = []
    for _ in range(CORE_STEPS):
        o.append(oracle.gdn_core(*gen.step(), S)[:, 0])
    return dict(generator="CoreSteps(B=1, seed=0)", steps=CORE_STEPS, o=np.stack(o, 1).astype(np.float32),
                S_sample=S[:, :, ::16, ::16].astype(np.float32), S_sum=S.sum(axis=(2, 3)),
                S_sumsq=(S * S).sum(axis=(2, 3)))


def block_c1(gate_act):
    lay = fn_synth.BlockLayer(B=1, config=1, layer=0)
    S, conv = lay.S0.astype(np.float64), lay.conv0.astype(np.float64)
    out = []
    for _ in range(BLOCK_STEPS):
        qkv, ab, z = lay.step()
        out.append(oracle.gdn_block(qkv, lay.conv_w, conv, ab, lay.dt_bias, lay.ssm_a, S, z, lay.norm_w, 16, 32,
                                    gate_act=gate_act)[:, 0])
    return dict(generator="BlockLayer(B=1, config=1, layer=0)", steps=BLOCK_STEPS, gate_act=gate_act,
                out=np.stack(out, 1).astype(np.float32), S_sample=S[:, :, ::16, ::16].astype(np.float32),
                S_sum=S.sum(axis=(2, 3)), S_sumsq=(S * S).sum(axis=(2, 3)))


def attn_c3():
    case = fn_synth.AttnCase(B=1, L=512)
    og, kr, vr = oracle.attn(case.qg, case.k, case.v, case.wq, case.wk, case.Kc, case.Vc, case.pos)
    return dict(generator="AttnCase(B=1, L=512)", og=og.astype(np.float32), k_row=kr.astype(np.float32),
                v_row=vr.astype(np.float32))


def main():
    np.savez_compressed(os.path.join(HERE, "gdn_core_c0.npz"), **core_c0())
    np.savez_compressed(os.path.join(HERE, "gdn_block_c1_sigmoid.npz"), **block_c1(0))
    np.savez_compressed(os.path.join(HERE, "gdn_block_c1_silu.npz"), **block_c1(1))
    np.savez_compressed(os.path.join(HERE, "attn_c3_l512.npz"), **attn_c3())


if __name__ == "__main__":
    main()

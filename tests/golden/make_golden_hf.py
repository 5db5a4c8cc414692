"""Writes golden fixtures of the DeltaNet path from an implementation independent of this repository: the
transformers library's Qwen3-Next routines (transformers.models.qwen3_next.modeling_qwen3_next, installed in this
image; not part of the reference and not this repository's oracle), on the seeded inputs of
faie2-flashnext_amd/fn_synth.py.  Inputs are not stored: the fixtures name the generator and seed.

* gdn_core_c0_hf.npz: config 0 (B=1, 16 q/k heads, 32 v heads, dk = dv = 128, S ~ N(0, 0.02)) for all 64 steps
  through torch_recurrent_gated_delta_rule (float32 inside, as the library computes it); o every 8th step and the
  last, and the final state's sampled entries and per-head sums.
* gdn_block_c1_silu_hf.npz: the fused block at config 1's shapes with the SiLU output gate
  for 16 steps, composed from causal_conv1d_update (float64), l2norm, softplus (threshold 20),
  torch_recurrent_gated_delta_rule (float32) and Qwen3NextRMSNormGated (float64); out every 4th step, the final
  state's summaries and conv state.

    python tests/golden/make_golden_hf.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "faie2-flashnext_amd")]

import torch  # noqa: E402
import transformers  # noqa: E402
from transformers.models.qwen3_next import modeling_qwen3_next as hf  # noqa: E402

import fn_synth  # noqa: E402

CORE_STEPS, CORE_EVERY = 64, 8
BLOCK_STEPS, BLOCK_EVERY = 16, 4
NKH, NVH, DK = 16, 32, 128


def _t(a, dtype=torch.float64):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype)


def _summary(S):
    S = np.asarray(S, np.float64)
    return dict(S_sample=S[:, :, ::16, ::16].astype(np.float32), S_sum=S.sum(axis=(2, 3)),
                S_sumsq=(S * S).sum(axis=(2, 3)))


def core_c0():
    gen = fn_synth.CoreSteps(B=1, seed=0)
    steps = [gen.step() for _ in range(CORE_STEPS)]
    q, k, v, beta, g = (np.concatenate([s[i] for s in steps], axis=1) for i in range(5))
    idx = np.arange(NVH) % NKH  # value head h reads key head h mod 16 (the reference's map)
    out, S = hf.torch_recurrent_gated_delta_rule(_t(q[:, :, idx], torch.float32), _t(k[:, :, idx], torch.float32),
                                                 _t(v, torch.float32), _t(g, torch.float32),
                                                 _t(beta, torch.float32), _t(gen.S0, torch.float32), True)
    o = out.numpy()[0]  # [steps][heads][dv]
    keep = sorted(set(range(CORE_EVERY - 1, CORE_STEPS, CORE_EVERY)) | {CORE_STEPS - 1})
    return dict(generator="CoreSteps(B=1, seed=0)", steps=CORE_STEPS, o_steps=np.array(keep, np.int32),
                o=o[keep].astype(np.float32), **_summary(S.numpy()))


def block_c1_silu():
    lay = fn_synth.BlockLayer(B=1, config=1, layer=0)
    steps = [lay.step() for _ in range(BLOCK_STEPS)]
    qkv, ab, z = (np.concatenate([s[i] for s in steps], axis=1) for i in range(3))
    B, nt, C = 1, BLOCK_STEPS, lay.C
    state = _t(lay.conv0).transpose(1, 2).contiguous()  # [B][C][3], oldest first
    x = hf.causal_conv1d_update(_t(qkv).transpose(1, 2), state, _t(lay.conv_w), None, "silu").transpose(1, 2)
    q = hf.l2norm(x[..., : NKH * DK].reshape(B, nt, NKH, DK))
    k = hf.l2norm(x[..., NKH * DK: 2 * NKH * DK].reshape(B, nt, NKH, DK))
    v = x[..., 2 * NKH * DK:].reshape(B, nt, NVH, DK)
    g = _t(lay.ssm_a) * torch.nn.functional.softplus(_t(ab[..., :NVH]) + _t(lay.dt_bias))
    beta = torch.sigmoid(_t(ab[..., NVH:]))
    idx = torch.arange(NVH) % NKH
    o, S = hf.torch_recurrent_gated_delta_rule(q[:, :, idx], k[:, :, idx], v, g, beta, _t(lay.S0), True)
    norm = hf.Qwen3NextRMSNormGated(DK, eps=1e-6).to(torch.float64)
    with torch.no_grad():
        norm.weight.copy_(_t(lay.norm_w))
        out = norm(o.to(torch.float64), _t(z).reshape(B, nt, NVH, DK)).reshape(B, nt, NVH * DK).numpy()[0]
    keep = list(range(BLOCK_EVERY - 1, BLOCK_STEPS, BLOCK_EVERY))
    return dict(generator="BlockLayer(B=1, config=1, layer=0)", steps=BLOCK_STEPS, gate_act=1,
                out_steps=np.array(keep, np.int32), out=out[keep].astype(np.float32),
                conv=state.transpose(1, 2).numpy()[0].astype(np.float32), **_summary(S.numpy()))


def main():
    meta = dict(source=np.array(f"transformers {transformers.__version__} qwen3_next, torch {torch.__version__}"))
    for name, fn in (("gdn_core_c0_hf.npz", core_c0), ("gdn_block_c1_silu_hf.npz", block_c1_silu)):
        np.savez_compressed(os.path.join(HERE, name), **fn(), **meta)
        print("wrote", name)


if __name__ == "__main__":
    main()

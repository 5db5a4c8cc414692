"""Pins of the float64 oracle (CPU only).  The reference ships no golden vectors for this path and its Python oracle
(flashnext/ref_fn.py) cannot run here, so each oracle function is pinned by what the mathematics fixes:

* the independent numpy twin (oracle/twin.py) on random cases of every shape option;
* closed forms and invariants of the delta rule, exact rational arithmetic on tiny heads;
* library routines that compute the same operations: transformers' Qwen3-Next causal_conv1d_update, l2norm,
  torch_recurrent_gated_delta_rule, Qwen3NextRMSNormGated, apply_rotary_pos_emb (float32 inside, so compared at
  float32 precision), torch's softplus and scaled_dot_product_attention in float64;
* the reference's stated conventions (fp32 RoPE angle, softplus threshold 20, sigmoid gate).
Each check is chosen so that a plausible slip (a transposed state, a dropped decay, the wrong tap order, the wrong
head map, a float64 RoPE angle) fails it.
"""

from fractions import Fraction

import numpy as np
import pytest

import fn_synth
import oracle
import oracle.twin as twin

RNG = np.random.default_rng(20261201)


def f32(x):
    return np.asarray(x, np.float32)


def rand_core(B, nt, nkh, nvh, dk, dv, rng):
    q = f32(rng.standard_normal((B, nt, nkh, dk)))
    k = f32(rng.standard_normal((B, nt, nkh, dk)))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = f32(rng.standard_normal((B, nt, nvh, dv)))
    beta = f32(rng.random((B, nt, nvh)))
    g = f32(-rng.random((B, nt, nvh)))
    S = rng.standard_normal((B, nvh, dk, dv)) * 0.1
    return q, k, v, beta, g, S


# ---------------------------------------------------------------------------------------------------------------
# C oracle == numpy twin


@pytest.mark.parametrize("head_map", [0, 1])
def test_twin_core(head_map):
    q, k, v, beta, g, S = rand_core(3, 4, 2, 6, 16, 8, RNG)
    S1, S2 = S.copy(), S.copy()
    o1 = oracle.gdn_core(q, k, v, beta, g, S1, head_map)
    o2 = twin.gdn_core(q, k, v, beta, g, S2, head_map)
    assert oracle.relerr(o1, o2) < 1e-13 and oracle.relerr(S1, S2) < 1e-13


@pytest.mark.parametrize("head_map,gate_act", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_twin_block(head_map, gate_act):
    B, nt, nkh, nvh, dk, dv = 2, 5, 2, 4, 16, 16
    C = 2 * nkh * dk + nvh * dv
    qkv = f32(RNG.standard_normal((B, nt, C)))
    cw = f32(RNG.normal(0, 0.3, (C, 4)))
    cs = RNG.standard_normal((B, 3, C)).astype(np.float32).astype(np.float64)
    ab = f32(RNG.standard_normal((B, nt, 2 * nvh)) * 8)  # some alpha + dt_bias above 20
    dtb = f32(RNG.standard_normal(nvh) * 8)
    sa = f32(-np.exp(RNG.normal(0, 0.5, nvh)))
    S = RNG.standard_normal((B, nvh, dk, dv)) * 0.02
    z = f32(RNG.standard_normal((B, nt, nvh * dv)))
    nw = f32(RNG.normal(1, 0.1, dv))
    c1, c2, S1, S2 = cs.copy(), cs.copy(), S.copy(), S.copy()
    o1 = oracle.gdn_block(qkv, cw, c1, ab, dtb, sa, S1, z, nw, nkh, nvh, dk, dv, head_map, gate_act)
    o2 = twin.gdn_block(qkv, cw, c2, ab, dtb, sa, S2, z, nw, nkh, nvh, dk, dv, head_map, gate_act)
    assert max(oracle.relerr(o1, o2), oracle.relerr(S1, S2), oracle.relerr(c1, c2)) < 1e-12


def test_twin_attn():
    B, nt, nq, nkv, hd, L = 3, 3, 8, 2, 32, 90
    qg = f32(RNG.standard_normal((B, nt, nq, 2, hd)))
    kn = f32(RNG.standard_normal((B, nt, nkv, hd)))
    vn = f32(RNG.standard_normal((B, nt, nkv, hd)))
    wq, wk = f32(RNG.normal(1, 0.1, hd)), f32(RNG.normal(1, 0.1, hd))
    K = f32(RNG.standard_normal((B, L, nkv, hd)))
    V = f32(RNG.standard_normal((B, L, nkv, hd)))
    pos = np.array([0, 41, 87], np.int32)
    a = oracle.attn(qg, kn, vn, wq, wk, K, V, pos, nrot=8, theta=1e4)
    b = twin.attn(qg, kn, vn, wq, wk, K, V, pos, nrot=8, theta=1e4)
    for x, y in zip(a, b):
        assert oracle.relerr(x, y) < 1e-12


# ---------------------------------------------------------------------------------------------------------------
# delta rule: closed forms, invariants, exact arithmetic


def _core1(q, k, v, beta, g, S, head_map=0):
    S = S.copy()
    o = oracle.gdn_core(q, k, v, beta, g, S, head_map)
    return o, S


def test_beta_zero_is_pure_decay():
    q, k, v, beta, g, S = rand_core(2, 1, 2, 4, 16, 8, RNG)
    beta[:] = 0
    o, S1 = _core1(q, k, v, beta, g, S)
    gam = np.exp(g[:, 0].astype(np.float64))[..., None, None]
    assert np.allclose(S1, gam * S, rtol=0, atol=1e-15)
    kidx = np.arange(4) % 2
    ref = np.einsum("bhij,bhi->bhj", gam * S, q[:, 0, kidx].astype(np.float64)) / 4.0
    assert np.allclose(o[:, 0], ref, atol=1e-14)


def test_zero_state_rank_one_write():
    q, k, v, beta, g, S = rand_core(2, 1, 2, 4, 16, 8, RNG)
    S[:] = 0
    o, S1 = _core1(q, k, v, beta, g, S)
    kidx = np.arange(4) % 2
    kk = k[:, 0, kidx].astype(np.float64)
    qq = q[:, 0, kidx].astype(np.float64)
    bb = beta[:, 0].astype(np.float64)
    ref_S = bb[..., None, None] * kk[..., :, None] * v[:, 0].astype(np.float64)[..., None, :]
    assert np.allclose(S1, ref_S, atol=1e-15)
    ref_o = (bb * (kk * qq).sum(-1))[..., None] * v[:, 0] / 4.0
    assert np.allclose(o[:, 0], ref_o, atol=1e-14)


def test_write_then_read_returns_v():
    """gamma = 1, beta = 1, |k| = 1: after the update, S'^T k = v exactly (delta rule stores v at key k)."""
    q, k, v, beta, g, S = rand_core(1, 1, 1, 2, 32, 16, RNG)
    beta[:] = 1
    g[:] = 0
    kk = k[:, 0, 0].astype(np.float64)
    k[:, 0, 0] = (kk / np.linalg.norm(kk)).astype(np.float32)
    _, S1 = _core1(q, k, v, beta, g, S)
    kd = k[0, 0, 0].astype(np.float64)
    nk2 = kd @ kd
    for h in range(2):
        # S'^T k = S^T k (1 - |k|^2) + v |k|^2  -> v when |k| = 1 (float32 k: |k|^2 = 1 up to rounding)
        ref = (S[0, h].T @ kd) * (1 - nk2) + v[0, 0, h] * nk2
        assert np.allclose(S1[0, h].T @ kd, ref, atol=1e-13)
        assert np.allclose(S1[0, h].T @ kd, v[0, 0, h], atol=1e-6)


def test_affine_in_v():
    q, k, v, beta, g, S = rand_core(1, 1, 2, 4, 16, 8, RNG)
    v2 = f32(RNG.standard_normal(v.shape))
    z = np.zeros_like(v)
    oa, Sa = _core1(q, k, v, beta, g, S)
    ob, Sb = _core1(q, k, v2, beta, g, S)
    oc, Sc = _core1(q, k, f32(v.astype(np.float64) + v2), beta, g, S)
    o0, S0 = _core1(q, k, z, beta, g, S)
    assert np.allclose(oc + o0, oa + ob, atol=1e-7)  # v + v2 rounded to fp32 once
    assert np.allclose(Sc + S0, Sa + Sb, atol=1e-7)


@pytest.mark.parametrize("head_map", [0, 1])
def test_batch_and_head_permutation(head_map):
    """Sequences are independent; value heads read the key head the map names (tiled h % nkh, grouped h / r)."""
    q, k, v, beta, g, S = rand_core(4, 2, 2, 4, 16, 8, RNG)
    perm = np.array([2, 0, 3, 1])
    o, S1 = _core1(q, k, v, beta, g, S, head_map)
    op, Sp = _core1(q[perm], k[perm], v[perm], beta[perm], g[perm], S[perm], head_map)
    assert np.array_equal(op, o[perm]) and np.array_equal(Sp, S1[perm])
    # swapping the two key heads is the same as permuting value heads onto the other key head
    kidx = np.arange(4) % 2 if head_map == 0 else np.arange(4) // 2
    sw = np.array([1, 0])
    vperm = np.array([np.nonzero(kidx == sw[kidx[h]])[0][list(np.nonzero(kidx == kidx[h])[0]).index(h)]
                      for h in range(4)])
    o2, S2 = _core1(q[:, :, sw], k[:, :, sw], v[:, :, vperm], beta[:, :, vperm], g[:, :, vperm], S[:, vperm], head_map)
    assert np.allclose(o2, o[:, :, vperm], atol=1e-15) and np.allclose(S2, S1[:, vperm], atol=1e-15)


def test_exact_rational_three_steps():
    """dk = dv = 4, one key head, two value heads, 3 steps: the oracle against exact rational arithmetic on the
    same (binary-exact) inputs; gamma and beta enter as the float64 values the oracle uses."""
    rng = np.random.default_rng(3)
    B, nt, nkh, nvh, dk, dv = 1, 3, 1, 2, 4, 4
    q, k, v, beta, g, S = rand_core(B, nt, nkh, nvh, dk, dv, rng)
    S = (np.round(S * 64) / 64).astype(np.float64)  # dyadic start
    Sx = S.copy()
    o = oracle.gdn_core(q, k, v, beta, g, Sx)
    Fr = Fraction
    Se = [[[Fr(float(S[0, h, i, j])) for j in range(dv)] for i in range(dk)] for h in range(nvh)]
    for t in range(nt):
        for h in range(nvh):
            gam = Fr(float(np.exp(np.float64(g[0, t, h]))))
            bet = Fr(float(beta[0, t, h]))
            kk = [Fr(float(x)) for x in k[0, t, 0]]
            qq = [Fr(float(x)) for x in q[0, t, 0]]
            vv = [Fr(float(x)) for x in v[0, t, h]]
            kv = [sum(Se[h][i][j] * kk[i] for i in range(dk)) for j in range(dv)]
            d = [(vv[j] - gam * kv[j]) * bet for j in range(dv)]
            Se[h] = [[gam * Se[h][i][j] + kk[i] * d[j] for j in range(dv)] for i in range(dk)]
            oe = [sum(Se[h][i][j] * qq[i] for i in range(dk)) / 2 for j in range(dv)]  # 1/sqrt(4)
            assert np.allclose(o[0, t, h], [float(x) for x in oe], rtol=0, atol=1e-14)
    for h in range(nvh):
        assert np.allclose(Sx[0, h], [[float(x) for x in row] for row in Se[h]], rtol=0, atol=1e-14)


# ---------------------------------------------------------------------------------------------------------------
# library routines (transformers Qwen3-Next; float32 inside, so compared at float32 precision)

torch = pytest.importorskip("torch")
hf = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")


def _expand(x, nvh, head_map):
    nkh = x.shape[2]
    idx = np.arange(nvh) % nkh if head_map == 0 else np.arange(nvh) // (nvh // nkh)
    return x[:, :, idx]


@pytest.mark.parametrize("head_map", [0, 1])
def test_hf_recurrent_gated_delta_rule(head_map):
    gen = fn_synth.CoreSteps(B=2, nkh=4, nvh=8, seed=9)
    steps = [gen.step() for _ in range(8)]
    q, k, v, beta, g = (np.concatenate([s[i] for s in steps], axis=1) for i in range(5))
    S = gen.S0.astype(np.float64)
    o = oracle.gdn_core(q, k, v, beta, g, S, head_map)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    out, st = hf.torch_recurrent_gated_delta_rule(T(_expand(q, 8, head_map)), T(_expand(k, 8, head_map)), T(v), T(g),
                                                   T(beta), T(gen.S0), True)
    assert oracle.relerr(out.numpy(), o) < 5e-6
    assert oracle.relerr(st.numpy(), S) < 5e-6


@pytest.mark.parametrize("gate_act", [0, 1])
def test_hf_composed_block(gate_act):
    """The whole fused block against a composition of library routines: causal_conv1d_update (float64), HF l2norm,
    torch softplus (threshold 20), torch_recurrent_gated_delta_rule, and the gated RMSNorm (HF's module for silu,
    its sigmoid twin for the reference's gate)."""
    B, nt, nkh, nvh, dk = 2, 6, 4, 8, 128
    lay = fn_synth.BlockLayer(B=B, nkh=nkh, nvh=nvh, config=1, layer=5)
    lay.dt_bias = f32(RNG.normal(0, 10, nvh))  # exercise both softplus branches
    C = lay.C
    st = [lay.step() for _ in range(nt)]
    qkv, ab, z = (np.concatenate([s[i] for s in st], axis=1) for i in range(3))
    S, conv = lay.S0.astype(np.float64), lay.conv0.astype(np.float64)
    got = oracle.gdn_block(qkv, lay.conv_w, conv, ab, lay.dt_bias, lay.ssm_a, S, z, lay.norm_w, nkh, nvh,
                           gate_act=gate_act)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))
    state = torch.zeros(B, C, 3, dtype=torch.float64)
    x = hf.causal_conv1d_update(T(qkv).transpose(1, 2), state, T(lay.conv_w), None, "silu").transpose(1, 2)
    q = hf.l2norm(x[..., : nkh * dk].reshape(B, nt, nkh, dk))
    k = hf.l2norm(x[..., nkh * dk: 2 * nkh * dk].reshape(B, nt, nkh, dk))
    v = x[..., 2 * nkh * dk:].reshape(B, nt, nvh, dk)
    a = T(ab[..., :nvh]) + T(lay.dt_bias)
    g = T(lay.ssm_a) * torch.nn.functional.softplus(a)
    beta = torch.sigmoid(T(ab[..., nvh:]))
    idx = torch.arange(nvh) % nkh
    o, _ = hf.torch_recurrent_gated_delta_rule(q[:, :, idx], k[:, :, idx], v, g, beta, T(lay.S0), True)
    o = o.to(torch.float64)
    zz = T(z).reshape(B, nt, nvh, dk)
    if gate_act == 1:
        norm = hf.Qwen3NextRMSNormGated(dk, eps=1e-6).to(torch.float64)
        with torch.no_grad():
            norm.weight.copy_(T(lay.norm_w))
            ref = norm(o, zz)
    else:
        ref = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + 1e-6) * T(lay.norm_w) * torch.sigmoid(zz)
    assert oracle.relerr(got, ref.reshape(B, nt, nvh * dk).detach().numpy()) < 1e-5
    assert np.array_equal(conv, state.transpose(1, 2).numpy())


def test_hf_rotary_and_fp32_angle():
    hd, nrot, theta = 256, 64, 1e7
    inv = oracle.rope_inv_freq(nrot, theta)
    inv_hf = (1.0 / (theta ** (torch.arange(0, nrot, 2, dtype=torch.int64).float() / nrot))).numpy()
    assert inv[0] == 1.0
    assert np.max(np.abs(inv.view(np.int32) - inv_hf.astype(np.float32).view(np.int32))) <= 1  # within 1 ulp
    x = f32(RNG.standard_normal((1, 1, 1, 2, hd)))
    w = np.ones(hd, np.float32)
    z = np.zeros((1, 1, 1, hd), np.float32)
    for pos in (0, 5, 131071):
        og, kr, _ = oracle.attn(f32(np.broadcast_to(x, (1, 1, 2, 2, hd))), x[:, :, :, 0], z, w, w,
                                np.zeros((1, pos + 1, 1, hd), np.float32), np.zeros((1, pos + 1, 1, hd), np.float32),
                                np.array([pos], np.int32), nrot=nrot, theta=theta, eps=1e-6)
        xn = x[0, 0, 0, 0].astype(np.float64)
        xn = xn / np.sqrt((xn * xn).mean() + 1e-6)
        ang = (np.float32(pos) * inv).astype(np.float32).astype(np.float64)  # fp32 product, then float64 trig
        cos = torch.from_numpy(np.concatenate([np.cos(ang), np.cos(ang)]))[None, None]
        sin = torch.from_numpy(np.concatenate([np.sin(ang), np.sin(ang)]))[None, None]
        t = torch.from_numpy(xn)[None, None, None]
        qe, _ = hf.apply_rotary_pos_emb(t, t, cos, sin)
        assert np.allclose(kr[0, 0, 0], qe.numpy()[0, 0, 0], atol=1e-12)
        if pos == 0:
            assert np.allclose(kr[0, 0, 0], xn, atol=1e-15)
        # rotation preserves each pair's norm
        a, b = kr[0, 0, 0, : nrot // 2], kr[0, 0, 0, nrot // 2: nrot]
        assert np.allclose(a * a + b * b, xn[: nrot // 2] ** 2 + xn[nrot // 2: nrot] ** 2, atol=1e-12)
    # a float64 angle would differ by ~1e-3 rad at pos 131071: the convention matters at the 1e-5 bar
    ang32 = (np.float32(131071) * inv).astype(np.float32).astype(np.float64)
    ang64 = 131071.0 * inv.astype(np.float64)
    assert np.max(np.abs(ang32 - ang64)) > 1e-4


def test_attention_special_cases_and_sdpa():
    B, nq, nkv, hd = 1, 8, 2, 32
    wq = np.ones(hd, np.float32)
    wk = np.ones(hd, np.float32)
    qg = f32(RNG.standard_normal((B, 1, nq, 2, hd)))
    kn = f32(RNG.standard_normal((B, 1, nkv, hd)))
    vn = f32(RNG.standard_normal((B, 1, nkv, hd)))
    gate = 1 / (1 + np.exp(-qg[0, 0, :, 1].astype(np.float64)))
    # one key: the output is that V row times the gate
    og, _, _ = oracle.attn(qg, kn, vn, wq, wk, np.zeros((1, 1, nkv, hd), np.float32),
                           np.zeros((1, 1, nkv, hd), np.float32), np.array([0], np.int32), nrot=8)
    for h in range(nq):
        assert np.allclose(og[0, 0, h], vn[0, 0, h // 4] * gate[h], atol=1e-14)
    # identical keys: uniform weights, the mean of V
    L = 7
    Kc = np.broadcast_to(kn[:, :1], (1, L, nkv, hd)).copy()
    Kc[:] = 0
    Vc = f32(RNG.standard_normal((1, L, nkv, hd)))
    og, kr, _ = oracle.attn(qg, kn * 0, vn, wq, wk, Kc, Vc, np.array([L], np.int32), nrot=8)
    allv = np.concatenate([Vc[0], vn[0]], 0).astype(np.float64)
    for h in range(nq):
        assert np.allclose(og[0, 0, h], allv[:, h // 4].mean(0) * gate[h], atol=1e-12)
    # dense softmax attention in float64 (torch SDPA), q head h on kv head h // (nq / nkv)
    L = 50
    Kc = f32(RNG.standard_normal((1, L, nkv, hd)))
    Vc = f32(RNG.standard_normal((1, L, nkv, hd)))
    og, kr, vr = oracle.attn(qg, kn, vn, wq, wk, Kc, Vc, np.array([L], np.int32), nrot=8)
    Q = twin._norm_rope(qg[0, 0, :, 0], wq, L, 8, oracle.rope_inv_freq(8, 1e7), 1e-6)
    K = torch.from_numpy(np.concatenate([Kc[0].astype(np.float64), kr[0]], 0)).permute(1, 0, 2)
    V = torch.from_numpy(np.concatenate([Vc[0].astype(np.float64), vr[0]], 0)).permute(1, 0, 2)
    Kr = K.repeat_interleave(nq // nkv, 0)
    Vr = V.repeat_interleave(nq // nkv, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(Q)[:, None], Kr, Vr)[:, 0]
    assert np.allclose(og[0, 0], ref.numpy() * gate, atol=1e-12)


def test_softplus_threshold_and_gate():
    """gamma = exp(ssm_a * softplus(a + dt_bias)) with softplus the identity above 20 (torch's default), seen
    through the state after one step from S = 0 and a second step."""
    nkh, nvh, dk = 1, 1, 128
    lay = fn_synth.BlockLayer(B=1, nkh=nkh, nvh=nvh, config=1, layer=1)
    for a_val in (-3.0, 0.5, 19.0, 25.0):
        S = np.zeros((1, 1, dk, dk))
        conv = np.zeros((1, 3, lay.C))
        qkv, ab, z = lay.step()
        ab[..., 0] = a_val
        oracle.gdn_block(qkv, lay.conv_w, conv, ab, lay.dt_bias, lay.ssm_a, S, z, lay.norm_w, nkh, nvh)
        S1 = S.copy()
        qkv2, ab2, z2 = lay.step()
        ab2[..., 0] = a_val
        ab2[..., 1] = -1e4  # beta = 0: the second step only decays
        oracle.gdn_block(qkv2, lay.conv_w, conv, ab2, lay.dt_bias, lay.ssm_a, S, z2, lay.norm_w, nkh, nvh)
        x = torch.tensor(float(ab2[0, 0, 0]) + float(lay.dt_bias[0]), dtype=torch.float64)
        gam = float(torch.exp(float(lay.ssm_a[0]) * torch.nn.functional.softplus(x)))
        assert np.allclose(S, gam * S1, rtol=1e-13, atol=1e-300)


# ---------------------------------------------------------------------------------------------------------------
# QSA indexer (faie2fn.cu:1480-1607)


def _ix_case(seed, B=2, nt=3, L=1024, pos=(700, 333)):
    rng = np.random.default_rng(seed)
    iqk = f32(rng.standard_normal((B, nt, 640)))
    wqn, wkn = f32(rng.normal(1, 0.1, 128)), f32(rng.normal(1, 0.1, 128))
    IK = np.zeros((B, L, 128), np.float32)
    pos = np.array(pos, np.int32)
    for b in range(B):
        IK[b, :pos[b]] = rng.standard_normal((pos[b], 128))
    return iqk, wqn, wkn, IK, pos


def test_twin_indexer():
    iqk, wqn, wkn, IK, pos = _ix_case(1)
    L = IK.shape[1]
    BK1, BK2 = np.zeros((2, L // 4, 128)), np.zeros((2, L // 4, 128))
    for b in range(2):
        oracle.ix_blocks(IK[b:b + 1], wkn, BK1[b:b + 1], 0, int(pos[b]) // 4)
    BK2[:] = BK1
    IK1, IK2 = IK.copy(), IK.copy()
    Q1 = oracle.ix_prep(iqk, wqn, wkn, IK1, BK1, pos)
    Q2 = twin.ix_prep(iqk, wqn, wkn, IK2, BK2, pos)
    assert oracle.relerr(Q1, Q2) < 1e-13 and np.array_equal(IK1, IK2) and oracle.relerr(BK1, BK2) < 1e-13
    s1 = oracle.ix_score(Q1, BK1, pos, L)
    s2 = twin.ix_score(Q2, BK2, pos, L)
    assert oracle.relerr(s1, s2) < 1e-13


def test_block_key_closed_form():
    """A block of four equal raw keys has that key's norm as its mean; block j is roped at position 4j."""
    rng = np.random.default_rng(5)
    IK = np.zeros((1, 256, 128), np.float32)
    x = f32(rng.standard_normal(128))
    IK[0, 40:44] = x
    w = f32(rng.normal(1, 0.1, 128))
    BK = np.zeros((1, 64, 128))
    oracle.ix_blocks(IK, w, BK, 10, 11)
    ref = twin._norm_rope(x, w, 40, 64, oracle.rope_inv_freq(64, 1e7), 1e-6)
    assert np.allclose(BK[0, 10], ref, atol=1e-14)


def test_selection_rule():
    """top-k by descending score; ties at the threshold keep the lowest index; queries with <= top complete blocks
    are dense (empty mask)."""
    rng = np.random.default_rng(6)
    nb = 300
    s = np.zeros((1, 2, 400))
    s[0, :, :nb] = rng.random(nb)
    m = oracle.ix_select(s, np.array([nb * 4 - 1]), top=50)
    order = np.lexsort((np.arange(nb), -s[0, 0, :nb]))  # independent: lexsort, index as the tie key
    assert set(np.nonzero(m[0, 0])[0]) == set(order[:50])
    s2 = np.zeros((1, 1, 400))
    s2[0, 0, :nb] = 0.5
    s2[0, 0, [7, 99]] = 1.0
    m2 = oracle.ix_select(s2, np.array([nb * 4 - 1]), top=5)
    assert sorted(np.nonzero(m2[0, 0])[0]) == [0, 1, 2, 7, 99]
    m3 = oracle.ix_select(s2, np.array([4 * 5 - 1]), top=5)  # nb = 5 <= top: dense
    assert not m3.any()


def test_masked_attention_reduces_to_dense():
    """All blocks kept == dense; nothing kept leaves exactly the incomplete tail block visible."""
    rng = np.random.default_rng(7)
    B, nq, nkv, hd = 1, 8, 2, 32
    qg = f32(rng.standard_normal((B, 1, nq, 2, hd)))
    kn, vn = f32(rng.standard_normal((B, 1, nkv, hd))), f32(rng.standard_normal((B, 1, nkv, hd)))
    w = np.ones(hd, np.float32)
    K, V = f32(rng.standard_normal((B, 256, nkv, hd))), f32(rng.standard_normal((B, 256, nkv, hd)))
    pos = np.array([205], np.int32)  # keys 0..205: 51 complete blocks (0..203) and the tail 204, 205
    dense = oracle.attn(qg, kn, vn, w, w, K, V, pos, nrot=8)[0]
    full = oracle.attn(qg, kn, vn, w, w, K, V, pos, nrot=8, mask=np.ones((1, 1, 64), np.uint8), top=4)[0]
    assert np.allclose(full, dense, atol=1e-15)
    few = oracle.attn(qg, kn, vn, w, w, K, V, pos, nrot=8, mask=np.zeros((1, 1, 64), np.uint8), top=100)[0]
    assert np.allclose(few, dense, atol=1e-15)  # nb = 51 <= top: dense whatever the mask says
    tail, kr, vr = oracle.attn(qg, kn, vn, w, w, K, V, pos, nrot=8, mask=np.zeros((1, 1, 64), np.uint8), top=4)
    inv = oracle.rope_inv_freq(8, 1e7)
    Q = twin._norm_rope(qg[0, 0, :, 0], w, 205, 8, inv, 1e-6)
    gate = 1 / (1 + np.exp(-qg[0, 0, :, 1].astype(np.float64)))
    for h in range(nq):
        g = h // 4
        keys = np.stack([K[0, 204, g].astype(np.float64), kr[0, 0, g]])
        vals = np.stack([V[0, 204, g].astype(np.float64), vr[0, 0, g]])
        sc = keys @ Q[h] / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        assert np.allclose(tail[0, 0, h], (p @ vals) / p.sum() * gate[h], atol=1e-14)


def _ix_dots_case(dots, ixd=128, nblk=3):
    """Qix [1][1][ixh][ixd], BKc [1][nblk][ixd] with q_h = a_h e_h and block key k_j = sum_h c_jh e_h, so that
    q_h . k_j = dots[j][h] exactly (one nonzero product per dot)."""
    dots = np.asarray(dots, np.float64)
    ixh = dots.shape[1]
    Q = np.zeros((1, 1, ixh, ixd))
    K = np.zeros((1, nblk, ixd))
    for h in range(ixh):
        Q[0, 0, h, h] = 2.0
    for j in range(dots.shape[0]):
        for h in range(ixh):
            K[0, j, h] = dots[j, h] / 2.0
    return Q, K


def test_ix_score_closed_forms():
    """orc_ix_score (k_ix_score, faie2fn.cu:1534-1555): score_j = sum_h relu(q_h . k_j) / sqrt(ixd), pinned by closed
    forms that each plausible misreading fails: one head positive and the rest negative gives that dot / sqrt(128);
    all heads negative give exactly 0; mixed signs give the sum of the positive dots only (relu of the summed dots
    would give their difference); the scale is 1/sqrt(128) (not 1/128 or 1); only the (pos + t + 1) / 4 complete
    blocks are scored."""
    dots = [[5.0, -1.0, -2.0, -3.0],      # one head positive
            [-1.0, -2.0, -0.5, -7.0],     # all negative
            [3.0, -2.0, 4.0, -6.0]]       # mixed: relu per head 7, relu of the sum 0
    Q, K = _ix_dots_case(dots, nblk=4)
    # pos 11, nt 1: (11 + 1) / 4 = 3 complete blocks; block 3 is left untouched
    sc = oracle.ix_score(Q, K, np.array([11]), max_ctx=16)
    r = np.sqrt(128.0)
    assert sc[0, 0, 0] == pytest.approx(5.0 / r, rel=1e-15)
    assert sc[0, 0, 1] == 0.0
    assert sc[0, 0, 2] == pytest.approx(7.0 / r, rel=1e-15)
    assert sc[0, 0, 3] == 0.0
    # a sequence one position shorter has one complete block fewer
    sc2 = oracle.ix_score(Q, K, np.array([10]), max_ctx=16)
    assert sc2[0, 0, 2] == 0.0 and sc2[0, 0, 0] == sc[0, 0, 0]


def test_ix_score_exact_brute_force():
    """Exact rational brute force at ixd = 4 (scale 1/2 exactly), 2 heads, 2 tokens, random small integers: the
    oracle's float64 scores equal sum_h max(0, q_h . k_j) / 2 computed in Fractions (integers make every float64
    product and sum exact)."""
    rng = np.random.default_rng(31)
    B, nt, ixh, ixd, ixr, max_ctx = 2, 2, 2, 4, 4, 32
    Q = rng.integers(-5, 6, size=(B, nt, ixh, ixd)).astype(np.float64)
    K = rng.integers(-5, 6, size=(B, max_ctx // ixr, ixd)).astype(np.float64)
    pos = np.array([9, 22])
    sc = oracle.ix_score(Q, K, pos, max_ctx, ixr)
    for b in range(B):
        for t in range(nt):
            nb = (pos[b] + t + 1) // ixr
            for j in range(max_ctx // ixr):
                want = Fraction(0)
                if j < nb:
                    for h in range(ixh):
                        p = sum(Fraction(int(Q[b, t, h, d])) * Fraction(int(K[b, j, d])) for d in range(ixd))
                        want += max(Fraction(0), p)
                    want /= 2
                assert Fraction(sc[b, t, j]) == want, (b, t, j)

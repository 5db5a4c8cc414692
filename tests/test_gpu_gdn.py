"""GPU parity of the DeltaNet kernels against the float64 oracle (per tensor per step, normwise <= 1e-5).

Every case prints what names it before the GPU call, so a failing run identifies itself.
"""

import numpy as np
import pytest

import fn_synth
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5  # max|gpu - ref| / max|ref| per tensor per step, the reference gate metric (gate_fn_ref.py:43)


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("B,head_map", [(1, 0), (3, 1)])
def test_core_config0_64_steps(fnlib, B, head_map):
    _say(f"gdn core config0 B={B} head_map={head_map} 64 steps")
    gen = fn_synth.CoreSteps(B=B, seed=0)
    S_gpu = gen.S0.copy()
    S_ref = gen.S0.astype(np.float64)
    for step in range(64):
        q, k, v, beta, g = gen.step()
        o_gpu = fnlib.gdn(q, k, v, beta, g, S_gpu, head_map=head_map)
        o_ref = oracle.gdn_core(q, k, v, beta, g, S_ref, head_map=head_map)
        eo, es = oracle.relerr(o_gpu, o_ref), oracle.relerr(S_gpu, S_ref)
        assert eo <= TOL and es <= TOL, (step, eo, es)


def test_core_multi_token_equals_steps(fnlib):
    """nt tokens in one call == nt calls of one token (state carried in registers across the token loop)."""
    _say("gdn core nt=5 vs 5 x nt=1")
    gen = fn_synth.CoreSteps(B=2, seed=5)
    steps = [gen.step() for _ in range(5)]
    cat = [np.concatenate([s[i] for s in steps], axis=1) for i in range(5)]
    S_a = gen.S0.copy()
    o_a = fnlib.gdn(*cat, S_a)
    S_ref = gen.S0.astype(np.float64)
    o_ref = oracle.gdn_core(*cat, S_ref)
    assert oracle.relerr(o_a, o_ref) <= TOL and oracle.relerr(S_a, S_ref) <= TOL


@pytest.mark.parametrize("gate_act,head_map", [(0, 0), (1, 0), (0, 1)])
def test_block_config1_steps(fnlib, gate_act, head_map):
    _say(f"gdn block config1 gate_act={gate_act} head_map={head_map} 48 steps")
    lay = fn_synth.BlockLayer(B=1, config=1, layer=3)
    S_gpu, S_ref = lay.S0.copy(), lay.S0.astype(np.float64)
    c_gpu, c_ref = lay.conv0.copy(), lay.conv0.astype(np.float64)
    for step in range(48):
        qkv, ab, z = lay.step()
        out = fnlib.gdn_block(qkv, lay.conv_w, c_gpu, ab, lay.dt_bias, lay.ssm_a, S_gpu, z, lay.norm_w, 16, 32,
                              head_map=head_map, gate_act=gate_act)
        ref = oracle.gdn_block(qkv, lay.conv_w, c_ref, ab, lay.dt_bias, lay.ssm_a, S_ref, z, lay.norm_w, 16, 32,
                               head_map=head_map, gate_act=gate_act)
        e = (oracle.relerr(out, ref), oracle.relerr(S_gpu, S_ref), oracle.relerr(c_gpu, c_ref))
        assert max(e) <= TOL, (step, e)


@pytest.mark.parametrize("nt", [2, 3, 5])
def test_block_multi_token(fnlib, nt):
    """nt tokens per call (taps inside the call from the qkv input, across calls from the conv ring)."""
    _say(f"gdn block nt={nt} x 3 calls, B=2")
    lay = fn_synth.BlockLayer(B=2, config=1, layer=7)
    S_gpu, S_ref = lay.S0.copy(), lay.S0.astype(np.float64)
    c_gpu, c_ref = lay.conv0.copy(), lay.conv0.astype(np.float64)
    for call in range(3):
        st = [lay.step() for _ in range(nt)]
        qkv, ab, z = (np.concatenate([s[i] for s in st], axis=1) for i in range(3))
        out = fnlib.gdn_block(qkv, lay.conv_w, c_gpu, ab, lay.dt_bias, lay.ssm_a, S_gpu, z, lay.norm_w, 16, 32)
        ref = oracle.gdn_block(qkv, lay.conv_w, c_ref, ab, lay.dt_bias, lay.ssm_a, S_ref, z, lay.norm_w, 16, 32)
        e = (oracle.relerr(out, ref), oracle.relerr(S_gpu, S_ref), oracle.relerr(c_gpu, c_ref))
        assert max(e) <= TOL, (call, e)


@pytest.mark.parametrize("nt,head_map", [(2, 0), (4, 1), (7, 0)])
def test_block_multi_token_bitwise_equals_steps(fnlib, nt, head_map):
    """One call of nt tokens (the multi-token kernel, 256 threads per head) reproduces nt one-token calls (the
    decode kernel, 512 threads per head) bit for bit: outputs, state and conv state."""
    _say(f"gdn block nt={nt} head_map={head_map} vs {nt} x nt=1, bitwise, B=3")
    lay = fn_synth.BlockLayer(B=3, config=1, layer=11)
    st = [lay.step() for _ in range(nt)]
    qkv, ab, z = (np.concatenate([s[i] for s in st], axis=1) for i in range(3))
    S_a, c_a = lay.S0.copy(), lay.conv0.copy()
    out_a = fnlib.gdn_block(qkv, lay.conv_w, c_a, ab, lay.dt_bias, lay.ssm_a, S_a, z, lay.norm_w, 16, 32,
                            head_map=head_map)
    S_b, c_b = lay.S0.copy(), lay.conv0.copy()
    out_b = np.concatenate([fnlib.gdn_block(s[0], lay.conv_w, c_b, s[1], lay.dt_bias, lay.ssm_a, S_b, s[2],
                                            lay.norm_w, 16, 32, head_map=head_map) for s in st], axis=1)
    assert out_a.shape == out_b.shape
    assert np.array_equal(out_a, out_b), np.abs(out_a - out_b).max()
    assert np.array_equal(S_a, S_b), np.abs(S_a - S_b).max()
    assert np.array_equal(c_a, c_b)


def test_block_device_ring_advances(fnlib):
    """Device entry point with the conv ring and a device position advanced by fn_advance_dev: 12 decode steps of
    B=3 sequences at different starting positions, checked against the oracle every step."""
    import hiprt

    _say("gdn block device ring, B=3, 12 steps")
    lay = fn_synth.BlockLayer(B=3, config=1, layer=11)
    B, C, nvh = 3, lay.C, 32
    ring = 4
    start = np.array([0, 5, 130], np.int32)
    pos = hiprt.Buf.like(start)
    # conv history of each sequence at its start position: random raw inputs in ring slots p-3..p-1
    rng = np.random.default_rng(99)
    hist = rng.standard_normal((B, 3, C)).astype(np.float32)
    ring_h = np.zeros((B, ring, C), np.float32)
    for b in range(B):
        for j in range(3):
            ring_h[b, (int(start[b]) - 3 + j) & (ring - 1)] = hist[b, j]
    d_ring, d_S = hiprt.Buf.like(ring_h), hiprt.Buf.like(lay.S0)
    d_w, d_dt, d_sa, d_nw = (hiprt.Buf.like(x) for x in (lay.conv_w, lay.dt_bias, lay.ssm_a, lay.norm_w))
    out = hiprt.Buf.empty((B, 1, nvh * 128))
    d_qkv, d_ab, d_z = hiprt.Buf.empty((B, 1, C)), hiprt.Buf.empty((B, 1, 2 * nvh)), hiprt.Buf.empty((B, 1, nvh * 128))
    S_ref, c_ref = lay.S0.astype(np.float64), hist.astype(np.float64)
    for step in range(12):
        qkv, ab, z = lay.step()
        d_qkv.upload(qkv), d_ab.upload(ab), d_z.upload(z)
        fnlib.gdn_block_dev(B, 16, nvh, 1, ring, pos.ptr, d_qkv.ptr, d_w.ptr, d_ring.ptr, d_ab.ptr, d_dt.ptr,
                            d_sa.ptr, d_S.ptr, d_z.ptr, d_nw.ptr, out.ptr, None)
        fnlib.advance_dev(pos.ptr, B, 1, None)
        hiprt.sync()
        ref = oracle.gdn_block(qkv, lay.conv_w, c_ref, ab, lay.dt_bias, lay.ssm_a, S_ref, z, lay.norm_w, 16, 32)
        e = (oracle.relerr(out.download(), ref), oracle.relerr(d_S.download(), S_ref))
        assert max(e) <= TOL, (step, e)
    assert pos.download().tolist() == (start + 12).tolist()
    # the ring now holds the last three raw inputs at their positions
    rh = d_ring.download()
    for b in range(B):
        p = int(start[b]) + 12
        got = np.stack([rh[b, (p - 3 + j) & (ring - 1)] for j in range(3)])
        assert np.array_equal(got, c_ref[b].astype(np.float32))


def test_block_batch64_subset(fnlib):
    """Config 2 shape (B = 64): batch entries are independent, so the oracle runs a subset of sequences."""
    _say("gdn block B=64, 4 steps, oracle on sequences 0, 31, 63")
    lay = fn_synth.BlockLayer(B=64, config=2, layer=0)
    pick = [0, 31, 63]
    S_gpu = lay.S0.copy()
    S_ref = lay.S0[pick].astype(np.float64)
    c_gpu = lay.conv0.copy()
    c_ref = lay.conv0[pick].astype(np.float64)
    for step in range(4):
        qkv, ab, z = lay.step()
        out = fnlib.gdn_block(qkv, lay.conv_w, c_gpu, ab, lay.dt_bias, lay.ssm_a, S_gpu, z, lay.norm_w, 16, 32)
        ref = oracle.gdn_block(qkv[pick], lay.conv_w, c_ref, ab[pick], lay.dt_bias, lay.ssm_a, S_ref, z[pick],
                               lay.norm_w, 16, 32)
        e = (oracle.relerr(out[pick], ref), oracle.relerr(S_gpu[pick], S_ref), oracle.relerr(c_gpu[pick], c_ref))
        assert max(e) <= TOL, (step, e)


def _bf16(a):
    """float32 -> BF16 bits, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16_f64(r):
    return (r.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("B,hidden,head_map,gate_act", [(3, 2048, 0, 0), (2, 4, 0, 0), (2, 2052, 0, 0), (2, 6144, 0, 0),
                                                       (64, 2048, 0, 0), (3, 2048, 1, 1)])
def test_block_xab_device(fnlib, B, hidden, head_map, gate_act):
    """fn_gdn_block_xab_dev (alpha/beta projection fused into the block): 5 decode steps, each against the oracle
    fed ab = w_ab . x in float64 over the same BF16 weights; hidden sizes one thread's share (4), not a multiple of
    the workgroup's stride (2052) and three strides (6144); B = 64 with the oracle on a subset; the grouped head map
    with the SiLU gate."""
    import hiprt

    _say(f"gdn block with fused alpha/beta projection, B={B}, hidden={hidden}, head_map={head_map}, "
         f"gate_act={gate_act}, 5 steps")
    nvh, ring = 32, 4
    lay = fn_synth.BlockLayer(B=B, config=1, layer=7)
    C = lay.C
    rng = np.random.default_rng(hidden + B)
    wab = _bf16(rng.normal(0.0, 1.0 / np.sqrt(hidden), (2 * nvh, hidden)))
    wab64 = _bf16_f64(wab)
    pick = list(range(B)) if B <= 4 else [0, 31, 63]
    pos = hiprt.Buf.like(np.zeros(B, np.int32))
    d_ring, d_S = hiprt.Buf.like(np.zeros((B, ring, C), np.float32)), hiprt.Buf.like(lay.S0)
    d_w, d_dt, d_sa, d_nw = (hiprt.Buf.like(x) for x in (lay.conv_w, lay.dt_bias, lay.ssm_a, lay.norm_w))
    d_wab = hiprt.Buf.like(wab)
    d_x, d_qkv, d_z = hiprt.Buf.empty((B, hidden)), hiprt.Buf.empty((B, 1, C)), hiprt.Buf.empty((B, 1, nvh * 128))
    out = hiprt.Buf.empty((B, 1, nvh * 128))
    S_ref = lay.S0[pick].astype(np.float64)
    c_ref = np.zeros((len(pick), 3, C))
    for step in range(5):
        qkv, _, z = lay.step()
        x = rng.standard_normal((B, hidden)).astype(np.float32)
        d_qkv.upload(qkv), d_z.upload(z), d_x.upload(x)
        fnlib.gdn_block_xab_dev(B, 16, nvh, ring, pos.ptr, d_qkv.ptr, d_w.ptr, d_ring.ptr, d_x.ptr, hidden, d_wab.ptr,
                                d_dt.ptr, d_sa.ptr, d_S.ptr, d_z.ptr, d_nw.ptr, out.ptr, None, head_map=head_map,
                                gate_act=gate_act)
        fnlib.advance_dev(pos.ptr, B, 1, None)
        hiprt.sync()
        ab = (x[pick].astype(np.float64) @ wab64.T)[:, None, :]
        ref = oracle.gdn_block(qkv[pick], lay.conv_w, c_ref, ab, lay.dt_bias, lay.ssm_a, S_ref, z[pick], lay.norm_w,
                               16, 32, head_map=head_map, gate_act=gate_act)
        e = (oracle.relerr(out.download()[pick], ref), oracle.relerr(d_S.download()[pick], S_ref))
        assert max(e) <= TOL, (step, e)
    for bf in (pos, d_ring, d_S, d_w, d_dt, d_sa, d_nw, d_wab, d_x, d_qkv, d_z, out):
        bf.free()

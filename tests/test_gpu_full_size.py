"""GPU parity at the benchmark configurations' own workloads (not reduced copies of them), through the device entry
points and the path engine, against the float64 oracle per tensor per step (normwise <= 1e-5).

* config 1: one fused DeltaNet layer at B = 1 over all 512 decode steps, with the sigmoid and the SiLU output gate;
* config 2: the B = 64 layer over all 128 steps, the oracle on three sequences (sequences are independent);
* config 4: the 48-layer hybrid engine (36 DeltaNet + 12 attention layers) at B = 16 with 32768 keys of context
  and at B = 64 with 4096 keys for three decode steps, and at B = 16 with 4096 keys for config 4's 256 steps, each
  run ending exactly at the cache's end, every layer checked every step on the first, (a middle) and the last
  sequence.

Config 3's sizes are in test_gpu_attn.py (test_attn_full_size_device).  Every case prints what names it.
"""

import numpy as np
import pytest

import fn
import fn_synth
import hiprt
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
NKH, NVH, DK, NQ, NKV, HD = 16, 32, 128, 16, 2, 256
SB = NVH * DK * DK * 4  # bytes of one sequence's DeltaNet state


def _say(*a):
    print(*a, flush=True)


class DevLayer:
    """One DeltaNet layer's device buffers (B sequences, one-token decode, conv ring of 4)."""

    def __init__(self, lay, start=0):
        B, C = lay.B, lay.C
        self.lay, self.B, self.C = lay, B, C
        self.S = hiprt.Buf.like(lay.S0)
        self.ring = hiprt.Buf.like(np.zeros((B, 4, C), np.float32))
        self.pos = hiprt.Buf.like(np.full(B, start, np.int32))
        self.w, self.dt, self.sa, self.nw = (hiprt.Buf.like(x) for x in (lay.conv_w, lay.dt_bias, lay.ssm_a,
                                                                          lay.norm_w))
        self.qkv, self.ab, self.z = (hiprt.Buf.empty(s) for s in ((B, 1, C), (B, 1, 2 * NVH), (B, 1, NVH * DK)))
        self.out = hiprt.Buf.empty((B, 1, NVH * DK))

    def step(self, fnlib, qkv, ab, z, gate_act=0):
        self.qkv.upload(qkv), self.ab.upload(ab), self.z.upload(z)
        fnlib.gdn_block_dev(self.B, NKH, NVH, 1, 4, self.pos.ptr, self.qkv.ptr, self.w.ptr, self.ring.ptr, self.ab.ptr,
                            self.dt.ptr, self.sa.ptr, self.S.ptr, self.z.ptr, self.nw.ptr, self.out.ptr, None,
                            gate_act=gate_act)
        fnlib.advance_dev(self.pos.ptr, self.B, 1, None)
        hiprt.sync()

    def seq_state(self, b):
        return hiprt.dtoh(self.S.ptr + b * SB, (NVH, DK, DK))

    def free(self):
        for x in (self.S, self.ring, self.pos, self.w, self.dt, self.sa, self.nw, self.qkv, self.ab, self.z, self.out):
            x.free()


def _ring_taps(ring_seq, p):
    """[3][C] raw inputs of positions p-3..p-1 from one sequence's ring [4][C]."""
    return np.stack([ring_seq[(p - 3 + j) & 3] for j in range(3)])


@pytest.mark.parametrize("gate_act", [0, 1])
def test_config1_layer_512_steps(fnlib, gate_act):
    """Config 1's decode length: one layer, B = 1, 512 steps on the device path, out, S and the conv taps against
    the oracle after every step (errors do not accumulate past the bar over the whole run)."""
    _say(f"full size: config 1 layer 0, B=1, 512 steps, gate_act={gate_act}")
    lay = fn_synth.BlockLayer(B=1, config=1, layer=0)
    d = DevLayer(lay)
    S_ref, c_ref = lay.S0.astype(np.float64), lay.conv0.astype(np.float64)
    worst = 0.0
    try:
        for step in range(512):
            qkv, ab, z = lay.step()
            d.step(fnlib, qkv, ab, z, gate_act)
            ref = oracle.gdn_block(qkv, lay.conv_w, c_ref, ab, lay.dt_bias, lay.ssm_a, S_ref, z, lay.norm_w, NKH, NVH,
                                   gate_act=gate_act)
            e = (oracle.relerr(d.out.download(), ref), oracle.relerr(d.S.download(), S_ref),
                 oracle.relerr(_ring_taps(d.ring.download()[0], step + 1), c_ref[0]))
            worst = max(worst, *e)
            assert max(e) <= TOL, (step, e)
            if step % 128 == 127:
                _say(f"  step {step + 1}: worst rel err so far {worst:.3e}")
    finally:
        d.free()


def test_config2_128_steps_subset(fnlib):
    """Config 2's workload: B = 64 sequences, all 128 steps, one launch per step over the whole batch; the oracle
    follows sequences 0, 31 and 63 (out, S and conv taps every step)."""
    _say("full size: config 2 layer 0, B=64, 128 steps, oracle on sequences 0, 31, 63")
    lay = fn_synth.BlockLayer(B=64, config=2, layer=0)
    pick = [0, 31, 63]
    d = DevLayer(lay)
    S_ref = lay.S0[pick].astype(np.float64)
    c_ref = lay.conv0[pick].astype(np.float64)
    worst = 0.0
    try:
        for step in range(128):
            qkv, ab, z = lay.step()
            d.step(fnlib, qkv, ab, z)
            ref = oracle.gdn_block(qkv[pick], lay.conv_w, c_ref, ab[pick], lay.dt_bias, lay.ssm_a, S_ref, z[pick],
                                   lay.norm_w, NKH, NVH)
            out = d.out.download()
            ring = d.ring.download()
            e = [oracle.relerr(out[pick], ref)]
            for i, b in enumerate(pick):
                e.append(oracle.relerr(d.seq_state(b), S_ref[i]))
                e.append(oracle.relerr(_ring_taps(ring[b], step + 1), c_ref[i]))
            worst = max(worst, *e)
            assert max(e) <= TOL, (step, e)
            if step % 32 == 31:
                _say(f"  step {step + 1}: worst rel err so far {worst:.3e}")
    finally:
        d.free()


def _k_row(K, b, g, p, max_ctx):
    """Row p of kv head g of sequence b from the key-tiled device K [B][nkv][max_ctx/64][hd/4][64][4]."""
    tile = (b * NKV + g) * (max_ctx // 64) + p // 64
    t = hiprt.dtoh(K + tile * 64 * HD * 4, (HD // 4, 64, 4))
    return t[:, p % 64, :].reshape(HD)


@pytest.mark.parametrize("B, L, pick, steps", [(16, 32768, [0, 15], 3), (64, 4096, [0, 31, 63], 3),
                                               (16, 4096, [0, 15], 256)])
def test_config4_hybrid_engine_full_context(fnlib, B, L, pick, steps):
    """Config 4 as the engine runs it: 48 layers in the reference's hybrid order, decode steps that end at the last
    row of the cache (caches filled in HBM): B = 16 with 32768 keys of context for 3 steps, the north star's batch of
    64 with 4096 keys for 3 steps, and config 4's 256 steps at B = 16 with 4096 keys (the attention oracle's cost at
    32K would make that run minutes long).  Every layer is checked every step on the picked sequences (first, middle,
    last): DeltaNet out, S and conv taps; attention og and the appended K/V rows."""
    nl = 48
    pos0 = L - steps
    _say(f"full size: config 4 engine, B={B}, {nl} layers, context {L}, {steps} steps, oracle on sequences {pick}")
    rng = np.random.default_rng(4004)
    fnlib.path_init(B, nl, attn_every=4, max_ctx=L)
    try:
        hiprt.htod(fnlib.path_buffer(0, "POS")[0], np.full(B, pos0, np.int32))
        ref = []
        for il in range(nl):
            if (il + 1) % 4:
                lay = fn_synth.BlockLayer(B=1, config=1, layer=il)
                for kind, arr in (("CONV_W", lay.conv_w), ("DT_BIAS", lay.dt_bias), ("SSM_A", lay.ssm_a),
                                  ("NORM_W", lay.norm_w)):
                    hiprt.htod(fnlib.path_buffer(il, kind)[0], arr)
                S_p, S_n = fnlib.path_buffer(il, "S")
                fnlib.fill_normal_dev(S_p, S_n // 4, 7000 + il, 0.0, 0.02)
                R_p, R_n = fnlib.path_buffer(il, "CONV_RING")
                fnlib.fill_normal_dev(R_p, R_n // 4, 8000 + il)
                hiprt.sync()
                C = lay.C
                ring = hiprt.dtoh(R_p, (B, 4, C))
                ref.append(dict(kind="gdn", lay=lay, C=C,
                                S=np.stack([hiprt.dtoh(S_p + b * SB, (NVH, DK, DK)) for b in pick]).astype(np.float64),
                                conv=np.stack([_ring_taps(ring[b], pos0) for b in pick]).astype(np.float64)))
            else:
                K_p, K_n = fnlib.path_buffer(il, "KC")
                V_p, V_n = fnlib.path_buffer(il, "VC")
                fnlib.fill_normal_dev(K_p, K_n // 4, 9000 + il)
                fnlib.fill_normal_dev(V_p, V_n // 4, 9500 + il)
                wq = rng.normal(1, 0.1, HD).astype(np.float32)
                wk = rng.normal(1, 0.1, HD).astype(np.float32)
                hiprt.htod(fnlib.path_buffer(il, "WQ")[0], wq)
                hiprt.htod(fnlib.path_buffer(il, "WK")[0], wk)
                hiprt.sync()
                per = K_n // 4 // B
                KV = []
                for b in pick:
                    Kd = hiprt.dtoh(K_p + b * per * 4, (per,))
                    Vd = hiprt.dtoh(V_p + b * per * 4, (per,))
                    KV.append(fn.kv_from_device(Kd, Vd, 1, L, NKV, HD))
                ref.append(dict(kind="attn", wq=wq, wk=wk, KV=KV, K_p=K_p, V_p=V_p))
            if il % 8 == 7:
                _say(f"  layers 0..{il} filled")
        worst = 0.0
        for step in range(steps):
            P = pos0 + step
            inputs = []
            for il in range(nl):
                R = ref[il]
                if R["kind"] == "gdn":
                    x = (rng.standard_normal((B, 1, R["C"])).astype(np.float32),
                         rng.standard_normal((B, 1, 2 * NVH)).astype(np.float32),
                         rng.standard_normal((B, 1, NVH * DK)).astype(np.float32))
                    for kind, arr in zip(("QKV", "AB", "Z"), x):
                        hiprt.htod(fnlib.path_buffer(il, kind)[0], arr)
                else:
                    x = (rng.standard_normal((B, 1, NQ, 2, HD)).astype(np.float32),
                         rng.standard_normal((B, 1, NKV, HD)).astype(np.float32),
                         rng.standard_normal((B, 1, NKV, HD)).astype(np.float32))
                    for kind, arr in zip(("QG", "K", "V"), x):
                        hiprt.htod(fnlib.path_buffer(il, kind)[0], arr)
                inputs.append(x)
            fnlib.path_step(1)
            for il in range(nl):
                R, x = ref[il], inputs[il]
                if R["kind"] == "gdn":
                    lay = R["lay"]
                    want = oracle.gdn_block(x[0][pick], lay.conv_w, R["conv"], x[1][pick], lay.dt_bias, lay.ssm_a,
                                            R["S"], x[2][pick], lay.norm_w, NKH, NVH)
                    out = hiprt.dtoh(fnlib.path_buffer(il, "OUT")[0], (B, 1, NVH * DK))
                    S_p = fnlib.path_buffer(il, "S")[0]
                    ring = hiprt.dtoh(fnlib.path_buffer(il, "CONV_RING")[0], (B, 4, R["C"]))
                    e = [oracle.relerr(out[pick], want)]
                    for i, b in enumerate(pick):
                        e.append(oracle.relerr(hiprt.dtoh(S_p + b * SB, (NVH, DK, DK)), R["S"][i]))
                        e.append(oracle.relerr(_ring_taps(ring[b], P + 1), R["conv"][i]))
                else:
                    og = hiprt.dtoh(fnlib.path_buffer(il, "OG")[0], (B, 1, NQ, HD))
                    e = []
                    for i, b in enumerate(pick):
                        Kr, Vr = R["KV"][i]
                        pos = np.array([P], np.int32)
                        want, wk_, wv_ = oracle.attn(x[0][b:b + 1], x[1][b:b + 1], x[2][b:b + 1], R["wq"], R["wk"],
                                                     Kr, Vr, pos)
                        e.append(oracle.relerr(og[b:b + 1], want))
                        for g in range(NKV):
                            e.append(oracle.relerr(_k_row(R["K_p"], b, g, P, L), wk_[0, 0, g]))
                            vrow = hiprt.dtoh(R["V_p"] + (((b * NKV + g) * L + P) * HD) * 4, (HD,))
                            e.append(oracle.relerr(vrow, wv_[0, 0, g]))
                        # the oracle's own cache grows by the rows it computed (the next step attends them)
                        Kr[0, P] = wk_[0, 0].astype(np.float32)
                        Vr[0, P] = wv_[0, 0].astype(np.float32)
                worst = max(worst, *e)
                assert max(e) <= TOL, (step, il, R["kind"], e)
            if steps <= 8 or step % 32 == 31:
                _say(f"  step {step + 1}: all {nl} layers within {worst:.3e}")
        assert list(hiprt.dtoh(fnlib.path_buffer(0, "POS")[0], (B,), np.int32)) == [L] * B
        with pytest.raises(RuntimeError, match="context full"):
            fnlib.path_step(1)
    finally:
        fnlib.free()

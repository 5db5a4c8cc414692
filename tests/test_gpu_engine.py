"""GPU tests of the path engine: the hybrid layer schedule (attention iff (il + 1) % 4 == 0) decoded step by step
through engine-owned state, checked against the float64 oracle per layer per step, and graph replay == eager."""

import numpy as np
import pytest

import fn
import fn_synth
import hiprt
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(*a):
    print(*a, flush=True)


class Hybrid:
    """Host-side mirror of a small hybrid stack: parameters, initial state, and the oracle state per layer."""

    def __init__(self, B, nl, max_ctx, pos0, seed=7):
        self.B, self.nl, self.max_ctx = B, nl, max_ctx
        self.pos = np.array(pos0, np.int32)
        rng = np.random.default_rng(seed)
        self.layers = []
        for il in range(nl):
            if (il + 1) % 4:
                lay = fn_synth.BlockLayer(B=B, config=1, layer=il, seed=seed * 100 + il)
                self.layers.append(dict(kind="gdn", lay=lay, S=lay.S0.astype(np.float64), conv=lay.conv0.astype(np.float64)))
            else:
                K = np.zeros((B, max_ctx, 2, 256), np.float32)
                V = np.zeros((B, max_ctx, 2, 256), np.float32)
                for b in range(B):
                    K[b, : self.pos[b]] = rng.standard_normal((self.pos[b], 2, 256))
                    V[b, : self.pos[b]] = rng.standard_normal((self.pos[b], 2, 256))
                self.layers.append(dict(kind="attn", K=K, V=V, wq=rng.normal(1, 0.1, 256).astype(np.float32),
                                        wk=rng.normal(1, 0.1, 256).astype(np.float32), rng=rng))

    def load(self, lib):
        """Initial state and parameters into the engine."""
        for il, L in enumerate(self.layers):
            if L["kind"] == "gdn":
                lay = L["lay"]
                for kind, arr in (("S", lay.S0), ("CONV_W", lay.conv_w), ("DT_BIAS", lay.dt_bias), ("SSM_A", lay.ssm_a),
                                  ("NORM_W", lay.norm_w)):
                    hiprt.htod(lib.path_buffer(il, kind)[0], arr)
            else:
                Kd, Vd = fn.kv_to_device(L["K"], L["V"])
                hiprt.htod(lib.path_buffer(il, "KC")[0], Kd)
                hiprt.htod(lib.path_buffer(il, "VC")[0], Vd)
                hiprt.htod(lib.path_buffer(il, "WQ")[0], L["wq"])
                hiprt.htod(lib.path_buffer(il, "WK")[0], L["wk"])
        hiprt.htod(lib.path_buffer(0, "POS")[0], self.pos)

    def inputs(self, step):
        """Per-layer inputs of one step (deterministic in step)."""
        out = []
        for il, L in enumerate(self.layers):
            rng = np.random.default_rng(1000 * step + il)
            if L["kind"] == "gdn":
                C = L["lay"].C
                out.append(dict(qkv=rng.standard_normal((self.B, 1, C)).astype(np.float32),
                                ab=rng.standard_normal((self.B, 1, 64)).astype(np.float32),
                                z=rng.standard_normal((self.B, 1, 4096)).astype(np.float32)))
            else:
                out.append(dict(qg=rng.standard_normal((self.B, 1, 16, 2, 256)).astype(np.float32),
                                k=rng.standard_normal((self.B, 1, 2, 256)).astype(np.float32),
                                v=rng.standard_normal((self.B, 1, 2, 256)).astype(np.float32)))
        return out


def _upload_inputs(lib, H, ins):
    for il, x in enumerate(ins):
        for name, arr in x.items():
            hiprt.htod(lib.path_buffer(il, name.upper())[0], arr)


def _outputs(lib, H):
    res = []
    for il, L in enumerate(H.layers):
        if L["kind"] == "gdn":
            p, n = lib.path_buffer(il, "OUT")
            res.append(hiprt.dtoh(p, (H.B, 1, 4096)))
        else:
            p, n = lib.path_buffer(il, "OG")
            res.append(hiprt.dtoh(p, (H.B, 1, 16, 256)))
    return res


def test_hybrid_engine_against_oracle(fnlib):
    B, nl, max_ctx, steps = 2, 8, 320, 4
    _say(f"engine hybrid B={B} nl={nl} max_ctx={max_ctx} {steps} steps vs oracle")
    H = Hybrid(B, nl, max_ctx, pos0=[100, 37])
    fnlib.path_init(B, nl, attn_every=4, max_ctx=max_ctx)
    try:
        assert fnlib.d.fn_dev_gb(0) > 0 and fnlib.d.fn_n_past() == 0
        H.load(fnlib)
        pos = H.pos.copy()
        for step in range(steps):
            ins = H.inputs(step)
            _upload_inputs(fnlib, H, ins)
            fnlib.path_step(1)
            outs = _outputs(fnlib, H)
            for il, (L, x, got) in enumerate(zip(H.layers, ins, outs)):
                if L["kind"] == "gdn":
                    lay = L["lay"]
                    ref = oracle.gdn_block(x["qkv"], lay.conv_w, L["conv"], x["ab"], lay.dt_bias, lay.ssm_a, L["S"],
                                           x["z"], lay.norm_w, 16, 32)
                    e = oracle.relerr(got, ref)
                else:
                    og, kr, vr = oracle.attn(x["qg"], x["k"], x["v"], L["wq"], L["wk"], L["K"], L["V"], pos)
                    for b in range(B):  # the oracle's cache grows like the engine's
                        L["K"][b, pos[b]] = kr[b, 0].astype(np.float32)
                        L["V"][b, pos[b]] = vr[b, 0].astype(np.float32)
                    e = oracle.relerr(got, og)
                assert e <= TOL, (step, il, L["kind"], e)
            pos += 1
        assert fnlib.d.fn_n_past() == steps
        assert hiprt.dtoh(fnlib.path_buffer(0, "POS")[0], (B,), np.int32).tolist() == pos.tolist()
        # DeltaNet state after the steps
        for il, L in enumerate(H.layers):
            if L["kind"] == "gdn":
                S = hiprt.dtoh(fnlib.path_buffer(il, "S")[0], L["S"].shape)
                assert oracle.relerr(S, L["S"]) <= TOL, il
        # fn_reset zeroes state and positions
        fnlib.reset()
        assert fnlib.d.fn_n_past() == 0
        assert not hiprt.dtoh(fnlib.path_buffer(0, "POS")[0], (B,), np.int32).any()
        assert not hiprt.dtoh(fnlib.path_buffer(0, "S")[0], (B, 32, 128, 128)).any()
    finally:
        fnlib.free()


def test_graph_replay_equals_eager(fnlib):
    """The captured step and the eagerly launched step give the same bits, over several replays with eager work
    and synchronisation between them."""
    B, nl, max_ctx, steps = 2, 4, 192, 3
    _say("engine graph vs eager")
    res = {}
    for graphs in (True, False):
        H = Hybrid(B, nl, max_ctx, pos0=[60, 129], seed=11)
        fnlib.path_init(B, nl, attn_every=4, max_ctx=max_ctx)
        try:
            fnlib.use_graphs(graphs)
            H.load(fnlib)
            outs = []
            for step in range(steps):
                _upload_inputs(fnlib, H, H.inputs(step))
                fnlib.path_step(1)
                outs.append(_outputs(fnlib, H))
            res[graphs] = outs
        finally:
            fnlib.free()
    for a, b in zip(res[True], res[False]):
        for x, y in zip(a, b):
            assert np.array_equal(x, y)


def test_engine_errors(fnlib):
    fnlib.path_init(1, 4, attn_every=4, max_ctx=128)
    try:
        with pytest.raises(RuntimeError, match="no such buffer"):
            fnlib.path_buffer(0, "KC")
        with pytest.raises(RuntimeError, match="out of range"):
            fnlib.path_buffer(4, "S")
    finally:
        fnlib.free()
    with pytest.raises(RuntimeError, match="not loaded"):
        fnlib.path_step(1)


def test_engine_context_full(fnlib):
    """Stepping a sequence past the attention cache fails before anything runs ("context full", the reference's
    forward check, faie2fn.cu:2468): a step that fits runs, the next one is refused, and so is a multi-step call that
    would cross the end; the positions are left as they were."""
    _say("engine context full")
    fnlib.path_init(2, 4, attn_every=4, max_ctx=64)
    try:
        pos = fnlib.path_buffer(0, "POS")[0]
        hiprt.htod(pos, np.array([10, 63], np.int32))
        fnlib.path_step(1)                       # the token at position 63 takes the last row of the cache
        with pytest.raises(RuntimeError, match="context full"):
            fnlib.path_step(1)
        assert list(hiprt.dtoh(pos, (2,), np.int32)) == [11, 64]
        hiprt.htod(pos, np.array([10, 61], np.int32))
        with pytest.raises(RuntimeError, match="context full"):
            fnlib.path_step(4)                   # 61 + 4 > 64
        fnlib.path_step(3)                       # 61 + 3 = 64 fits
        assert list(hiprt.dtoh(pos, (2,), np.int32)) == [13, 64]
        hiprt.htod(pos, np.array([-1, 0], np.int32))
        with pytest.raises(RuntimeError, match="negative position"):
            fnlib.path_step(1)
        assert fnlib.dev_status() == 0
    finally:
        fnlib.free()

"""GPU parity of the whole model: fn_load of a synthetic GGUF with the reference model's structure (tensor names,
metadata, weight formats; small dimensions), then fn_forward over a token sequence against the float64 model oracle
(oracle/model.py): logits of every call and the residual streams after every layer (fn_debug_layers) within 1e-5
normwise, the argmax token equal wherever the oracle's top two logits are apart.

The sequence runs past the indexer's threshold (top 8 blocks of 4 keys), so the attention layer switches from dense
to sparse inside it; calls take 1 to 8 tokens.  Layer 1 carries the per-layer n-gram embedding (as in the reference
model), and the sequence holds EOS tokens, which cut the n-gram contexts.  Every case prints what names it before
the GPU calls.
"""

import numpy as np
import pytest

import model_synth as ms
import oracle.model as om

pytestmark = pytest.mark.gpu

TOL = 1e-5
CHUNKS = [1, 3, 8, 2, 8, 8, 5, 8, 8, 7, 1, 8, 8, 4]   # 79 tokens


def _say(*a):
    print(*a, flush=True)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "tiny.gguf")
    kv, ts = ms.write_model(path, ms.TINY_DIMS, seed=11)
    return path, kv, ts


def _run(fnlib, ref, ids, debug):
    """fn_forward over ids in CHUNKS, checked against the oracle after every call; returns the GPU logits."""
    outs = []
    i = 0
    worst = [0.0, 0.0]
    NL, HCD = ref.NL, ref.HC * ref.D
    for c, nt in enumerate(CHUNKS):
        tok = ids[i:i + nt]
        i += nt
        buf = np.zeros((NL, nt, HCD), np.float32) if debug else None
        fnlib.debug_layers(buf)
        am, lg = fnlib.forward(tok, logits=True)
        want, want_am, hs, _ = ref.forward(tok)
        e = _rel(lg, want)
        worst[0] = max(worst[0], e)
        assert e <= TOL, (c, nt, e)
        if debug:
            for il in range(NL):
                eh = _rel(buf[il], hs[il])
                worst[1] = max(worst[1], eh)
                assert eh <= TOL, (c, il, eh)
        for t in range(nt):
            top2 = np.sort(want[t])[-2:]
            if top2[1] - top2[0] > 1e-4 * abs(top2[1]):
                assert am[t] == want_am[t], (c, t)
        outs.append(lg)
    fnlib.debug_layers(None)
    _say(f"  worst normwise error: logits {worst[0]:.3e}, residual streams {worst[1]:.3e}")
    return np.concatenate(outs)


def test_model_forward_matches_oracle(fnlib, model_file):
    path, kv, ts = model_file
    _say(f"model forward: tiny synthetic model, {sum(CHUNKS)} tokens in calls of {CHUNKS}, per-layer debug")
    fnlib.load(path, "", max_ctx=256)
    try:
        assert fnlib.d.fn_split() == ms.TINY_DIMS["NL"] and fnlib.d.fn_dev_gb(0) > 0
        ref = om.Model(kv, ts, max_ctx=256)
        ids = np.random.default_rng(2).integers(0, ms.TINY_DIMS["VOCAB"], size=sum(CHUNKS))
        ids[[0, 9, 10, 33, 60]] = ms.TINY_DIMS["ple_eos"]
        _run(fnlib, ref, ids, debug=True)
        assert fnlib.d.fn_n_past() == sum(CHUNKS)
    finally:
        fnlib.free()


def test_model_graphs_equal_eager_and_reset(fnlib, model_file):
    """The same tokens through captured graphs and eagerly give the same bits; fn_reset returns the model to its
    first state (DeltaNet state, conv rings and the position; the caches are overwritten from position 0)."""
    path, kv, ts = model_file
    _say("model forward: graphs vs eager, reset")
    fnlib.load(path, "", max_ctx=256)
    try:
        ids = np.random.default_rng(4).integers(0, ms.TINY_DIMS["VOCAB"], size=20)
        res = []
        for graphs in (True, False, True):
            fnlib.d.fn_use_graphs(1 if graphs else 0)
            fnlib.reset()
            out = [fnlib.forward(ids[k:k + 5], logits=True)[1] for k in range(0, 20, 5)]
            res.append(np.concatenate(out))
        assert np.array_equal(res[0], res[1]) and np.array_equal(res[0], res[2])
    finally:
        fnlib.free()


def test_model_errors(fnlib, model_file):
    path, kv, ts = model_file
    _say("model forward: argument and context checks")
    fnlib.load(path, "", max_ctx=256)
    try:
        with pytest.raises(RuntimeError, match="nt out of range"):
            fnlib.forward(np.zeros(9, np.int32))
        with pytest.raises(RuntimeError, match="vocabulary"):
            fnlib.forward([ms.TINY_DIMS["VOCAB"]])
        ids = np.zeros(8, np.int32)
        for _ in range(32):
            fnlib.forward(ids)
        assert fnlib.d.fn_n_past() == 256
        with pytest.raises(RuntimeError, match="context full"):
            fnlib.forward([1])
    finally:
        fnlib.free()
    assert fnlib.d.fn_n_past() == -1


def _stale_status_bit(fnlib):
    """Leave FN_STATUS_POS in the device's status word: a GQA decode call whose new token lies past its cache."""
    import hiprt

    B, nq, nkv, hd, max_ctx = 1, 16, 2, 256, 64
    rng = np.random.default_rng(1)
    bufs = [hiprt.Buf.like(rng.standard_normal(n).astype(np.float32)) for n in
            (B * nkv * max_ctx * hd, B * nkv * max_ctx * hd, B * nq * 2 * hd, B * nkv * hd, B * nkv * hd, hd, hd)]
    K, V, qg, k, v, wq, wk = bufs
    pos = hiprt.Buf.like(np.array([max_ctx], np.int32))
    nsplit = fnlib.attn_nsplit(B, nkv, 1, max_ctx)
    wb = fnlib.attn_work_bytes(B, nq, 1, nsplit)
    work, og = hiprt.Buf(wb), hiprt.Buf.empty((B, 1, nq, hd))
    fnlib.attn_dev(B, nq, nkv, 1, max_ctx, pos.ptr, qg.ptr, k.ptr, v.ptr, wq.ptr, wk.ptr, K.ptr, V.ptr, nsplit,
                   work.ptr, wb, og.ptr, None)
    hiprt.sync()
    for b in (*bufs, pos, work, og):
        b.free()


def test_model_forward_after_split_override_and_stale_status(fnlib, model_file):
    """The forward holds no work buffer for a split-K GEMV: after fn_gemv_override asks for 3 splits its GEMVs keep
    their own plan (same bits as without the override).  A status bit another entry point left in the device's
    status word is not the forward's: the model records its kernels' misuse in a word of its own, so the call
    succeeds and leaves the other word as it found it."""
    import fn

    path, kv, ts = model_file
    ids = np.random.default_rng(6).integers(0, ms.TINY_DIMS["VOCAB"], size=12)
    _say("model forward: after fn_gemv_override(ks=3) and with a stale FN_STATUS_POS bit")
    fnlib.load(path, "", max_ctx=256)
    try:
        base = np.concatenate([fnlib.forward(ids[k:k + 4], logits=True)[1] for k in range(0, 12, 4)])
        fnlib.reset()
        fnlib.gemv_override(ks=3)
        try:
            over = np.concatenate([fnlib.forward(ids[k:k + 4], logits=True)[1] for k in range(0, 12, 4)])
        finally:
            fnlib.gemv_override()
        assert np.array_equal(base, over)
        fnlib.reset()
        _stale_status_bit(fnlib)
        assert fnlib.dev_status(clear=False) & fn.STATUS_POS
        again = np.concatenate([fnlib.forward(ids[k:k + 4], logits=True)[1] for k in range(0, 12, 4)])
        assert np.array_equal(base, again)
        assert fnlib.dev_status() == fn.STATUS_POS
        assert fnlib.dev_status() == 0
    finally:
        fnlib.free()


def test_model_two_shards_equal_one_file(fnlib, model_file, tmp_path):
    """The n-gram table in a second file (the reference model's layout) gives the same bits as one file."""
    path, kv, ts = model_file
    s1, s2 = str(tmp_path / "s1.gguf"), str(tmp_path / "s2.gguf")
    ms.write_model(s1, ms.TINY_DIMS, seed=11, shard2=s2)
    ids = np.random.default_rng(5).integers(0, ms.TINY_DIMS["VOCAB"], size=16)
    out = []
    for a, b in ((path, ""), (s1, s2)):
        _say(f"model forward: shards {a!r} {b!r}")
        fnlib.load(a, b, max_ctx=256)
        try:
            out.append(np.concatenate([fnlib.forward(ids[k:k + 4], logits=True)[1] for k in range(0, 16, 4)]))
        finally:
            fnlib.free()
    assert np.array_equal(out[0], out[1])


def test_model_ple_load_checks(fnlib, tmp_path):
    """A table with fewer rows than the n-gram heads address, and a second shard that is missing, fail the load."""
    kv, ts = ms.model_tensors(ms.TINY_DIMS, seed=3)
    T = ms.TINY_DIMS
    short = sum(T["ple_sizes"]) - 1
    ts2 = [t if t[0] != "per_layer_token_embd.weight" else
           (t[0], t[1], [T["ple_hd"], short], t[3][: short * T["ple_hd"] // 32 * 18]) for t in ts]
    p = str(tmp_path / "short.gguf")
    ms.write_gguf(p, kv, ts2)
    _say("model load: short n-gram table")
    with pytest.raises(RuntimeError, match="n-gram heads reach"):
        fnlib.load(p, "", max_ctx=256)
    _say("model load: missing second shard")
    with pytest.raises(RuntimeError, match="cannot open"):
        fnlib.load(p, str(tmp_path / "absent.gguf"), max_ctx=256)
    assert fnlib.d.fn_n_past() == -1


def test_model_quantized_hyper_connections(fnlib, tmp_path):
    """Hyper-connection weights in a block format take the general path (low-rank kernel, up GEMV, mix kernel) in
    place of the fused BF16 up-and-mix kernel; both match the oracle."""
    p = str(tmp_path / "hcq.gguf")
    kv, ts = ms.write_model(p, ms.TINY_DIMS, seed=12, types={"hc": ms.Q8_0})
    _say("model forward: Q8_0 hyper-connection weights, 20 tokens")
    fnlib.load(p, "", max_ctx=256)
    try:
        ref = om.Model(kv, ts, max_ctx=256)
        ids = np.random.default_rng(3).integers(0, ms.TINY_DIMS["VOCAB"], size=20)
        for k, nt in ((0, 1), (1, 8), (9, 3), (12, 8)):
            am, lg = fnlib.forward(ids[k:k + nt], logits=True)
            want, _, _, _ = ref.forward(ids[k:k + nt])
            assert _rel(lg, want) <= TOL, (k, nt, _rel(lg, want))
    finally:
        fnlib.free()


# the reference model's widths in two layers (a DeltaNet layer, then an attention layer that carries the n-gram
# embedding): hidden 2560, 16 / 48 DeltaNet heads, 24 / 2 attention heads, hyper-connections 4 of rank 320, experts
# and the shared expert of 640; fewer experts and a small vocabulary keep the float64 oracle quick
MEDIUM_DIMS = dict(ms.TINY_DIMS, D=2560, NL=2, attn_every=2, NH=24, NKV=2, NE=8, NEU=2, FFE=640, FFS=640, NKH=16,
                   NVH=48, HC=4, HCR=320, VOCAB=4096, ple_hd=320, ple_heads_per_ngram=4)


def test_model_reference_widths(fnlib, tmp_path):
    """Every kernel of the forward at the reference model's row lengths and projection shapes (the grouped
    projections at 10240 / 6144 / 96 and 12288 / 512 / 512 / 640 rows, 80-group rows in the GEMVs and expert rows,
    the up-and-mix kernel at rank 320), one- and several-token calls, within 1e-5 of the oracle."""
    p = str(tmp_path / "medium.gguf")
    kv, ts = ms.write_model(p, MEDIUM_DIMS, seed=21)
    _say("model forward: reference widths, 2 layers, 20 tokens in calls of 1, 8, 3, 8")
    fnlib.load(p, "", max_ctx=256)
    try:
        ref = om.Model(kv, ts, max_ctx=256)
        ids = np.random.default_rng(6).integers(0, MEDIUM_DIMS["VOCAB"], size=20)
        ids[[4, 13]] = MEDIUM_DIMS["ple_eos"]
        i = 0
        for nt in (1, 8, 3, 8):
            am, lg = fnlib.forward(ids[i:i + nt], logits=True)
            want, want_am, _, _ = ref.forward(ids[i:i + nt])
            e = _rel(lg, want)
            _say(f"  nt={nt}: logits error {e:.3e}")
            assert e <= TOL, (i, nt, e)
            for t in range(nt):
                top2 = np.sort(want[t])[-2:]
                if top2[1] - top2[0] > 1e-4 * abs(top2[1]):
                    assert am[t] == want_am[t], (i, t)
            i += nt
    finally:
        fnlib.free()


def test_model_token_count_invariance(fnlib, tmp_path):
    """Token t of an 8-token call gets the bits of one-token calls in a model without attention layers (every
    DeltaNet, hyper-connection, projection and expert kernel sums per token in a fixed order, whatever the launch
    shape); with attention layers, whose several-token kernel runs on the matrix cores, within 1e-6."""
    out = {}
    for name, dims in (("no attention", dict(ms.TINY_DIMS, attn_every=0)), ("hybrid", ms.TINY_DIMS)):
        p = str(tmp_path / "inv.gguf")
        ms.write_model(p, dims, seed=11)
        _say(f"model forward: 8-token calls vs one-token calls, {name}")
        fnlib.load(p, "", max_ctx=256)
        try:
            ids = np.random.default_rng(3).integers(0, dims["VOCAB"], size=24)
            fnlib.reset()
            a = np.concatenate([fnlib.forward(ids[k:k + 8], logits=True)[1] for k in range(0, 24, 8)])
            fnlib.reset()
            b = np.concatenate([fnlib.forward(ids[k:k + 1], logits=True)[1] for k in range(24)])
            out[name] = (a, b)
        finally:
            fnlib.free()
    a, b = out["no attention"]
    assert np.array_equal(a, b)
    a, b = out["hybrid"]
    assert _rel(a, b) <= 1e-6


@pytest.mark.parametrize("ne,neu", [(24, 10), (40, 17), (600, 10)])
def test_model_expert_counts(fnlib, tmp_path, ne, neu):
    """The reference model's 10 experts a token, and 17 (the MoE output kernel then takes its items in two passes a
    wave for one token, and the several-token kernel three chunks of weight words), and 600 experts (more than 512:
    the routing holds 16 logits a lane instead of 8), against the oracle."""
    dims = dict(ms.TINY_DIMS, NE=ne, NEU=neu)
    p = str(tmp_path / "experts.gguf")
    kv, ts = ms.write_model(p, dims, seed=13)
    _say(f"model forward: {ne} experts, {neu} a token, 12 tokens in calls of 1, 8, 3")
    fnlib.load(p, "", max_ctx=256)
    try:
        ref = om.Model(kv, ts, max_ctx=256)
        ids = np.random.default_rng(7).integers(0, dims["VOCAB"], size=12)
        i = 0
        for nt in (1, 8, 3):
            _, lg = fnlib.forward(ids[i:i + nt], logits=True)
            want, _, _, _ = ref.forward(ids[i:i + nt])
            assert _rel(lg, want) <= TOL, (ne, neu, i, nt, _rel(lg, want))
            i += nt
    finally:
        fnlib.free()


@pytest.mark.parametrize("ne,neu", [(24, 10), (40, 17)])
def test_model_moe_override_same_bits(fnlib, tmp_path, ne, neu):
    """fn_moe_override's dn_wpt picks the MoE output kernel: 1 runs the 16-row kernel for one-token calls too, 4 the
    4-row kernel for several-token calls too (grid rows x tokens).  Both give the automatic choice's bits, through
    the graphs captured after the override (fn_use_graphs drops the earlier ones) and eagerly; 17 experts a token
    take the 4-row kernel's items in two passes."""
    dims = dict(ms.TINY_DIMS, NE=ne, NEU=neu)
    p = str(tmp_path / "moe.gguf")
    ms.write_model(p, dims, seed=17)
    ids = np.random.default_rng(8).integers(0, dims["VOCAB"], size=12)

    def run():
        fnlib.reset()
        out, i = [], 0
        for nt in (1, 8, 3):
            out.append(fnlib.forward(ids[i:i + nt], logits=True)[1])
            i += nt
        return np.concatenate(out)

    fnlib.load(p, "", max_ctx=256)
    try:
        base = run()
        for w, graphs in ((1, True), (4, True), (1, False), (4, False)):
            _say(f"model forward: {neu} experts a token, fn_moe_override dn_wpt={w}, graphs {graphs}")
            fnlib.moe_override(w)
            fnlib.use_graphs(graphs)
            assert np.array_equal(run(), base), (neu, w, graphs)
    finally:
        fnlib.moe_override(-1)
        fnlib.free()

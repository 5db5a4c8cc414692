"""CPU checks of the model loader's file handling and of the model oracle (no GPU).

* The GGUF writer (model_synth) and the library's reader (fn_model_dims: parse + shapes, no device work) agree on
  every shape of the synthetic model; malformed files fail with a message that names the problem.
* The whole-model oracle (oracle/model.py) is pinned piece by piece by closed forms: the hyper-connection read with
  zero up / inject weights, the routing rule on exact ties, the write with unit inject weights, and one layer's
  MoE against a hand-assembled sum.
"""

import os
import struct

import numpy as np
import pytest

import fn
import model_synth as ms
import oracle.model as om


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    kv, ts = ms.write_model(path, ms.TINY_DIMS, seed=3)
    return path, kv, ts


def test_reader_reads_the_written_shapes(fnlib, tiny):
    path, kv, ts = tiny
    d = fnlib.model_dims(path)
    T = ms.TINY_DIMS
    assert (d["D"], d["NL"], d["NH"], d["NKV"], d["NE"], d["NEU"], d["FFE"], d["FFS"]) == \
        (T["D"], T["NL"], T["NH"], T["NKV"], T["NE"], T["NEU"], T["FFE"], T["FFS"])
    assert (d["NKH"], d["NVH"], d["HC"], d["HCR"], d["VOCAB"], d["attn_every"]) == \
        (T["NKH"], T["NVH"], T["HC"], T["HCR"], T["VOCAB"], T["attn_every"])
    assert (d["HD"], d["DS"], d["NROT"], d["IXH"], d["IXD"], d["top"]) == (256, 128, 64, 4, 128, T["top_k"] // 4)
    assert d["DINNER"] == T["NVH"] * 128 and d["CONVCH"] == 2 * T["NKH"] * 128 + T["NVH"] * 128


def test_reader_reads_ple_and_two_shards(fnlib, tmp_path):
    """The PLE shapes come from the metadata; a model whose table sits in a second file reads the same from the
    first (the reference model's shard layout)."""
    a, b, c = str(tmp_path / "one.gguf"), str(tmp_path / "s1.gguf"), str(tmp_path / "s2.gguf")
    ms.write_model(a, ms.TINY_DIMS, seed=1)
    ms.write_model(b, ms.TINY_DIMS, seed=1, shard2=c)
    d = fnlib.model_dims(a)
    T = ms.TINY_DIMS
    assert (d["PLE_LAYERS"], d["PLE_HEADS"], d["PLE_HD"]) == (1, 2 * T["ple_heads_per_ngram"], T["ple_hd"])
    assert fnlib.model_dims(b) == d
    r = ms.REFERENCE_DIMS
    assert 2 * r["ple_heads_per_ngram"] * r["ple_hd"] == r["D"] and len(r["ple_sizes"]) == 2 * r["ple_heads_per_ngram"]


def test_reader_alignment_and_version(fnlib, tmp_path):
    """A GGUF v2 file and one with general.alignment = 64 parse to the same shapes."""
    kv, ts = ms.model_tensors(ms.TINY_DIMS, seed=1)
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    ms.write_gguf(a, kv, ts, alignment=64, version=2)
    ms.write_gguf(b, kv, ts)
    assert fnlib.model_dims(a) == fnlib.model_dims(b)


def _err(fnlib, path):
    with pytest.raises(RuntimeError) as e:
        fnlib.model_dims(path)
    return str(e.value)


def test_reader_rejects_malformed_files(fnlib, tmp_path, tiny):
    path, kv, ts = tiny
    raw = open(path, "rb").read()
    p = str(tmp_path / "x.gguf")
    open(p, "wb").write(b"GGUX" + raw[4:])
    assert "bad magic" in _err(fnlib, p)
    open(p, "wb").write(raw[:4] + struct.pack("<I", 9) + raw[8:])
    assert "version 9" in _err(fnlib, p)
    open(p, "wb").write(raw[:200])
    assert "truncated" in _err(fnlib, p)
    open(p, "wb").write(raw[: len(raw) - 1000])
    assert "outside the file" in _err(fnlib, p)
    assert "cannot open" in _err(fnlib, str(tmp_path / "missing.gguf"))
    # dimensions whose byte count wraps 64 bits (2^33 rows x 2^32 x 2^32) are refused, not wrapped into range
    name, ty, dims, data = ts[0]
    ms.write_gguf(p, kv, [(name, ty, [dims[0], 1 << 33, 1 << 32, 1 << 32], data)] + list(ts[1:]))
    assert "implausible dimensions" in _err(fnlib, p)


def test_reader_rejects_unbuilt_shapes(fnlib, tmp_path):
    p = str(tmp_path / "y.gguf")
    kv, ts = ms.model_tensors(ms.TINY_DIMS, seed=2)
    k2 = dict(kv)
    k2["qwen4exp.attention.key_length"] = 128
    ms.write_gguf(p, k2, ts)
    assert "head dims" in _err(fnlib, p)
    k2 = dict(kv)
    k2["qwen4exp.attention.head_count"] = 6           # 3 query heads per kv head
    ms.write_gguf(p, k2, ts)
    assert "4, 8 or 12" in _err(fnlib, p)
    k2 = dict(kv)
    k2["qwen4exp.ple.head_vocab_sizes"] = [97] * 7                 # one size short of the 8 heads
    ms.write_gguf(p, k2, ts)
    assert "PLE" in _err(fnlib, p)
    k2 = dict(kv)
    k2["qwen4exp.embedding_length_per_layer_input"] = 48           # 8 heads x 48 != D
    ms.write_gguf(p, k2, ts)
    assert "PLE" in _err(fnlib, p)
    k2 = dict(kv)
    k2["qwen4exp.ple.layers"] = [4]                                # layer outside the model
    ms.write_gguf(p, k2, ts)
    assert "PLE" in _err(fnlib, p)
    k2 = dict(kv)
    del k2["general.architecture"]
    ms.write_gguf(p, k2, ts)
    assert "architecture" in _err(fnlib, p)


def test_load_before_device_checks_the_file(fnlib, tmp_path):
    """fn_load reports file problems with the reference's -1 + fn_error() convention (faie2fn.cu:2531-2535)."""
    d = fnlib.d
    assert d.fn_load(str(tmp_path / "none.gguf").encode(), b"", 4096, 0) == -1
    assert b"cannot open" in d.fn_error()
    with pytest.raises(RuntimeError, match="not loaded"):
        fnlib.forward([1, 2])


def test_load_plans_every_tensor_before_the_device(fnlib, tmp_path):
    """fn_load walks its tensor table over the file before it touches the device: a missing tensor, a tensor of
    another shape and an n-gram table shorter than its heads address fail with a message naming the tensor (here,
    without a GPU), and leave no model loaded."""
    kv, ts = ms.model_tensors(ms.TINY_DIMS, seed=3)
    T = ms.TINY_DIMS
    p = str(tmp_path / "bad.gguf")
    ms.write_gguf(p, kv, [t for t in ts if t[0] != "blk.2.ssm_out.weight"])
    with pytest.raises(RuntimeError, match=r"blk\.2\.ssm_out\.weight missing"):
        fnlib.load(p, "", max_ctx=256)
    # one row fewer in a BF16 weight (rows of D values, 2 bytes each)
    row = T["D"] * 2
    ts2 = [t if t[0] != "blk.1.ssm_alpha.weight" else (t[0], t[1], [T["D"], T["NVH"] - 1], t[3][: (T["NVH"] - 1) * row])
           for t in ts]
    ms.write_gguf(p, kv, ts2)
    with pytest.raises(RuntimeError, match=r"blk\.1\.ssm_alpha\.weight has shape \[256, 3, 1\], expected 256 columns x 4"):
        fnlib.load(p, "", max_ctx=256)
    short = sum(T["ple_sizes"]) - 1
    ts3 = [t if t[0] != "per_layer_token_embd.weight" else
           (t[0], t[1], [T["ple_hd"], short], t[3][: short * T["ple_hd"] // 32 * 18]) for t in ts]
    ms.write_gguf(p, kv, ts3)
    with pytest.raises(RuntimeError, match="n-gram heads reach"):
        fnlib.load(p, "", max_ctx=256)
    assert fnlib.d.fn_n_past() == -1


# ---- oracle pins ----


@pytest.fixture(scope="module")
def oracle_model(tiny):
    path, kv, ts = tiny
    return om.Model(kv, ts, max_ctx=256)


def test_hc_read_closed_forms(oracle_model):
    """With the up weight zero, sigmoid(0) = 1/2 for every stream, so x = mean_s(hn_s) / 2; with the inject rows
    zero, inj = 2 sigmoid(0) = 1 for every stream (tile_mix, faie2fn.cu:873-888)."""
    m = oracle_model
    rng = np.random.default_rng(5)
    hn = rng.standard_normal((3, m.HC * m.D))
    name_d, name_u, name_i = "output_hc_down.weight", "blk.0.hc_attn_up.weight", "blk.0.hc_attn_inject.weight"
    saved = dict(m._w)
    try:
        m._w[(name_u,)] = np.zeros((m.HC * m.D, m.HCR))
        m._w[(name_d, name_i)] = np.concatenate([m.w(name_d), np.zeros((m.HC, m.HC * m.D))])
        x, inj = m.hc_read(hn, name_d, name_u, name_i)
    finally:
        m._w = saved
    assert np.allclose(x, hn.reshape(3, m.HC, m.D).mean(1) / 2, rtol=1e-14, atol=0)
    assert np.array_equal(inj, np.ones((3, m.HC)))


def test_groupnorm_closed_form(oracle_model):
    """A stream of constant c normalizes to sign(c) * w / sqrt(1 + eps / c^2)."""
    m = oracle_model
    h = np.full((1, m.HC * m.D), 3.0)
    w = np.arange(m.HC * m.D, dtype=np.float64)
    out = m.groupnorm(h, w)
    assert np.allclose(out, w / np.sqrt(1 + m.eps / 9.0), rtol=1e-15)


def test_route_ties_and_weights(oracle_model):
    """Equal logits: the lowest expert indices win (repeated argmax, faie2fn.cu:1749-1751); weights are the
    renormalized softmax of the chosen ones, so equal logits give equal weights 1 / NEU."""
    m = oracle_model
    l = np.zeros((2, m.NE))
    l[1, 5] = 1.0
    sel, w = m.route(l)
    assert list(sel[0]) == list(range(m.NEU)) and np.allclose(w[0], 1.0 / m.NEU)
    assert sel[1][0] == 5 and list(sel[1][1:]) == [i for i in range(m.NE) if i != 5][: m.NEU - 1]
    e = np.exp(1.0)
    assert np.allclose(w[1], np.array([e] + [1.0] * (m.NEU - 1)) / (e + m.NEU - 1))


def test_moe_layer_hand_sum(oracle_model):
    """One token through blk.0's MoE equals the hand-assembled sum over its routed experts plus the gated shared
    expert, each expert SwiGLU(gate, up) then down (k_tmoe_gu / k_tmoe_down / k_hc_add, faie2fn.cu:1047-1183,
    1298-1318)."""
    m = oracle_model
    p = "blk.0."
    rng = np.random.default_rng(6)
    x = rng.standard_normal((1, m.D))
    y, sel = m.ffn(0, x)
    rl = (x @ m.w(p + "ffn_gate_inp.weight").T)[0]
    pr = np.exp(rl - rl.max())
    top = np.argsort(-pr, kind="stable")[: m.NEU]
    assert list(top) == list(sel[0])
    want = np.zeros(m.D)
    for e in top:
        g = m.w(p + "ffn_gate_exps.weight")[e * m.FFE:(e + 1) * m.FFE] @ x[0]
        u = m.w(p + "ffn_up_exps.weight")[e * m.FFE:(e + 1) * m.FFE] @ x[0]
        a = g / (1 + np.exp(-g)) * u
        want += pr[e] / pr[top].sum() * (m.w(p + "ffn_down_exps.weight")[e * m.D:(e + 1) * m.D] @ a)
    sg = (x @ m.w(p + "ffn_gate_shexp.weight").T)[0]
    su = (x @ m.w(p + "ffn_up_shexp.weight").T)[0]
    sd = m.w(p + "ffn_down_shexp.weight") @ (sg / (1 + np.exp(-sg)) * su)
    gate = (x @ m.w(p + "ffn_gate_inp_shexp.weight").T)[0, 0]
    want += sd / (1 + np.exp(-gate))
    assert np.allclose(y[0], want, rtol=1e-12, atol=1e-12)


def test_oracle_forward_runs_and_is_deterministic(oracle_model):
    m = oracle_model
    m.reset()
    l1, a1, h1, _ = m.forward([3, 17, 250])
    m.reset()
    l2, a2, h2, _ = m.forward([3, 17, 250])
    assert np.array_equal(l1, l2) and np.array_equal(a1, a2) and np.isfinite(l1).all()
    assert h1.shape == (m.NL, 3, m.HC * m.D)
    m.reset()


# ---- per-layer n-gram embedding pins ----


def test_ple_hash_matches_uint64_arithmetic(oracle_model):
    """The rows of every head equal the hash in numpy's wrapping uint64 arithmetic (ids widened with their sign),
    an independent statement of the reference's unsigned long long products (k_ple_ids, faie2fn.cu:1810-1823); the
    tiny model's multipliers make every product wrap."""
    m = oracle_model
    m.reset()
    rng = np.random.default_rng(8)
    m.toks = [int(v) for v in rng.integers(0, m.VOCAB, 40)]
    m.toks[10] = m.ple_eos
    mult = np.array(m.ple_mult, np.uint64)
    assert all(int(v) * 300 >= 1 << 64 for v in m.ple_mult)
    H = m.ple_heads
    with np.errstate(over="ignore"):
        for p in range(40):
            tok = np.array(m.toks, np.int64).view(np.uint64)
            eos = np.array([m.ple_eos], np.int64).view(np.uint64)[0]
            p1 = tok[p - 1] if p >= 1 else eos
            p2 = tok[p - 2] if p >= 2 and p1 != eos else eos
            big = (tok[p] * mult[0]) ^ (p1 * mult[1])
            tri = big ^ (p2 * mult[2])
            want = [int((big if hd < H // 2 else tri) % np.uint64(m.ple_size[hd])) + m.ple_off[hd] for hd in range(H)]
            assert m.ple_rows(p) == want, p
    m.reset()


def test_ple_hash_context_rules(oracle_model):
    """Bigram heads never see the token two back; trigram heads see it unless the previous token is EOS; the first
    position's context is EOS (k_ple_ids, faie2fn.cu:1817-1821)."""
    m = oracle_model
    H = m.ple_heads
    m.toks = [5, 9, 11]
    r = m.ple_rows(2)
    m.toks = [6, 9, 11]
    r2 = m.ple_rows(2)
    assert r[: H // 2] == r2[: H // 2] and r[H // 2:] != r2[H // 2:]
    m.toks = [5, m.ple_eos, 11]
    r = m.ple_rows(2)
    m.toks = [6, m.ple_eos, 11]
    assert m.ple_rows(2) == r
    m.toks = [m.ple_eos, m.ple_eos, 11]
    assert m.ple_rows(2) == r                    # the cut context reads EOS, whatever sits before it
    m.toks = [11]
    assert m.ple_rows(0) == r                    # position 0: previous token and the one before are EOS
    m.reset()


def test_ple_gate_closed_forms(oracle_model):
    """key = h with unit norm weights: gate = sqrt(sqrt(D) ms / (ms + eps)) per stream (ms the stream's mean
    square); key = -h gives the negative root; key = 0 gives gate 0, sigmoid 1/2; gvn = RMSNorm of the scaled value
    (k_ple_gate, faie2fn.cu:1843-1875)."""
    m = oracle_model
    HC, D = m.HC, m.D
    rng = np.random.default_rng(9)
    h = rng.standard_normal((2, HC * D)) * np.repeat(np.array([0.5, 1.0, 2.0, 3.0]), D)
    val = rng.standard_normal((2, D))
    one = np.ones(HC * D)
    ms_ = (h.reshape(2, HC, D) ** 2).mean(-1)
    for sgn in (1.0, -1.0):
        gv, gvn = m.ple_gate(sgn * h, val, h, one, one, one)
        gate = sgn * np.sqrt(np.sqrt(D) * ms_ / (ms_ + m.eps))
        sg = 1 / (1 + np.exp(-gate))
        want = sg[:, :, None] * val[:, None, :]
        assert np.allclose(gv.reshape(2, HC, D), want, rtol=1e-13, atol=0)
        msv = (want ** 2).mean(-1, keepdims=True)
        assert np.allclose(gvn.reshape(2, HC, D), want / np.sqrt(msv + m.eps), rtol=1e-13, atol=0)
    gv, _ = m.ple_gate(np.zeros_like(h), val, h, one, one, one)
    assert np.array_equal(gv.reshape(2, HC, D), np.broadcast_to(0.5 * val[:, None, :], (2, HC, D)))


def test_ple_conv_taps_and_history(oracle_model):
    """Weights (0,0,0,1) read the current value, (1,0,0,0) the value 9 steps back, (0,1,0,0) 6 back, (0,0,1,0)
    3 back; the history afterwards is the last 9 inputs (k_ple_conv, faie2fn.cu:1878-1896)."""
    m = oracle_model
    n = m.HC * m.D
    il = m.ple_layers[0]
    rng = np.random.default_rng(10)
    hist = rng.standard_normal((9, n))
    gvn = rng.standard_normal((5, n))
    gv = rng.standard_normal((5, n))
    x = np.concatenate([hist, gvn])
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    for tap, back in ((3, 0), (2, 3), (1, 6), (0, 9)):
        w = np.zeros((n, 4))
        w[:, tap] = 1.0
        m.ple_hist[il] = hist.copy()
        out = m.ple_conv(il, gv, gvn, w)
        want = gv + silu(np.stack([x[9 + t - back] for t in range(5)]))
        assert np.allclose(out, want, rtol=1e-14, atol=1e-15), tap
        assert np.array_equal(m.ple_hist[il], x[5:14])
    m.reset()

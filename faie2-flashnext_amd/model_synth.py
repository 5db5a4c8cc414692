"""Synthetic FAIE2-FlashNext models as GGUF files: a GGUF writer and seeded random weights in the reference model's
tensor layout (engine/faie2fn.cu:2578-2671 names, flashnext/inspect_fn.txt shapes), at any size.

No checkpoint of the reference model is available here, so fn_load / fn_forward are exercised on models written by
this module: the same tensor names, metadata keys and weight formats as the reference's GGUF, with small dimensions
(tests) or the reference's own (benchmarks).  Quantized weights are random block bytes whose scale fields are set so
that each weight matrix has values of standard deviation about 1 / sqrt(columns).
"""

import struct

import numpy as np

# GGUF value types
_U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64 = 4, 5, 6, 7, 8, 9, 10, 11
# ggml type ids and (values, bytes) per block
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS, BF16 = 0, 1, 8, 12, 13, 14, 20, 21, 23, 30
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ2_S, Q2_0 = 16, 17, 18, 22, 42
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
         IQ4_NL: (32, 18), IQ3_S: (256, 110), IQ4_XS: (256, 136), BF16: (1, 2), IQ2_XXS: (256, 66), IQ2_XS: (256, 74),
         IQ3_XXS: (256, 98), IQ2_S: (256, 82), Q2_0: (64, 18)}
# byte offsets of the fp16 scale fields inside a block (d, and dmin for the K formats with a minimum)
SCALES = {Q8_0: [0], Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208], IQ4_NL: [0], IQ3_S: [0], IQ4_XS: [0], IQ2_XXS: [0],
          IQ2_XS: [0], IQ3_XXS: [0], IQ2_S: [0], Q2_0: [0]}


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, value):
    """One GGUF key/value pair; ints as u32 / i32 / i64 by range, floats as f32, lists as arrays of i64 or i32."""
    out = _s(key)
    if isinstance(value, bool):
        return out + struct.pack("<IB", _BOOL, int(value))
    if isinstance(value, str):
        return out + struct.pack("<I", _STR) + _s(value)
    if isinstance(value, float):
        return out + struct.pack("<If", _F32, value)
    if isinstance(value, int):
        if 0 <= value < 2 ** 32:
            return out + struct.pack("<II", _U32, value)
        return out + struct.pack("<Iq", _I64, value)
    if isinstance(value, (list, tuple)):
        vals = list(value)
        if all(isinstance(v, int) and -2 ** 31 <= v < 2 ** 31 for v in vals):
            return out + struct.pack("<IIQ", _ARR, _I32, len(vals)) + struct.pack(f"<{len(vals)}i", *vals)
        return out + struct.pack("<IIQ", _ARR, _I64, len(vals)) + struct.pack(f"<{len(vals)}q", *vals)
    raise TypeError(f"{key}: unsupported value {value!r}")


def write_gguf(path, kv, tensors, alignment=32, version=3):
    """Write a GGUF file.  kv: dict of metadata; tensors: list of (name, ggml type, dims (ne[0] first), raw bytes)."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kv) + (alignment != 32))
    body = b"".join(_kv(k, v) for k, v in kv.items())
    if alignment != 32:
        body += _kv("general.alignment", alignment)
    infos, off = b"", 0
    offsets = []
    for name, ty, dims, raw in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        infos += _s(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        infos += struct.pack("<IQ", ty, off)
        off += len(raw)
    header = head + body + infos
    with open(path, "wb") as f:
        f.write(header)
        pad = (-len(header)) % alignment
        f.write(b"\0" * pad)
        pos = 0
        for (name, ty, dims, raw), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(raw)
            pos = o + len(raw)


def _f16_bits(x):
    return np.float16(x).view(np.uint16)


# root mean square of a value of each format with every fp16 scale field 1.0 and uniformly random code bytes
# (code ranges: Q8_0 int8; IQ4 levels x (ls - 32) for IQ4_XS; IQ3_S (1 + 2 sc) x grid magnitudes; Q6_K int8 scale x
# (q - 32); Q4_K / Q5_K 6-bit scale x 4 / 5-bit code)
_RMS = {Q8_0: 73.9, IQ4_NL: 67.4, IQ4_XS: 67.4 * 18.5, IQ3_S: 18.5 * 7.6, Q6_K: 73.9 * 18.5, Q4_K: 36.5 * 8.8,
        Q5_K: 36.5 * 18.0, IQ2_XXS: 53.4, IQ2_XS: 55.8, IQ2_S: 56.7, IQ3_XXS: 141.4, Q2_0: 1.225}


def _code_bytes(n, rng, pool):
    """n uniformly random bytes, or (with a pool) n bytes of the pool repeated from a random start: as random-looking
    to a decoder and written at copy speed, for benchmark models of tens of GB"""
    if pool is None:
        return rng.integers(0, 256, size=n, dtype=np.uint8)
    out = np.empty(n, np.uint8)
    i, pos = 0, int(rng.integers(0, len(pool)))
    while i < n:
        k = min(n - i, len(pool) - pos)
        out[i:i + k] = pool[pos:pos + k]
        i, pos = i + k, 0
    return out


def random_weight(ty, rows, cols, rng, std=None, pool=None):
    """Raw GGUF bytes of a rows x cols weight of type ty with values of spread ~ std (default 1 / sqrt(cols)): normal
    values for the float types; for the block formats random code bytes with every fp16 scale field set to the one
    value that gives that spread."""
    std = 1.0 / np.sqrt(cols) if std is None else std
    if ty == F32:
        return rng.normal(0.0, std, rows * cols).astype(np.float32).tobytes()
    if ty in (BF16, F16):
        v = rng.normal(0.0, std, rows * cols).astype(np.float32)
        if ty == F16:
            return v.astype(np.float16).tobytes()
        u = v.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).tobytes()
    qk, bb = BLOCK[ty]
    raw = _code_bytes(rows * (cols // qk) * bb, rng, pool)
    blk = raw.reshape(-1, bb)
    bits = np.frombuffer(_f16_bits(std / _RMS[ty]).tobytes(), np.uint8)
    for o in SCALES[ty]:
        blk[:, o] = bits[0]
        blk[:, o + 1] = bits[1]
    return raw if pool is not None else raw.tobytes()  # (a uint8 array serves the writer as well as bytes)


# the reference model's shapes (flashnext/inspect_fn.txt), and a small model of the same structure for tests
# (PLE: the per-layer n-gram embedding of the layers in ple_layers; its hash constants and head sizes are the
# reference model's, flashnext/inspect_fn.txt:37-45)
REFERENCE_DIMS = dict(D=2560, NL=48, NH=24, NKV=2, NE=512, NEU=10, FFE=640, FFS=640, NKH=16, NVH=48, HC=4, HCR=320,
                      top_k=2048, VOCAB=248320, attn_every=4, ple_layers=[1], ple_heads_per_ngram=8, ple_hd=160,
                      ple_eos=248044, ple_mult=[23703573157769, 20109073645365, 8052911324071],
                      ple_sizes=[20000003, 20000023, 20000033, 20000047, 20000059, 20000063, 20000069, 20000077,
                                 20000081, 20000093, 20000107, 20000147, 20000153, 20000159, 20000161, 20000171])
# the tiny model's multipliers are large enough that the hash products wrap modulo 2^64, and its EOS is an ordinary
# token id, so short random sequences cross it
TINY_DIMS = dict(D=256, NL=4, NH=8, NKV=2, NE=8, NEU=2, FFE=64, FFS=64, NKH=2, NVH=4, HC=4, HCR=32, top_k=32, VOCAB=320,
                 attn_every=4, ple_layers=[1], ple_heads_per_ngram=4, ple_hd=32, ple_eos=7,
                 ple_mult=[0x7F4A7C159E3779B9, 0x5851F42D4C957F2D, 0x14057B7EF767814F],
                 ple_sizes=[97, 101, 103, 107, 109, 113, 127, 131])

# weight formats of the reference model by tensor (flashnext/inspect_fn.txt:75-164): layer-dependent formats as
# tuples cycled over the layers (routed experts: IQ2_XS / IQ2_XXS / IQ2_S / IQ3_XXS gate and up, IQ4_NL / Q2_0 down)
TYPES = dict(token_embd=IQ3_S, output=Q5_K, hc=BF16, attn_qkv=IQ4_XS, attn_gate=(IQ3_S, Q6_K), ssm_ab=BF16,
             ssm_out=Q8_0, attn_q=IQ4_XS, attn_k=IQ4_XS, attn_v=Q6_K, attn_output=Q8_0, indexer=BF16, router=BF16,
             shexp_gate=IQ4_XS, shexp_up=IQ3_S, shexp_down=Q8_0, exps_gate=(IQ2_XS, IQ2_XXS, IQ2_S, IQ3_XXS),
             exps_up=(IQ2_XS, IQ2_XXS, IQ2_S, IQ3_XXS), exps_down=(IQ4_NL, Q2_0), ple=BF16, ple_table=IQ4_NL)


def pick(ty, il):
    """the format of layer il: a tuple of formats cycles over the layers"""
    return ty[il % len(ty)] if isinstance(ty, tuple) else ty


def model_tensors(dims, seed=0, types=None, fast=False):
    """(metadata, tensors) of a synthetic model with the reference's tensor names and layouts.  fast: block-format
    code bytes come from a repeated 64 MiB random pool (benchmark models)."""
    T = dict(TYPES, **(types or {}))
    rng = np.random.default_rng(seed)
    pool = rng.integers(0, 256, size=64 << 20, dtype=np.uint8) if fast else None
    d = dict(dims)
    D, NL, NH, NKV, NE, NEU = d["D"], d["NL"], d["NH"], d["NKV"], d["NE"], d["NEU"]
    FFE, FFS, NKH, NVH, HC, HCR, V = d["FFE"], d["FFS"], d["NKH"], d["NVH"], d["HC"], d["HCR"], d["VOCAB"]
    HD, DS, IXH, IXD = 256, 128, 4, 128
    HCD, DINNER = HC * D, NVH * DS
    CONV = 2 * NKH * DS + DINNER
    a = "qwen4exp."
    kv = {"general.architecture": "qwen4exp", "general.name": "synthetic FAIE2-FlashNext",
          a + "block_count": NL, a + "embedding_length": D, a + "attention.head_count": NH,
          a + "attention.head_count_kv": NKV, a + "rope.freq_base": 1e7,
          a + "attention.layer_norm_rms_epsilon": 1e-6, a + "expert_count": NE, a + "expert_used_count": NEU,
          a + "attention.key_length": HD, a + "attention.value_length": HD, a + "expert_feed_forward_length": FFE,
          a + "expert_shared_feed_forward_length": FFS, a + "ssm.conv_kernel": 4, a + "ssm.state_size": DS,
          a + "ssm.group_count": NKH, a + "ssm.time_step_rank": NVH, a + "ssm.inner_size": DINNER,
          a + "full_attention_interval": d["attn_every"], a + "rope.dimension_count": 64,
          a + "hyper_connection.count": HC, a + "hyper_connection.low_rank": HCR,
          a + "attention.indexer.head_count": IXH, a + "attention.indexer.key_length": IXD,
          a + "attention.indexer.top_k": d["top_k"]}
    ple = list(d.get("ple_layers", []))
    if ple:
        sizes = list(d["ple_sizes"])
        offs = [int(v) for v in np.concatenate([[0], np.cumsum(sizes)[:-1]])]
        kv.update({a + "ple.layers": ple, a + "ple.ngram_size": 3, a + "ple.heads_per_ngram": d["ple_heads_per_ngram"],
                   a + "ple.conv_kernel": 4, a + "ple.eos_token_id": d["ple_eos"],
                   a + "embedding_length_per_layer_input": d["ple_hd"], a + "ple.layer_multipliers": list(d["ple_mult"]),
                   a + "ple.head_offsets": offs, a + "ple.head_vocab_sizes": sizes})
    ts = []

    def W(name, ty, rows, cols, n3=1, std=None):
        raw = random_weight(ty, rows * n3, cols, rng, std, pool)
        dims_ = [cols, rows] + ([n3] if n3 > 1 else [])
        ts.append((name, ty, dims_, raw))

    def V_(name, n, mean=0.0, std=1.0, dims_=None):
        ts.append((name, F32, dims_ or [n], rng.normal(mean, std, n).astype(np.float32).tobytes()))

    W("token_embd.weight", T["token_embd"], V, D, std=1.0)
    W("output.weight", T["output"], V, D)
    V_("output_hc_norm.weight", HCD, 1.0, 0.1)
    W("output_hc_down.weight", T["hc"], HCR, HCD)
    W("output_hc_up.weight", T["hc"], HCD, HCR)
    for il in range(NL):
        p = f"blk.{il}."
        attn = d["attn_every"] > 0 and (il + 1) % d["attn_every"] == 0
        for part in ("attn", "ffn"):
            V_(p + f"hc_{part}_norm.weight", HCD, 1.0, 0.1)
            W(p + f"hc_{part}_down.weight", T["hc"], HCR, HCD)
            W(p + f"hc_{part}_inject.weight", T["hc"], HC, HCD)
            W(p + f"hc_{part}_up.weight", T["hc"], HCD, HCR)
        if not attn:
            W(p + "attn_qkv.weight", T["attn_qkv"], CONV, D)
            W(p + "attn_gate.weight", pick(T["attn_gate"], il), DINNER, D)
            W(p + "ssm_alpha.weight", T["ssm_ab"], NVH, D)
            W(p + "ssm_beta.weight", T["ssm_ab"], NVH, D)
            W(p + "ssm_out.weight", T["ssm_out"], D, DINNER)
            V_(p + "ssm_conv1d.weight", CONV * 4, 0.0, 0.3, dims_=[4, CONV])
            V_(p + "ssm_dt.bias", NVH, 0.0, 0.5)
            ts.append((p + "ssm_a", F32, [NVH], (-np.exp(rng.normal(0.0, 0.5, NVH))).astype(np.float32).tobytes()))
            V_(p + "ssm_norm.weight", DS, 1.0, 0.1)
        else:
            W(p + "attn_q.weight", T["attn_q"], NH * 2 * HD, D)
            W(p + "attn_k.weight", T["attn_k"], NKV * HD, D)
            W(p + "attn_v.weight", T["attn_v"], NKV * HD, D)
            W(p + "attn_output.weight", T["attn_output"], D, NH * HD)
            V_(p + "attn_q_norm.weight", HD, 1.0, 0.1)
            V_(p + "attn_k_norm.weight", HD, 1.0, 0.1)
            W(p + "indexer.q_proj.weight", T["indexer"], IXH * IXD, D)
            W(p + "indexer.k_proj.weight", T["indexer"], IXD, D)
            V_(p + "indexer.q_norm.weight", IXD, 1.0, 0.1)
            V_(p + "indexer.k_norm.weight", IXD, 1.0, 0.1)
        if il in ple:
            W(p + "ple_key.weight", T["ple"], HCD, D)
            W(p + "ple_value.weight", T["ple"], D, D)
            for nm in ("key", "query", "conv"):
                V_(p + f"ple_norm_{nm}.weight", HCD, 1.0, 0.1)
            ts.append((p + "ple_conv1d.weight", F16, [4, HCD],
                       rng.normal(0.0, 0.3, HCD * 4).astype(np.float16).tobytes()))
        W(p + "ffn_gate_inp.weight", T["router"], NE, D, std=2.0 / np.sqrt(D))
        ts.append((p + "ffn_gate_inp_shexp.weight", T["router"], [D],
                   random_weight(T["router"], 1, D, rng)))
        W(p + "ffn_gate_shexp.weight", T["shexp_gate"], FFS, D)
        W(p + "ffn_up_shexp.weight", T["shexp_up"], FFS, D)
        W(p + "ffn_down_shexp.weight", T["shexp_down"], D, FFS)
        W(p + "ffn_gate_exps.weight", pick(T["exps_gate"], il), FFE, D, NE)
        W(p + "ffn_up_exps.weight", pick(T["exps_up"], il), FFE, D, NE)
        W(p + "ffn_down_exps.weight", pick(T["exps_down"], il), D, FFE, NE)
    if ple:
        W("per_layer_token_embd.weight", T["ple_table"], sum(d["ple_sizes"]), d["ple_hd"], std=1.0)
    return kv, ts


def write_model(path, dims=None, seed=0, types=None, shard2=None, fast=False):
    """Write a synthetic model GGUF; returns (metadata, tensors) as written.  With shard2, the n-gram table goes to
    that second file instead (as in the reference model's two shards)."""
    kv, ts = model_tensors(dims or TINY_DIMS, seed, types, fast)
    if shard2:
        table = [t for t in ts if t[0] == "per_layer_token_embd.weight"]
        write_gguf(path, kv, [t for t in ts if t[0] != "per_layer_token_embd.weight"])
        write_gguf(shard2, {"general.architecture": kv["general.architecture"]}, table)
    else:
        write_gguf(path, kv, ts)
    return kv, ts

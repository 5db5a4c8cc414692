"""Float64 CPU oracle of the decode-attention path (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py import this package, and only as
the checker: the product path (libfaie2fn.so and its ctypes layer) never routes through it.

Two independent restatements of the reference arithmetic live here:

* ``liboracle_fn.so`` built from ``fn_oracle.c`` (C, float64, OpenMP), bound below with ctypes;
* ``oracle.twin``, a vectorised numpy float64 twin written separately, used to cross-check the C oracle.

Pinning status of each function (what checks it beyond retyping its formula) is recorded in the tests:
``tests/test_oracle_pins.py`` (closed forms, invariants, exact rational brute force, the transformers Qwen3-Next
library routines, C oracle == numpy twin) and ``tests/test_quant_pins.py`` (the GGUF weight decode: numpy twin,
blocks packed from chosen codes, library fp16 / bf16 conversions).
"""

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_fn.so")

_F32 = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_F64 = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_I32 = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_U8 = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")

_lib = None


def build():
    """Compile liboracle_fn.so with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-B", "-C", HERE], check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        d = C.CDLL(LIB_PATH)
        d.orc_set_threads.argtypes = [C.c_int]
        d.orc_max_threads.restype = C.c_int
        d.orc_gdn_core.argtypes = [C.c_int] * 7 + [_F32] * 5 + [_F64, _F64]
        d.orc_gdn_block.argtypes = ([C.c_int] * 8 + [_F32, _F32, _F64, _F32, _F32, _F32, _F64, _F32, _F32,
                                                      C.c_double, _F64])
        d.orc_rope_inv_freq.argtypes = [C.c_int, C.c_double, _F32]
        d.orc_attn.argtypes = ([C.c_int] * 5 + [C.c_double, C.c_double, C.c_int, _I32] + [_F32] * 5 +
                               [C.c_int, _F32, _F32, _F64, _F64, _F64])
        d.orc_attn_masked.argtypes = ([C.c_int] * 5 + [C.c_double, C.c_double, C.c_int, _I32] + [_F32] * 5 +
                                      [C.c_int, _F32, _F32, _U8, C.c_int, C.c_int, C.c_int, _F64, _F64, _F64])
        d.orc_ix_prep.argtypes = ([C.c_int] * 6 + [C.c_double, C.c_double, C.c_int, _I32, _F32, _F32, _F32, _F64,
                                                   _F32, _F64])
        d.orc_ix_blocks.argtypes = ([C.c_int] * 4 + [C.c_double, C.c_double] + [C.c_int] * 3 + [_F32, _F32, _F64])
        d.orc_ix_score.argtypes = [C.c_int] * 6 + [_I32, _F64, _F64, _F64]
        d.orc_f16_to_f32.argtypes = [C.c_uint16]
        d.orc_f16_to_f32.restype = C.c_float
        d.orc_qblock.argtypes = [C.c_uint32, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        d.orc_dequant.argtypes = [C.c_uint32, _U8, C.c_int, C.c_int, _F32]
        d.orc_gemv.argtypes = [C.c_uint32, _U8, C.c_int, C.c_int, _F32, C.c_int, _F64]
        _lib = d
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def set_threads(n):
    lib().orc_set_threads(int(n))


def max_threads():
    return lib().orc_max_threads()


def gdn_core(q, k, v, beta, g, S, head_map=0):
    """DeltaNet core on normalised q, k.  q,k [B,nt,nkh,dk]; v [B,nt,nvh,dv]; beta, g [B,nt,nvh]; S [B,nvh,dk,dv]
    float64, updated in place.  Returns o [B,nt,nvh,dv] float64."""
    B, nt, nkh, dk = q.shape
    nvh, dv = v.shape[2], v.shape[3]
    assert S.dtype == np.float64 and S.flags.c_contiguous and S.shape == (B, nvh, dk, dv)
    o = np.zeros((B, nt, nvh, dv), np.float64)
    lib().orc_gdn_core(B, nkh, nvh, dk, dv, head_map, nt, _f32(q), _f32(k), _f32(v), _f32(beta), _f32(g), S, o)
    return o


def gdn_block(qkv, conv_w, conv_state, ab, dt_bias, ssm_a, S, z, norm_w, nkh, nvh, dk=128, dv=128, head_map=0,
              gate_act=0, eps=1e-6):
    """Fused DeltaNet block.  qkv [B,nt,C]; conv_w [C,4]; conv_state [B,3,C] float64 (in place); ab [B,nt,2nvh];
    dt_bias, ssm_a [nvh]; S [B,nvh,dk,dv] float64 (in place); z [B,nt,nvh*dv]; norm_w [dv].
    Returns out [B,nt,nvh*dv] float64."""
    B, nt, Cc = qkv.shape
    assert Cc == 2 * nkh * dk + nvh * dv
    assert conv_state.dtype == np.float64 and conv_state.flags.c_contiguous and conv_state.shape == (B, 3, Cc)
    assert S.dtype == np.float64 and S.flags.c_contiguous and S.shape == (B, nvh, dk, dv)
    out = np.zeros((B, nt, nvh * dv), np.float64)
    lib().orc_gdn_block(B, nkh, nvh, dk, dv, head_map, gate_act, nt, _f32(qkv), _f32(conv_w), conv_state, _f32(ab),
                        _f32(dt_bias), _f32(ssm_a), S, _f32(z), _f32(norm_w), float(eps), out)
    return out


def rope_inv_freq(nrot, theta):
    inv = np.zeros(nrot // 2 + 1, np.float32)
    lib().orc_rope_inv_freq(nrot, float(theta), inv)
    return inv[: nrot // 2]


def attn(qg, knew, vnew, wq, wk, Kc, Vc, pos, nrot=64, theta=1e7, eps=1e-6, mask=None, ixr=4, top=512):
    """GQA decode.  qg [B,nt,nq,2,hd]; knew, vnew [B,nt,nkv,hd]; Kc, Vc [B,max_ctx,nkv,hd] fp32 (rows < pos[b]
    read); pos [B] int; mask [B,nt,nblocks] uint8 (QSA block mask, applied to tokens with more than `top` complete
    blocks of ixr keys) or None (dense).  Returns (og [B,nt,nq,hd], k_rows [B,nt,nkv,hd], v_rows) float64."""
    B, nt, nq, two, hd = qg.shape
    assert two == 2
    nkv = knew.shape[2]
    max_ctx = Kc.shape[1]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert pos.shape == (B,) and int(pos.max()) <= max_ctx
    kro = np.zeros((B, nt, nkv, hd), np.float64)
    vro = np.zeros((B, nt, nkv, hd), np.float64)
    og = np.zeros((B, nt, nq, hd), np.float64)
    if mask is None:
        lib().orc_attn(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, pos, _f32(qg), _f32(knew), _f32(vnew),
                       _f32(wq), _f32(wk), max_ctx, _f32(Kc), _f32(Vc), kro, vro, og)
    else:
        mask = np.ascontiguousarray(mask, dtype=np.uint8)
        assert mask.shape[:2] == (B, nt)
        lib().orc_attn_masked(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, pos, _f32(qg), _f32(knew),
                              _f32(vnew), _f32(wq), _f32(wk), max_ctx, _f32(Kc), _f32(Vc), mask, mask.shape[2], ixr, top,
                              kro, vro, og)
    return og, kro, vro


def ix_prep(iqk, wqn, wkn, IKc, BKc, pos, ixh=4, ixd=128, ixr=4, nrot=64, theta=1e7, eps=1e-6):
    """QSA indexer prep.  iqk [B,nt,ixh*ixd+ixd]; IKc [B,max_ctx,ixd] float32 and BKc [B,max_ctx/ixr,ixd] float64
    are updated in place (raw keys appended; blocks completed by this call filled).  Returns Qix [B,nt,ixh,ixd]."""
    B, nt, row = iqk.shape
    assert row == ixh * ixd + ixd
    max_ctx = IKc.shape[1]
    assert IKc.dtype == np.float32 and IKc.flags.c_contiguous and BKc.dtype == np.float64 and BKc.flags.c_contiguous
    Qix = np.zeros((B, nt, ixh, ixd), np.float64)
    lib().orc_ix_prep(B, nt, ixh, ixd, ixr, nrot, float(theta), float(eps), max_ctx,
                      np.ascontiguousarray(pos, dtype=np.int32), _f32(iqk), _f32(wqn), _f32(wkn), Qix, IKc, BKc)
    return Qix


def ix_blocks(IKc, wkn, BKc, j0, j1, ixr=4, nrot=64, theta=1e7, eps=1e-6):
    """Block keys of blocks [j0, j1) of every sequence from the raw keys, into BKc (float64, in place)."""
    B, max_ctx, ixd = IKc.shape
    lib().orc_ix_blocks(B, ixd, ixr, nrot, float(theta), float(eps), max_ctx, j0, j1, _f32(IKc), _f32(wkn), BKc)


def ix_score(Qix, BKc, pos, max_ctx, ixr=4):
    """scores [B,nt,max_ctx/ixr] float64 (entries past each token's complete blocks stay 0)."""
    B, nt, ixh, ixd = Qix.shape
    sc = np.zeros((B, nt, max_ctx // ixr), np.float64)
    lib().orc_ix_score(B, nt, ixh, ixd, ixr, max_ctx, np.ascontiguousarray(pos, dtype=np.int32), _f64(Qix), _f64(BKc), sc)
    return sc


def ix_select(scores, pos, top=512, ixr=4):
    """Block mask [B,nt,nblocks] uint8 of k_ix_select (faie2fn.cu:1557-1607): for a token with nb > top complete
    blocks, the top highest-scoring ones, ties at the threshold kept lowest index first (a stable sort on the
    descending score); other tokens get an all-zero mask (their attention is dense)."""
    B, nt, nbmax = scores.shape
    mask = np.zeros((B, nt, nbmax), np.uint8)
    for b in range(B):
        for t in range(nt):
            nb = (int(pos[b]) + t + 1) // ixr
            if nb <= top:
                continue
            order = np.argsort(-scores[b, t, :nb], kind="stable")
            mask[b, t, order[:top]] = 1
    return mask


def qblock(qtype):
    """(values, bytes) per GGUF block of a weight format this oracle decodes."""
    qk, bb = C.c_int(), C.c_int()
    if not lib().orc_qblock(int(qtype), C.byref(qk), C.byref(bb)):
        raise ValueError(f"unsupported type {qtype}")
    return qk.value, bb.value


def f16_to_f32(bits):
    return float(lib().orc_f16_to_f32(int(bits)))


def dequant(qtype, raw, rows, cols):
    """GGUF rows -> float32 [rows][cols], the values ggml's dequantize_row_* returns."""
    out = np.zeros((rows, cols), np.float32)
    if lib().orc_dequant(int(qtype), np.ascontiguousarray(raw, np.uint8).reshape(-1), rows, cols, out):
        raise ValueError("unsupported type or shape")
    return out


def gemv(qtype, raw, rows, cols, x):
    """float64 y [nt][rows] = decoded W @ x[t] for x [nt][cols]."""
    x = _f32(np.atleast_2d(x))
    y = np.zeros((x.shape[0], rows), np.float64)
    if lib().orc_gemv(int(qtype), np.ascontiguousarray(raw, np.uint8).reshape(-1), rows, cols, x, x.shape[0], y):
        raise ValueError("unsupported type or shape")
    return y


def relerr(got, ref):
    """Normwise error max|got - ref| / max|ref| (the reference's gate metric, flashnext/gate_fn_ref.py:43)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    num = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    if den == 0.0:
        return num
    return num / den

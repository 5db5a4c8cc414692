"""Float64 CPU oracle of the decode-attention path (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py import this package, and only as
the checker: the product path (libfaie2fn.so and its ctypes layer) never routes through it.

Two independent restatements of the reference arithmetic live here:

* ``liboracle_fn.so`` built from ``fn_oracle.c`` (C, float64, OpenMP), bound below with ctypes;
* ``oracle.twin``, a vectorised numpy float64 twin written separately, used to cross-check the C oracle.

Pinning status of each function (what checks it beyond retyping its formula) is recorded in the tests:
``tests/test_oracle_pins.py`` (closed forms, invariants, exact rational brute force, the transformers Qwen3-Next
library routines) and ``tests/test_oracle_twin.py`` (C oracle == numpy twin).
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


def attn(qg, knew, vnew, wq, wk, Kc, Vc, pos, nrot=64, theta=1e7, eps=1e-6):
    """GQA decode.  qg [B,nt,nq,2,hd]; knew, vnew [B,nt,nkv,hd]; Kc, Vc [B,max_ctx,nkv,hd] fp32 (rows < pos[b]
    read); pos [B] int.  Returns (og [B,nt,nq,hd], k_rows [B,nt,nkv,hd], v_rows [B,nt,nkv,hd]) float64."""
    B, nt, nq, two, hd = qg.shape
    assert two == 2
    nkv = knew.shape[2]
    max_ctx = Kc.shape[1]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert pos.shape == (B,) and int(pos.max()) <= max_ctx
    kro = np.zeros((B, nt, nkv, hd), np.float64)
    vro = np.zeros((B, nt, nkv, hd), np.float64)
    og = np.zeros((B, nt, nq, hd), np.float64)
    lib().orc_attn(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, pos, _f32(qg), _f32(knew), _f32(vnew), _f32(wq),
                   _f32(wk), max_ctx, _f32(Kc), _f32(Vc), kro, vro, og)
    return og, kro, vro


def relerr(got, ref):
    """Normwise error max|got - ref| / max|ref| (the reference's gate metric, flashnext/gate_fn_ref.py:43)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    num = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    if den == 0.0:
        return num
    return num / den

"""ctypes host layer for libfaie2fn.so, the MI355X decode-attention engine of FAIE2-FlashNext.

Linux counterpart of the reference's ``flashnext/fn.py`` (class ``FN``, flashnext/fn.py:21-66): the same
argtypes for the reference's entry points, the same ``check()`` that turns a -1 into ``RuntimeError(fn_error())``,
plus the path hooks of this library (``gdn``, ``gdn_block``, ``attn``) and thin wrappers of its device-buffer
entry points.  The library path comes from the ``lib`` argument, else ``$FN_DLL``, else the ``libfaie2fn.so``
built next to this file.  There is no fallback: if the library is missing the constructor raises.
"""

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libfaie2fn.so")
VOCAB = 248320
HCD = 10240
NL = 48

P = np.ctypeslib.ndpointer
F32 = P(np.float32, flags="C_CONTIGUOUS")
I32 = P(np.int32, flags="C_CONTIGUOUS")
U8 = P(np.uint8, flags="C_CONTIGUOUS")
VP = C.c_void_p

# every symbol include/faie2fn.h declares
SYMBOLS = (
    "fn_error", "fn_free", "fn_load", "fn_split", "fn_dev_gb", "fn_n_past", "fn_last_ms", "fn_reset",
    "fn_use_graphs", "fn_forward", "fn_debug_layers", "fn_test_dequant", "fn_gemv_override", "fn_gemv_waves",
    "fn_pdl", "fn_early", "fn_moe_var", "fn_moe_override", "fn_gemv_plan", "fn_bench_hot", "fn_bench_gemv",
    "fn_bench_route", "fn_test_gemv",
    "fn_test_gdn", "fn_test_gdn_block", "fn_test_attn",
    "fn_gdn_block_dev", "fn_gdn_core_dev", "fn_attn_dev", "fn_attn_work_bytes", "fn_attn_nsplit", "fn_advance_dev",
    "fn_fill_normal_dev", "fn_copy_dev",
    "fn_path_init", "fn_path_buffer", "fn_path_step",
    "fn_attn_qsa_dev", "fn_attn_qsa_work_bytes", "fn_ix_blocks_dev", "fn_test_attn_qsa",
    "fn_gemv_packed_bytes", "fn_gemv_pack_dev", "fn_dequant_dev", "fn_gemv_work_bytes", "fn_gemv_dev",
    "fn_gdn_verify_dev", "fn_advance_by_dev", "fn_gdn_block_xab_dev",
    "fn_attn_noalloc_dev", "fn_dev_status", "fn_model_dims", "fn_gemv_group_dev", "fn_stage_events",
    "fn_bench_gdn", "fn_bench_attn",
)

# the shapes fn_model_dims writes, in order (include/faie2fn.h section 6)
MODEL_DIMS = ("D", "NL", "NH", "NKV", "HD", "NROT", "NE", "NEU", "FFE", "FFS", "DS", "NKH", "NVH", "DINNER", "CONVCH",
              "attn_every", "HC", "HCR", "IXH", "IXD", "top", "VOCAB", "PLE_LAYERS", "PLE_HEADS", "PLE_HD")

# status bits of fn_dev_status (include/faie2fn.h)
STATUS_POS, STATUS_KR = 1, 2

# bytes of the device array fn_attn_noalloc_dev takes its workspace from (FN_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 32 << 20

# GGUF type ids of the weight formats this library reads (engine/faie2fn.cu:78-81), and (values, bytes) per block
QTYPES = dict(Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14, IQ2_XXS=16, IQ2_XS=17, IQ3_XXS=18, IQ4_NL=20, IQ3_S=21, IQ2_S=22,
              IQ4_XS=23, BF16=30, Q2_0=42)
QBLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 16: (256, 66), 17: (256, 74), 18: (256, 98),
          20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136), 30: (1, 2), 42: (64, 18)}


def row_bytes(qtype, cols):
    """GGUF bytes of one row of `cols` values."""
    qk, bb = QBLOCK[int(qtype)]
    return cols // qk * bb

# buffer kinds of fn_path_buffer (include/faie2fn.h)
BUF = dict(S=0, CONV_RING=1, QKV=2, AB=3, Z=4, OUT=5, CONV_W=6, DT_BIAS=7, SSM_A=8, NORM_W=9, KC=10, VC=11, QG=12,
           K=13, V=14, OG=15, WQ=16, WK=17, POS=18)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def kv_to_device(Kc, Vc):
    """Reference-layout caches [B][T][nkv][hd] (T a multiple of 64) -> the device layouts of fn_attn_dev:
    K key-tiled [B][nkv][T/64][hd/4][64][4], V head-major [B][nkv][T][hd]."""
    B, T, nkv, hd = Kc.shape
    if T % 64 or hd % 4:
        raise ValueError("cache rows must be a multiple of 64 and head_dim a multiple of 4")
    Kd = Kc.reshape(B, T // 64, 64, nkv, hd // 4, 4).transpose(0, 3, 1, 4, 2, 5)
    Vd = Vc.transpose(0, 2, 1, 3)
    return np.ascontiguousarray(Kd, np.float32), np.ascontiguousarray(Vd, np.float32)


def kv_from_device(Kd, Vd, B, T, nkv, hd):
    """Inverse of kv_to_device."""
    K = np.asarray(Kd).reshape(B, nkv, T // 64, hd // 4, 64, 4).transpose(0, 2, 4, 1, 3, 5).reshape(B, T, nkv, hd)
    V = np.asarray(Vd).reshape(B, nkv, T, hd).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(K), np.ascontiguousarray(V)


class FN:
    def __init__(self, lib=None):
        path = lib or os.environ.get("FN_DLL") or LIB
        if not os.path.exists(path):
            raise RuntimeError(f"libfaie2fn.so not found at {path}: build it first (__graft_entry__.build())")
        d = self.d = C.CDLL(path)
        # the reference's bindings (flashnext/fn.py:26-34)
        d.fn_error.restype = C.c_char_p
        d.fn_load.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int]
        d.fn_forward.argtypes = [I32, C.c_int, C.c_void_p, C.c_void_p]
        d.fn_debug_layers.argtypes = [C.c_void_p]
        d.fn_test_dequant.argtypes = [C.c_uint32, U8, C.c_int, C.c_int, F32]
        d.fn_test_gemv.argtypes = [C.c_uint32, U8, C.c_int, C.c_int, F32, C.c_int, F32]
        d.fn_dev_gb.restype = C.c_double
        d.fn_dev_gb.argtypes = [C.c_int]
        d.fn_last_ms.restype = C.c_double
        # path hooks
        i = C.c_int
        d.fn_test_gdn.argtypes = [i] * 7 + [F32] * 7
        d.fn_test_gdn_block.argtypes = [i] * 8 + [F32] * 9 + [C.c_float, F32]
        d.fn_test_attn.argtypes = ([i] * 5 + [C.c_float, C.c_float, i, i, I32] + [F32] * 7 + [i, F32])
        d.fn_gdn_block_dev.argtypes = [i] * 9 + [VP] * 10 + [C.c_float, VP, VP]
        d.fn_gdn_core_dev.argtypes = [i] * 7 + [VP] * 7 + [VP]
        d.fn_gdn_verify_dev.argtypes = [i] * 9 + [VP, VP, i] + [VP] * 11 + [C.c_float, VP, VP]
        d.fn_gdn_block_xab_dev.argtypes = [i] * 8 + [VP] * 5 + [i] + [VP] * 6 + [C.c_float, VP, VP]
        d.fn_advance_by_dev.argtypes = [VP, VP, i, VP]
        d.fn_attn_dev.argtypes = ([i] * 5 + [C.c_float, C.c_float, i, i] + [VP] * 8 + [i, VP, C.c_size_t, VP, VP])
        d.fn_attn_noalloc_dev.argtypes = ([i] * 5 + [C.c_float, C.c_float, i, i] + [VP] * 8 + [i, VP, VP])
        d.fn_attn_work_bytes.restype = C.c_size_t
        d.fn_attn_work_bytes.argtypes = [i] * 5
        d.fn_attn_nsplit.argtypes = [i] * 4
        d.fn_advance_dev.argtypes = [VP, i, i, VP]
        d.fn_fill_normal_dev.argtypes = [VP, C.c_size_t, C.c_uint64, C.c_float, C.c_float, VP]
        d.fn_copy_dev.argtypes = [VP, VP, C.c_size_t, VP]
        d.fn_stage_events.argtypes = [C.POINTER(VP), C.c_int]
        d.fn_bench_gdn.argtypes = [C.c_int] * 5 + [C.POINTER(C.c_float)]
        d.fn_bench_attn.argtypes = [C.c_int] * 6 + [C.POINTER(C.c_float)]
        d.fn_path_init.argtypes = [i] * 11
        d.fn_path_buffer.argtypes = [i, i, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
        d.fn_path_step.argtypes = [i, C.POINTER(C.c_float)]
        d.fn_use_graphs.argtypes = [i]
        f = C.c_float
        d.fn_attn_qsa_dev.argtypes = [i] * 5 + [f, f, i, i] + [VP] * 13 + [i, i, VP, C.c_size_t, VP, VP]
        d.fn_attn_qsa_work_bytes.restype = C.c_size_t
        d.fn_attn_qsa_work_bytes.argtypes = [i] * 7
        d.fn_ix_blocks_dev.argtypes = [i] * 4 + [VP] * 3 + [i, f, f, VP]
        d.fn_test_attn_qsa.argtypes = [i] * 5 + [f, f, i, i, I32] + [F32] * 11 + [i, i, F32, VP, VP]
        d.fn_n_past.restype = C.c_int
        u32, sz = C.c_uint32, C.c_size_t
        d.fn_gemv_plan.argtypes = [u32, i, i, I32]
        d.fn_bench_gemv.argtypes = [u32, i, i, i, i, C.POINTER(C.c_float)]
        d.fn_bench_route.argtypes = [i, i, i, VP, i, VP, VP, VP]
        d.fn_gemv_override.argtypes = [i] * 4
        d.fn_gemv_waves.argtypes = [i]
        d.fn_model_dims.argtypes = [C.c_char_p, I32, i]
        d.fn_dev_status.argtypes = [i]
        d.fn_bench_hot.argtypes = [i]
        d.fn_gemv_packed_bytes.restype = sz
        d.fn_gemv_packed_bytes.argtypes = [u32, i, i]
        d.fn_gemv_pack_dev.argtypes = [u32, VP, i, i, VP, VP]
        d.fn_dequant_dev.argtypes = [u32, VP, i, i, VP, VP]
        d.fn_gemv_work_bytes.restype = sz
        d.fn_gemv_work_bytes.argtypes = [u32, i, i, i]
        d.fn_gemv_dev.argtypes = [u32, VP, i, i, VP, i, VP, VP, sz, VP]
        d.fn_gemv_group_dev.argtypes = [i, VP, VP, i, VP, VP, i, VP, VP]

    def check(self, rc):
        if rc != 0:
            raise RuntimeError(self.d.fn_error().decode())

    # ---- the reference's methods (flashnext/fn.py:40-66) ----
    def load(self, shard1, shard2="", max_ctx=32768, split=0):
        self.check(self.d.fn_load(shard1.encode(), (shard2 or "").encode(), max_ctx, split))
        self.vocab = self.model_dims(shard1)["VOCAB"]

    def model_dims(self, path):
        """The model shapes fn_load reads from a GGUF file (no device work)."""
        out = np.zeros(32, np.int32)
        n = self.d.fn_model_dims(path.encode(), out, len(out))
        if n < 0:
            raise RuntimeError(self.d.fn_error().decode())
        return dict(zip(MODEL_DIMS, out[:n].tolist()))

    def reset(self):
        self.check(self.d.fn_reset())

    def forward(self, tokens, logits=False):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        am = np.zeros(len(t), np.int32)
        lg = np.zeros((len(t), getattr(self, "vocab", VOCAB)), np.float32) if logits else None
        self.check(self.d.fn_forward(t, len(t), lg.ctypes.data if logits else None, am.ctypes.data))
        return (am, lg) if logits else am

    def debug_layers(self, buf):
        self.check(self.d.fn_debug_layers(buf.ctypes.data if buf is not None else None))

    def dequant(self, qtype, raw, rows, cols):
        out = np.zeros((rows, cols), np.float32)
        self.check(self.d.fn_test_dequant(int(qtype), np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1), rows, cols,
                                          out))
        return out

    def gemv(self, qtype, raw, rows, cols, x):
        nt = x.shape[0]
        y = np.zeros((nt, rows), np.float32)
        self.check(self.d.fn_test_gemv(int(qtype), np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1), rows, cols,
                                       _f32(x), nt, y))
        return y

    def gemv_plan(self, qtype, rows, cols):
        """{values per group, 16-lane groups per row (wpt), split-K, rows per workgroup pass, waves per workgroup,
        workgroups along the rows (0: persistent), groups per row} of a weight."""
        out = np.zeros(7, np.int32)
        self.check(self.d.fn_gemv_plan(int(qtype), rows, cols, out))
        return [int(v) for v in out]

    def bench_gemv(self, qtype, rows, cols, nt=1, iters=50):
        """ms per GEMV call, weights cold (fn_bench_hot(0)) or hot."""
        ms = C.c_float(0.0)
        self.check(self.d.fn_bench_gemv(int(qtype), rows, cols, nt, iters, C.byref(ms)))
        return ms.value

    def bench_route(self, variant, part, nt, iters=1):
        """MoE routing of nt tokens on router partials part [ks][8][528]: (sel [nt][10], weights [nt][10], ms per
        call); variant 0 ranks every expert, 1 is the model's one-wave routing."""
        part = np.ascontiguousarray(part, dtype=np.float32)
        if part.ndim != 3 or part.shape[1:] != (8, 528):
            raise ValueError("part must be [ks][8][528] float32")
        sel = np.zeros((nt, 10), np.int32)
        w = np.zeros((nt, 10), np.float32)
        ms = np.zeros(1, np.float32)
        self.check(self.d.fn_bench_route(variant, nt, part.shape[0], part.ctypes.data, iters, sel.ctypes.data,
                                         w.ctypes.data, ms.ctypes.data))
        return sel, w, float(ms[0])

    def gemv_override(self, ks=0, lpr=0, kernel=0, waves_per_cu=0):
        """Force the GEMV plan (0 = automatic): split-K, lanes per row (16, 32, 64; passed as the reference's wpt,
        16-lane groups per row), kernel (1 x in chunks, 2 x staged once, 3 / 4 x staged once with the deep / short
        walk) and the resident waves per CU the persistent grid is sized for."""
        wpt = int(lpr) // 16 if int(lpr) in (16, 32, 64) else (5 if lpr else 0)  # 5: an invalid split (ignored)
        self.d.fn_gemv_override(wpt, int(ks), int(kernel), int(waves_per_cu))

    def moe_override(self, waves_per_row=-1):
        """Force the MoE output kernel by the waves that share one output row (the reference's dn_wpt): 1 = 16 rows
        a workgroup, 2 or more = 4 rows a workgroup; negative = automatic.  Graphs captured before keep their kernel
        (use_graphs drops them)."""
        self.d.fn_moe_override(0, 0, int(waves_per_row), 0)

    def bench_hot(self, on):
        self.d.fn_bench_hot(1 if on else 0)

    # ---- path hooks (host arrays, synchronous) ----
    def gdn(self, q, k, v, beta, g, S, head_map=0):
        """DeltaNet core.  q,k [B,nt,nkh,dk]; v [B,nt,nvh,dv]; beta, g [B,nt,nvh]; S [B,nvh,dk,dv] float32,
        updated in place.  Returns o [B,nt,nvh,dv]."""
        B, nt, nkh, dk = q.shape
        nvh, dv = v.shape[2], v.shape[3]
        if S.dtype != np.float32 or not S.flags.c_contiguous or S.shape != (B, nvh, dk, dv):
            raise ValueError("S must be a C-contiguous float32 [B, nvh, dk, dv] array")
        o = np.zeros((B, nt, nvh, dv), np.float32)
        self.check(self.d.fn_test_gdn(B, nkh, nvh, dk, dv, head_map, nt, _f32(q), _f32(k), _f32(v), _f32(beta),
                                      _f32(g), S, o))
        return o

    def gdn_block(self, qkv, conv_w, conv_state, ab, dt_bias, ssm_a, S, z, norm_w, nkh, nvh, dk=128, dv=128,
                  head_map=0, gate_act=0, eps=1e-6):
        """Fused DeltaNet block.  conv_state [B,3,C] and S [B,nvh,dk,dv] float32 are updated in place.
        Returns out [B,nt,nvh*dv]."""
        B, nt, Cc = qkv.shape
        for name, arr, shape in (("conv_state", conv_state, (B, 3, Cc)), ("S", S, (B, nvh, dk, dv))):
            if arr.dtype != np.float32 or not arr.flags.c_contiguous or arr.shape != shape:
                raise ValueError(f"{name} must be a C-contiguous float32 {shape} array")
        out = np.zeros((B, nt, nvh * dv), np.float32)
        self.check(self.d.fn_test_gdn_block(B, nkh, nvh, dk, dv, head_map, gate_act, nt, _f32(qkv), _f32(conv_w),
                                            conv_state, _f32(ab), _f32(dt_bias), _f32(ssm_a), S, _f32(z),
                                            _f32(norm_w), float(eps), out))
        return out

    def attn(self, qg, k, v, wq, wk, Kc, Vc, pos, nrot=64, theta=1e7, eps=1e-6, nsplit=0):
        """GQA decode.  qg [B,nt,nq,2,hd]; k, v [B,nt,nkv,hd]; Kc, Vc [B,max_ctx,nkv,hd] float32 (rows
        pos[b]..pos[b]+nt-1 are written in place); pos [B].  Returns og [B,nt,nq,hd]."""
        B, nt, nq, two, hd = qg.shape
        nkv = k.shape[2]
        max_ctx = Kc.shape[1]
        for name, arr in (("Kc", Kc), ("Vc", Vc)):
            if arr.dtype != np.float32 or not arr.flags.c_contiguous or arr.shape != (B, max_ctx, nkv, hd):
                raise ValueError(f"{name} must be a C-contiguous float32 [B, max_ctx, nkv, hd] array")
        og = np.zeros((B, nt, nq, hd), np.float32)
        self.check(self.d.fn_test_attn(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, max_ctx,
                                       np.ascontiguousarray(pos, dtype=np.int32), _f32(qg), _f32(k), _f32(v), _f32(wq),
                                       _f32(wk), Kc, Vc, int(nsplit), og))
        return og

    def attn_qsa(self, qg, k, v, wq, wk, Kc, Vc, iqk, wqn, wkn, IKc, pos, top=512, nsplit=0, nrot=64, theta=1e7,
                 eps=1e-6):
        """Sparse (QSA) GQA decode.  As attn(), plus iqk [B,nt,640], wqn, wkn [128], IKc [B,max_ctx,128] float32
        (new raw index keys written in place).  Returns (og [B,nt,nq,hd], scores [B,nt,max_ctx/4],
        mask [B,nt,max_ctx/4] uint8)."""
        B, nt, nq, two, hd = qg.shape
        nkv = k.shape[2]
        max_ctx = Kc.shape[1]
        for name, arr, shape in (("Kc", Kc, (B, max_ctx, nkv, hd)), ("Vc", Vc, (B, max_ctx, nkv, hd)),
                                 ("IKc", IKc, (B, max_ctx, 128))):
            if arr.dtype != np.float32 or not arr.flags.c_contiguous or arr.shape != shape:
                raise ValueError(f"{name} must be a C-contiguous float32 {shape} array")
        og = np.zeros((B, nt, nq, hd), np.float32)
        sc = np.zeros((B, nt, max_ctx // 4), np.float32)
        mask = np.zeros((B, nt, max_ctx // 4), np.uint8)
        self.check(self.d.fn_test_attn_qsa(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, max_ctx,
                                           np.ascontiguousarray(pos, dtype=np.int32), _f32(qg), _f32(k), _f32(v),
                                           _f32(wq), _f32(wk), Kc, Vc, _f32(iqk), _f32(wqn), _f32(wkn), IKc, int(top),
                                           int(nsplit), og, sc.ctypes.data, mask.ctypes.data))
        return og, sc, mask

    # ---- device entry points (integers are device addresses; stream is a HIP stream handle or 0) ----
    def gdn_block_dev(self, B, nkh, nvh, nt, ring, pos, qkv, conv_w, conv_ring, ab, dt_bias, ssm_a, S, z, norm_w,
                      out, stream=0, dk=128, dv=128, head_map=0, gate_act=0, eps=1e-6):
        self.check(self.d.fn_gdn_block_dev(B, nkh, nvh, dk, dv, head_map, gate_act, nt, ring, pos, qkv, conv_w,
                                           conv_ring, ab, dt_bias, ssm_a, S, z, norm_w, float(eps), out, stream))

    def gdn_block_xab_dev(self, B, nkh, nvh, ring, pos, qkv, conv_w, conv_ring, x, hidden, w_ab, dt_bias, ssm_a, S,
                          z, norm_w, out, stream=0, dk=128, dv=128, head_map=0, gate_act=0, eps=1e-6):
        """One decode token of the fused block with the alpha/beta projection inside: ab = w_ab . x (w_ab BF16
        [2 nvh][hidden], x fp32 [B][hidden], both device pointers) instead of a precomputed ab."""
        self.check(self.d.fn_gdn_block_xab_dev(B, nkh, nvh, dk, dv, head_map, gate_act, ring, pos, qkv, conv_w,
                                               conv_ring, x, hidden, w_ab, dt_bias, ssm_a, S, z, norm_w, float(eps),
                                               out, stream))

    def gdn_verify_dev(self, B, nkh, nvh, nt, ring, pos, kr, rnt, rqkv, rab, qkv, conv_w, conv_ring, ab, dt_bias,
                       ssm_a, S, z, norm_w, out, stream=0, dk=128, dv=128, head_map=0, gate_act=0, eps=1e-6):
        """Verify step with deferred commit (include/faie2fn.h): replay kr[b] accepted tokens of the previous call,
        write the committed state, then run nt new tokens without writing state."""
        self.check(self.d.fn_gdn_verify_dev(B, nkh, nvh, dk, dv, head_map, gate_act, nt, ring, pos, kr, rnt, rqkv,
                                            rab, qkv, conv_w, conv_ring, ab, dt_bias, ssm_a, S, z, norm_w, float(eps),
                                            out, stream))

    def advance_by_dev(self, pos, kr, B, stream=0):
        self.check(self.d.fn_advance_by_dev(pos, kr, B, stream))

    def gdn_core_dev(self, B, nkh, nvh, nt, q, k, v, beta, g, S, o, stream=0, dk=128, dv=128, head_map=0):
        self.check(self.d.fn_gdn_core_dev(B, nkh, nvh, dk, dv, head_map, nt, q, k, v, beta, g, S, o, stream))

    def attn_work_bytes(self, B, nq, nt, nsplit, hd=256):
        return int(self.d.fn_attn_work_bytes(B, nq, nt, hd, nsplit))

    def attn_nsplit(self, B, nkv, nt, ctx):
        return int(self.d.fn_attn_nsplit(B, nkv, nt, ctx))

    def attn_dev(self, B, nq, nkv, nt, max_ctx, pos, qg, k, v, wq, wk, Kc, Vc, nsplit, work, work_bytes, og,
                 stream=0, hd=256, nrot=64, theta=1e7, eps=1e-6):
        self.check(self.d.fn_attn_dev(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, max_ctx, pos, qg, k, v, wq,
                                      wk, Kc, Vc, nsplit, work, work_bytes, og, stream))

    def attn_noalloc_dev(self, B, nq, nkv, nt, max_ctx, pos, qg, k, v, wq, wk, Kc, Vc, nsplit, og, stream=0, hd=256,
                         nrot=64, theta=1e7, eps=1e-6):
        self.check(self.d.fn_attn_noalloc_dev(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, max_ctx, pos, qg, k,
                                              v, wq, wk, Kc, Vc, nsplit, og, stream))

    def attn_qsa_work_bytes(self, B, nq, nt, nsplit, max_ctx, top=512, hd=256):
        return int(self.d.fn_attn_qsa_work_bytes(B, nq, nt, hd, nsplit, max_ctx, top))

    def attn_qsa_dev(self, B, nq, nkv, nt, max_ctx, pos, qg, k, v, wq, wk, Kc, Vc, iqk, wqn, wkn, IKc, BKc, top, nsplit,
                     work, work_bytes, og, stream=0, hd=256, nrot=64, theta=1e7, eps=1e-6):
        self.check(self.d.fn_attn_qsa_dev(B, nq, nkv, hd, nrot, float(theta), float(eps), nt, max_ctx, pos, qg, k, v,
                                          wq, wk, Kc, Vc, iqk, wqn, wkn, IKc, BKc, top, nsplit, work, work_bytes, og,
                                          stream))

    def ix_blocks_dev(self, B, max_ctx, j0, j1, IKc, wkn, BKc, stream=0, nrot=64, theta=1e7, eps=1e-6):
        self.check(self.d.fn_ix_blocks_dev(B, max_ctx, j0, j1, IKc, wkn, BKc, nrot, float(theta), float(eps), stream))

    def dev_status(self, clear=True):
        """FN_STATUS_* bits the kernels recorded on the current device (synchronizes it); cleared unless clear=False."""
        r = self.d.fn_dev_status(1 if clear else 0)
        if r < 0:
            raise RuntimeError(self.d.fn_error().decode())
        return r

    def advance_dev(self, pos, B, nt, stream=0):
        self.check(self.d.fn_advance_dev(pos, B, nt, stream))

    def fill_normal_dev(self, ptr, n, seed, mean=0.0, std=1.0, stream=0):
        self.check(self.d.fn_fill_normal_dev(ptr, n, seed, float(mean), float(std), stream))

    def copy_dev(self, dst, src, nbytes, stream=0):
        self.check(self.d.fn_copy_dev(dst, src, nbytes, stream))

    def bench_gdn(self, B, nkh=16, nvh=32, nt=1, iters=20):
        """µs per layer-step of the fused DeltaNet block, cold state, graph-replayed (fn_bench_gdn)."""
        us = C.c_float(0.0)
        self.check(self.d.fn_bench_gdn(B, nkh, nvh, nt, iters, C.byref(us)))
        return us.value

    def bench_attn(self, B, ctx, nq=16, nkv=2, nt=1, iters=20):
        """µs per layer-step of GQA decode at context ctx, cold caches, graph-replayed (fn_bench_attn)."""
        us = C.c_float(0.0)
        self.check(self.d.fn_bench_attn(B, nq, nkv, ctx, nt, iters, C.byref(us)))
        return us.value

    def stage_events(self, handles):
        """Record handles[0], handles[1], ... after each kernel launch of the attention entry points (an empty list
        clears); handles are hipEvent_t values (hiprt.Event.handle)."""
        arr = (VP * max(1, len(handles)))(*handles)
        self.check(self.d.fn_stage_events(arr, len(handles)))

    def gemv_packed_bytes(self, qtype, rows, cols):
        return int(self.d.fn_gemv_packed_bytes(int(qtype), rows, cols))

    def gemv_work_bytes(self, qtype, rows, cols, nt):
        return int(self.d.fn_gemv_work_bytes(int(qtype), rows, cols, nt))

    def gemv_pack_dev(self, qtype, raw, rows, cols, packed, stream=0):
        self.check(self.d.fn_gemv_pack_dev(int(qtype), raw, rows, cols, packed, stream))

    def dequant_dev(self, qtype, packed, rows, cols, out, stream=0):
        self.check(self.d.fn_dequant_dev(int(qtype), packed, rows, cols, out, stream))

    def gemv_dev(self, qtype, packed, rows, cols, x, nt, y, work, work_bytes, stream=0):
        self.check(self.d.fn_gemv_dev(int(qtype), packed, rows, cols, x, nt, y, work, work_bytes, stream))

    def gemv_group_dev(self, types, rows, cols, packed, x, nt, ys, stream=0):
        n = len(types)
        ty = (C.c_uint32 * n)(*[int(t) for t in types])
        rw = (C.c_int * n)(*[int(r) for r in rows])
        pk = (VP * n)(*packed)
        yp = (VP * n)(*ys)
        self.check(self.d.fn_gemv_group_dev(n, ty, rw, cols, pk, x, nt, yp, stream))

    # ---- path engine ----
    def path_init(self, B, nl, attn_every=4, nkh=16, nvh=32, nq=16, nkv=2, max_ctx=4096, head_map=0, gate_act=0,
                  nsplit=0):
        self.check(self.d.fn_path_init(B, nl, attn_every, nkh, nvh, nq, nkv, max_ctx, head_map, gate_act, nsplit))

    def path_buffer(self, il, kind):
        """(device address, bytes) of buffer `kind` (a BUF name or number) of layer il."""
        k = BUF[kind] if isinstance(kind, str) else int(kind)
        p, n = C.c_void_p(), C.c_size_t()
        self.check(self.d.fn_path_buffer(il, k, C.byref(p), C.byref(n)))
        return p.value, n.value

    def path_step(self, steps=1, timed=False):
        """steps decode steps through all layers; returns HIP-event ms per step when timed."""
        ms = C.c_float(0.0)
        self.check(self.d.fn_path_step(steps, C.byref(ms) if timed else None))
        return ms.value if timed else None

    def use_graphs(self, on):
        self.check(self.d.fn_use_graphs(1 if on else 0))

    def free(self):
        self.d.fn_free()

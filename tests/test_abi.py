"""CPU checks of the C ABI: the library loads without a GPU, exports every symbol include/faie2fn.h declares, the
reference's model-level entries fail with the reference's -1 + fn_error() convention, and argument validation
rejects bad calls before any device work."""

import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import fn

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "faie2fn.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fn_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_symbols() == sorted(fn.SYMBOLS)


def test_library_exports_every_declared_symbol(fnlib):
    for name in header_symbols():
        assert hasattr(fnlib.d, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", fn.LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(fn_\w+)$", out, flags=re.M))
    assert set(header_symbols()) <= exported


def test_reference_entries_report_not_built(fnlib):
    d = fnlib.d
    assert d.fn_load(b"a.gguf", b"b.gguf", 4096, 0) == -1
    assert b"cannot open a.gguf" in d.fn_error()
    with pytest.raises(RuntimeError, match="not loaded"):
        fnlib.reset()
    with pytest.raises(RuntimeError, match="not loaded"):
        fnlib.forward([1, 2, 3])
    assert d.fn_split() == -1 and d.fn_n_past() == -1
    assert d.fn_dev_gb(0) == -1.0 and d.fn_last_ms() == -1.0
    d.fn_pdl(0), d.fn_early(0), d.fn_moe_var(1), d.fn_bench_hot(1), d.fn_free()


def test_validation_before_device_work(fnlib):
    d = fnlib.d
    z = np.zeros(16, np.float32)
    # dk != 128 is rejected by the launcher; shapes < 1 by the hook
    assert d.fn_test_gdn(0, 1, 1, 128, 128, 0, 1, z, z, z, z, z, z, z) == -1
    assert b"bad shape" in d.fn_error()
    # device entry points validate before launching
    assert d.fn_gdn_block_dev(1, 16, 32, 64, 64, 0, 0, 1, 4, *([None] * 10), 1e-6, None, None) == -1
    assert b"dk = dv = 128" in d.fn_error()
    assert d.fn_gdn_block_dev(1, 16, 32, 128, 128, 0, 0, 2, 4, *([None] * 10), 1e-6, None, None) == -1
    assert b"ring - 3" in d.fn_error()
    assert d.fn_gdn_block_dev(1, 16, 32, 128, 128, 0, 0, 1, 6, *([None] * 10), 1e-6, None, None) == -1
    assert b"power of two" in d.fn_error()
    assert d.fn_gdn_block_dev(1, 16, 30, 128, 128, 0, 0, 1, 4, *([None] * 10), 1e-6, None, None) == -1
    assert b"multiple of nkh" in d.fn_error()
    assert d.fn_gdn_block_dev(1, 16, 32, 128, 128, 0, 0, 1, 4, *([None] * 10), 1e-6, None, None) == -1
    assert b"null pointer" in d.fn_error()
    assert d.fn_attn_dev(1, 16, 2, 128, 64, 1e7, 1e-6, 1, 64, *([None] * 8), 1, None, 0, None, None) == -1
    assert b"head_dim 256" in d.fn_error()
    assert d.fn_attn_dev(1, 16, 2, 256, 64, 1e7, 1e-6, 1, 100, *([None] * 8), 1, None, 0, None, None) == -1
    assert b"multiple of 64" in d.fn_error()
    assert d.fn_attn_dev(1, 16, 3, 256, 64, 1e7, 1e-6, 1, 128, *([None] * 8), 1, None, 0, None, None) == -1
    assert b"multiple of nkv" in d.fn_error()
    assert d.fn_attn_dev(1, 16, 2, 256, 65, 1e7, 1e-6, 1, 128, *([None] * 8), 1, None, 0, None, None) == -1
    assert b"nrot" in d.fn_error()
    # the host hook checks positions against the cache before touching the device
    qg = np.zeros((1, 1, 16, 2, 256), np.float32)
    kv = np.zeros((1, 1, 2, 256), np.float32)
    w = np.ones(256, np.float32)
    K = np.zeros((1, 8, 2, 256), np.float32)
    with pytest.raises(RuntimeError, match="max_ctx"):
        fnlib.attn(qg, kv, kv, w, w, K, K.copy(), np.array([8], np.int32))
    with pytest.raises(ValueError):
        fnlib.gdn_block(np.zeros((1, 1, 8192), np.float32), np.zeros((8192, 4), np.float32),
                        np.zeros((1, 3, 8192), np.float64), np.zeros((1, 1, 64), np.float32), np.zeros(32, np.float32),
                        np.zeros(32, np.float32), np.zeros((1, 32, 128, 128), np.float32),
                        np.zeros((1, 1, 4096), np.float32), np.zeros(128, np.float32), 16, 32)


def test_attn_split_heuristic_and_workspace(fnlib):
    # about 512 workgroups; long contexts keep >= 4 tiles per workgroup, short ones go one tile wide
    assert fnlib.attn_nsplit(1, 2, 1, 131072) == 256
    assert fnlib.attn_nsplit(1, 2, 1, 32768) == 128
    assert fnlib.attn_nsplit(16, 2, 1, 32768) == 16
    assert fnlib.attn_nsplit(1, 2, 1, 4096) == 64
    assert fnlib.attn_nsplit(1, 2, 1, 1) == 1
    for B, nq, nt, ns in ((1, 16, 1, 512), (16, 16, 1, 32), (2, 24, 3, 7)):
        wb = fnlib.attn_work_bytes(B, nq, nt, ns)
        assert wb >= 4 * (B * nt * nq * 256 + B * nt * nq * ns * 258)
    assert fnlib.attn_work_bytes(0, 16, 1, 1) == 0


def test_gemv_hooks_validate_before_device_work(fnlib):
    """The reference's GEMV hooks reject unsupported formats and shapes with -1 + fn_error() (faie2fn.cu:2753,
    2918) before touching a device."""
    z8 = np.zeros(1 << 16, np.uint8)
    x = np.zeros((9, 256), np.float32)
    with pytest.raises(RuntimeError, match="unsupported type 19"):        # IQ1_S: not a format of the model
        fnlib.dequant(19, z8, 1, 256)
    with pytest.raises(RuntimeError, match="unsupported shape"):          # K-quant row not a whole super-block
        fnlib.dequant(12, z8, 1, 288)
    with pytest.raises(RuntimeError, match="nt must be 1..8"):
        fnlib.gemv(8, z8, 1, 256, x)
    with pytest.raises(RuntimeError, match="unsupported type 0"):         # F32 has no block decode
        fnlib.gemv(0, z8, 1, 256, x[:1])
    assert fnlib.gemv_packed_bytes(19, 4, 256) == 0 and fnlib.gemv_work_bytes(8, 4, 256, 9) == 0
    assert fnlib.gemv_packed_bytes(21, 4, 256) >= 4 * 110          # IQ3_S is read
    with pytest.raises(RuntimeError, match="unsupported"):
        fnlib.gemv_plan(1, 4, 256)


def test_gemv_plan_shapes(fnlib):
    """Plans of the projection shapes around the path (the benchmark configs' hidden 2048 and the reference model's 2560)."""
    for qtype, rows, cols in [(23, 10240, 2560), (8, 2560, 6144), (30, 96, 2560), (14, 512, 2560), (23, 8192, 2048),
                              (21, 6144, 2560)]:
        gv, wpt, ks, rpw, waves, grid, ngroups = fnlib.gemv_plan(qtype, rows, cols)
        lpr = 16 * wpt
        assert (gv, waves) == (32, 8) and lpr in (16, 32, 64) and rpw == 8 * 64 // lpr
        assert grid == 0 and ngroups == cols // 32  # persistent grid by default
        assert 1 <= ks <= ngroups
        assert fnlib.gemv_work_bytes(qtype, rows, cols, 3) == (ks * 3 * rows * 4 if ks > 1 else 0)
        assert fnlib.gemv_packed_bytes(qtype, rows, cols) >= rows * fn.row_bytes(qtype, cols)
    assert fnlib.gemv_plan(23, 10240, 2560)[2] == 1           # no split-K by default
    fnlib.gemv_override(3)
    try:
        assert fnlib.gemv_plan(23, 10240, 2560)[2] == 3
    finally:
        fnlib.gemv_override(0)
    auto = fnlib.gemv_plan(8, 2560, 6144)
    fnlib.gemv_override(lpr=16)                                  # forced lanes per row; an invalid value is ignored
    try:
        assert fnlib.gemv_plan(23, 10240, 2560)[1::3] == [1, 8]
        fnlib.gemv_override(lpr=48)
        assert fnlib.gemv_plan(8, 2560, 6144) == auto
    finally:
        fnlib.gemv_override(0)


def test_forced_gemv_plan_reads_back(fnlib):
    """flashnext/sweep_gemv_fn.py's forced loop: fn_gemv_override(wpt, ks, 0, 16) then fn_gemv_plan, keeping the
    plans whose out[1] == wpt and out[2] == ks.  Every wpt this library builds (1, 2, 4 sixteen-lane groups per row)
    and every ks reads back as forced; wpt 8 and 16 (no such split here) read back as the automatic choice, so the
    script's filter skips them instead of mislabelling them."""
    d = fnlib.d
    auto = fnlib.gemv_plan(23, 10240, 2560)
    saved = d.fn_gemv_override.argtypes, d.fn_gemv_plan.argtypes
    d.fn_gemv_override.argtypes = [C.c_int] * 4       # as the sweep binds them
    d.fn_gemv_plan.argtypes = [C.c_uint32, C.c_int, C.c_int, C.POINTER(C.c_int)]
    kept = []
    try:
        for wpt in (1, 2, 4, 8, 16):
            for ks in (1, 2, 4, 8, 16):
                d.fn_gemv_override(wpt, ks, 0, 16)
                plan = (C.c_int * 7)()
                assert d.fn_gemv_plan(23, 10240, 2560, plan) == 0
                if plan[1] == wpt and plan[2] == ks:
                    kept.append((wpt, ks))
                else:
                    assert wpt in (8, 16) and plan[1] == auto[1] and plan[2] == ks
    finally:
        d.fn_gemv_override(0, 0, 0, 0)
        d.fn_gemv_override.argtypes, d.fn_gemv_plan.argtypes = saved
    assert kept == [(w, k) for w in (1, 2, 4) for k in (1, 2, 4, 8, 16)]
    assert fnlib.gemv_plan(23, 10240, 2560) == auto


def test_gemv_waves_switches_the_grid(fnlib):
    """fn_gemv_waves, the reference's persistent-grid switch (faie2fn.cu:2075, 2793, driven by
    flashnext/ab_waves_fn.py): 0 gives one workgroup per row tile, any other value the persistent grid again; the plan
    of the weight reflects it and nothing else in the plan changes."""
    d = fnlib.d
    d.fn_gemv_waves.argtypes = [C.c_int]  # as ab_waves_fn.py binds it
    base = fnlib.gemv_plan(23, 10240, 2560)
    try:
        d.fn_gemv_waves(0)
        flat = fnlib.gemv_plan(23, 10240, 2560)
        assert flat[5] == (10240 + flat[3] - 1) // flat[3] and flat[:5] + flat[6:] == base[:5] + base[6:]
        for w in (1, 2, 4):
            d.fn_gemv_waves(w)
            assert fnlib.gemv_plan(23, 10240, 2560) == base
    finally:
        d.fn_gemv_waves(1)


def test_verify_validates_before_device_work(fnlib):
    """fn_gdn_verify_dev rejects a replay stride that does not fit the ring and missing replay inputs before any
    launch."""
    d = fnlib.d
    p = [1] * 11  # non-null stand-ins for rqkv .. norm_w: validation fails before anything is dereferenced
    assert len(d.fn_gdn_verify_dev.argtypes) == 26
    # rnt = 2 with ring 4: 2 + 3 taps > 4
    assert d.fn_gdn_verify_dev(1, 16, 32, 128, 128, 0, 0, 1, 4, 1, 1, 2, *p, 1e-6, 1, None) == -1
    assert b"ring - 3" in d.fn_error()
    # rnt = 1 but no replay inputs
    assert d.fn_gdn_verify_dev(1, 16, 32, 128, 128, 0, 0, 1, 4, 1, 1, 1, None, None, *p[:9], 1e-6, 1, None) == -1
    assert b"null pointer" in d.fn_error()
    assert d.fn_advance_by_dev(None, None, 1, None) == -1


def test_block_xab_validates_before_device_work(fnlib):
    """fn_gdn_block_xab_dev rejects a missing weight or input, a hidden size that is not a positive multiple of 4 and
    misaligned x / w_ab before any launch (the pointers are stand-ins: validation fails before any is used)."""
    d = fnlib.d
    assert len(d.fn_gdn_block_xab_dev.argtypes) == 23
    a = 4096  # aligned stand-in address

    def call(x=a, hidden=2048, w=a):
        return d.fn_gdn_block_xab_dev(1, 16, 32, 128, 128, 0, 0, 4, a, a, a, a, x, hidden, w, a, a, a, a, a, 1e-6, a,
                                      None)

    assert call(w=None) == -1 and b"null pointer" in d.fn_error()
    assert call(x=None) == -1 and b"null pointer" in d.fn_error()
    assert call(hidden=2046) == -1 and b"multiple of 4" in d.fn_error()
    assert call(hidden=0) == -1 and b"multiple of 4" in d.fn_error()
    assert call(x=a + 4) == -1 and b"16-byte aligned" in d.fn_error()
    assert call(w=a + 8) == -1 and b"16-byte aligned" in d.fn_error()


def test_noalloc_attn_rejects_oversize(fnlib):
    """fn_attn_noalloc_dev refuses shapes whose workspace exceeds its built-in device array, before touching the
    device; shapes that fit are sized by the same fn_attn_work_bytes as fn_attn_dev."""
    d = fnlib.d
    assert len(d.fn_attn_noalloc_dev.argtypes) == 20
    big = fnlib.attn_work_bytes(64, 16, 8, 64)
    assert big > fn.NOALLOC_SCRATCH_BYTES
    assert d.fn_attn_noalloc_dev(64, 16, 2, 256, 64, 1e7, 1e-6, 8, 4096, *([None] * 8), 64, None, None) == -1
    assert b"workspace" in d.fn_error() and str(fn.NOALLOC_SCRATCH_BYTES).encode() in d.fn_error()
    assert d.fn_attn_noalloc_dev(1, 16, 2, 256, 64, 1e7, 1e-6, 1, 4096, *([None] * 8), 0, None, None) == -1
    # the decode shapes of the benchmark fit: B = 16 at 32K and B = 1 at 128K with their automatic split counts
    for B, L in ((16, 32768), (1, 131072), (1, 4096)):
        assert fnlib.attn_work_bytes(B, 16, 1, fnlib.attn_nsplit(B, 2, 1, L)) <= fn.NOALLOC_SCRATCH_BYTES


def test_gemv_group_refuses_bad_arguments(fnlib):
    """fn_gemv_group_dev checks its parts before any launch: 1 to 4 of them, formats and shapes the library reads,
    no null weight, output or x."""
    d = fnlib.d
    assert d.fn_gemv_group_dev(0, None, None, 2560, None, None, 1, None, None) == -1
    assert d.fn_gemv_group_dev(5, None, None, 2560, None, None, 1, None, None) == -1
    assert b"1 to 4 parts" in d.fn_error()
    ty = (C.c_uint32 * 2)(23, 30)
    rows = (C.c_int * 2)(64, 8)
    fake = (C.c_void_p * 2)(4096, 8192)
    assert d.fn_gemv_group_dev(2, ty, rows, 2560, fake, None, 1, fake, None) == -1  # x null
    assert d.fn_gemv_group_dev(2, ty, rows, 2500, fake, 4096, 1, fake, None) == -1  # 2500: not whole blocks
    assert b"unsupported shape" in d.fn_error()
    bad = (C.c_uint32 * 2)(23, 99)
    assert d.fn_gemv_group_dev(2, bad, rows, 2560, fake, 4096, 1, fake, None) == -1
    assert b"unsupported type" in d.fn_error()
    nul = (C.c_void_p * 2)(4096, None)
    assert d.fn_gemv_group_dev(2, ty, rows, 2560, nul, 4096, 1, fake, None) == -1
    assert b"null part" in d.fn_error()
    assert d.fn_gemv_group_dev(2, ty, rows, 2560, fake, 4096, 9, fake, None) == -1
    assert b"nt must be" in d.fn_error()
    # a plane past 4 GiB (the GEMV kernels address planes with 32-bit offsets) is refused before any launch
    big = (C.c_int * 2)(64, 1100000)  # BF16, 4096 bytes a row: 4.5 GB
    assert d.fn_gemv_group_dev(2, ty, big, 2048, fake, 4096, 1, fake, None) == -1
    assert b"exceeds 4 GiB" in d.fn_error()


def test_gemv_refuses_planes_past_4gib(fnlib):
    """fn_gemv_dev refuses a weight with a plane over 4 GiB before any launch (the GEMV kernels address each plane
    with 32-bit offsets)."""
    d = fnlib.d
    assert d.fn_gemv_dev(30, 4096, 1100000, 2048, 4096, 1, 8192, None, 0, None) == -1  # BF16 rows of 4096 B: 4.5 GB
    assert b"exceeds 4 GiB" in d.fn_error()


def test_bench_route_refuses_bad_arguments(fnlib):
    """fn_bench_route checks its arguments before any device work (engine/faie2fn.cu:2875's arguments)."""
    d = fnlib.d
    part = np.zeros((1, 8, 528), np.float32)
    sel = np.zeros(80, np.int32)
    w = np.zeros(80, np.float32)
    ms = np.zeros(1, np.float32)
    args = lambda v, nt, ks, it: (v, nt, ks, part.ctypes.data, it, sel.ctypes.data, w.ctypes.data,  # noqa: E731
                                  ms.ctypes.data)
    assert d.fn_bench_route(*args(2, 1, 1, 1)) == -1
    assert b"variant" in d.fn_error()
    assert d.fn_bench_route(*args(0, 9, 1, 1)) == -1
    assert b"nt must be" in d.fn_error()
    assert d.fn_bench_route(*args(1, 1, 0, 1)) == -1
    assert b"ks must be" in d.fn_error()
    assert d.fn_bench_route(*args(1, 1, 1, 0)) == -1
    assert b"iters" in d.fn_error()
    assert d.fn_bench_route(0, 1, 1, None, 1, None, None, None) == -1
    assert b"null pointer" in d.fn_error()
    with pytest.raises(ValueError):
        fnlib.bench_route(0, np.zeros((1, 8, 500), np.float32), 1)


def test_bench_hooks_check_shapes_before_the_device(fnlib):
    """fn_bench_gdn / fn_bench_attn reject shapes they cannot time before touching a device (these run without a
    GPU)."""
    for args, msg in (((0, 16, 32, 1, 20), "B >= 1"), ((1, 16, 30, 1, 20), "multiple of nkh"),
                      ((1, 16, 32, 9, 20), "nt 1..8"), ((1, 16, 32, 1, 0), "iters")):
        with pytest.raises(RuntimeError, match=msg):
            fnlib.bench_gdn(*args[:1], nkh=args[1], nvh=args[2], nt=args[3], iters=args[4])
    with pytest.raises(RuntimeError, match="4, 8 or 12"):
        fnlib.bench_attn(1, 4096, nq=16, nkv=8)
    with pytest.raises(RuntimeError, match="ctx >= nt"):
        fnlib.bench_attn(1, 2, nt=4)


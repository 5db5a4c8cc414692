"""The path's timing hooks through the C ABI (fn_bench_gdn, fn_bench_attn): they run on the device and report
plausible microseconds per layer-step (bounded below by the HBM time of the algorithmic bytes at 8 TB/s, above by
a generous latency bound), and agree with the HBM-bound bench figures of the same shapes."""

import pytest

import fn_synth

pytestmark = pytest.mark.gpu

PEAK = 8e12  # B/s


def _say(*a):
    print(*a, flush=True)


def test_bench_gdn(fnlib):
    for B, nt in ((64, 1), (1, 1), (16, 4)):
        _say(f"fn_bench_gdn B={B} nt={nt}")
        us = fnlib.bench_gdn(B, nt=nt, iters=10)
        floor = fn_synth.gdn_block_bytes(B) / PEAK * 1e6 if nt == 1 else 0.0
        assert floor < us < 500.0, (B, nt, us)
        _say(f"  {us:.2f} us per layer-step")
    us = fnlib.bench_gdn(64, iters=10)
    assert us < 1.5 * fn_synth.gdn_block_bytes(64) / 5.0e12 * 1e6  # at least 5 TB/s / 1.5 on the headline shape


def test_bench_attn(fnlib):
    for B, ctx, nt in ((1, 4096, 1), (16, 32768, 1), (1, 32768, 4)):
        _say(f"fn_bench_attn B={B} ctx={ctx} nt={nt}")
        us = fnlib.bench_attn(B, ctx, nt=nt, iters=10)
        floor = fn_synth.attn_bytes(B, ctx, nt=nt) / PEAK * 1e6
        assert floor < us < 5000.0, (B, ctx, nt, us)
        _say(f"  {us:.2f} us per layer-step")

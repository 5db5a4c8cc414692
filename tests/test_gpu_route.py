"""GPU parity of the MoE routing benchmark hook fn_bench_route (engine/faie2fn.cu:2875) against the oracle.

The reference's check (flashnext/route_fn.py:29-44): random router partials part [ks][8][528], ties forced in on a
third of the cases (logits copied onto others within one split, so the sums tie exactly) and many exact ties on a
seventh (logits rounded to integers); every variant picks the same experts with the same weight bits.  Here both
variants (0: a rank per expert, 1: the model forward's one-wave routing) must agree bit for bit with each other, and
with the float64 routing of the model restatement (oracle/model.py Model.route: softmax, the 10 most probable,
ties to the lower expert, renormalized) on the logits summed from the partials in split order as float32 (the
GOut convention, faie2fn.cu:1245-1250): picks exact, weights within 1e-5.

Every case prints what names it before the GPU call.
"""

import types

import numpy as np
import pytest

import oracle.model as om

pytestmark = pytest.mark.gpu

RSG, MAXT, NE, NEU = 528, 8, 512, 10
TOL = 1e-5
ROUTER = types.SimpleNamespace(NE=NE, NEU=NEU)


def _say(*a):
    print(*a, flush=True)


def _logits(part, nt):
    s = part[0, :nt, :NE].copy()
    for k in range(1, part.shape[0]):
        s = (s + part[k, :nt, :NE]).astype(np.float32)
    return s.astype(np.float64)


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    for trial in range(n):
        ks = int(rng.integers(1, 6))
        nt = int(rng.integers(1, 9))
        part = (rng.standard_normal((ks, MAXT, RSG)) * rng.choice([0.1, 1, 4])).astype(np.float32)
        if trial % 3 == 0:
            part[1:] = 0
            for t in range(nt):
                src = rng.integers(0, NE, 20)
                dst = rng.integers(0, NE, 20)
                part[0, t, dst] = part[0, t, src]
        if trial % 7 == 0:
            part[:, :, :NE] = np.round(part[:, :, :NE])
        yield trial, ks, nt, part


def test_route_variants_agree_with_oracle(fnlib):
    for trial, ks, nt, part in _cases(60, 1):
        _say(f"route trial {trial}: ks {ks} nt {nt}")
        sel0, w0, _ = fnlib.bench_route(0, part, nt)
        sel1, w1, _ = fnlib.bench_route(1, part, nt)
        assert np.array_equal(sel0, sel1), trial
        assert np.array_equal(w0.view(np.uint32), w1.view(np.uint32)), trial
        sel, w = om.Model.route(ROUTER, _logits(part, nt))
        assert np.array_equal(sel1, sel), trial
        assert np.abs(w1 - w).max() <= TOL, trial


def test_route_all_equal_and_extremes(fnlib):
    """Closed forms: all logits equal picks experts 0..9 at weight 1/10; one logit 1000 above the rest gives that
    expert weight 1 (exp(-1000) is zero in float32, so the others tie at zero) and the rest in index order."""
    part = np.zeros((2, MAXT, RSG), np.float32)
    part[0, 1, 300] = 500.0
    part[1, 1, 300] = 500.0
    for v in (0, 1):
        _say(f"route closed forms, variant {v}")
        sel, w, _ = fnlib.bench_route(v, part, 2)
        assert list(sel[0]) == list(range(NEU)) and np.all(w[0] == np.float32(0.1))
        assert sel[1][0] == 300 and list(sel[1][1:]) == list(range(NEU - 1))
        assert w[1][0] == 1.0 and np.all(w[1][1:] == 0.0)


def test_route_reports_time(fnlib):
    part = np.random.default_rng(2).standard_normal((5, MAXT, RSG)).astype(np.float32)
    for v in (0, 1):
        for nt in (1, 8):
            _say(f"route timing, variant {v}, nt {nt}")
            _, _, ms = fnlib.bench_route(v, part, nt, iters=50)
            assert 0.0 < ms < 1.0

"""Pin the CPU oracle against the reference's own golden vectors.

fixtures/small-{fp32,mixed}/expected were written by the reference's PyTorch model
(reference/export.py:46-70): 201 events of the Small fixture config (L=1, d=64, H=4, dh=16,
F=128, W=64, f=32), covering the first event, a partial window, eviction, several ring
revolutions and a warm reset before event 131. Every event's score, hidden state and the
complete K/V cache are compared, with the reference's tolerances (bench/Main.cpp:72,
docs/NumericalPolicy.md).
"""
import numpy as np
import pytest

from oracle.pyoracle import Oracle
from streamtx import numerical


def run_fixture(g, accumulate):
    ck = g.checkpoint
    oracle = Oracle(ck.config, ck.tensors, mixed=ck.mixed, accumulate=accumulate)
    for i, score, keys, values, hidden in g.expected_state():
        if i in g.resets:
            oracle.reset()
        got = oracle.step(g.trace[i])
        pos, k, v, h = oracle.snapshot()
        yield i, got, score, (k, v, h), (keys, values, hidden), pos


@pytest.mark.parametrize('accumulate', ['float', 'double'])
def test_fp32_fixture_every_event(golden, accumulate):
    g = golden('small-fp32')
    last_reset = 0
    for i, got, score, (k, v, h), (rk, rv, rh), pos in run_fixture(g, accumulate):
        if i in g.resets:
            last_reset = i
        assert pos == i - last_reset + 1
        assert numerical.fp32_failures([got], [score]) == 0, (i, got, score)
        for a, r, name in ((k, rk, 'keys'), (v, rv, 'values'), (h, rh, 'hidden')):
            assert numerical.fp32_failures(a, r) == 0, (i, name, float(np.abs(a - r).max()))


@pytest.mark.parametrize('accumulate', ['float', 'double'])
def test_mixed_fixture_policy_v3(golden, accumulate):
    g = golden('small-mixed')
    scores, refs = [], []
    for i, got, score, (k, v, h), (rk, rv, rh), pos in run_fixture(g, accumulate):
        scores.append(got)
        refs.append(score)
        res = numerical.mixed_state_passes(k, v, h, rk, rv, rh)
        assert res['passed'], (i, res['failures'][:2])
    res = numerical.score_errors(scores, refs, g.config.layers)
    assert res['passed'], res


@pytest.mark.parametrize('accumulate', ['float', 'double'])
def test_fp32_fixture_within_strict_bound(golden, accumulate):
    """Tighter than the reference's own gate: every score, hidden coordinate and cache entry
    within 1e-6 + 1e-5 |ref| of the PyTorch FP32 fixture."""
    g = golden('small-fp32')
    for i, got, score, (k, v, h), (rk, rv, rh), pos in run_fixture(g, accumulate):
        assert numerical.fp32_strict_failures([got], [score]) == 0, (i, got, score)
        for a, r in ((k, rk), (v, rv), (h, rh)):
            assert numerical.fp32_strict_failures(a, r) == 0, i


def test_mixed_cache_entries_are_fp16_values(golden):
    g = golden('small-mixed')
    for i, got, score, (k, v, h), *_ in run_fixture(g, 'float'):
        for a in (k, v, h):
            assert np.array_equal(a, a.astype(np.float16).astype(np.float32))
        if i > 10:
            break

"""Persistent mailbox backend: lifecycle (the reference's tests/Lifecycle.cu Persistent cases)
and bit-for-bit agreement with the fused backend, through the C ABI."""
import time

import numpy as np
import pytest

from oracle.pyoracle import Oracle
from streamtx import Backend, ModelConfig, Runtime, RuntimeOptions, synthetic_checkpoint

pytestmark = pytest.mark.gpu

U64_MAX = (1 << 64) - 1
IDLE = 10.0  # seconds: bounds how long a worker outlives a failed test


def persistent(model, blocks, **kw):
    kw.setdefault('idle_seconds', IDLE)
    print(f'[case] backend=PERSISTENT blocks={blocks} {kw}', flush=True)
    return Runtime(model, RuntimeOptions(backend=Backend.PERSISTENT, blocks=blocks, **kw))


@pytest.mark.parametrize('mode', ['fp32', 'mixed'])
@pytest.mark.parametrize('blocks', [1, 4])
def test_reset_repeated_scores_and_restart(golden, mode, blocks):
    # tests/Lifecycle.cu:17-47: repeated zero scores still complete distinct sequence IDs;
    # each reconstruction starts an independent state and mailbox sequence.
    g = golden(f'small-{mode}')
    c = g.config
    event = np.zeros(c.features, dtype=np.float32)
    for _ in range(2):
        rt = persistent(g.checkpoint, blocks)
        oracle = Oracle(c, g.checkpoint.tensors, mixed=g.checkpoint.mixed)
        for i in range(3 * c.window + 9):
            if i in (1, c.window, 2 * c.window + 3):
                rt.reset()
                rt.reset()
                oracle.reset()
                assert rt.snapshot()[0] == 0
            assert rt.step(event) == oracle.step(event) == 0.0
            assert rt.snapshot()[0] == oracle.position
        rt.stop()
        rt.stop()
        with pytest.raises(RuntimeError):
            rt.step(event)
        with pytest.raises(RuntimeError):
            rt.reset()
        rt.close()


@pytest.mark.parametrize('blocks', [1, 4])
def test_finite_event_budget(golden, blocks):
    # tests/Lifecycle.cu:49-64: RESET does not consume the RUN budget.
    g = golden('small-fp32')
    event = np.zeros(g.config.features, dtype=np.float32)
    with persistent(g.checkpoint, blocks, max_events=2) as rt:
        assert rt.step(event) == 0.0
        rt.reset()
        assert rt.step(event) == 0.0
        with pytest.raises(RuntimeError, match='exited'):
            rt.step(event)
        rt.stop()


def test_idle_exit(golden):
    # tests/Lifecycle.cu:65-71
    g = golden('small-fp32')
    event = np.zeros(g.config.features, dtype=np.float32)
    with persistent(g.checkpoint, 1, idle_seconds=0.001) as rt:
        time.sleep(0.1)
        with pytest.raises(RuntimeError, match='exited'):
            rt.step(event)
        rt.stop()


@pytest.mark.parametrize('blocks', [1, 4])
def test_sequence_exhaustion_still_allows_stop(golden, blocks):
    # tests/Lifecycle.cu:74-90: the last sequence ID is reserved for STOP.
    g = golden('small-fp32')
    event = np.zeros(g.config.features, dtype=np.float32)
    with persistent(g.checkpoint, blocks, initial_sequence=U64_MAX - 2) as rt:
        assert rt.step(event) == 0.0
        with pytest.raises(RuntimeError, match='exhausted'):
            rt.step(event)
        with pytest.raises(RuntimeError, match='exhausted'):
            rt.reset()
        rt.stop()
        rt.stop()


def test_initial_sequence_leaving_no_room_is_rejected(golden):
    g = golden('small-fp32')
    with pytest.raises(RuntimeError):
        persistent(g.checkpoint, 1, initial_sequence=U64_MAX - 1)


@pytest.mark.parametrize('blocks', [1, 4, 0])
def test_fixture_trace_equals_fused_bit_for_bit(golden, blocks):
    g = golden('small-fp32')
    results = []
    for make in (lambda: persistent(g.checkpoint, blocks),
                 lambda: Runtime(g.checkpoint, RuntimeOptions(backend=Backend.FUSED, blocks=blocks))):
        with make() as rt:
            scores = []
            for i, e in enumerate(g.trace):
                if i in g.resets:
                    rt.reset()
                scores.append(rt.step(e))
            results.append((np.array(scores, dtype=np.float32), rt.snapshot()))
    (s0, st0), (s1, st1) = results
    np.testing.assert_array_equal(s0, s1)
    assert st0[0] == st1[0]
    for a, b in zip(st0[1:], st1[1:]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize('mode', ['fp32', 'mixed'])
def test_snapshots_while_worker_runs(golden, mode):
    # The reference's validation snapshots a live persistent runtime between commands
    # (scripts/validate.py:55-74). The worker serves each snapshot and keeps running: every
    # snapshot equals the fused backend's at the same event, and returns promptly (a copy
    # that waited for the worker would only return after the idle budget).
    g = golden(f'small-{mode}')
    points = {5, 17, 40, 63, 64, 90}
    states = []
    for make in (lambda: persistent(g.checkpoint, 0),
                 lambda: Runtime(g.checkpoint, RuntimeOptions(backend=Backend.FUSED, blocks=0))):
        got = []
        with make() as rt:
            for i, e in enumerate(g.trace[:100]):
                if i == 70:
                    rt.reset()
                rt.step(e)
                if i in points:
                    t0 = time.perf_counter()
                    got.append(rt.snapshot())
                    assert time.perf_counter() - t0 < 2.0
        states.append(got)
    for a, b in zip(*states):
        assert a[0] == b[0]
        for x, y in zip(a[1:], b[1:]):
            np.testing.assert_array_equal(x, y)


def test_main_shape_matches_oracle():
    c = ModelConfig(8, 512, 8, 2048, 128, 512)
    w = synthetic_checkpoint(c, seed=7)
    events = np.random.default_rng(7).standard_normal((150, c.features)).astype(np.float32)
    oracle = Oracle(c, w, accumulate='double', threads=8)
    with persistent((c, w, False), 0) as rt:
        for i, e in enumerate(events):
            if i == 131:
                rt.reset()
                oracle.reset()
            got, ref = rt.step(e), oracle.step(e)
            assert abs(got - ref) <= 1e-6 + 1e-5 * abs(ref), (i, got, ref)
        pos, k, v, h = rt.snapshot()
        opos, ok, ov, oh = oracle.snapshot()
        assert pos == opos
        for a, o in ((k, ok), (v, ov), (h, oh)):
            np.testing.assert_allclose(a, o, rtol=1e-5, atol=1e-6)

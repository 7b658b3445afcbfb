"""Resident batches (st_batch_create_resident): B streams in one launch of the fused step per
step, stream s on its own workgroups with its own state, the weights shared.

Bars, through the C ABI:
  - every stream is bit-identical to a single-stream FUSED runtime fed the same events and
    resets: scores, K/V rings, hidden state and position (the step's results do not depend on
    the grid, and each stream runs the unchanged fused step);
  - every stream against its own CPU oracle (FP64-accumulating): FP32 within 1e-6 + 1e-5|r|;
  - per-stream reset touches only its stream; device_run equals stepping bit for bit;
  - more streams than the resident limit are refused.
"""
import numpy as np
import pytest

from oracle.pyoracle import Oracle
from streamtx import (Backend, BatchRuntime, ModelConfig, Runtime, RuntimeOptions, WeightStorage, numerical,
                      round_bf16, synthetic_checkpoint)

pytestmark = pytest.mark.gpu

STRICT = dict(atol=1e-6, rtol=1e-5)

SHAPES = {
    'small': ModelConfig(4, 256, 4, 1024, 64, 256),
    'main': ModelConfig(8, 512, 8, 2048, 128, 512),
    # head dim 32, 32 features (padded input rows), window 256
    'ref-main': ModelConfig(2, 128, 4, 256, 256, 32),
    # head dim 48 (the LDS attention path)
    'dh48': ModelConfig(2, 96, 2, 192, 40, 96),
    # weights beyond the Infinity Cache: the non-temporal weight-load instantiation
    'large': ModelConfig(12, 1024, 16, 4096, 512, 1024),
}


def resident(model, streams, weight_dtype=WeightStorage.AS_MODEL):
    c = model[0]
    print(f'[case] resident batch streams={streams} layers={c.layers} width={c.width} window={c.window} '
          f'mixed={model[2]} weights={WeightStorage(weight_dtype).name}', flush=True)
    return BatchRuntime(model, streams, weight_dtype, resident=True)


def _events(config, seed, steps, streams):
    return np.random.default_rng(seed).standard_normal((steps, streams, config.features)).astype(np.float32)


def _same_state(a, b):
    assert a[0] == b[0]
    for x, y in zip(a[1:], b[1:]):
        assert np.array_equal(x, y)


@pytest.mark.parametrize('name,mixed,weights,streams,steps,resets', [
    ('small', False, WeightStorage.AS_MODEL, 3, 80, {1: 50}),
    ('small', True, WeightStorage.AS_MODEL, 5, 70, {4: 20}),
    ('main', False, WeightStorage.BF16, 4, 40, {2: 17}),
    ('main', False, WeightStorage.AS_MODEL, 16, 12, {}),
    # one stream on the whole grid, and the 32-stream limit (8 workgroups per stream): the W = 128
    # window filled, then 24 full-window steps
    ('main', False, WeightStorage.BF16, 1, 152, {}),
    ('main', False, WeightStorage.BF16, 32, 152, {5: 70}),
    ('dh48', False, WeightStorage.AS_MODEL, 7, 50, {0: 9}),
    ('large', False, WeightStorage.AS_MODEL, 2, 6, {1: 3}),
])
def test_every_stream_equals_fused_runtime(name, mixed, weights, streams, steps, resets):
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=21, mixed=mixed)
    events = _events(c, 21, steps, streams)
    scores = np.empty((steps, streams), dtype=np.float32)
    with resident((c, w, mixed), streams, weights) as rt:
        for i in range(steps):
            for b, at in resets.items():
                if at == i:
                    rt.reset(b)
            scores[i] = rt.step(events[i])
        states = [rt.snapshot(b) for b in range(streams)]
    opts = RuntimeOptions(backend=Backend.FUSED, blocks=0, weight_dtype=weights)
    for b in range(streams):
        with Runtime((c, w, mixed), opts) as single:
            for i in range(steps):
                if resets.get(b) == i:
                    single.reset()
                assert single.step(events[i, b]) == scores[i, b], (b, i)
            _same_state(states[b], single.snapshot())


@pytest.mark.parametrize('name,streams,steps,resets', [
    ('ref-main', 5, 270, {3: 100}),
    ('small', 2, 80, {}),
])
def test_every_stream_matches_oracle(name, streams, steps, resets):
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=22)
    events = _events(c, 22, steps, streams)
    oracles = [Oracle(c, w, accumulate='double', threads=8) for _ in range(streams)]
    with resident((c, w, False), streams) as rt:
        for i in range(steps):
            for b, at in resets.items():
                if at == i:
                    rt.reset(b)
                    oracles[b].reset()
            got = rt.step(events[i])
            for b in range(streams):
                ref = oracles[b].step(events[i, b])
                assert numerical.fp32_strict_failures([got[b]], [ref], **STRICT) == 0, (i, b, got[b], ref)
        for b in range(streams):
            state, ref = rt.snapshot(b), oracles[b].snapshot()
            assert state[0] == ref[0]
            for x, y in zip(state[1:], ref[1:]):
                assert numerical.fp32_strict_failures(x, y, **STRICT) == 0, float(np.abs(x - y).max())


@pytest.mark.parametrize('resident_path', [True, False], ids=['resident', 'graph'])
def test_main_bf16w_single_stream_batch_matches_oracle(resident_path):
    """Batched Main with bfloat16 weights at B = 1, the configuration the benchmark reports, on
    the resident kernel and on the phase-kernel graph: the W = 128 window filled, then 24
    full-window steps, every score and the final state against the FP64-accumulating oracle on
    the bfloat16-rounded weights (the exact equivalent of bfloat16 storage with FP32 compute)."""
    c = SHAPES['main']
    w = synthetic_checkpoint(c, seed=4)
    oracle = Oracle(c, {k: round_bf16(v) for k, v in w.items()}, accumulate='double', threads=8)
    steps = c.window + 24
    events = _events(c, 4, steps, 1)
    if resident_path:
        rt = resident((c, w, False), 1, WeightStorage.BF16)
    else:
        print('[case] graph batch streams=1 main bf16w', flush=True)
        rt = BatchRuntime((c, w, False), 1, WeightStorage.BF16)
    with rt:
        for i in range(steps):
            got = rt.step(events[i])[0]
            ref = oracle.step(events[i, 0])
            assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (i, got, ref)
        state, ref = rt.snapshot(0), oracle.snapshot()
    assert state[0] == ref[0] == steps
    for x, y in zip(state[1:], ref[1:]):
        assert numerical.fp32_strict_failures(x, y, **STRICT) == 0, float(np.abs(x - y).max())


def test_device_run_equals_stepping_and_reset_is_per_stream():
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=23)
    streams, steps = 6, 40
    events = _events(c, 23, steps, streams)
    with resident((c, w, False), streams) as a, resident((c, w, False), streams) as b:
        for i in range(steps):
            a.step(events[i])
        mean, per = b.device_run(events)
        assert mean > 0 and per.shape == (steps,)
        for s in range(streams):
            _same_state(a.snapshot(s), b.snapshot(s))
        # Reset stream 2 of one batch only: the other streams keep their state.
        before = [b.snapshot(s) for s in range(streams)]
        b.reset(2)
        pos, keys, values, hidden = b.snapshot(2)
        assert pos == 0 and not keys.any() and not values.any() and not hidden.any()
        for s in range(streams):
            if s != 2:
                _same_state(before[s], b.snapshot(s))
        # Both batches then step on: the streams that were not reset agree bit for bit.
        more = _events(c, 24, 5, streams)
        for i in range(5):
            x, y = a.step(more[i]), b.step(more[i])
            assert np.array_equal(np.delete(x, 2), np.delete(y, 2))


def test_stream_count_limit():
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=25)
    for bad in (0, 33):
        with pytest.raises(RuntimeError, match='Resident batches take 1 to 32 streams'):
            BatchRuntime((c, w, False), bad, resident=True)

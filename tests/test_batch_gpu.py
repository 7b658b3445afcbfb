"""Batched independent streams (st_batch_*): B streams over one set of weights, the
projections as MFMA GEMMs over the streams.

Bars, through the C ABI:
  - every stream against its own CPU oracle (FP64-accumulating): FP32 within 1e-6 + 1e-5|r|
    per step, for the score and the stream's complete carried state;
  - a stream's results do not depend on the batch around it: stream b of a batch of B is
    bit-identical to a batch of 1 fed the same events (every output element of the MFMA
    tiles and the split-K reduction is a function of that stream's row only);
  - per-stream reset touches only its stream; device_run equals stepping bit for bit;
  - eager launches (st_batch_set_eager) equal the graph replay bit for bit.
"""
import numpy as np
import pytest

from oracle.pyoracle import Oracle
from streamtx import BatchRuntime, ModelConfig, WeightStorage, numerical, round_bf16, synthetic_checkpoint
from streamtx.runtime import _check, library

pytestmark = pytest.mark.gpu

STRICT = dict(atol=1e-6, rtol=1e-5)

SHAPES = {
    'small': ModelConfig(4, 256, 4, 1024, 64, 256),
    'main': ModelConfig(8, 512, 8, 2048, 128, 512),
    # head dim 32, 32 features (padded input rows), window 256
    'ref-main': ModelConfig(2, 128, 4, 256, 256, 32),
    # head dim 48
    'dh48': ModelConfig(2, 96, 2, 192, 40, 96),
    # head dim 128: attention's general per-pass loop (two 64-element passes per row)
    'dh128': ModelConfig(2, 256, 2, 512, 48, 256),
    # Large's width and FFN (d = 1024, F = 4096): the longest K-slices and the widest operands
    'wide': ModelConfig(2, 1024, 16, 4096, 40, 1024),
    # 29 features: events that are not whole 16-byte pieces, a padded input projection
    'odd': ModelConfig(2, 64, 2, 128, 24, 29),
}


def batch(model, streams, weight_dtype=WeightStorage.AS_MODEL):
    c = model[0]
    print(f'[case] batch streams={streams} layers={c.layers} width={c.width} window={c.window} '
          f'weights={WeightStorage(weight_dtype).name}', flush=True)
    return BatchRuntime(model, streams, weight_dtype)


def _events(config, seed, steps, streams):
    return np.random.default_rng(seed).standard_normal((steps, streams, config.features)).astype(np.float32)


def _check_state(state, oracle_state):
    assert state[0] == oracle_state[0]
    for a, o in zip(state[1:], oracle_state[1:]):
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, float(np.abs(a - o).max())


@pytest.mark.parametrize('name,streams,steps,resets', [
    ('small', 19, 80, {7: 50, 18: 3}),
    ('ref-main', 17, 270, {0: 100}),
    ('dh48', 3, 60, {1: 41}),
    ('dh128', 5, 60, {2: 30}),
    ('main', 16, 24, {5: 11}),
    ('wide', 3, 48, {1: 20}),
    ('odd', 5, 60, {4: 31}),
])
def test_every_stream_matches_oracle(name, streams, steps, resets):
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=11)
    events = _events(c, 11, steps, streams)
    oracles = [Oracle(c, w, accumulate='double', threads=8) for _ in range(streams)]
    with batch((c, w, False), streams) as rt:
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
            _check_state(rt.snapshot(b), oracles[b].snapshot())


@pytest.mark.parametrize('name,streams,steps', [('main', 16, 20), ('wide', 5, 16), ('odd', 5, 40)])
def test_bf16_weights_match_oracle_on_rounded_weights(name, streams, steps):
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=12)
    rounded = {k: round_bf16(v) for k, v in w.items()}
    events = _events(c, 12, steps, streams)
    oracles = [Oracle(c, rounded, accumulate='double', threads=8) for _ in range(streams)]
    with batch((c, w, False), streams, WeightStorage.BF16) as rt:
        for i in range(steps):
            got = rt.step(events[i])
            for b in range(streams):
                ref = oracles[b].step(events[i, b])
                assert numerical.fp32_strict_failures([got[b]], [ref], **STRICT) == 0, (i, b, got[b], ref)
        for b in (0, streams // 2, streams - 1):
            _check_state(rt.snapshot(b), oracles[b].snapshot())


@pytest.mark.parametrize('weight_dtype,mixed,streams,steps', [
    (WeightStorage.AS_MODEL, False, 40, 70), (WeightStorage.BF16, False, 40, 70), (WeightStorage.AS_MODEL, True, 40, 70),
    # 130 streams: the large-batch workgroup shapes of every projection
    (WeightStorage.BF16, False, 130, 20), (WeightStorage.AS_MODEL, True, 130, 20),
    # 256 streams: mixed mode's attention takes four passes of loads (against eight passes with
    # V loaded early for a batch of one), past the window
    (WeightStorage.AS_MODEL, True, 256, 70)])
def test_stream_independent_of_batch(weight_dtype, mixed, streams, steps):
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=13, mixed=mixed)
    events = _events(c, 13, steps, streams)
    picks = (0, 21, streams - 1)
    with batch((c, w, mixed), streams, weight_dtype) as rt:
        many = np.stack([rt.step(events[i]) for i in range(steps)])
        states = [rt.snapshot(b) for b in picks]
    for b, state in zip(picks, states):
        with batch((c, w, mixed), 1, weight_dtype) as one:
            alone = np.array([one.step(events[i, b:b + 1])[0] for i in range(steps)], dtype=np.float32)
            np.testing.assert_array_equal(alone, many[:, b])
            ref = one.snapshot(0)
        assert ref[0] == state[0]
        for x, y in zip(ref[1:], state[1:]):
            np.testing.assert_array_equal(x, y)


# head dim 128: mixed mode's attention through the per-pass loop
@pytest.mark.parametrize('name,streams,steps', [('main', 16, 40), ('small', 19, 90), ('dh128', 6, 60),
                                                ('wide', 3, 48), ('odd', 5, 60)])
def test_mixed_streams_meet_the_reference_policy(name, streams, steps):
    # Mixed mode: FP16 weights and K/V with the reference's cast points; each stream against
    # the mixed oracle under the reference's numerical policy v3 (include/Numerical.hpp).
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=16, mixed=True)
    events = _events(c, 16, steps, streams)
    oracles = [Oracle(c, w, mixed=True, threads=8) for _ in range(streams)]
    scores = np.empty((steps, streams), dtype=np.float32)
    refs = np.empty_like(scores)
    with batch((c, w, True), streams) as rt:
        for i in range(steps):
            if i == steps // 2:
                r = min(3, streams - 1)
                rt.reset(r)
                oracles[r].reset()
            scores[i] = rt.step(events[i])
            refs[i] = [o.step(events[i, b]) for b, o in enumerate(oracles)]
        for b in range(streams):
            pos, k, v, h = rt.snapshot(b)
            opos, ok, ov, oh = oracles[b].snapshot()
            assert pos == opos
            for a in (k, v, h):
                assert np.array_equal(a, a.astype(np.float16).astype(np.float32))
            res = numerical.mixed_state_passes(k, v, h, ok, ov, oh)
            assert res['passed'], (b, res['failures'][:2])
    for b in range(streams):
        res = numerical.score_errors(scores[:, b], refs[:, b], c.layers)
        assert res['passed'], (b, res)


def test_reset_one_and_all_and_device_run_equals_stepping():
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=14)
    streams, steps = 5, 30
    events = _events(c, 14, steps, streams)
    with batch((c, w, False), streams) as rt:
        for i in range(10):
            rt.step(events[i])
        before = [rt.snapshot(b) for b in range(streams)]
        rt.reset(2)
        after = [rt.snapshot(b) for b in range(streams)]
        assert after[2][0] == 0
        for a in after[2][1:]:
            assert not a.any()
        for b in (0, 1, 3, 4):
            assert after[b][0] == before[b][0] == 10
            for x, y in zip(after[b][1:], before[b][1:]):
                np.testing.assert_array_equal(x, y)
        rt.reset()
        assert all(rt.snapshot(b)[0] == 0 for b in range(streams))
        stepped = np.stack([rt.step(events[i]) for i in range(steps)])
        states = [rt.snapshot(b) for b in range(streams)]
        rt.reset()
        mean, per = rt.device_run(events)
        assert mean > 0 and per.shape == (steps,) and np.all(per > 0)
        for b in range(streams):
            traced = rt.snapshot(b)
            assert traced[0] == states[b][0] == steps
            for x, y in zip(traced[1:], states[b][1:]):
                np.testing.assert_array_equal(x, y)
        # the scores of the last device-run step are the stepped ones
        rt.reset()
        for i in range(steps - 1):
            rt.step(events[i])
        np.testing.assert_array_equal(rt.step(events[-1]), stepped[-1])


@pytest.mark.parametrize('weights,streams', [(WeightStorage.BF16, 64), (WeightStorage.BF16, 256),
                                             (WeightStorage.AS_MODEL, 64)])
def test_large_rings_read_non_temporally_match_a_batch_of_one(weights, streams):
    # Main with FP32 K/V: from 64 streams the K/V rings and the weights exceed the Infinity
    # Cache, and attention reads K/V with non-temporal loads (and other loop forms); a batch of
    # one reads them with ordinary loads. Scores and state must agree bit for bit.
    c = SHAPES['main']
    w = synthetic_checkpoint(c, seed=17)
    steps = 36
    events = _events(c, 17, steps, streams)
    picks = (0, streams // 2, streams - 1)
    with batch((c, w, False), streams, weights) as rt:
        many = np.stack([rt.step(events[i]) for i in range(steps)])
        states = [rt.snapshot(b) for b in picks]
    for b, state in zip(picks, states):
        with batch((c, w, False), 1, weights) as one:
            alone = np.array([one.step(events[i, b:b + 1])[0] for i in range(steps)], dtype=np.float32)
            np.testing.assert_array_equal(alone, many[:, b])
            ref = one.snapshot(0)
        assert ref[0] == state[0] == steps
        for x, y in zip(ref[1:], state[1:]):
            np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize('weights,mixed,streams', [
    (WeightStorage.BF16, False, 256),
    (WeightStorage.AS_MODEL, True, 70),
])
def test_eager_launches_equal_the_graph_replay(weights, mixed, streams):
    c = SHAPES['main']
    w = synthetic_checkpoint(c, seed=16, mixed=mixed)
    steps = c.window + 8
    events = _events(c, 16, steps, streams)
    runs = []
    for eager in (False, True):
        with batch((c, w, mixed), streams, weights) as rt:
            rt.set_eager(eager)
            scores = [rt.step(events[i]) for i in range(4)]
            rt.device_run(events[4:steps - 1])
            scores.append(rt.step(events[steps - 1]))
            runs.append((np.stack(scores), [rt.snapshot(b) for b in (0, streams // 2, streams - 1)]))
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert a[0] == b[0] == steps
        for x, y in zip(a[1:], b[1:]):
            np.testing.assert_array_equal(x, y)


def test_invalid_arguments_are_rejected():
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=15)
    for streams in (0, 257):
        with pytest.raises(RuntimeError, match='Streams'):
            BatchRuntime((c, w, False), streams)
    with pytest.raises(RuntimeError, match='bfloat16'):
        BatchRuntime((c, synthetic_checkpoint(c, seed=15, mixed=True), True), 4, WeightStorage.BF16)
    odd = ModelConfig(1, 40, 1, 40, 8, 40)
    with pytest.raises(RuntimeError, match='multiples of 16'):
        BatchRuntime((odd, synthetic_checkpoint(odd, seed=15), False), 4)
    with batch((c, w, False), 4) as rt:
        with pytest.raises(RuntimeError, match='out of range'):
            rt.reset(4)
        with pytest.raises(RuntimeError, match='out of range'):
            rt.snapshot(-1)
        with pytest.raises(ValueError):
            rt.step(np.zeros((3, c.features), dtype=np.float32))
        with pytest.raises(RuntimeError, match='eager'):
            _check(library().st_batch_set_eager(rt._handle(), 2))

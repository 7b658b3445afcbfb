"""The reference's device-primitive edge cases (tests/Primitives.cu), restated at the level of
the whole step through the C ABI, plus the runtime's own boundary cases.

  - RoPE at absolute positions 0, 255, 10007 (traced steps) and past 10^6 (a device trace of
    1,000,003 events): rotated q / k rows against the textbook rotation of the projected rows
    in float64, with the reference's tolerance 1e-5 + 1e-4|x| (tests/Primitives.cu:190-218);
  - softmax over window lengths 1..512 (tests/Primitives.cu:220-264): logits of about +-10
    against the FP64-accumulating oracle, and logits spanning about +-10^4 (chunk maxima of one
    head thousands apart, most combine weights underflowing to 0) against the float64 softmax
    of the step's own q and K/V within the FP32 logit-rounding bound;
  - odd shapes: FFN 127 and 31 features (tests/Primitives.cu:104-153), a window that is not a
    multiple of the attention chunk with head dim 48;
  - the hand-sized layer of tests/Primitives.cu:322-414 (width 8, 2 heads of 4, window 3, at
    t = 3 the ring wraps onto slot 0): every traced operation against its closed form;
  - a state poisoned with NaN (NaN events fill every ring row), then RESET: the following steps
    match the oracle on every backend (the reference's poisoned-slot case, tests/Primitives.cu:
    15-98, and a RESET after non-finite state);
  - epoch rebase: starting 10 steps below the epoch limit, every backend crosses the rebase
    and stays bit-identical to a runtime that never rebases;
  - mapped staging (src/cuda/Runtime.cu:43-48,435-450): bit-identical to pinned copies.
"""
import os

import numpy as np
import pytest

from oracle.pyoracle import Oracle
from streamtx import Backend, ModelConfig, Runtime, RuntimeOptions, numerical, round_half, synthetic_checkpoint

pytestmark = pytest.mark.gpu

STRICT = dict(atol=1e-6, rtol=1e-5)
REFERENCE_BAR = dict(atol=1e-5, rtol=1e-4)
THREADS = min(16, os.cpu_count() or 1)
EPOCH_LIMIT = 0xF0000000


def _runtime(model, backend, **kw):
    kw.setdefault('blocks', 0)
    print(f'[case] backend={Backend(backend).name} {kw}', flush=True)
    return Runtime(model, RuntimeOptions(backend=backend, **kw))


def _events(config, seed, count):
    return np.random.default_rng(seed).standard_normal((count, config.features), dtype=np.float32)


def _rms(x, g, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * g


def _rotate(rows, position, dim):
    """Adjacent-pair RoPE of rows [heads*dim] at `position`: the angle in FP32 as the
    reference computes it (float(t) * powf(10000, -i/dim)), the rotation in float64."""
    i = np.arange(0, dim, 2, dtype=np.float32)
    angle = (np.float32(position) * np.power(np.float32(10000.0), -i / np.float32(dim))).astype(np.float64)
    a = np.asarray(rows, np.float64).reshape(-1, dim // 2, 2)
    co, si = np.cos(angle), np.sin(angle)
    return np.stack([a[..., 0] * co - a[..., 1] * si, a[..., 0] * si + a[..., 1] * co], -1).reshape(-1)


def _close(actual, expected, atol, rtol):
    a, e = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    bad = np.abs(a - e) > atol + rtol * np.abs(e)
    assert not bad.any(), (int(bad.sum()), float(np.abs(a - e).max()))


# ---- RoPE at absolute positions

ROPE = ModelConfig(1, 128, 4, 256, 2, 32)  # the reference's AbsolutePositions shape


@pytest.mark.parametrize('position', [0, 255, 10007])
def test_rope_at_absolute_positions_traced(position):
    c = ROPE
    w = synthetic_checkpoint(c, seed=31)
    with _runtime((c, w, False), Backend.CUDA) as rt:
        if position:
            rt.device_run(np.zeros((position, c.features), np.float32), reset=True)
        e = _events(c, 31, 1)[0]
        t = rt.trace_step(e)
        pos, keys, _, _ = rt.snapshot()
    assert pos == position + 1
    for m in ('q', 'k'):
        _close(t[f'layers.0.{m}'], _rotate(t[f'layers.0.{m}.linear'], position, c.dim), **REFERENCE_BAR)
    np.testing.assert_array_equal(t['layers.0.k'].reshape(c.heads, c.dim), keys[0, :, position % c.window])


def test_rope_past_a_million_positions():
    # 1,000,003 events in one device trace (zeros, then three random events): the last two
    # ring rows are k at positions 1,000,001 and 1,000,002, checked against the closed form
    # rope(W_k . norm1(W_in . e)) with float64 projections.
    c = ROPE
    w = synthetic_checkpoint(c, seed=32)
    count = 1_000_003
    events = np.zeros((count, c.features), np.float32)
    events[-3:] = _events(c, 32, 3)
    with _runtime((c, w, False), Backend.FUSED, blocks=1) as rt:
        rt.device_trace(events)
        pos, keys, values, _ = rt.snapshot()
    del events
    assert pos == count
    last = _events(c, 32, 3)
    for j, position in ((1, count - 2), (2, count - 1)):
        x = w['input'].astype(np.float64) @ last[j]
        z = _rms(x, w['layers.0.norm1'], c.epsilon)
        k = _rotate(w['layers.0.k'].astype(np.float64) @ z, position, c.dim)
        v = w['layers.0.v'].astype(np.float64) @ z
        slot = position % c.window
        _close(keys[0, :, slot].reshape(-1), k, **REFERENCE_BAR)
        _close(values[0, :, slot].reshape(-1), v, **REFERENCE_BAR)


# ---- softmax over disparate logits

def test_softmax_mixing_logits_match_oracle():
    # W_q scaled so that q.k / sqrt(dh) (otherwise of standard deviation ~0.02^2 * width = 0.05)
    # spans about +-10: many slots of the 512-slot window mix, over 32 chunks per head.
    c = ModelConfig(1, 128, 2, 256, 512, 128)
    w = synthetic_checkpoint(c, seed=33)
    w['layers.0.q'] = (w['layers.0.q'] * np.float32(200.0)).astype(np.float32)
    events = _events(c, 33, c.window + 40)
    oracle = Oracle(c, w, accumulate='double', threads=THREADS)
    with _runtime((c, w, False), Backend.FUSED) as rt:
        for i, e in enumerate(events):
            got, ref = rt.step(e), oracle.step(e)
            assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (i, got, ref)
        state = rt.snapshot()
    ostate = oracle.snapshot()
    assert state[0] == ostate[0]
    for a, o in zip(state[1:], ostate[1:]):
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, float(np.abs(a - o).max())


@pytest.mark.parametrize('config', [ModelConfig(1, 128, 4, 256, 512, 32), ModelConfig(1, 128, 2, 256, 512, 128)])
def test_softmax_disparate_chunk_maxima_within_rounding_bound(config):
    # W_q scaled by 2e5: logits span about +-1e4, so the chunk maxima of one head differ by
    # thousands and almost every combine weight exp(m_c - M) underflows to 0. Each traced
    # attention output is compared with the float64 softmax over the valid window computed from
    # the step's own q and the K/V ring, within the bound that FP32 rounding of the logits
    # allows: logits within d_j = gamma(2 dh + 2) sum_i |q_i k_ji| / sqrt(dh) of their exact
    # values move the output by at most (exp(2 max d_j) - 1) sum_j p_j |v_j - attn| (plus the
    # rounding of the weighted sum). That bound is tight where one slot dominates, so a
    # dropped, repeated or misordered chunk (an O(1) change) fails it; near-tied slots widen it
    # as they widen the FP32 computation's own error. The K/V ring does not depend on the
    # attention (one layer) and is held to the strict bar against the oracle.
    c = config
    w = synthetic_checkpoint(c, seed=33)
    w['layers.0.q'] = (w['layers.0.q'] * np.float32(2e5)).astype(np.float32)
    events = _events(c, 33, c.window + 40)
    oracle = Oracle(c, w, accumulate='double', threads=THREADS)
    u = 2.0 ** -24
    checked = 0
    with _runtime((c, w, False), Backend.CUDA) as rt:
        for i, e in enumerate(events):
            oracle.step(e)
            if not (i % 23 == 0 or i >= c.window - 1):
                rt.step(e)
                continue
            t = rt.trace_step(e)
            pos, keys, values, _ = rt.snapshot()
            valid = min(pos, c.window)
            slots = [(pos - valid + j) % c.window for j in range(valid)]
            q = t['layers.0.q'].astype(np.float64).reshape(c.heads, c.dim)
            attn = t['layers.0.attention'].astype(np.float64).reshape(c.heads, c.dim)
            assert np.isfinite(attn).all()
            for h in range(c.heads):
                k = keys[0, h, slots].astype(np.float64)
                v = values[0, h, slots].astype(np.float64)
                logits = k @ q[h] / np.sqrt(c.dim)
                p = np.exp(logits - logits.max())
                p /= p.sum()
                want = p @ v
                delta = (2 * c.dim + 2) * u / (1 - (2 * c.dim + 2) * u) * (np.abs(k) @ np.abs(q[h])) / np.sqrt(c.dim)
                delta += u * np.abs(logits)
                spread = p @ np.abs(v - want)
                bound = (np.exp(2 * delta.max()) - 1) * spread + 64 * u * (p @ np.abs(v)) + 1e-7
                err = np.abs(attn[h] - want)
                assert np.all(err <= bound), (i, h, float(err.max()), float(bound[np.argmax(err - bound)]))
            checked += 1
        state = rt.snapshot()
    assert checked > 40
    ostate = oracle.snapshot()
    assert state[0] == ostate[0]
    for a, o in zip(state[1:3], ostate[1:3]):
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, float(np.abs(a - o).max())


# ---- odd shapes

@pytest.mark.parametrize('mixed', [False, True])
@pytest.mark.parametrize('config', [ModelConfig(2, 64, 2, 127, 16, 31), ModelConfig(2, 96, 2, 192, 37, 96)])
def test_odd_shapes_match_oracle(config, mixed):
    c = config
    w = synthetic_checkpoint(c, seed=34, mixed=mixed)
    events = _events(c, 34, 3 * c.window + 5)
    reset_at = 2 * c.window + 1
    for backend, blocks in ((Backend.FUSED, 0), (Backend.FUSED, 3), (Backend.CUDA, 0)):
        oracle = Oracle(c, w, mixed=mixed, accumulate='float' if mixed else 'double', threads=THREADS)
        scores, refs = [], []
        with _runtime((c, w, mixed), backend, blocks=blocks) as rt:
            for i, e in enumerate(events):
                if i == reset_at:
                    rt.reset()
                    oracle.reset()
                got, ref = rt.step(e), oracle.step(e)
                scores.append(got)
                refs.append(ref)
                if not mixed:
                    assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (i, got, ref)
            state = rt.snapshot()
        ostate = oracle.snapshot()
        assert state[0] == ostate[0]
        if mixed:
            assert numerical.score_errors(scores, refs, c.layers)['passed']
            assert numerical.mixed_state_passes(*state[1:], *ostate[1:])['passed']
        else:
            for a, o in zip(state[1:], ostate[1:]):
                assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, float(np.abs(a - o).max())


# ---- the hand-sized layer

@pytest.mark.parametrize('mixed', [False, True])
def test_hand_sized_layer_at_t3_window3(mixed):
    # tests/Primitives.cu:322-414: width 8, 2 heads of 4, FFN 8, window 3, 4 features; at t = 3
    # the new K/V row overwrites slot 0. Weights (i % 11 - 5) / 8 as there, norm weights 1.
    c = ModelConfig(1, 8, 2, 8, 3, 4)
    w = {}
    for name, shape in (('input', (8, 4)), ('layers.0.q', (8, 8)), ('layers.0.k', (8, 8)), ('layers.0.v', (8, 8)),
                        ('layers.0.out', (8, 8)), ('layers.0.gate', (8, 8)), ('layers.0.up', (8, 8)),
                        ('layers.0.down', (8, 8)), ('score', (1, 8))):
        n = shape[0] * shape[1]
        w[name] = ((np.arange(n) % 11 - 5) * 0.125).astype(np.float32).reshape(shape)
    for name in ('layers.0.norm1', 'layers.0.norm2', 'final_norm'):
        w[name] = np.ones(8, np.float32)
    cast = (lambda v: round_half(np.asarray(v, np.float32))) if mixed else (lambda v: np.asarray(v, np.float64))
    tol = dict(atol=1e-3, rtol=0) if mixed else dict(atol=2e-6, rtol=2e-5)
    events = [np.array([.25, -.5, .75, 1], np.float32) * (1 + 0.1 * i) for i in range(4)]
    with _runtime((c, w, mixed), Backend.CUDA) as rt:
        for e in events[:3]:
            rt.step(e)
        t = rt.trace_step(events[3])
        pos, keys, values, hidden = rt.snapshot()
    assert pos == 4
    W = {k: v.astype(np.float64) for k, v in w.items()}
    _close(t['input'], cast(W['input'] @ events[3]), **tol)
    x = t['input']
    n1 = t['layers.0.norm1.norm']
    _close(n1, cast(_rms(x, 1.0, c.epsilon)), **tol)
    for m in ('q', 'k'):
        lin = t[f'layers.0.{m}.linear']
        _close(lin, cast(W[f'layers.0.{m}'] @ n1), **tol)
        _close(t[f'layers.0.{m}'], cast(_rotate(lin, 3, c.dim)), **tol)
    _close(t['layers.0.v'], cast(W['layers.0.v'] @ n1), **tol)
    # The ring: slot 0 holds t = 3's row, slots 1 and 2 those of t = 1 and t = 2.
    np.testing.assert_array_equal(keys[0, :, 0].reshape(-1), t['layers.0.k'])
    np.testing.assert_array_equal(values[0, :, 0].reshape(-1), t['layers.0.v'])
    q = t['layers.0.q'].reshape(c.heads, c.dim).astype(np.float64)
    attention = []
    for h in range(c.heads):
        order = [1, 2, 0]  # chronological slots at t = 3: positions 1, 2, 3
        k = keys[0, h, order].astype(np.float64)
        v = values[0, h, order].astype(np.float64)
        logits = k @ q[h] / np.sqrt(c.dim)
        p = np.exp(logits - logits.max())
        attention.append(p @ v / p.sum())
    _close(t['layers.0.attention'], cast(np.concatenate(attention)), **tol)
    out = t['layers.0.out.linear']
    _close(out, cast(W['layers.0.out'] @ t['layers.0.attention']), **tol)
    _close(t['layers.0.attention_residual'], cast(x + out), **tol)
    xr = t['layers.0.attention_residual']
    n2 = t['layers.0.norm2.norm']
    _close(n2, cast(_rms(xr, 1.0, c.epsilon)), **tol)
    g, u = t['layers.0.gate.linear'], t['layers.0.up.linear']
    _close(g, cast(W['layers.0.gate'] @ n2), **tol)
    _close(u, cast(W['layers.0.up'] @ n2), **tol)
    g64 = np.asarray(g, np.float64)
    _close(t['layers.0.activation'], cast(g64 / (1 + np.exp(-g64)) * u), **tol)
    _close(t['layers.0.hidden'], cast(xr + t['layers.0.down.linear']), **tol)
    np.testing.assert_array_equal(hidden[0], t['layers.0.hidden'])
    fin = _rms(t['layers.0.hidden'], 1.0, c.epsilon)
    _close(t['final_norm.norm'], cast(fin), **tol)
    _close(t['score.linear'], W['score'] @ t['final_norm.norm'], **tol)


# ---- poisoned state, then RESET

@pytest.mark.parametrize('backend', [Backend.FUSED, Backend.CUDA, Backend.GRAPH, Backend.PERSISTENT])
def test_reset_recovers_from_nan_state(backend):
    c = ModelConfig(2, 256, 4, 512, 48, 256)
    w = synthetic_checkpoint(c, seed=35)
    nan = np.full(c.features, np.nan, np.float32)
    events = _events(c, 35, 2 * c.window + 7)
    oracle = Oracle(c, w, accumulate='double', threads=THREADS)
    kw = dict(idle_seconds=10.0) if backend == Backend.PERSISTENT else {}
    with _runtime((c, w, False), backend, **kw) as rt:
        for _ in range(c.window + 3):
            assert np.isnan(rt.step(nan))
        _, keys, _, _ = rt.snapshot()
        assert np.isnan(keys).all()
        rt.reset()
        for i, e in enumerate(events):
            got, ref = rt.step(e), oracle.step(e)
            assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (i, got, ref)
        state = rt.snapshot()
    ostate = oracle.snapshot()
    assert state[0] == ostate[0]
    for a, o in zip(state[1:], ostate[1:]):
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0


# ---- epoch rebase

@pytest.mark.parametrize('backend', [Backend.FUSED, Backend.GRAPH, Backend.CUDA, Backend.PERSISTENT])
def test_epoch_rebase_is_invisible(backend):
    c = ModelConfig(2, 256, 4, 512, 32, 256)
    w = synthetic_checkpoint(c, seed=36)
    events = _events(c, 36, 40)
    per_step = 5 * c.layers + 3
    kw = dict(idle_seconds=10.0) if backend == Backend.PERSISTENT else {}
    results = []
    for epoch in (0, EPOCH_LIMIT - 10 * per_step + 3):
        with _runtime((c, w, False), backend, initial_epoch=epoch, **kw) as rt:
            scores = []
            for i, e in enumerate(events):
                if i == 25:
                    rt.reset()
                scores.append(rt.step(e))
            results.append((np.array(scores, np.float32), rt.snapshot()))
    (s0, st0), (s1, st1) = results
    np.testing.assert_array_equal(s1, s0)
    assert st1[0] == st0[0]
    for a, b in zip(st1[1:], st0[1:]):
        np.testing.assert_array_equal(a, b)


def test_epoch_rebase_device_trace_and_budget():
    c = ModelConfig(2, 256, 4, 512, 32, 256)
    w = synthetic_checkpoint(c, seed=37)
    events = _events(c, 37, 30)
    per_step = 5 * c.layers + 3
    near = EPOCH_LIMIT - 10 * per_step + 3
    traced = []
    for epoch in (0, near):
        with _runtime((c, w, False), Backend.FUSED, initial_epoch=epoch) as rt:
            rt.device_trace(events)
            traced.append(rt.snapshot())
    assert traced[0][0] == traced[1][0] == len(events)
    for a, b in zip(traced[0][1:], traced[1][1:]):
        np.testing.assert_array_equal(a, b)
    # The persistent worker's RUN budget survives its relaunch at the rebase.
    with _runtime((c, w, False), Backend.PERSISTENT, initial_epoch=near, max_events=20, idle_seconds=10.0) as rt:
        for e in events[:20]:
            rt.step(e)
        with pytest.raises(RuntimeError, match='exited'):
            rt.step(events[20])


# ---- mapped staging

@pytest.mark.parametrize('backend', [Backend.CUDA, Backend.GRAPH, Backend.FUSED, Backend.CUBLAS, Backend.CUBLAS_GRAPH])
def test_mapped_staging_equals_pinned_copies(backend):
    c = ModelConfig(2, 256, 4, 512, 24, 200)
    w = synthetic_checkpoint(c, seed=38)
    events = _events(c, 38, 60)
    results = []
    for mapped in (False, True):
        with _runtime((c, w, False), backend, mapped=mapped) as rt:
            info = rt.info()
            assert info['transport'] == ('mapped-stream-sync' if mapped else 'pinned-copy-stream-sync')
            scores = [rt.step(e) for e in events[:40]]
            rt.device_run(events[40:])
            results.append((np.array(scores, np.float32), rt.snapshot()))
    (s0, st0), (s1, st1) = results
    np.testing.assert_array_equal(s1, s0)
    for a, b in zip(st1, st0):
        np.testing.assert_array_equal(a, b)


# Events of 29 features (the staged row's tail is padding): the mapped staging kernel moves the
# padded row in 16-byte pieces; FP32 and mixed.
@pytest.mark.parametrize('backend,mixed', [(Backend.FUSED, False), (Backend.FUSED, True), (Backend.GRAPH, True)])
def test_mapped_staging_of_a_ragged_event(backend, mixed):
    c = ModelConfig(2, 128, 2, 256, 20, 29)
    w = synthetic_checkpoint(c, seed=39, mixed=mixed)
    events = _events(c, 39, 50)
    results = []
    for mapped in (False, True):
        with _runtime((c, w, mixed), backend, mapped=mapped) as rt:
            scores = [rt.step(e) for e in events]
            results.append((np.array(scores, np.float32), rt.snapshot()))
    (s0, st0), (s1, st1) = results
    np.testing.assert_array_equal(s1, s0)
    for a, b in zip(st1, st0):
        np.testing.assert_array_equal(a, b)

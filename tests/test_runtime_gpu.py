"""GPU parity of libstamd.so against the reference's golden vectors and the CPU oracle.

Every test calls the HIP path through the C ABI (streamtx.runtime). Bars:
  - reference fixtures: the reference's tolerances (FP32 1e-5 + 1e-4|r|, mixed v3 policy);
  - CPU oracle (FP64-accumulating referee): FP32 within 1e-6 + 1e-5|r| per step, for the
    score and the complete carried state;
  - backends (staged, graph, fused, grid sizes): bit-identical to each other.
"""
import numpy as np
import pytest

import fp32bar
from oracle.pyoracle import Oracle
from streamtx import (Backend, ModelConfig, Runtime, RuntimeOptions, WeightStorage, numerical, round_bf16,
                      synthetic_checkpoint)

pytestmark = pytest.mark.gpu

STRICT = dict(atol=1e-6, rtol=1e-5)
# GRAPH with a full grid captures the fused kernel as one node; with one workgroup it captures
# the staged phase sequence.
BACKENDS = [(Backend.CUDA, 0), (Backend.GRAPH, 0), (Backend.GRAPH, 1), (Backend.FUSED, 1), (Backend.FUSED, 4),
            (Backend.FUSED, 0)]
# Vendor GEMV baselines (rocBLAS projections): same parity bars, their own summation order.
VENDOR = [(Backend.CUBLAS, 0), (Backend.CUBLAS_GRAPH, 0)]


def runtime(model, backend, blocks, **kw):
    print(f'[case] backend={Backend(backend).name} blocks={blocks} {kw}', flush=True)
    return Runtime(model, RuntimeOptions(backend=backend, blocks=blocks, **kw))


@pytest.mark.parametrize('backend,blocks', BACKENDS + VENDOR)
def test_fp32_fixture_every_event(golden, backend, blocks):
    g = golden('small-fp32')
    oracle = Oracle(g.config, g.checkpoint.tensors, accumulate='double')
    with runtime(g.checkpoint, backend, blocks) as rt:
        for i, score, keys, values, hidden in g.expected_state():
            if i in g.resets:
                rt.reset()
                oracle.reset()
            got = rt.step(g.trace[i])
            ref = oracle.step(g.trace[i])
            pos, k, v, h = rt.snapshot()
            _, ok, ov, oh = oracle.snapshot()
            assert pos == oracle.position
            assert numerical.fp32_failures([got], [score]) == 0, (i, got, score)
            assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (i, got, ref)
            for a, r, o in ((k, keys, ok), (v, values, ov), (h, hidden, oh)):
                assert numerical.fp32_failures(a, r) == 0, i
                assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, (i, float(np.abs(a - o).max()))


@pytest.mark.parametrize('backend,blocks', [(Backend.CUDA, 0), (Backend.GRAPH, 0), (Backend.FUSED, 0),
                                            (Backend.CUBLAS, 0), (Backend.CUBLAS_GRAPH, 0)])
def test_mixed_fixture_policy_v3(golden, backend, blocks):
    g = golden('small-mixed')
    scores, refs = [], []
    with runtime(g.checkpoint, backend, blocks) as rt:
        for i, score, keys, values, hidden in g.expected_state():
            if i in g.resets:
                rt.reset()
            scores.append(rt.step(g.trace[i]))
            refs.append(score)
            _, k, v, h = rt.snapshot()
            res = numerical.mixed_state_passes(k, v, h, keys, values, hidden)
            assert res['passed'], (i, res['failures'][:2])
            for a in (k, v, h):
                assert np.array_equal(a, a.astype(np.float16).astype(np.float32))
    res = numerical.score_errors(scores, refs, g.config.layers)
    assert res['passed'], res


def _stream(config, seed, count):
    return np.random.default_rng(seed).standard_normal((count, config.features)).astype(np.float32)


SHAPES = {
    # the Small, Main and Large configurations with features = d_model (SwiGLU, RoPE, norm weights 1)
    'small': ModelConfig(4, 256, 4, 1024, 64, 256),
    'main': ModelConfig(8, 512, 8, 2048, 128, 512),
    'large': ModelConfig(12, 1024, 16, 4096, 512, 1024),
    # reference fixture shapes with head dim 32 (configs/main.json, configs/large.json)
    'ref-main': ModelConfig(2, 128, 4, 256, 256, 32),
    'ref-large': ModelConfig(4, 256, 8, 512, 512, 32),
    # head dim 48 (not a power of two): attention reads K/V rows in place from the FIFO
    'dh48': ModelConfig(2, 96, 2, 192, 40, 96),
    # 48 active chunks per head at full window: the general partial-combine path
    'long-window': ModelConfig(1, 128, 2, 256, 1536, 128),
}


@pytest.mark.parametrize('name,steps,reset_at', [('small', 160, 137), ('main', 40, None), ('large', 12, None),
                                                 ('ref-main', 300, 261), ('ref-large', 64, None),
                                                 ('dh48', 100, 57), ('long-window', 1540, None)])
def test_fused_matches_oracle_at_shape(name, steps, reset_at):
    # FP32 bar against the FP64 referee, or (deep models) no worse than the reference's own
    # FP32 algorithm, the float oracle (tests/fp32bar.py).
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=1)
    events = _stream(c, 1, steps)
    oracle = Oracle(c, w, accumulate='double', threads=8)
    oracle32 = Oracle(c, w, accumulate='float', threads=8)
    scores, refs, refs32 = [], [], []
    with runtime((c, w, False), Backend.FUSED, 0) as rt:
        for i, e in enumerate(events):
            if i == reset_at:
                rt.reset()
                oracle.reset()
                oracle32.reset()
            scores.append(rt.step(e))
            refs.append(oracle.step(e))
            refs32.append(oracle32.step(e))
        state = rt.snapshot()
    fp32bar.check(scores, refs, refs32, f'{name} scores')
    ostate, ostate32 = oracle.snapshot(), oracle32.snapshot()
    assert state[0] == ostate[0]
    for name_, a, o, o32 in zip(('keys', 'values', 'hidden'), state[1:], ostate[1:], ostate32[1:]):
        fp32bar.check(a, o, o32, f'{name} {name_}')


@pytest.mark.parametrize('name,steps', [('small', 150), ('main', 140), ('ref-main', 64), ('dh48', 50)])
def test_backends_are_bit_identical(name, steps):
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=2)
    events = _stream(c, 2, steps)
    results = []
    for backend, blocks in BACKENDS:
        with runtime((c, w, False), backend, blocks) as rt:
            scores = np.array([rt.step(e) for e in events], dtype=np.float32)
            results.append((scores, rt.snapshot()))
    base_scores, base_state = results[0]
    for scores, state in results[1:]:
        np.testing.assert_array_equal(scores, base_scores)
        assert state[0] == base_state[0]
        for a, b in zip(state[1:], base_state[1:]):
            np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize('mixed', [False, True])
def test_zero_input_scores_zero(mixed):
    c = ModelConfig(2, 256, 4, 512, 16, 256)
    w = synthetic_checkpoint(c, seed=4, mixed=mixed)
    zero = np.zeros(c.features, dtype=np.float32)
    with runtime((c, w, mixed), Backend.FUSED, 0) as rt:
        for i in range(3 * c.window + 9):
            if i in (1, c.window, 2 * c.window + 3):
                rt.reset()
                rt.reset()
                assert rt.snapshot()[0] == 0
            assert rt.step(zero) == 0.0


@pytest.mark.parametrize('backend', [Backend.FUSED, Backend.GRAPH])
def test_device_trace_equals_stepping(backend):
    c = SHAPES['main']
    w = synthetic_checkpoint(c, seed=5)
    events = _stream(c, 5, 70)
    with runtime((c, w, False), backend, 0) as rt:
        for e in events:
            rt.step(e)
        stepped = rt.snapshot()
        mean, per = rt.device_trace(events)
        traced = rt.snapshot()
    assert mean > 0 and per.shape == (len(events),) and np.all(per > 0)
    assert traced[0] == stepped[0]
    for a, b in zip(traced[1:], stepped[1:]):
        np.testing.assert_array_equal(a, b)


def test_bf16_weights_equal_fp32_model_on_rounded_weights():
    c = SHAPES['main']
    w = synthetic_checkpoint(c, seed=6)
    rounded = {k: round_bf16(v) for k, v in w.items()}
    oracle = Oracle(c, rounded, accumulate='double', threads=8)
    events = _stream(c, 6, 40)
    with runtime((c, w, False), Backend.FUSED, 0, weight_dtype=WeightStorage.BF16) as rt:
        for e in events:
            got, ref = rt.step(e), oracle.step(e)
            assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (got, ref)
        _, k, v, h = rt.snapshot()
    _, ok, ov, oh = oracle.snapshot()
    for a, o in ((k, ok), (v, ov), (h, oh)):
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0


def test_mixed_baseline_shape_policy_v3():
    c = SHAPES['main']
    w = synthetic_checkpoint(c, seed=7, mixed=True)
    events = _stream(c, 7, 40)
    oracle = Oracle(c, w, mixed=True, threads=8)
    scores, refs = [], []
    with runtime((c, w, True), Backend.FUSED, 0) as rt:
        for e in events:
            scores.append(rt.step(e))
            refs.append(oracle.step(e))
        _, k, v, h = rt.snapshot()
    _, ok, ov, oh = oracle.snapshot()
    assert numerical.mixed_state_passes(k, v, h, ok, ov, oh)['passed']
    assert numerical.score_errors(scores, refs, c.layers)['passed']


def test_cooperative_grid_limit_and_info():
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=8)
    with runtime((c, w, False), Backend.FUSED, 0) as rt:
        info = rt.info()
    assert info['environment']['arch'].startswith('gfx950')
    assert info['blocks'] == info['environment']['compute_units']
    assert info['legal_cooperative_blocks'] >= info['blocks']
    assert info['fused_launch'] in ('plain', 'cooperative')
    assert info['weight_loads'] == 'temporal'  # about 17 MB of weights stay in the 256 MB Infinity Cache
    with pytest.raises(RuntimeError, match='occupancy limit'):
        Runtime((c, w, False), RuntimeOptions(backend=Backend.FUSED, blocks=info['legal_cooperative_blocks'] + 1))
    with runtime((c, w, False), Backend.GRAPH, 0) as rt:
        assert rt.info()['fused_launch'] == ('graph node (plain)' if info['fused_launch'] == 'plain'
                                             else 'n/a (phase sequence)')
    with runtime((c, w, False), Backend.GRAPH, 1) as rt:
        assert rt.info()['fused_launch'] == 'n/a (phase sequence)'


def test_stopped_runtime_rejects_commands():
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=9)
    with runtime((c, w, False), Backend.GRAPH, 0) as rt:
        rt.step(np.ones(c.features, np.float32))
        rt.stop()
        rt.stop()
        with pytest.raises(RuntimeError, match='stopped'):
            rt.step(np.ones(c.features, np.float32))
        with pytest.raises(RuntimeError, match='stopped'):
            rt.reset()


@pytest.mark.parametrize('name,steps,reset_at', [('main', 140, 131), ('dh48', 60, 41)])
def test_vendor_backends_match_oracle_and_graph_replays_match_eager(name, steps, reset_at):
    # The rocBLAS baseline against the oracle at the FP32 bar, and its captured graph against
    # eager launches bit for bit (graph replays interleaved with the host's own work).
    c = SHAPES[name]
    w = synthetic_checkpoint(c, seed=9)
    events = _stream(c, 9, steps)
    oracle = Oracle(c, w, accumulate='double', threads=8)
    results = []
    for backend in (Backend.CUBLAS, Backend.CUBLAS_GRAPH):
        scores = []
        with runtime((c, w, False), backend, 0) as rt:
            for i, e in enumerate(events):
                if i == reset_at:
                    rt.reset()
                    if backend == Backend.CUBLAS:
                        oracle.reset()
                got = rt.step(e)
                scores.append(got)
                if backend == Backend.CUBLAS:
                    ref = oracle.step(e)
                    assert numerical.fp32_strict_failures([got], [ref], **STRICT) == 0, (i, got, ref)
            results.append((np.array(scores, dtype=np.float32), rt.snapshot()))
    (s0, st0), (s1, st1) = results
    np.testing.assert_array_equal(s0, s1)
    _, ok, ov, oh = oracle.snapshot()
    for a, b, o in zip(st0[1:], st1[1:], (ok, ov, oh)):
        np.testing.assert_array_equal(a, b)
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, float(np.abs(a - o).max())


@pytest.mark.parametrize('fixture', ['main-mixed', 'small-fp32'])
def test_trace_step_preserves_execution(golden, fixture):
    # tests/Lifecycle.cu:108-137: traced steps give the scores and leave the state of ordinary
    # steps, bit for bit.
    g = golden(fixture)
    c = g.config
    with runtime(g.checkpoint, Backend.CUDA, 4) as rt:
        scores = [rt.step(e) for e in g.trace[:12]]
        state = rt.snapshot()
        rt.reset()
        for i, e in enumerate(g.trace[:12]):
            trace = rt.trace_step(e)
            assert trace['layers.0.attention'].shape == (c.width,)
            assert trace['score.linear'][0] == scores[i]
            if g.checkpoint.mixed:
                for name, v in trace.items():
                    # every cast point is FP16; the raw event and the uncast score are not
                    if not name.endswith('.pre_cast') and name != 'input.operand' and not name.startswith('score.'):
                        assert np.array_equal(v, v.astype(np.float16).astype(np.float32)), name
        traced = rt.snapshot()
    assert traced[0] == state[0]
    for a, b in zip(traced[1:], state[1:]):
        np.testing.assert_array_equal(a, b)


def _rms(x, g, eps):
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * g


def test_trace_entries_satisfy_the_model_equations():
    # The diagnostic entries against the model's closed forms (float64 numpy), and the phase
    # outputs against the carried state.
    c = ModelConfig(2, 128, 4, 256, 16, 96)
    w = synthetic_checkpoint(c, seed=21)
    events = _stream(c, 21, 20)
    tol = dict(atol=2e-6, rtol=2e-5)
    with runtime((c, w, False), Backend.CUDA, 0) as rt:
        for e in events[:19]:
            rt.step(e)
        t = rt.trace_step(events[19])
        pos, keys, values, hidden = rt.snapshot()
    position, slot = pos - 1, (pos - 1) % c.window
    lin = lambda name, m, v: np.testing.assert_allclose(t[name + '.linear'], m @ v.astype(np.float64), **tol)
    np.testing.assert_array_equal(t['input.operand'], events[19])
    lin('input', w['input'], events[19])
    np.testing.assert_allclose(t['input'], t['input.linear'], **tol)
    x = t['input']
    dh = c.dim
    inv = 10000.0 ** (-np.arange(0, dh, 2, dtype=np.float32) / dh)
    ang = np.float32(position) * inv.astype(np.float32)
    co, si = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
    for l in range(c.layers):
        p = f'layers.{l}.'
        np.testing.assert_array_equal(t[p + 'norm1.operand'], x)
        np.testing.assert_allclose(t[p + 'norm1.norm'], _rms(x, w[p + 'norm1'], c.epsilon), **tol)
        n1 = t[p + 'norm1.norm']
        for m in ('q', 'k', 'v'):
            np.testing.assert_array_equal(t[p + m + '.operand'], n1)
            lin(p + m, w[p + m], n1)
        for m in ('q', 'k'):
            a = t[p + m + '.linear'].reshape(c.heads, dh // 2, 2).astype(np.float64)
            rot = np.stack([a[..., 0] * co - a[..., 1] * si, a[..., 0] * si + a[..., 1] * co], -1)
            np.testing.assert_allclose(t[p + m], rot.reshape(-1), **tol)
        np.testing.assert_allclose(t[p + 'v'], t[p + 'v.linear'], **tol)
        np.testing.assert_array_equal(t[p + 'k'].reshape(c.heads, dh), keys[l, :, slot])
        np.testing.assert_array_equal(t[p + 'v'].reshape(c.heads, dh), values[l, :, slot])
        lin(p + 'out', w[p + 'out'], t[p + 'attention'])
        np.testing.assert_allclose(t[p + 'attention_residual'], x + t[p + 'out.linear'], **tol)
        x = t[p + 'attention_residual']
        np.testing.assert_allclose(t[p + 'norm2.norm'], _rms(x, w[p + 'norm2'], c.epsilon), **tol)
        for m in ('gate', 'up'):
            lin(p + m, w[p + m], t[p + 'norm2.norm'])
        gv, uv = t[p + 'gate.linear'].astype(np.float64), t[p + 'up.linear']
        np.testing.assert_allclose(t[p + 'activation'], gv / (1 + np.exp(-gv)) * uv, **tol)
        lin(p + 'down', w[p + 'down'], t[p + 'activation'])
        np.testing.assert_allclose(t[p + 'hidden'], x + t[p + 'down.linear'], **tol)
        np.testing.assert_array_equal(t[p + 'hidden'], hidden[l])
        x = t[p + 'hidden']
    np.testing.assert_allclose(t['final_norm.norm'], _rms(x, w['final_norm'], c.epsilon), **tol)
    np.testing.assert_allclose(t['score.linear'], w['score'] @ t['final_norm.norm'].astype(np.float64), **tol)


def test_trace_step_requires_staged_backend():
    c = ModelConfig(1, 64, 4, 128, 8, 32)
    w = synthetic_checkpoint(c, seed=22)
    with runtime((c, w, False), Backend.FUSED, 0) as rt:
        with pytest.raises(RuntimeError, match='staged'):
            rt.trace_step(np.zeros(c.features, dtype=np.float32))


@pytest.mark.parametrize('backend', [Backend.FUSED, Backend.PERSISTENT])
def test_scheduled_arrivals_step_every_kept_event_in_order(backend):
    # bench/Main.cpp:282-342: offered events go through a bounded queue; the consumer steps
    # the kept ones in order, so their scores equal plain stepping of the same subsequence.
    c = SHAPES['small']
    w = synthetic_checkpoint(c, seed=23)
    events = _stream(c, 23, 400)
    kw = dict(idle_seconds=10.0) if backend == Backend.PERSISTENT else {}
    with runtime((c, w, False), backend, 0, **kw) as rt:
        r = rt.scheduled_run(events, rate=4000.0, queue=4096)
        s = r['summary']
        assert s['offered'] == 400 and s['dropped'] == 0 and s['completed'] == 400
        assert np.all(r['intended_ns'] <= r['enqueue_ns']) and np.all(r['enqueue_ns'] <= r['submit_ns'])
        assert np.all(r['submit_ns'] < r['complete_ns'])
        assert np.all(np.diff(r['submit_ns']) > 0)
        assert s['service']['p50_us'] > 0 and s['arrival']['p50_us'] >= s['service']['p50_us']
        rt.reset()
        # A one-slot queue offered faster than service drops events; the kept ones still run in order.
        r2 = rt.scheduled_run(events[:200], rate=1e6, queue=1)
        kept = ~r2['dropped']
        assert r2['summary']['dropped'] > 0 and kept.sum() == r2['summary']['completed'] > 0
        assert np.all(np.isnan(r2['scores'][~kept]))
    with runtime((c, w, False), Backend.FUSED, 0) as ref:
        plain = np.array([ref.step(e) for e in events], dtype=np.float32)
        np.testing.assert_array_equal(r['scores'], plain)
        ref.reset()
        plain2 = np.array([ref.step(e) for e in events[:200][kept]], dtype=np.float32)
        np.testing.assert_array_equal(r2['scores'][kept], plain2)

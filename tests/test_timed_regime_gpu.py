"""GPU parity in the regime the benchmark times, and at the benchmark configurations' full
stream lengths, through the C ABI.

  - Large (d 1024, 12 layers, 16 heads x 64, FFN 4096, W 512) in FP32, bfloat16-weight and
    mixed storage at the configured 4096 events: every score (511 to fill the window, then
    3585 full-window steps, 32 attention chunks per head, the ring wrapping seven times) and
    the complete carried state at three points are compared with the oracle;
  - Small (512 events, seed 0) and Main (2048 events, seed 1) FP32 at their configured stream
    lengths on the staged, graph, fused and persistent backends: bit-identical to each other
    and within the FP32 bar of the FP64-accumulating oracle;
  - the Main window sweep, W in {32, 64, 256, 512}, 2048 events each, bfloat16 weights (FP32
    bar against the oracle on the rounded weights) and mixed mode (the reference's policy v3
    against the mixed oracle);
  - batched Main with bfloat16 weights at B = 64 and 256: sampled streams against their own
    oracle (stream b's inputs from seed 4 + b).

Bars: FP32 |a - r| <= 1e-6 + 1e-5 |r| per score and state element against the FP64 referee
(bit-identical across backends), or at Large depth no worse than the reference's own FP32
algorithm (tests/fp32bar.py); mixed: numerical.score_errors / mixed_state_passes (policy v3).
"""
import os
import threading

import numpy as np
import pytest

import fp32bar
from oracle.pyoracle import Oracle
from streamtx import (Backend, BatchRuntime, ModelConfig, Runtime, RuntimeOptions, WeightStorage, numerical,
                      round_bf16, synthetic_checkpoint)

pytestmark = pytest.mark.gpu

STRICT = dict(atol=1e-6, rtol=1e-5)
THREADS = min(16, os.cpu_count() or 1)
LARGE = ModelConfig(12, 1024, 16, 4096, 512, 1024)
MAIN = ModelConfig(8, 512, 8, 2048, 128, 512)
SMALL = ModelConfig(4, 256, 4, 1024, 64, 256)


def _events(config, seed, count):
    return np.random.default_rng(seed).standard_normal((count, config.features), dtype=np.float32)


def _runtime(model, backend, **kw):
    kw.setdefault('blocks', 0)
    print(f'[case] backend={Backend(backend).name} {kw}', flush=True)
    return Runtime(model, RuntimeOptions(backend=backend, **kw))


def _assert_state_strict(state, oracle_state):
    assert state[0] == oracle_state[0]
    for a, o in zip(state[1:], oracle_state[1:]):
        bad = numerical.fp32_strict_failures(a, o, **STRICT)
        assert bad == 0, (bad, float(np.abs(a - o).max()))


def _host_isa():
    """'v3' (the oracle's AVX2 build, bit-identical results, faster) on hosts that have it."""
    try:
        flags = set(open('/proc/cpuinfo').read().split())
    except OSError:
        return 'portable'
    return 'v3' if {'avx2', 'fma', 'bmi2', 'movbe'} <= flags else 'portable'


def _oracle_scores(oracles, events, snap_at=()):
    """Step every oracle through all events, each in its own thread (the C oracle releases the
    GIL in its calls). Returns the scores [oracle][event] and the snapshots taken after the
    events in snap_at."""
    scores = [np.empty(len(events), dtype=np.float64) for _ in oracles]
    snaps = [{} for _ in oracles]

    def work(k):
        o = oracles[k]
        for i, e in enumerate(events):
            scores[k][i] = o.step(e)
            if i in snap_at:
                snaps[k][i] = o.snapshot()

    threads = [threading.Thread(target=work, args=(k,)) for k in range(len(oracles))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    return scores, snaps


@pytest.mark.parametrize('precision', ['fp32', 'bf16w', 'mixed'])
def test_large_configured_stream_matches_oracle(precision):
    """Large at its configured stream length: 4096 events from seed 3 (511 to fill the window,
    then 3585 full-window steps with 32 attention chunks per head and the ring wrapping seven
    times). Every score is compared, and the complete carried state after the last fill event,
    half way and at the end."""
    c = LARGE
    mixed = precision == 'mixed'
    w = synthetic_checkpoint(c, seed=3, mixed=mixed)
    count = 4096
    events = _events(c, 3, count)
    snap_at = (c.window - 2, count // 2 - 1, count - 1)
    isa = _host_isa()
    if precision == 'bf16w':
        rounded = {k: round_bf16(v) for k, v in w.items()}
        oracles = [Oracle(c, rounded, accumulate=a, threads=THREADS // 2, isa=isa) for a in ('double', 'float')]
        storage = WeightStorage.BF16
    elif mixed:
        oracles = [Oracle(c, w, mixed=True, threads=THREADS, isa=isa)]
        storage = WeightStorage.AS_MODEL
    else:
        oracles = [Oracle(c, w, accumulate=a, threads=THREADS // 2, isa=isa) for a in ('double', 'float')]
        storage = WeightStorage.AS_MODEL
    scores, states = np.empty(count, dtype=np.float32), {}
    with _runtime((c, w, mixed), Backend.FUSED, weight_dtype=storage) as rt:
        # Large's weights (430-860 MB) exceed the Infinity Cache: they stream non-temporally.
        assert rt.info()['weight_loads'] == 'non-temporal'
        for i, e in enumerate(events):
            scores[i] = rt.step(e)
            if i in snap_at:
                states[i] = rt.snapshot()
    print(f'[large {precision}] {count} GPU steps done; running the oracle(s) on {THREADS} threads ({isa})',
          flush=True)
    refs, snaps = _oracle_scores(oracles, events, snap_at)
    print(f'[large {precision}] max |score - oracle| over {count} steps: {float(np.max(np.abs(scores - refs[0]))):.3g}',
          flush=True)
    for i in snap_at:
        assert states[i][0] == snaps[0][i][0] == i + 1
    if mixed:
        assert numerical.score_errors(scores, refs[0], c.layers)['passed']
        for i in snap_at:
            assert numerical.mixed_state_passes(*states[i][1:], *snaps[0][i][1:])['passed'], i
        return
    # FP32 bar, or no worse than the reference's own FP32 algorithm by both measures
    # (tests/fp32bar.py); the margins go to gpurun_out/parity_margins.jsonl.
    m = fp32bar.check(scores, refs[0], refs[1], f'large {precision} scores, {count} events')
    print(f'[large {precision}] {m}', flush=True)
    for i in snap_at:
        for name, a, o, o32 in zip(('keys', 'values', 'hidden'), states[i][1:], snaps[0][i][1:], snaps[1][i][1:]):
            m = fp32bar.check(a, o, o32, f'large {precision} {name} after event {i}')
            print(f'[large {precision}] {m}', flush=True)


@pytest.mark.parametrize('name,config,seed,steps', [('small', SMALL, 0, 512), ('main', MAIN, 1, 2048)])
def test_configured_stream_length_all_backends(name, config, seed, steps):
    c = config
    w = synthetic_checkpoint(c, seed=seed)
    events = _events(c, seed, steps)
    oracle = Oracle(c, w, accumulate='double', threads=THREADS)
    refs = np.array([oracle.step(e) for e in events], dtype=np.float64)
    ostate = oracle.snapshot()
    results = {}
    for backend in (Backend.CUDA, Backend.GRAPH, Backend.FUSED, Backend.PERSISTENT):
        kw = dict(idle_seconds=10.0) if backend == Backend.PERSISTENT else {}
        with _runtime((c, w, False), backend, **kw) as rt:
            scores = np.array([rt.step(e) for e in events], dtype=np.float32)
            results[backend] = (scores, rt.snapshot())
    base_scores, base_state = results[Backend.FUSED]
    bad = numerical.fp32_strict_failures(base_scores, refs, **STRICT)
    assert bad == 0, (bad, float(np.abs(base_scores - refs).max()))
    _assert_state_strict(base_state, ostate)
    for backend, (scores, state) in results.items():
        np.testing.assert_array_equal(scores, base_scores, err_msg=Backend(backend).name)
        assert state[0] == base_state[0] == steps
        for a, b in zip(state[1:], base_state[1:]):
            np.testing.assert_array_equal(a, b, err_msg=Backend(backend).name)


@pytest.mark.parametrize('mode', ['bf16w', 'mixed'])
@pytest.mark.parametrize('window', [32, 64, 256, 512])
def test_main_window_sweep_matches_oracle(mode, window):
    c = ModelConfig(MAIN.layers, MAIN.width, MAIN.heads, MAIN.ffn, window, MAIN.features)
    mixed = mode == 'mixed'
    w = synthetic_checkpoint(c, seed=2, mixed=mixed)
    events = _events(c, 2, 2048)
    if mixed:
        oracle = Oracle(c, w, mixed=True, threads=THREADS)
    else:
        oracle = Oracle(c, {k: round_bf16(v) for k, v in w.items()}, accumulate='double', threads=THREADS)
    storage = WeightStorage.AS_MODEL if mixed else WeightStorage.BF16
    scores, refs = [], []
    with _runtime((c, w, mixed), Backend.FUSED, weight_dtype=storage) as rt:
        for e in events:
            scores.append(rt.step(e))
            refs.append(oracle.step(e))
        state = rt.snapshot()
    ostate = oracle.snapshot()
    if mixed:
        assert numerical.score_errors(scores, refs, c.layers)['passed']
        assert state[0] == ostate[0]
        assert numerical.mixed_state_passes(*state[1:], *ostate[1:])['passed']
    else:
        bad = numerical.fp32_strict_failures(scores, refs, **STRICT)
        assert bad == 0, (bad, float(np.max(np.abs(np.array(scores) - np.array(refs)))))
        _assert_state_strict(state, ostate)


@pytest.mark.parametrize('streams', [64, 256])
def test_batched_main_sampled_streams_match_oracle(streams):
    c = MAIN
    w = synthetic_checkpoint(c, seed=4)
    rounded = {k: round_bf16(v) for k, v in w.items()}
    steps = c.window + 24
    sample = sorted({0, 1, streams // 2, streams - 1})
    events = np.stack([_events(c, 4 + b, steps) for b in range(streams)], axis=1)  # [steps, B, features]
    oracles = {b: Oracle(c, rounded, accumulate='double', threads=THREADS) for b in sample}
    print(f'[case] batch streams={streams} steps={steps} sample={sample}', flush=True)
    with BatchRuntime((c, w, False), streams, WeightStorage.BF16) as rt:
        for i in range(steps):
            got = rt.step(events[i])
            for b in sample:
                ref = oracles[b].step(events[i, b])
                assert numerical.fp32_strict_failures([got[b]], [ref], **STRICT) == 0, (i, b, got[b], ref)
        for b in sample:
            _assert_state_strict(rt.snapshot(b), oracles[b].snapshot())

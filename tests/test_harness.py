"""The benchmark driver (stream-bench) and the stored-oracle writer, without a GPU.

The driver keeps the reference's bench/Main.cpp contract. These tests cover:
  - its building blocks (harness_selftest: SHA-256 known answers, nearest-rank percentiles, the
    error thresholds, JSON and the parser's rejections), the FP16 decode of mixed checkpoints
    against numpy for all 65,536 bit patterns, the checkpoint and config checks with their
    error exit (1), and the stream-sparse-oracle-v1 archive that oracle/sparse_oracle.py writes
    (bench/Oracle.cpp:47-84);
  - the whole driver on the CPU, with the runtime ABI served by tests/cpu_runtime.cpp (the C
    oracle behind st_runtime.h, first on LD_LIBRARY_PATH): correctness against the reference's
    fixtures with their resets and against a stored oracle with --reset-every, a planted score
    error (exit 2), a stored oracle for other replay settings (exit 1), service, scheduled
    (including drops from a full queue), device and transport modes with the reference's
    result keys and CSV columns, and a max-events budget below warmup plus events (exit 1).
"""
import csv
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

from harness_layout import build_stand_in, gate, plant_score_error, reference_checkpoint, reference_fixture

ROOT = Path(__file__).resolve().parent.parent
BENCH = ROOT / 'streaming-transformer_amd' / 'lib' / 'stream-bench'
SELFTEST = ROOT / 'tests' / '_build' / 'harness_selftest'


def run(*args, env=None):
    return subprocess.run([str(BENCH), *map(str, args)], capture_output=True, text=True, timeout=120, env=env)


@pytest.fixture(scope='module')
def built():
    if not BENCH.exists() or not SELFTEST.exists():
        from streamtx import build
        build.build_consumers()
    return BENCH


def test_selftest_known_answers(built):
    out = subprocess.run([str(SELFTEST)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr


def test_fp16_decode_matches_numpy_for_every_bit_pattern(built):
    out = subprocess.run([str(SELFTEST), 'halves'], capture_output=True, text=True, timeout=60).stdout.split()
    got = np.array([int(x, 16) for x in out], dtype=np.uint32)
    want = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    assert got.shape == want.shape and np.array_equal(got, want)


def test_help_and_option_errors(built, tmp_path):
    out = run('--help')
    assert out.returncode == 0 and '--mode correctness' in out.stdout
    for bad in (['--bogus', '1'], ['--events'], ['--events', '1', '--events', '2'], ['--mode', 'nope'],
                ['--events', '0'], ['--backend', 'cpu', '--mode', 'correctness']):
        out = run(*bad, '--output', tmp_path / 'r')
        assert out.returncode == 1 and out.stderr.strip(), bad


@pytest.mark.parametrize('name', ['small-fp32', 'small-mixed'])
def test_checkpoint_hashes_and_config_checks(built, tmp_path, name):
    weights, config = reference_fixture(name, tmp_path / name)
    # A well-formed fixture passes every check before the runtime: the hash of the whole archive
    # and of each tensor (computed by the driver's own SHA-256) match the manifest, so the run
    # fails only where the runtime starts (no GPU here) or, on a GPU host, completes.
    out = run('--mode', 'correctness', '--backend', 'fused', '--weights', weights, '--config', config,
              '--events', '201', '--output', tmp_path / 'out' / 'r')
    assert out.returncode in (0, 1)
    if out.returncode == 1:
        assert 'hash' not in out.stderr and 'Shape' not in out.stderr and 'Configuration' not in out.stderr, out.stderr
    # A config that differs from the checkpoint's
    other = json.loads(config.read_text())
    other['window'] += 1
    bad_config = tmp_path / 'other.json'
    bad_config.write_text(json.dumps(other))
    out = run('--mode', 'service', '--weights', weights, '--config', bad_config, '--output', tmp_path / 'r')
    assert out.returncode == 1 and 'Configuration differs from checkpoint' in out.stderr
    # One flipped byte in the tensors
    raw = bytearray((weights / 'tensors.bin').read_bytes())
    raw[100] ^= 1
    (weights / 'tensors.bin').write_bytes(bytes(raw))
    out = run('--mode', 'service', '--weights', weights, '--config', config, '--output', tmp_path / 'r')
    assert out.returncode == 1 and 'Checkpoint hash mismatch' in out.stderr


def test_sparse_oracle_archive(tmp_path):
    from oracle.pyoracle import Oracle
    from oracle.sparse_oracle import write
    from streamtx import load_checkpoint
    weights, _ = reference_checkpoint('small-fp32', tmp_path / 'w')
    out = write(weights, tmp_path / 'oracle', events=150, reset_every=61, snapshot_every=32)
    manifest = json.loads((out / 'manifest.json').read_text())
    raw = (out / 'tensors.bin').read_bytes()
    ck = load_checkpoint(weights)
    assert manifest['format'] == 'stream-sparse-oracle-v1' and manifest['events'] == 150
    assert manifest['reset_every'] == 61 and manifest['snapshot_every'] == 32
    assert manifest['state_events'] == [0, 32, 64, 96, 128, 149]
    assert manifest['config'] == ck.manifest['config'] and manifest['mode'] == 'fp32'
    assert manifest['checkpoint_sha256'] == ck.manifest['sha256']
    assert manifest['trace_sha256'] == hashlib.sha256((weights / 'trace.bin').read_bytes()).hexdigest()
    assert manifest['sha256'] == hashlib.sha256(raw).hexdigest()
    t = {x['name']: np.frombuffer(raw[x['offset']:x['offset'] + x['nbytes']], dtype='<f4') for x in manifest['tensors']}
    c = ck.config
    cache = c.layers * c.width * c.window
    assert t['scores'].size == 150 and t['keys'].size == 6 * cache and t['hidden'].size == 6 * c.layers * c.width
    # The same events through the oracle directly, resets included
    trace = np.fromfile(weights / 'trace.bin', dtype='<f4').reshape(-1, c.features)
    oracle = Oracle(c, ck.tensors)
    for i in range(150):
        if i and i % 61 == 0:
            oracle.reset()
        assert oracle.step(trace[i % len(trace)]) == t['scores'][i]
        if i == 149:
            _, k, v, h = oracle.snapshot()
            assert np.array_equal(k.ravel(), t['keys'][-cache:]) and np.array_equal(h.ravel(), t['hidden'][-c.layers * c.width:])


# ---------------------------------------------------------------------------------------------
# the driver end to end on the CPU stand-in runtime

CPU_RUNTIME = ROOT / 'tests' / '_build' / 'cpu_runtime' / 'libstamd.so'


@pytest.fixture(scope='module')
def cpu_env(built):
    """Environment that loads tests/cpu_runtime.cpp (over the C oracle) as libstamd.so."""
    import os
    build_stand_in()
    env = dict(os.environ)
    env['LD_LIBRARY_PATH'] = f'{CPU_RUNTIME.parent}:' + env.get('LD_LIBRARY_PATH', '')
    return env


@pytest.fixture(scope='module')
def cpu_fixtures(tmp_path_factory):
    base = tmp_path_factory.mktemp('cpu_fixtures')
    out = {name: reference_fixture(name, base / name) for name in ('small-fp32', 'small-mixed')}
    out['main-fp32'] = reference_checkpoint('main-fp32', base / 'main-fp32')
    return out


@pytest.mark.parametrize('precision', ['fp32', 'mixed'])
def test_cpu_driver_fixture_correctness(cpu_env, cpu_fixtures, tmp_path, precision):
    weights, config = cpu_fixtures[f'small-{precision}']
    out = run('--mode', 'correctness', '--backend', 'fused', '--weights', weights, '--config', config,
              '--events', 201, '--output', tmp_path / 'r', env=cpu_env)
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'r.json').read_text())
    assert 'CPU stand-in' in result['environment']['gpu']
    gate(result, 'fused', precision, 201)
    # every event's score and full state (201 snapshots) with the reset before event 131
    c = json.loads(config.read_text())
    assert result['scores']['elements'] == 201 and result['hidden']['elements'] == 201 * c['layers'] * c['width']
    assert result['keys']['elements'] == 201 * c['layers'] * c['width'] * c['window']
    if precision == 'mixed':
        # per head row and per layer relative L2 entries: 201 events x (H*W rows, L layers) x 2
        rows = c['heads'] * c['window'] * c['layers']
        assert result['cache_head_relative_l2_diagnostic']['elements'] == 2 * 201 * rows
        assert result['cache_relative_l2_gate']['elements'] == 2 * 201 * c['layers']
        assert result['hidden_relative_l2_gate']['elements'] == 201 * c['layers']
    rows = list(csv.DictReader(open(tmp_path / 'r.csv')))
    assert len(rows) == 201 and list(rows[0]) == ['event', 'intended_ns', 'enqueue_ns', 'submit_ns', 'complete_ns',
                                                  'score', 'dropped']
    np.testing.assert_allclose([float(r['score']) for r in rows],
                               np.load(ROOT / 'tests' / 'golden' / f'small-{precision}' / 'expected.npz')['scores'],
                               rtol=2e-2 if precision == 'mixed' else 1e-4, atol=2e-3 if precision == 'mixed' else 1e-5)


def test_cpu_driver_without_the_fixture_resets_fails(cpu_env, cpu_fixtures, tmp_path):
    """resets.json is part of the fixture: without the reset before event 131 the stand-in
    keeps its state, which then differs from the expected archive (exit 2, the failures start
    at event 131)."""
    weights, config = cpu_fixtures['small-fp32']
    (weights / 'resets.json').rename(weights / 'resets.json.off')
    try:
        out = run('--mode', 'correctness', '--backend', 'cuda', '--weights', weights, '--config', config,
                  '--events', 201, '--output', tmp_path / 'r', env=cpu_env)
    finally:
        (weights / 'resets.json.off').rename(weights / 'resets.json')
    assert out.returncode == 2, out.stderr[-2000:]
    result = json.loads((tmp_path / 'r.json').read_text())
    assert result['scores']['failed'] > 0 and result['scores']['examples'][0]['index'] >= 131


def test_cpu_driver_stored_oracle_planted_error_and_other_replay(cpu_env, cpu_fixtures, tmp_path):
    from oracle.sparse_oracle import write
    weights, config = cpu_fixtures['main-fp32']
    oracle = write(weights, tmp_path / 'oracle', events=130, reset_every=47, snapshot_every=40)
    args = ('--mode', 'correctness', '--backend', 'persistent', '--weights', weights, '--config', config,
            '--events', 130, '--reset-every', 47, '--expected', oracle)
    out = run(*args, '--output', tmp_path / 'ok', env=cpu_env)
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'ok.json').read_text())
    gate(result, 'persistent', 'fp32', 130)
    c = json.loads(config.read_text())
    assert result['keys']['elements'] == 5 * c['layers'] * c['width'] * c['window']  # events 0, 40, 80, 120, 129
    assert result['scores']['max_abs'] == 0  # the stand-in is the stored oracle's own arithmetic
    plant_score_error(oracle, 77, 0.05)
    out = run(*args, '--output', tmp_path / 'planted', env=cpu_env)
    assert out.returncode == 2, out.stderr[-2000:]
    planted = json.loads((tmp_path / 'planted.json').read_text())
    assert planted['scores']['failed'] == 1 and planted['scores']['examples'][0]['index'] == 77
    out = run(*args[:-4], '--reset-every', 48, '--expected', oracle, '--output', tmp_path / 'other', env=cpu_env)
    assert out.returncode == 1 and 'differs from requested' in out.stderr


def test_cpu_driver_service_scheduled_device_transport(cpu_env, cpu_fixtures, tmp_path):
    weights, config = cpu_fixtures['small-fp32']
    common = ('--weights', weights, '--config', config)
    out = run('--mode', 'service', '--backend', 'graph', *common, '--events', 150, '--warmup', 7,
              '--output', tmp_path / 'service', env=cpu_env)
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'service.json').read_text())
    assert result['completed'] == 150 and result['warmup'] == 7 and result['dropped'] == 0
    for key in ('service', 'arrival', 'queueing', 'injection'):
        assert set(result[key]) == {'p50_us', 'p95_us', 'p99_us', 'p999_us_diagnostic', 'worst_us'}
    assert result['scores']['elements'] == 0 and result['expected_source'] == 'fixture'
    # Scheduled at a modest rate: nothing dropped, every event stepped once, in order of arrival.
    out = run('--mode', 'scheduled', '--backend', 'fused', *common, '--events', 300, '--warmup', 0,
              '--rate', 5000, '--queue', 64, '--output', tmp_path / 'sched', env=cpu_env)
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'sched.json').read_text())
    assert result['completed'] + result['dropped'] == 300 and result['queue_capacity'] == 64
    offsets = np.arange(300, dtype=np.float64) * 1e9 / 5000
    assert result['schedule_sha256'] == hashlib.sha256(offsets.tobytes()).hexdigest()
    rows = list(csv.DictReader(open(tmp_path / 'sched.csv')))
    done = [r for r in rows if r['dropped'] == '0']
    assert all(float(r['submit_ns']) >= float(r['enqueue_ns']) >= float(r['intended_ns']) for r in done)
    submits = [float(r['submit_ns']) for r in done]
    assert submits == sorted(submits)
    # Bursts of 16 into a queue of 4 at a rate the stand-in cannot keep: events are dropped,
    # and every one is either stepped or dropped.
    out = run('--mode', 'scheduled', '--backend', 'fused', *common, '--events', 320, '--warmup', 0,
              '--rate', 200000, '--bursty', 1, '--queue', 4, '--output', tmp_path / 'drops', env=cpu_env)
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'drops.json').read_text())
    assert result['dropped'] > 0 and result['completed'] + result['dropped'] == 320 and result['bursty'] is True
    rows = list(csv.DictReader(open(tmp_path / 'drops.csv')))
    assert sum(r['dropped'] == '1' for r in rows) == result['dropped']
    out = run('--mode', 'device', '--backend', 'fused', *common, '--events', 20, '--output', tmp_path / 'device',
              env=cpu_env)
    assert out.returncode == 0 and json.loads((tmp_path / 'device.json').read_text())['events'] == 20
    out = run('--mode', 'gpu-ping', '--events', 5, '--output', tmp_path / 'nested' / 'dir' / 'pp', env=cpu_env)
    assert out.returncode == 0 and json.loads((tmp_path / 'nested' / 'dir' / 'pp.json').read_text())['mode'] == 'gpu-ping'
    # A max-events budget that does not cover warmup plus the run is refused (exit 1); one that
    # does is accepted.
    out = run('--mode', 'service', *common, '--events', 50, '--warmup', 10, '--max-events', 59,
              '--output', tmp_path / 'budget', env=cpu_env)
    assert out.returncode == 1 and 'max-events must cover' in out.stderr
    out = run('--mode', 'service', *common, '--events', 50, '--warmup', 10, '--max-events', 60,
              '--output', tmp_path / 'budget', env=cpu_env)
    assert out.returncode == 0, out.stderr[-2000:]


def test_cpu_driver_rejects_malformed_numbers(cpu_env, cpu_fixtures, tmp_path):
    weights, config = cpu_fixtures['small-fp32']
    for bad in (['--events', '12x'], ['--rate', '1e3q', '--mode', 'scheduled'], ['--warmup', '-1'], ['--queue', '0', '--mode', 'scheduled'],
                ['--expected', 'cpu', '--mode', 'correctness']):
        out = run('--weights', weights, '--config', config, *bad, '--output', tmp_path / 'r', env=cpu_env)
        assert out.returncode == 1 and out.stderr.strip(), (bad, out.stderr)

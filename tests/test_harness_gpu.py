"""The benchmark driver (stream-bench) and a C++ consumer of the C ABI on the GPU.

- correctness mode on the reference's small fixtures (201 events: first event, partial and
  full window, eviction, several ring revolutions, a warm reset) for every backend, with the
  checks of the reference's correctness gate (bench/gates.py:104-161) on the result file;
- correctness against a stored oracle (stream-sparse-oracle-v1 written from the C oracle)
  with --reset-every, on Main, and the same oracle with one planted score error, which must
  exit 2;
- service, scheduled, device and transport modes: exit 0 and the reference's result keys and
  CSV columns;
- tests/abi_consumer.cpp: the reference's lifecycle checks (tests/Lifecycle.cu) through the
  ABI as a Stream::Runtime shim binds it.
"""
import csv
import hashlib
import json
import subprocess
from pathlib import Path

import pytest

from harness_layout import gate, plant_score_error, reference_checkpoint, reference_fixture

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
BENCH = ROOT / 'streaming-transformer_amd' / 'lib' / 'stream-bench'
CONSUMER = ROOT / 'tests' / '_build' / 'abi_consumer'


def bench(*args, timeout=240):
    print('stream-bench', *map(str, args), flush=True)
    return subprocess.run([str(BENCH), *map(str, args)], capture_output=True, text=True, timeout=timeout)


@pytest.fixture(scope='module')
def fixtures(tmp_path_factory):
    base = tmp_path_factory.mktemp('fixtures')
    out = {name: reference_fixture(name, base / name) for name in ('small-fp32', 'small-mixed')}
    for name in ('main-fp32', 'main-mixed'):
        out[name] = reference_checkpoint(name, base / name)
    return out


VARIANTS = [('cuda', 1), ('cuda', 4), ('graph', 1), ('graph', 4), ('fused', 1), ('fused', 0),
            ('persistent', 1), ('persistent', 4), ('cublas', 4), ('cublas-graph', 4)]


@pytest.mark.parametrize('precision', ['fp32', 'mixed'])
@pytest.mark.parametrize('backend,blocks', VARIANTS)
def test_fixture_correctness(fixtures, tmp_path, backend, blocks, precision):
    weights, config = fixtures[f'small-{precision}']
    out = bench('--mode', 'correctness', '--backend', backend, '--blocks', blocks, '--weights', weights,
                '--config', config, '--events', 201, '--output', tmp_path / 'r')
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'r.json').read_text())
    gate(result, backend, precision, 201)
    assert result['expected_source'] == 'fixture'
    # The reset schedule of resets.json was applied: 201 events, reset before event 131.
    assert result['scores']['elements'] == 201 and result['hidden']['elements'] == 201 * 64


@pytest.mark.parametrize('precision', ['fp32', 'mixed'])
def test_stored_oracle_correctness_and_planted_error(fixtures, tmp_path, precision):
    from oracle.sparse_oracle import write
    weights, config = fixtures[f'main-{precision}']
    oracle = write(weights, tmp_path / 'oracle', events=300, reset_every=97, snapshot_every=64)
    for backend, blocks in (('fused', 0), ('persistent', 4)):
        out = bench('--mode', 'correctness', '--backend', backend, '--blocks', blocks, '--weights', weights,
                    '--config', config, '--events', 300, '--reset-every', 97, '--expected', oracle,
                    '--output', tmp_path / backend)
        assert out.returncode == 0, out.stderr[-2000:]
        result = json.loads((tmp_path / f'{backend}.json').read_text())
        gate(result, backend, precision, 300)
        assert result['expected_manifest_sha256'] == hashlib.sha256((oracle / 'manifest.json').read_bytes()).hexdigest()
        c = json.loads(config.read_text())
        assert result['keys']['elements'] == 6 * c['layers'] * c['width'] * c['window']  # the 6 stored events
    # The planted mistake goes into the oracle, on the CPU: one score off by 0.05.
    plant_score_error(oracle, 123, 0.05)
    out = bench('--mode', 'correctness', '--backend', 'fused', '--blocks', 0, '--weights', weights, '--config',
                config, '--events', 300, '--reset-every', 97, '--expected', oracle, '--output', tmp_path / 'planted')
    assert out.returncode == 2, out.stderr[-2000:]
    result = json.loads((tmp_path / 'planted.json').read_text())
    assert result['scores']['failed'] == 1 and result['scores']['examples'][0]['index'] == 123
    # A stored oracle for other replay settings is refused (exit 1)
    out = bench('--mode', 'correctness', '--backend', 'fused', '--weights', weights, '--config', config,
                '--events', 300, '--reset-every', 100, '--expected', oracle, '--output', tmp_path / 'other')
    assert out.returncode == 1 and 'differs from requested' in out.stderr


def test_service_scheduled_device_and_transport_modes(fixtures, tmp_path):
    weights, config = fixtures['main-fp32']
    out = bench('--mode', 'service', '--backend', 'graph', '--blocks', 4, '--weights', weights, '--config', config,
                '--events', 300, '--warmup', 20, '--output', tmp_path / 'service')
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'service.json').read_text())
    assert result['completed'] == 300 and result['warmup'] == 20 and result['service']['p50_us'] > 0
    for key in ('p50_us', 'p95_us', 'p99_us', 'p999_us_diagnostic', 'worst_us'):
        assert key in result['service'] and key in result['arrival']
    rows = list(csv.DictReader(open(tmp_path / 'service.csv')))
    assert len(rows) == 300 and list(rows[0]) == ['event', 'intended_ns', 'enqueue_ns', 'submit_ns', 'complete_ns',
                                                  'score', 'dropped']
    out = bench('--mode', 'scheduled', '--backend', 'fused', '--blocks', 0, '--weights', weights, '--config', config,
                '--events', 400, '--warmup', 10, '--rate', 2000, '--queue', 64, '--output', tmp_path / 'sched')
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'sched.json').read_text())
    assert result['completed'] + result['dropped'] == 400 and result['rate_per_second'] == 2000
    assert result['queue_capacity'] == 64 and len(result['schedule_sha256']) == 64
    out = bench('--mode', 'device', '--backend', 'fused', '--blocks', 0, '--weights', weights, '--config', config,
                '--events', 64, '--output', tmp_path / 'device')
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads((tmp_path / 'device.json').read_text())
    assert result['device_us_per_event'] > 0 and result['events'] == 64
    out = bench('--mode', 'ping-pong', '--events', 200, '--output', tmp_path / 'pp')
    assert out.returncode == 0, out.stderr[-2000:]
    assert json.loads((tmp_path / 'pp.json').read_text())
    assert (tmp_path / 'pp.csv').read_text().startswith('sequence,host_observation_us,device_round_trip_or_wait_cycles')


def test_abi_consumer_lifecycle(fixtures):
    args = [str(CONSUMER), str(fixtures['small-fp32'][0]), str(fixtures['small-mixed'][0]),
            str(fixtures['main-mixed'][0])]
    print(*args, flush=True)
    out = subprocess.run(args, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, out.stdout[-3000:] + out.stderr[-2000:]
    assert out.stdout.count('PASS') == 5

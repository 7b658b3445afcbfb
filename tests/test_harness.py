"""The benchmark driver (stream-bench) and the stored-oracle writer, without a GPU.

The driver keeps the reference's bench/Main.cpp contract; these tests cover what runs before
a runtime exists: its building blocks (harness_selftest: SHA-256 known answers, nearest-rank
percentiles, the error thresholds, JSON), the FP16 decode of mixed checkpoints against numpy
for all 65,536 bit patterns, the checkpoint and config checks with their error exit (1), and
the stream-sparse-oracle-v1 archive that oracle/sparse_oracle.py writes (bench/Oracle.cpp:47-84).
"""
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

from harness_layout import reference_checkpoint, reference_fixture

ROOT = Path(__file__).resolve().parent.parent
BENCH = ROOT / 'streaming-transformer_amd' / 'lib' / 'stream-bench'
SELFTEST = ROOT / 'tests' / '_build' / 'harness_selftest'


def run(*args):
    return subprocess.run([str(BENCH), *map(str, args)], capture_output=True, text=True, timeout=120)


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

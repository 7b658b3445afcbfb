"""The reference's validation matrix on the GPU, through the benchmark driver (stream-bench)
against stored oracles (stream-sparse-oracle-v1 from the C oracle).

  - adversarial input families (scripts/extended_validation.py:26-84): zeros, constant,
    impulses, alternating and repeated events (reference/export.py:12-28) on the reference's
    small, main and large checkpoints, FP32 and mixed, 3W+9 events with a reset before event
    2W+3, through the staged (cuda), vendor GEMV (cublas) and persistent backends;
  - the window variants (scripts/check_windows.py:14-30): all 30 checkpoints
    {small,main,large}-w{32,64,128,256,512}-{fp32,mixed} with their own 3W+9-event traces and
    resets, through the staged, captured vendor GEMV (cublas-graph) and persistent backends.
    large-w512 is the large checkpoint itself (same weights, config and trace).
Every score is compared, and the full K/V and hidden state at the stored snapshots (every
event on small; on main and large every min(8 or 64, W/8) events, and the last one), under the driver's
gate: FP32 1e-5 + 1e-4|r|, mixed the reference's policy v3 (bench/Main.cpp:354-409).
"""
import json
import shutil
import subprocess
from pathlib import Path

import pytest

from harness_layout import GOLDEN, adversarial_trace, gate, reference_checkpoint, window_fixture
from oracle.sparse_oracle import write as stored_oracle

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
BENCH = ROOT / 'streaming-transformer_amd' / 'lib' / 'stream-bench'
SNAPSHOT_EVERY = {'small': 1, 'main': 8, 'large': 64}


def snapshot_every(size, window):
    """Stored snapshot spacing: every event on small, else at most every W/8 events."""
    return min(SNAPSHOT_EVERY[size], max(1, window // 8))
KINDS = ('zeros', 'constant', 'impulses', 'alternating', 'repeated')


def run_gate(weights, config, trace, events, reset, oracle, backend, blocks, precision, out):
    args = ['--mode', 'correctness', '--backend', backend, '--blocks', str(blocks), '--weights', str(weights),
            '--config', str(config), '--trace', str(trace), '--events', str(events), '--reset-every', str(reset),
            '--expected', str(oracle), '--output', str(out)]
    print('stream-bench', *args, flush=True)
    r = subprocess.run([str(BENCH), *args], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (backend, blocks, r.stderr[-2000:])
    result = json.loads(Path(str(out) + '.json').read_text())
    gate(result, backend, precision, events)
    return result


@pytest.mark.parametrize('mode', ['fp32', 'mixed'])
@pytest.mark.parametrize('size', ['small', 'main', 'large'])
def test_adversarial_families(tmp_path, size, mode):
    weights, config = reference_checkpoint(f'{size}-{mode}', tmp_path / 'ckpt')
    c = json.loads(config.read_text())
    w, f = c['window'], c['features']
    events, reset = 3 * w + 9, 2 * w + 3
    backends = [('cuda', 4), ('cublas', 4), ('persistent', 4)] + ([('persistent', 1)] if size == 'small' else [])
    for kind in KINDS:
        trace = tmp_path / f'{kind}.bin'
        adversarial_trace(events, f, kind).tofile(trace)
        oracle = stored_oracle(weights, tmp_path / f'{kind}-oracle', trace=trace, events=events, reset_every=reset,
                               snapshot_every=snapshot_every(size, w))
        for backend, blocks in backends:
            result = run_gate(weights, config, trace, events, reset, oracle, backend, blocks, mode,
                              tmp_path / f'{kind}-{backend}-{blocks}')
            if kind == 'zeros':
                # zero input: every score is exactly 0 (tests/Lifecycle.cu:38,60-62)
                assert result['scores']['max_abs'] == 0.0, (backend, blocks)
        shutil.rmtree(oracle)


@pytest.mark.parametrize('mode', ['fp32', 'mixed'])
@pytest.mark.parametrize('size', ['small', 'main', 'large'])
def test_window_variant_checkpoints(tmp_path, size, mode):
    for window in (32, 64, 128, 256, 512):
        name = f'{size}-w{window}-{mode}'
        weights, config = window_fixture(name, tmp_path / name)
        resets = json.loads((weights / 'resets.json').read_text())
        assert resets == [2 * window + 3]
        events = 3 * window + 9
        oracle = stored_oracle(weights, tmp_path / f'{name}-oracle', events=events, reset_every=resets[0],
                               snapshot_every=snapshot_every(size, window))
        for backend, blocks in (('cuda', 4), ('cublas-graph', 4), ('persistent', 4)):
            run_gate(weights, config, weights / 'trace.bin', events, resets[0], oracle, backend, blocks, mode,
                     tmp_path / f'{name}-{backend}')
        shutil.rmtree(tmp_path / f'{name}-oracle')

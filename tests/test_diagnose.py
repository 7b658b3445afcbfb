"""Per-operation diagnosis without a GPU (the reference's stream-diagnose / CpuTrace pair,
bench/Diagnose.cpp:12-68, src/cpu/Cpu.cpp:29-57).

  - the oracle's trace mode leaves exactly the state of an ordinary step (the reference's
    trace-equals-execution regression, tests/Lifecycle.cu:108-137), and reports the
    reference's entries in execution order with the right sizes;
  - every traced operation meets its closed form on its own operands: FP32 dot bound for the
    projections, exact casts, RMSNorm, SwiGLU and the residual adds (streamtx.diagnose);
  - stream-diagnose run over the CPU stand-in runtime (tests/cpu_runtime.cpp, the oracle behind
    the ABI) writes the same archive, byte for byte, as oracle/stage_archive.py;
  - a difference planted in one archive, on the CPU, is located at its event, stage and
    coordinate as the first divergence; archives of different fixtures are refused.
"""
import hashlib
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from harness_layout import reference_checkpoint
from oracle.pyoracle import Oracle
from oracle.stage_archive import write as oracle_archive
from streamtx import load_checkpoint
from streamtx.diagnose import compare, execution_order, isolated_checks, read_archive

ROOT = Path(__file__).resolve().parent.parent
DIAGNOSE = ROOT / 'streaming-transformer_amd' / 'lib' / 'stream-diagnose'
GOLDEN = ROOT / 'tests' / 'golden'


def fixture(name, target):
    """tests/golden/<name> as a reference fixture directory: checkpoint, trace.bin, resets.json."""
    weights, _ = reference_checkpoint(name, target / name)
    shutil.copyfile(GOLDEN / name / 'resets.json', weights / 'resets.json')
    return weights


@pytest.mark.parametrize('name', ['small-fp32', 'small-mixed'])
def test_oracle_trace_preserves_execution(name):
    ck = load_checkpoint(GOLDEN / name / 'checkpoint')
    c = ck.config
    events = np.fromfile(GOLDEN / name / 'trace.bin', dtype='<f4').reshape(-1, c.features)
    traced, plain = Oracle(c, ck.tensors, mixed=ck.mixed), Oracle(c, ck.tensors, mixed=ck.mixed)
    order = execution_order(c.layers)
    for i, e in enumerate(events):
        if i == 131:
            traced.reset()
            plain.reset()
        score, t = traced.trace_step(e)
        assert score == plain.step(e)
        assert list(t) == order  # the reference's names, in execution order
        assert score == t['score.linear'][0] == t['score.pre_cast'][0]
    for a, b in zip(traced.snapshot()[1:], plain.snapshot()[1:]):
        assert np.array_equal(a, b)
    d, F, f = c.width, c.ffn, c.features
    sizes = {k: v.size for k, v in t.items()}
    assert sizes['input.operand'] == f and sizes['layers.0.gate.linear'] == F and sizes['layers.0.down.operand'] == F
    assert sum(sizes.values()) == f + 7 * d + 2 + c.layers * (28 * d + 6 * F)


@pytest.mark.parametrize('name', ['small-fp32', 'small-mixed', 'main-mixed'])
def test_oracle_operations_meet_their_closed_forms(tmp_path, name):
    weights = fixture(name, tmp_path)
    out = oracle_archive(weights, tmp_path / 'oracle')
    _, stages = read_archive(out)
    ck = load_checkpoint(weights)
    checks = isolated_checks(stages, ck.tensors, ck.config, ck.mixed)
    assert len(checks['linear']) == 2 + 7 * ck.config.layers
    for n, r in checks['linear'].items():
        assert r['fp32_dot_bound_violations'] == 0 and r['cast_mismatches'] == 0, (n, r)
        assert r['max_fraction_of_dot_bound'] < 0.5, (n, r)
    for n, r in checks['nonlinear'].items():
        assert r['failed'] == 0 and r['nonfinite'] == 0, (n, r)


@pytest.fixture(scope='module')
def cpu_env():
    """The CPU stand-in runtime as libstamd.so (built by test_harness's fixture when run there)."""
    import os
    from harness_layout import build_stand_in
    lib = build_stand_in()
    if not DIAGNOSE.exists():
        from streamtx import build
        build.build_consumers()
    env = dict(os.environ)
    env['LD_LIBRARY_PATH'] = f'{lib.parent}:' + env.get('LD_LIBRARY_PATH', '')
    return env


@pytest.mark.parametrize('name', ['small-fp32', 'main-mixed'])
def test_stream_diagnose_archive_equals_oracle_archive(cpu_env, tmp_path, name):
    weights = fixture(name, tmp_path)
    out = subprocess.run([str(DIAGNOSE), str(weights), str(tmp_path / 'native')], capture_output=True, text=True,
                         env=cpu_env, timeout=300)
    assert out.returncode == 0, out.stderr
    oracle_archive(weights, tmp_path / 'oracle')
    native = json.loads((tmp_path / 'native' / 'manifest.json').read_text())
    ref = json.loads((tmp_path / 'oracle' / 'manifest.json').read_text())
    for key in ('version', 'dtype', 'layout', 'events', 'event_elements', 'stages', 'checkpoint_sha256',
                'trace_sha256', 'resets', 'sha256'):
        assert native[key] == ref[key], key
    assert native['backend'] == 'cuda' and native['events'] == (201 if name == 'small-fp32' else 777)
    assert (tmp_path / 'native' / 'stages.bin').read_bytes() == (tmp_path / 'oracle' / 'stages.bin').read_bytes()
    report = compare(tmp_path / 'native', tmp_path / 'oracle', weights)
    assert report['first_divergence'] is None and report['stages_over_bar'] == []


def test_planted_difference_is_located(tmp_path):
    weights = fixture('small-fp32', tmp_path)
    a = oracle_archive(weights, tmp_path / 'a')
    b = tmp_path / 'b'
    shutil.copytree(a, b)
    manifest = json.loads((b / 'manifest.json').read_text())
    stage = next(s for s in manifest['stages'] if s['name'] == 'layers.0.gate.pre_cast')
    raw = bytearray((b / 'stages.bin').read_bytes())
    at = 4 * (150 * manifest['event_elements'] + stage['offset_elements'] + 5)
    v = np.frombuffer(bytes(raw[at:at + 4]), dtype='<f4')[0]
    raw[at:at + 4] = np.float32(v + 0.5).tobytes()
    (b / 'stages.bin').write_bytes(bytes(raw))
    manifest['sha256'] = hashlib.sha256(bytes(raw)).hexdigest()
    (b / 'manifest.json').write_text(json.dumps(manifest))
    report = compare(b, a, weights)
    assert report['first_divergence']['event'] == 150
    assert report['first_divergence']['stage'] == 'layers.0.gate.pre_cast'
    assert report['first_divergence']['coordinate'] == 5
    assert report['stages_over_bar'] == ['layers.0.gate.pre_cast']
    # the isolated check of that projection sees its pre-cast value off its own operands
    assert report['isolated']['linear']['layers.0.gate']['fp32_dot_bound_violations'] == 1
    # an archive of another fixture is refused
    other = fixture('small-mixed', tmp_path / 'm')
    with pytest.raises(ValueError):
        compare(oracle_archive(other, tmp_path / 'c'), a, weights)


def test_stream_diagnose_usage_errors(cpu_env, tmp_path):
    weights = fixture('small-fp32', tmp_path)
    for args in ([], [str(weights)], [str(weights), str(tmp_path / 'o'), 'cpu'], [str(weights), str(tmp_path / 'o'), 'x']):
        out = subprocess.run([str(DIAGNOSE), *args], capture_output=True, text=True, env=cpu_env, timeout=60)
        assert out.returncode == 1 and out.stderr.strip(), args

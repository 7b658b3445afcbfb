"""Per-operation diagnosis on the GPU: stream-diagnose (the staged backend through
st_runtime_trace_step) against the oracle's archive of the same fixture, every event of the
reference's small and main fixtures with their resets (bench/Diagnose.cpp:12-68,
scripts/diagnose_native.py:31-140).

Bars, stage by stage over all events: FP32 |a - e| <= 1e-5 + 1e-4 |e| (the reference's
diagnostic bar); mixed: the policy-v3 bar (absolute term 2e-3 * (layer + 1) * max(1, RMS of
the expected vector), relative 2e-2). On the GPU archive's own operands: every projection
within the FP32 dot bound gamma(2n) * sum|x w| with exact casts, every norm, SwiGLU and residual
add at its exact value. The first divergence from the oracle is printed: where the two runs
first part, at one cast boundary.
"""
import json
import shutil
import subprocess
from pathlib import Path

import pytest

from harness_layout import reference_checkpoint
from oracle.stage_archive import write as oracle_archive
from streamtx.diagnose import compare

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
DIAGNOSE = ROOT / 'streaming-transformer_amd' / 'lib' / 'stream-diagnose'
GOLDEN = ROOT / 'tests' / 'golden'


@pytest.mark.parametrize('name', ['small-fp32', 'small-mixed', 'main-fp32', 'main-mixed'])
def test_gpu_operations_match_oracle(tmp_path, name):
    weights, _ = reference_checkpoint(name, tmp_path / name)
    shutil.copyfile(GOLDEN / name / 'resets.json', weights / 'resets.json')
    print(f'[case] stream-diagnose {name}', flush=True)
    out = subprocess.run([str(DIAGNOSE), str(weights), str(tmp_path / 'gpu'), 'cuda'], capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    oracle_archive(weights, tmp_path / 'oracle')
    report = compare(tmp_path / 'gpu', tmp_path / 'oracle', weights)
    (tmp_path / 'report.json').write_text(json.dumps(report, indent=2))
    mixed = report['mode'] == 'mixed'
    worst = max(report['stages'].items(), key=lambda kv: kv[1]['max_abs'])
    print(f'[{name}] events={report["events"]} stages={len(report["stages"])} first divergence: '
          f'{report["first_divergence"]}; largest stage difference {worst[0]} {worst[1]["max_abs"]:.3g}', flush=True)
    assert report['stages_over_bar'] == [], {n: report['stages'][n]['examples'][:2] for n in report['stages_over_bar']}
    for n, r in report['isolated']['linear'].items():
        assert r['fp32_dot_bound_violations'] == 0 and r['cast_mismatches'] == 0, (n, r)
    for n, r in report['isolated']['nonlinear'].items():
        assert r['failed'] == 0 and r['nonfinite'] == 0, (n, r)
    if not mixed:
        for s in report['stages'].values():
            assert s['failed'] == 0

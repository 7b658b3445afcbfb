"""The PyTorch-ROCm comparison (the reference's bench/torch_bench.py counterpart) on the GPU.

bench.py --torch-baseline writes the same step with PyTorch operators in FP32, eager and
captured in a hipGraph, in a child process (torch brings its own HIP runtime). The test runs
it on the Small shape and checks that every graph replay equals its eager step exactly and that
torch's scores agree with the HIP runtime's on the same events within the reference's FP32
score gate (1e-5 + 1e-4 |score|, bench/Main.cpp:66).
"""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize('config', ['small', 'main'])
def test_torch_comparison_agrees_with_the_runtime(config):
    cmd = [sys.executable, str(ROOT / 'bench.py'), '--torch-baseline', '--config', config, '--warmup', '4']
    print(*cmd, flush=True)
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, out.stderr[-2000:]
    result = json.loads([ln for ln in out.stdout.splitlines() if ln.startswith('{')][-1])
    assert result['graph_replay_vs_eager_max_abs'] == 0.0
    assert result['score_max_abs_diff_vs_runtime'] <= 1e-5 + 1e-4 * 1.0, result
    assert result['eager_p50_us'] > 0 and result['graph_p50_us'] > 0
    assert result['torch'].startswith('2.')

"""The batched projections' operand layouts (act_index, half_index in batch_kernels.hpp), checked
on the CPU by tests/layout_selftest.hip, built with hipcc from the library's header: bijective,
16-row x KB-column blocks as contiguous runs in MFMA lane order, runs of four columns."""
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
BUILD = HERE / '_build'


def _hipcc():
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and Path(cand).exists():
            return cand
    return None


def test_operand_layouts():
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip('hipcc not found')
    BUILD.mkdir(parents=True, exist_ok=True)
    fd, exe = tempfile.mkstemp(prefix='layout_selftest.', dir=BUILD)
    os.close(fd)
    try:
        subprocess.run([hipcc, '-O2', '-std=c++17', '--offload-arch=gfx950', '-o', exe, str(HERE / 'layout_selftest.hip')],
                       check=True, capture_output=True, text=True)
        run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    finally:
        os.unlink(exe)
    assert run.returncode == 0, run.stdout[-3000:]
    assert run.stdout.strip().endswith('OK: 0 failure(s)'), run.stdout[-3000:]

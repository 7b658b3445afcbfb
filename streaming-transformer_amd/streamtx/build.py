"""Build libstamd.so for gfx950 with hipcc (in-tree, so the library travels with the repo)."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent.parent
SOURCES = [PACKAGE_DIR / 'csrc' / 'runtime.hip']
DEPENDS = SOURCES + list((PACKAGE_DIR / 'csrc').glob('*.hpp')) + [PACKAGE_DIR.parent / 'include' / 'st_runtime.h']
OUTPUT = PACKAGE_DIR / 'lib' / 'libstamd.so'

HIPCC_FLAGS = [
    '-O3', '--offload-arch=gfx950', '-std=c++17', '-fPIC', '-shared', '-fno-strict-aliasing',
    # keep packed-FP32 VALU instructions out of the generated code
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    # rocBLAS for the vendor GEMV backends
    '-L/opt/rocm/lib', '-lrocblas', '-Wl,-rpath,/opt/rocm/lib',
]


def hipcc() -> str:
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError('hipcc not found')


def build(force: bool = True, verbose: bool = False) -> Path:
    """Compile libstamd.so. With force=False, skip when the library is newer than its sources."""
    if not force and OUTPUT.exists():
        newest = max(p.stat().st_mtime for p in DEPENDS)
        if OUTPUT.stat().st_mtime >= newest:
            return OUTPUT
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUTPUT.with_suffix('.so.tmp')
    cmd = [hipcc(), *HIPCC_FLAGS, '-o', str(tmp), *map(str, SOURCES)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed ({proc.returncode}):\n{proc.stderr[-4000:]}')
    if verbose:
        sys.stderr.write(proc.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == '__main__':
    print(build(verbose=True))

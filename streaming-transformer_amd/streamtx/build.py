"""Build libstamd.so for gfx950 with hipcc (in-tree, so the library travels with the repo)."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent.parent
SOURCES = [PACKAGE_DIR / 'csrc' / 'runtime.hip', PACKAGE_DIR / 'csrc' / 'batch.hip']
DEPENDS = SOURCES + list((PACKAGE_DIR / 'csrc').glob('*.hpp')) + [PACKAGE_DIR.parent / 'include' / 'st_runtime.h']
OUTPUT = PACKAGE_DIR / 'lib' / 'libstamd.so'

COMPILE_FLAGS = [
    '-O3', '--offload-arch=gfx950', '-std=c++17', '-fPIC', '-fno-strict-aliasing',
    # keep packed-FP32 VALU instructions out of the generated code
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
]
# Per translation unit: the batched phase kernels take their arguments preloaded into SGPRs
# (their first loads then wait for no argument load); the fused single-stream kernel is faster
# without, so runtime.hip keeps the default.
UNIT_FLAGS = {'batch.hip': ['-mllvm', '-amdgpu-kernarg-preload-count=16']}
LINK_FLAGS = [
    '--offload-arch=gfx950', '-fPIC', '-shared',
    # rocBLAS for the vendor GEMV backends
    '-L/opt/rocm/lib', '-lrocblas', '-Wl,-rpath,/opt/rocm/lib',
]


def hipcc() -> str:
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError('hipcc not found')


HARNESS_DIR = PACKAGE_DIR / 'harness'
HARNESS = OUTPUT.parent / 'stream-bench'
DIAGNOSE = OUTPUT.parent / 'stream-diagnose'
TESTS_DIR = PACKAGE_DIR.parent / 'tests'
ABI_CONSUMER = TESTS_DIR / '_build' / 'abi_consumer'
HARNESS_SELFTEST = TESTS_DIR / '_build' / 'harness_selftest'


def _cxx(source: Path, output: Path, rpath: str) -> None:
    """A host-only C++ consumer of the C ABI, linked against libstamd.so."""
    output.parent.mkdir(parents=True, exist_ok=True)
    cmd = [os.environ.get('CXX', 'g++'), '-O2', '-std=c++17', '-Wall', '-Wextra',
           f'-I{PACKAGE_DIR.parent / "include"}', f'-I{HARNESS_DIR}', '-o', str(output), str(source),
           f'-L{OUTPUT.parent}', '-lstamd', f'-Wl,-rpath,{rpath}', '-pthread']
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'{cmd[0]} failed ({proc.returncode}):\n{proc.stderr[-4000:]}')


def build_consumers() -> tuple[Path, Path, Path]:
    """The benchmark driver (stream-bench) and the per-operation diagnostic (stream-diagnose),
    next to the library, and two test programs under tests/_build (test infrastructure): the
    C++ ABI consumer and the driver's self-test."""
    _cxx(HARNESS_DIR / 'stream_bench.cpp', HARNESS, '$ORIGIN')
    _cxx(HARNESS_DIR / 'stream_diagnose.cpp', DIAGNOSE, '$ORIGIN')
    _cxx(TESTS_DIR / 'abi_consumer.cpp', ABI_CONSUMER, '$ORIGIN/../../streaming-transformer_amd/lib')
    _cxx(TESTS_DIR / 'harness_selftest.cpp', HARNESS_SELFTEST, '$ORIGIN/../../streaming-transformer_amd/lib')
    return HARNESS, ABI_CONSUMER, HARNESS_SELFTEST


def build(force: bool = True, verbose: bool = False) -> Path:
    """Compile libstamd.so. With force=False, skip when the library is newer than its sources."""
    if not force and OUTPUT.exists():
        newest = max(p.stat().st_mtime for p in DEPENDS)
        if OUTPUT.stat().st_mtime >= newest:
            return OUTPUT
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    # The translation units compile in parallel, each to an object beside the library.
    objects = [OUTPUT.parent / (src.stem + '.o.tmp') for src in SOURCES]
    procs = [subprocess.Popen([hipcc(), *COMPILE_FLAGS, *UNIT_FLAGS.get(src.name, []), '-c', '-o', str(obj), str(src)],
                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
             for src, obj in zip(SOURCES, objects)]
    try:
        for src, proc in zip(SOURCES, procs):
            _, err = proc.communicate()
            if proc.returncode != 0:
                raise RuntimeError(f'hipcc failed on {src.name} ({proc.returncode}):\n{err[-4000:]}')
            if verbose:
                sys.stderr.write(err)
        tmp = OUTPUT.with_suffix('.so.tmp')
        cmd = [hipcc(), *LINK_FLAGS, '-o', str(tmp), *map(str, objects)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f'hipcc link failed ({proc.returncode}):\n{proc.stderr[-4000:]}')
        os.replace(tmp, OUTPUT)
    finally:
        for p in procs:
            if p.poll() is None:
                p.kill()
        for obj in objects:
            obj.unlink(missing_ok=True)
    return OUTPUT


if __name__ == '__main__':
    print(build(verbose=True))

"""Reference-layout fixture directories for the benchmark driver's tests.

The driver (stream-bench) reads fixtures the way the reference's bench/Main.cpp does:
`--weights DIR` holding manifest.json + tensors.bin (the checkpoint), trace.bin and
resets.json, with the expected outputs in DIR/expected/ (manifest.json + tensors.bin holding
float32 scores[E], hidden[E,L,d], keys/values[E,L,H,W,dh]; reference/export.py:46-70), and a
config file equal to the checkpoint's config. tests/golden keeps the reference's small
fixtures compactly (the K/V row written by each event instead of the full cache per event);
this helper expands them back into that layout.
"""
from __future__ import annotations

import hashlib
import json
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / 'golden'))
from make_golden import rebuild_cache  # noqa: E402

GOLDEN = HERE / 'golden'
ROOT = HERE.parent
STAND_IN = HERE / '_build' / 'cpu_runtime' / 'libstamd.so'


def build_stand_in() -> Path:
    """tests/cpu_runtime.cpp over the C oracle, built as libstamd.so for the driver's CPU tests.

    Built under a private name and renamed into place, so test processes running at once never
    load a partly written library.
    """
    STAND_IN.parent.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix='libstamd.', suffix='.so.tmp', dir=STAND_IN.parent)
    os.close(fd)
    try:
        subprocess.run(['g++', '-O2', '-std=c++17', '-shared', '-fPIC', '-fopenmp', f'-I{ROOT / "include"}',
                        f'-I{ROOT / "oracle"}', '-o', tmp, str(HERE / 'cpu_runtime.cpp'), '-x', 'c',
                        '-ffp-contract=off', str(ROOT / 'oracle' / 'stream_oracle.c'), '-lm'],
                       check=True, capture_output=True, text=True)
        os.replace(tmp, STAND_IN)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return STAND_IN


def write_archive(directory: Path, tensors: dict, **fields) -> None:
    """manifest.json + tensors.bin with float32 tensors, the archive SHA-256 and extra fields."""
    directory.mkdir(parents=True, exist_ok=True)
    data = bytearray()
    table = []
    for name, array in tensors.items():
        blob = np.ascontiguousarray(array, dtype='<f4').tobytes()
        table.append(dict(name=name, shape=list(np.shape(array)), dtype='float32', offset=len(data), nbytes=len(blob),
                          sha256=hashlib.sha256(blob).hexdigest()))
        data.extend(blob)
    (directory / 'tensors.bin').write_bytes(bytes(data))
    manifest = dict(fields, tensors=table, sha256=hashlib.sha256(bytes(data)).hexdigest())
    (directory / 'manifest.json').write_text(json.dumps(manifest, indent=2) + '\n')


def reference_fixture(name: str, target: Path) -> tuple[Path, Path]:
    """Expand tests/golden/<name> into target/ in the reference's layout.
    Returns (weights directory, config file)."""
    source = GOLDEN / name
    target.mkdir(parents=True, exist_ok=True)
    for f in ('manifest.json', 'tensors.bin'):
        shutil.copyfile(source / 'checkpoint' / f, target / f)
    for f in ('trace.bin', 'resets.json'):
        shutil.copyfile(source / f, target / f)
    manifest = json.loads((source / 'checkpoint' / 'manifest.json').read_text())
    config = manifest['config']
    expected = np.load(source / 'expected.npz')
    resets = set(int(r) for r in expected['resets'])
    keys = np.stack([c.copy() for c in rebuild_cache(expected['key_rows'], resets, config['window'])])
    values = np.stack([c.copy() for c in rebuild_cache(expected['value_rows'], resets, config['window'])])
    write_archive(target / 'expected', dict(scores=expected['scores'], hidden=expected['hidden'], keys=keys,
                                            values=values),
                  version=1, byte_order='little', orientation='out_in', config=config, mode=manifest['mode'],
                  resets=sorted(resets))
    config_file = target / 'config.json'
    config_file.write_text(json.dumps(config, indent=2) + '\n')
    return target, config_file


def reference_checkpoint(name: str, target: Path) -> tuple[Path, Path]:
    """tests/golden/<name> (a checkpoint and its trace, no expected outputs) in the reference's
    layout. Returns (weights directory, config file)."""
    source = GOLDEN / name
    target.mkdir(parents=True, exist_ok=True)
    for f in ('manifest.json', 'tensors.bin'):
        shutil.copyfile(source / 'checkpoint' / f, target / f)
    shutil.copyfile(source / 'trace.bin', target / 'trace.bin')
    config = json.loads((source / 'checkpoint' / 'manifest.json').read_text())['config']
    config_file = target / 'config.json'
    config_file.write_text(json.dumps(config, indent=2) + '\n')
    return target, config_file


GATE_METRICS = ('scores', 'keys', 'values', 'hidden')


def gate(result, backend, precision, count):
    """The per-run checks of the reference's correctness gate (bench/gates.py:125-161) on a
    stream-bench result file."""
    assert result['mode'] == 'correctness' and result['dropped'] == 0 and result['completed'] == count
    assert result['backend'] == backend and result['precision'] == precision
    for metric in GATE_METRICS:
        e = result[metric]
        assert e['elements'] > 0 and e['failed'] == 0 and e['nonfinite'] == 0, (metric, e)
    for metric in ('cache_relative_l2_gate', 'hidden_relative_l2_gate'):
        assert result[metric]['failed'] == 0 and result[metric]['nonfinite'] == 0
    assert len(result['provenance']['executable_sha256']) == 64


def plant_score_error(oracle_dir: Path, index: int, delta: float) -> None:
    """Add `delta` to stored score `index` of a stream-sparse-oracle-v1 archive and re-hash it
    (the planted mistake of the stored-oracle tests goes into the oracle, on the CPU)."""
    manifest = json.loads((oracle_dir / 'manifest.json').read_text())
    raw = bytearray((oracle_dir / 'tensors.bin').read_bytes())
    entry = next(t for t in manifest['tensors'] if t['name'] == 'scores')
    at = entry['offset'] + 4 * index
    value = np.frombuffer(bytes(raw[at:at + 4]), dtype='<f4')[0] + np.float32(delta)
    raw[at:at + 4] = np.float32(value).tobytes()
    (oracle_dir / 'tensors.bin').write_bytes(bytes(raw))
    manifest['sha256'] = hashlib.sha256(bytes(raw)).hexdigest()
    (oracle_dir / 'manifest.json').write_text(json.dumps(manifest))


def window_fixture(name: str, target: Path) -> tuple[Path, Path]:
    """tests/golden/windows/<name> (e.g. 'large-w128-mixed') rebuilt as a reference fixture
    directory: the variant's manifest, trace and resets with its base checkpoint's tensors
    (the same bytes, checked by make_golden.py). Returns (weights directory, config file)."""
    source = GOLDEN / 'windows' / name
    size, _, mode = name.split('-')
    target.mkdir(parents=True, exist_ok=True)
    for f in ('manifest.json', 'trace.bin', 'resets.json'):
        shutil.copyfile(source / f, target / f)
    shutil.copyfile(GOLDEN / f'{size}-{mode}' / 'checkpoint' / 'tensors.bin', target / 'tensors.bin')
    config = json.loads((source / 'manifest.json').read_text())['config']
    config_file = target / 'config.json'
    config_file.write_text(json.dumps(config, indent=2) + '\n')
    return target, config_file


def adversarial_trace(count: int, features: int, kind: str, seed: int = 123) -> np.ndarray:
    """The reference's input families (reference/export.py:12-28): N(0,1) events from
    numpy's default_rng(seed) as little-endian float32, then 'zeros', 'constant' (0.25),
    'impulses' (1.0 at feature 0 of every 17th event, zeros elsewhere), 'alternating' (every
    feature +1 on even events, -1 on odd ones), 'repeated' (events cycling through the first
    7) or 'random' (unchanged)."""
    x = np.random.default_rng(seed).standard_normal((count, features)).astype('<f4')
    if kind == 'zeros':
        x.fill(0)
    elif kind == 'constant':
        x.fill(0.25)
    elif kind == 'impulses':
        x.fill(0)
        x[::17, 0] = 1
    elif kind == 'alternating':
        x[:] = ((-1.0) ** np.arange(count))[:, None]
    elif kind == 'repeated':
        x[:] = x[np.arange(count) % min(count, 7)]
    elif kind != 'random':
        raise ValueError(kind)
    return x

"""CPU checks of the C ABI library: it loads, exports every declared entry point, and
rejects invalid configurations and options before touching a device
(ModelConfig::validate, src/runtime/Model.cpp:22-29; RuntimeOptions checks,
src/cuda/Runtime.cu:178-183)."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from streamtx import Backend, ModelConfig, Runtime, RuntimeOptions, WeightStorage, library, synthetic_checkpoint
from streamtx.runtime import LIBRARY_PATH, _Options

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / 'include' / 'st_runtime.h').read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(st_[a-z_]+)\s*\(', text)))


def test_library_exports_every_declared_function():
    assert LIBRARY_PATH.exists(), 'run __graft_entry__.build() first'
    out = subprocess.run(['nm', '-D', '--defined-only', str(LIBRARY_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r'\s[TW]\s+(\S+)', out))
    names = declared_functions()
    assert len(names) >= 11
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    lib = library()
    for n in names:
        assert hasattr(lib, n)


def test_options_default_matches_reference_defaults():
    o = _Options()
    library().st_options_default(ctypes.byref(o))
    assert o.backend == int(Backend.GRAPH) and o.blocks == 1 and o.idle_seconds == 30.0
    assert o.max_events == 0 and o.initial_sequence == 0 and not o.mapped and not o.backoff


@pytest.mark.parametrize('field,value', [('heads', 3), ('layers', 17), ('width', 2048), ('ffn', 5000),
                                         ('window', 0), ('features', 2000), ('epsilon', 0.0)])
def test_invalid_config_rejected(field, value):
    base = dict(layers=1, width=64, heads=4, ffn=128, window=64, features=32, epsilon=1e-5)
    c = ModelConfig(**base)
    w = synthetic_checkpoint(c, seed=0)
    bad = ModelConfig(**{**base, field: value})
    with pytest.raises(RuntimeError, match='Invalid or unsupported model dimensions'):
        Runtime((bad, w, False), RuntimeOptions(backend=Backend.FUSED))


@pytest.mark.parametrize('opts,msg', [
    (dict(idle_seconds=0), 'idle budget'),
    (dict(blocks=-1), 'idle budget'),
    (dict(initial_sequence=2**64 - 2), 'Initial sequence'),
    (dict(backend=Backend.CUBLAS, weight_dtype=WeightStorage.BF16), 'own weight storage'),
])
def test_invalid_options_rejected(opts, msg):
    c = ModelConfig(1, 64, 4, 128, 64, 32)
    w = synthetic_checkpoint(c, seed=0)
    with pytest.raises(RuntimeError, match=msg):
        Runtime((c, w, False), RuntimeOptions(**opts))


def test_shape_mismatch_rejected_on_device_or_before():
    c = ModelConfig(1, 64, 4, 128, 64, 32)
    w = synthetic_checkpoint(c, seed=0)
    w['layers.0.q'] = np.zeros((64, 63), np.float32)
    with pytest.raises((RuntimeError, ValueError)):
        Runtime((c, w, False), RuntimeOptions(backend=Backend.FUSED))


@pytest.mark.parametrize('mode,count,msg', [('bogus', 10, 'Unknown transport mode'), ('empty', 0, 'count')])
def test_transport_bench_rejects_arguments(mode, count, msg):
    # Validated before any device work (Stream::transportBench, include/Runtime.hpp:46).
    from streamtx import transport_bench
    with pytest.raises(RuntimeError, match=msg):
        transport_bench(mode, count)

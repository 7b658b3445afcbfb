"""Python wrapper of the C oracle (oracle/stream_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the reference the GPU results are compared with. The product
path never imports this module.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / '_build' / 'libstream_oracle.so'
# The same C source built for x86-64-v3 (AVX2) hosts, for timing; bit-identical results.
LIBRARY_V3 = HERE / '_build' / 'libstream_oracle_v3.so'

# Canonical tensor order of so_create (oracle/stream_oracle.h).
_LAYER_ORDER = ('norm1', 'norm2', 'q', 'k', 'v', 'out', 'gate', 'up', 'down')


class _Config(ctypes.Structure):
    _fields_ = [('layers', ctypes.c_int32), ('width', ctypes.c_int32), ('heads', ctypes.c_int32),
                ('ffn', ctypes.c_int32), ('window', ctypes.c_int32), ('features', ctypes.c_int32),
                ('epsilon', ctypes.c_float)]


_libs = {}
# void fn(void* user, const char* name, const float* values, int count)
_TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int)


def build() -> Path:
    subprocess.run(['make', '-s', '-C', str(HERE)], check=True)
    return LIBRARY


def library(isa: str = 'portable') -> ctypes.CDLL:
    """The oracle library: 'portable' (x86-64 baseline) or 'v3' (AVX2 hosts)."""
    if isa not in _libs:
        path = LIBRARY if isa == 'portable' else LIBRARY_V3
        if not path.exists():
            build()
        lib = ctypes.CDLL(str(path))
        F = ctypes.POINTER(ctypes.c_float)
        lib.so_create.argtypes = [ctypes.POINTER(_Config), ctypes.c_int, ctypes.c_int, ctypes.POINTER(F)]
        lib.so_create.restype = ctypes.c_void_p
        lib.so_destroy.argtypes = [ctypes.c_void_p]
        lib.so_step.argtypes = [ctypes.c_void_p, F]
        lib.so_step.restype = ctypes.c_float
        lib.so_step_trace.argtypes = [ctypes.c_void_p, F, _TRACE_FN, ctypes.c_void_p]
        lib.so_step_trace.restype = ctypes.c_float
        lib.so_reset.argtypes = [ctypes.c_void_p]
        lib.so_position.argtypes = [ctypes.c_void_p]
        lib.so_position.restype = ctypes.c_uint64
        lib.so_snapshot.argtypes = [ctypes.c_void_p, F, F, F]
        lib.so_set_threads.argtypes = [ctypes.c_void_p, ctypes.c_int]
        lib.so_round_half.argtypes = [ctypes.c_float]
        lib.so_round_half.restype = ctypes.c_float
        lib.so_round_bf16.argtypes = [ctypes.c_float]
        lib.so_round_bf16.restype = ctypes.c_float
        lib.so_half_bits.argtypes = [ctypes.c_float]
        lib.so_half_bits.restype = ctypes.c_uint16
        lib.so_bf16_bits.argtypes = [ctypes.c_float]
        lib.so_bf16_bits.restype = ctypes.c_uint16
        _libs[isa] = lib
    return _libs[isa]


def _fptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Oracle:
    """The reference CPU step (src/cpu/Cpu.cpp:59-141) restated in C.

    config: any object with layers/width/heads/ffn/window/features/epsilon; tensors: name ->
    float32 array. accumulate: 'float' (the reference's arithmetic) or 'double' (referee).
    isa: 'portable' or 'v3' (the AVX2 build, same results; used to time the CPU baseline).
    """

    def __init__(self, config, tensors, mixed=False, accumulate='float', threads=1, isa='portable'):
        self.config = config
        self._lib = library(isa)
        self.mixed = bool(mixed)
        names = ['input', 'final_norm', 'score']
        for layer in range(config.layers):
            names += [f'layers.{layer}.{n}' for n in _LAYER_ORDER]
        self._keep = [np.ascontiguousarray(tensors[n], dtype=np.float32) for n in names]
        ptrs = (ctypes.POINTER(ctypes.c_float) * len(names))(*[_fptr(a) for a in self._keep])
        cfg = _Config(config.layers, config.width, config.heads, config.ffn, config.window, config.features,
                      config.epsilon)
        self._h = self._lib.so_create(ctypes.byref(cfg), int(self.mixed), int(accumulate == 'double'), ptrs)
        if not self._h:
            raise ValueError('Invalid or unsupported model dimensions')
        if threads > 1:
            self._lib.so_set_threads(self._h, threads)

    def __del__(self):
        if getattr(self, '_h', None):
            self._lib.so_destroy(self._h)
            self._h = None

    def step(self, event) -> float:
        x = np.ascontiguousarray(event, dtype=np.float32)
        return float(self._lib.so_step(self._h, _fptr(x)))

    def trace_step(self, event):
        """One step with the per-operation trace (so_step_trace, the reference's CpuTrace):
        returns (score, {name: float32 array}) with the entries in execution order."""
        x = np.ascontiguousarray(event, dtype=np.float32)
        entries = {}

        def take(_user, name, values, count):
            entries[name.decode()] = np.ctypeslib.as_array(values, shape=(count,)).copy()

        callback = _TRACE_FN(take)
        score = float(self._lib.so_step_trace(self._h, _fptr(x), callback, None))
        return score, entries

    def reset(self) -> None:
        self._lib.so_reset(self._h)

    @property
    def position(self) -> int:
        return int(self._lib.so_position(self._h))

    def snapshot(self):
        c = self.config
        dim = c.width // c.heads
        keys = np.empty((c.layers, c.heads, c.window, dim), dtype=np.float32)
        values = np.empty_like(keys)
        hidden = np.empty((c.layers, c.width), dtype=np.float32)
        self._lib.so_snapshot(self._h, _fptr(keys), _fptr(values), _fptr(hidden))
        return self.position, keys, values, hidden


def round_half(x: float) -> float:
    return float(library().so_round_half(x))


def round_bf16(x: float) -> float:
    return float(library().so_round_bf16(x))

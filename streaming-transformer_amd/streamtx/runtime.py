"""ctypes binding of libstamd.so, mirroring Stream::Runtime (include/Runtime.hpp:7-46).

Same names and meaning as the reference interface: ``Runtime(model, options)``, ``step``,
``reset``, ``stop``, ``snapshot``, ``info``, ``device_trace``, plus ``probe()``. Failures
raise ``RuntimeError`` with the library's message, as the reference throws
``std::runtime_error``. There is no fallback: if the HIP library is missing or cannot be
loaded, constructing a runtime raises.
"""
from __future__ import annotations

import ctypes
import enum
import json
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .model import Checkpoint, ModelConfig

PACKAGE_DIR = Path(__file__).resolve().parent.parent
LIBRARY_PATH = PACKAGE_DIR / 'lib' / 'libstamd.so'


class Backend(enum.IntEnum):
    """Stream::Backend (include/Runtime.hpp:7)."""
    CUDA = 0          # staged HIP phase kernels
    GRAPH = 1         # staged sequence captured in a hipGraph
    CUBLAS = 2        # vendor GEMV baseline: rocBLAS projections, HIP kernels for the rest
    CUBLAS_GRAPH = 3  # the same captured in a hipGraph
    FUSED = 4         # one launch per step (plain once the grid is shown co-resident)
    PERSISTENT = 5    # resident kernel + host mailbox


class WeightStorage(enum.IntEnum):
    AS_MODEL = 0
    BF16 = 1


@dataclass
class RuntimeOptions:
    """Stream::RuntimeOptions (include/Runtime.hpp:8-19) plus weight storage.
    blocks = workgroups of 512 threads; 0 = one per compute unit."""
    backend: Backend = Backend.GRAPH
    blocks: int = 1
    backoff: bool = False
    mapped: bool = False
    vector_matvec: bool = False
    fused_attention: bool = False
    max_events: int = 0
    initial_sequence: int = 0
    idle_seconds: float = 30.0
    weight_dtype: WeightStorage = WeightStorage.AS_MODEL
    initial_epoch: int = 0  # first epoch of the device's tagged dataflow (0 = 1); tests only


class _Config(ctypes.Structure):
    _fields_ = [('layers', ctypes.c_int32), ('width', ctypes.c_int32), ('heads', ctypes.c_int32),
                ('ffn', ctypes.c_int32), ('window', ctypes.c_int32), ('features', ctypes.c_int32),
                ('epsilon', ctypes.c_float)]


class _Options(ctypes.Structure):
    _fields_ = [('backend', ctypes.c_int32), ('blocks', ctypes.c_int32), ('backoff', ctypes.c_int32),
                ('mapped', ctypes.c_int32), ('vector_matvec', ctypes.c_int32),
                ('fused_attention', ctypes.c_int32), ('max_events', ctypes.c_uint64),
                ('initial_sequence', ctypes.c_uint64), ('idle_seconds', ctypes.c_double),
                ('weight_dtype', ctypes.c_int32), ('initial_epoch', ctypes.c_uint32)]


class _Tensor(ctypes.Structure):
    _fields_ = [('name', ctypes.c_char_p), ('rank', ctypes.c_int32), ('shape', ctypes.c_int32 * 2),
                ('data', ctypes.POINTER(ctypes.c_float))]


_lib = None


def library(path: os.PathLike | None = None) -> ctypes.CDLL:
    """Load libstamd.so (once). Raises RuntimeError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(path or os.environ.get('STAMD_LIBRARY', LIBRARY_PATH))
    if not path.exists():
        raise RuntimeError(f'HIP library not built: {path} (run __graft_entry__.build())')
    lib = ctypes.CDLL(str(path))
    P, F, D = ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_double)
    lib.st_options_default.argtypes = [ctypes.POINTER(_Options)]
    lib.st_options_default.restype = None
    lib.st_runtime_create.argtypes = [ctypes.POINTER(_Config), ctypes.c_int32, ctypes.POINTER(_Tensor),
                                      ctypes.c_size_t, ctypes.POINTER(_Options), ctypes.POINTER(P)]
    lib.st_runtime_destroy.argtypes = [P]
    lib.st_runtime_destroy.restype = None
    lib.st_runtime_step.argtypes = [P, F, F]
    lib.st_runtime_reset.argtypes = [P]
    lib.st_runtime_stop.argtypes = [P]
    lib.st_runtime_snapshot.argtypes = [P, ctypes.POINTER(ctypes.c_uint64), F, F, F]
    lib.st_runtime_device_trace.argtypes = [P, F, ctypes.c_size_t, D, D]
    lib.st_runtime_device_run.argtypes = [P, F, ctypes.c_size_t, ctypes.c_int32, D, D]
    lib.st_runtime_device_trace_noalloc.argtypes = [P, ctypes.c_void_p, ctypes.c_size_t, D, D]
    lib.st_runtime_phase_times.argtypes = [P, F, D, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.st_runtime_trace_step.argtypes = [P, F, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t), F,
                                          ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.st_runtime_scheduled_run.argtypes = [P, F, ctypes.c_size_t, ctypes.c_double, ctypes.c_size_t, ctypes.c_int32,
                                             D, D, D, D, F, ctypes.POINTER(ctypes.c_uint8)]
    lib.st_runtime_info_json.argtypes = [P, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.st_probe_json.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.st_transport_bench.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int32, ctypes.c_char_p,
                                       ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.st_last_error.argtypes = []
    lib.st_last_error.restype = ctypes.c_char_p
    lib.st_batch_create.argtypes = [ctypes.POINTER(_Config), ctypes.c_int32, ctypes.POINTER(_Tensor),
                                    ctypes.c_size_t, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(P)]
    lib.st_batch_create_resident.argtypes = lib.st_batch_create.argtypes
    lib.st_batch_destroy.argtypes = [P]
    lib.st_batch_destroy.restype = None
    lib.st_batch_step.argtypes = [P, F, F]
    lib.st_batch_reset.argtypes = [P, ctypes.c_int32]
    lib.st_batch_snapshot.argtypes = [P, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64), F, F, F]
    lib.st_batch_device_run.argtypes = [P, F, ctypes.c_size_t, D, D]
    lib.st_batch_set_eager.argtypes = [P, ctypes.c_int32]
    for name in ('st_batch_create', 'st_batch_create_resident', 'st_batch_step', 'st_batch_reset', 'st_batch_snapshot',
                 'st_batch_device_run', 'st_batch_set_eager',
                 'st_runtime_create', 'st_runtime_step', 'st_runtime_reset', 'st_runtime_stop',
                 'st_runtime_snapshot', 'st_runtime_device_trace', 'st_runtime_device_trace_noalloc',
                 'st_runtime_device_run', 'st_runtime_phase_times',
                 'st_runtime_trace_step', 'st_runtime_scheduled_run',
                 'st_runtime_info_json',
                 'st_probe_json', 'st_transport_bench'):
        getattr(lib, name).restype = ctypes.c_int
    _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        raise RuntimeError(library().st_last_error().decode() or f'libstamd error {status}')


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _json(fn, *args) -> dict:
    needed = ctypes.c_size_t(0)
    _check(fn(*args, None, 0, ctypes.byref(needed)))
    buf = ctypes.create_string_buffer(needed.value)
    _check(fn(*args, buf, needed.value, ctypes.byref(needed)))
    return json.loads(buf.value.decode())


def _marshal(config, tensors):
    """(st_config, kept arrays, st_tensor array) for a create call. Every named tensor is
    passed; the library validates names, shapes and the config."""
    cfg = _Config(config.layers, config.width, config.heads, config.ffn, config.window,
                  config.features, config.epsilon)
    keep, items = [], []
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name], dtype=np.float32)
        keep.append(a)
        t = _Tensor()
        t.name = name.encode()
        t.rank = a.ndim
        t.shape[0] = a.shape[0]
        t.shape[1] = a.shape[1] if a.ndim > 1 else 0
        t.data = _fptr(a)
        items.append(t)
    return cfg, keep, (_Tensor * len(items))(*items)


def probe() -> dict:
    """Stream::probe() (src/cuda/Runtime.cu:134-161)."""
    return _json(library().st_probe_json)


def transport_bench(mode: str, count: int, backoff: bool = False, output: str | None = None) -> dict:
    """Stream::transportBench (include/Runtime.hpp:46): ping-pong, gpu-ping, empty,
    empty-graph or copy; per-sample CSV to `output` when given."""
    lib = library()
    args = (mode.encode(), int(count), int(bool(backoff)), output.encode() if output else None)
    needed = ctypes.c_size_t(0)
    # One call runs the benchmark; the report is sized generously and re-read only if needed.
    buf = ctypes.create_string_buffer(1 << 16)
    _check(lib.st_transport_bench(*args, buf, len(buf), ctypes.byref(needed)))
    if needed.value > len(buf):
        raise RuntimeError('transport report exceeds 64 KiB')
    return json.loads(buf.value.decode())


class Runtime:
    """Stream::Runtime over the C ABI. ``model`` is a Checkpoint, or a (config, tensors,
    mixed) triple. Not thread-safe; one outstanding command (docs/transport.md:14)."""

    def __init__(self, model, options: RuntimeOptions | None = None):
        if isinstance(model, Checkpoint):
            config, tensors, mixed = model.config, model.tensors, model.mixed
        else:
            config, tensors, mixed = model
        self.config: ModelConfig = config
        self.mixed = bool(mixed)
        self.options = options or RuntimeOptions()
        lib = library()
        cfg, keep, array = _marshal(config, tensors)
        o = self.options
        opts = _Options(int(o.backend), int(o.blocks), int(o.backoff), int(o.mapped), int(o.vector_matvec),
                        int(o.fused_attention), int(o.max_events), int(o.initial_sequence),
                        float(o.idle_seconds), int(o.weight_dtype), int(o.initial_epoch))
        handle = ctypes.c_void_p()
        _check(lib.st_runtime_create(ctypes.byref(cfg), int(self.mixed), array, len(array), ctypes.byref(opts),
                                     ctypes.byref(handle)))
        self._h = handle
        self._score = np.zeros(1, dtype=np.float32)

    def close(self) -> None:
        """Stop the worker and free device resources (~Runtime)."""
        if getattr(self, '_h', None):
            library().st_runtime_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _handle(self):
        if not self._h:
            raise RuntimeError('Runtime is closed')
        return self._h

    def step(self, event) -> float:
        x = np.ascontiguousarray(event, dtype=np.float32)
        if x.size != self.config.features:
            raise ValueError('event must hold `features` floats')
        _check(library().st_runtime_step(self._handle(), _fptr(x), _fptr(self._score)))
        return float(self._score[0])

    def reset(self) -> None:
        _check(library().st_runtime_reset(self._handle()))

    def stop(self) -> None:
        _check(library().st_runtime_stop(self._handle()))

    def snapshot(self):
        """(position, keys[L,H,W,dh], values[L,H,W,dh], hidden[L,width]) as FP32."""
        c = self.config
        keys = np.empty((c.layers, c.heads, c.window, c.dim), dtype=np.float32)
        values = np.empty_like(keys)
        hidden = np.empty((c.layers, c.width), dtype=np.float32)
        pos = ctypes.c_uint64(0)
        _check(library().st_runtime_snapshot(self._handle(), ctypes.byref(pos), _fptr(keys), _fptr(values),
                                             _fptr(hidden)))
        return int(pos.value), keys, values, hidden

    def device_trace(self, inputs):
        """Runtime::deviceTrace: reset, run a preloaded trace; (mean us, per-event us)."""
        x = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, self.config.features)
        per = np.empty(x.shape[0], dtype=np.float64)
        mean = ctypes.c_double(0)
        _check(library().st_runtime_device_trace(self._handle(), _fptr(x), x.shape[0], ctypes.byref(mean),
                                                 per.ctypes.data_as(ctypes.POINTER(ctypes.c_double))))
        return float(mean.value), per

    def device_trace_noalloc(self, device_events: int, count: int, per_event: bool = True):
        """st_runtime_device_trace_noalloc: `count` events already in device memory at address
        `device_events` (count*features floats, unpadded); the call allocates nothing.
        (mean us, per-event us or None)."""
        per = np.empty(count, dtype=np.float64) if per_event else None
        mean = ctypes.c_double(0)
        _check(library().st_runtime_device_trace_noalloc(
            self._handle(), ctypes.c_void_p(device_events), int(count), ctypes.byref(mean),
            per.ctypes.data_as(ctypes.POINTER(ctypes.c_double)) if per is not None else None))
        return float(mean.value), per

    def device_run(self, inputs, reset: bool = False):
        """Per-launch device timing (extension): one step per launch, HIP events on the
        runtime's stream; continues the current state unless reset. (mean us, per-event us)."""
        x = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, self.config.features)
        per = np.empty(x.shape[0], dtype=np.float64)
        mean = ctypes.c_double(0)
        _check(library().st_runtime_device_run(self._handle(), _fptr(x), x.shape[0], int(reset),
                                               ctypes.byref(mean),
                                               per.ctypes.data_as(ctypes.POINTER(ctypes.c_double))))
        return float(mean.value), per

    def phase_times(self, event):
        """One fused step with stamps (extension): (array [phases, workgroups, 8] of
        microseconds since workgroup 0 started the step: phase start, stream wave 1 done,
        all stream waves done, staging done, three progress marks of stream wave 1, spare;
        step end)."""
        x = np.ascontiguousarray(event, dtype=np.float32)
        count = ctypes.c_size_t(0)
        lib = library()
        _check(lib.st_runtime_phase_times(self._handle(), _fptr(x), None, 0, ctypes.byref(count)))
        n = count.value
        out = np.empty(n, dtype=np.float64)
        _check(lib.st_runtime_phase_times(self._handle(), _fptr(x),
                                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), n,
                                          ctypes.byref(count)))
        phases = 5 * self.config.layers + 2
        return out[:-1].reshape(phases, -1, 8), float(out[-1])

    def trace_step(self, event) -> dict:
        """Runtime::traceStep (staged backend): one real step; {name: FP32 array} of the
        operation/cast boundaries, in the reference's naming."""
        x = np.ascontiguousarray(event, dtype=np.float32)
        if x.size != self.config.features:
            raise ValueError('event must hold `features` floats')
        lib = library()
        needed, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
        _check(lib.st_runtime_trace_step(self._handle(), _fptr(x), None, 0, ctypes.byref(needed), None, 0,
                                         ctypes.byref(total)))
        names = ctypes.create_string_buffer(needed.value)
        values = np.empty(total.value, dtype=np.float32)
        _check(lib.st_runtime_trace_step(self._handle(), _fptr(x), names, needed.value, ctypes.byref(needed),
                                         _fptr(values), total.value, ctypes.byref(total)))
        return {name: values[o:o + n].copy() for name, (o, n) in json.loads(names.value.decode()).items()}

    def scheduled_run(self, events, rate: float, queue: int = 4096, bursty: bool = False) -> dict:
        """Scheduled arrivals (bench/Main.cpp:282-342): arrays intended/enqueue/submit/complete
        (ns), scores and dropped, plus the latency distributions of bench/analyze.py:32-52
        (service = complete - submit, arrival = complete - intended, queueing = submit -
        enqueue, injection = enqueue - intended; microseconds, nearest rank)."""
        x = np.ascontiguousarray(events, dtype=np.float32).reshape(-1, self.config.features)
        n = x.shape[0]
        D = ctypes.POINTER(ctypes.c_double)
        out = {k: np.empty(n, dtype=np.float64) for k in ('intended_ns', 'enqueue_ns', 'submit_ns', 'complete_ns')}
        scores = np.empty(n, dtype=np.float32)
        dropped = np.zeros(n, dtype=np.uint8)
        _check(library().st_runtime_scheduled_run(
            self._handle(), _fptr(x), n, float(rate), int(queue), int(bool(bursty)),
            *(out[k].ctypes.data_as(D) for k in ('intended_ns', 'enqueue_ns', 'submit_ns', 'complete_ns')),
            _fptr(scores), dropped.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))))
        kept = dropped == 0

        def dist(v):
            v = np.sort(np.asarray(v, dtype=np.float64))
            if not len(v):
                return {}
            r = {name: float(v[int(np.ceil(q * len(v))) - 1]) for name, q in
                 (('p50_us', .5), ('p95_us', .95), ('p99_us', .99), ('p999_us', .999))}
            return dict(r, worst_us=float(v[-1]))

        summary = dict(offered=n, completed=int(kept.sum()), dropped=int((~kept).sum()),
                       service=dist((out['complete_ns'][kept] - out['submit_ns'][kept]) / 1e3),
                       arrival=dist((out['complete_ns'][kept] - out['intended_ns'][kept]) / 1e3),
                       queueing=dist((out['submit_ns'][kept] - out['enqueue_ns'][kept]) / 1e3),
                       injection=dist((out['enqueue_ns'] - out['intended_ns']) / 1e3))
        return dict(out, scores=scores, dropped=dropped.astype(bool), summary=summary)

    def info(self) -> dict:
        return _json(library().st_runtime_info_json, self._handle())


class BatchRuntime:
    """`streams` independent streams over one set of weights (extension; the reference is
    single-stream, docs/Architecture.md:3). Each stream behaves like its own Runtime on the
    same events; a step advances all of them. FP32 checkpoints, weights stored as
    ``weight_dtype`` (WeightStorage).

    ``resident=False``: a graph of phase kernels with MFMA projections over the streams
    (1..256 streams; every stream's results bit-identical for any batch size).
    ``resident=True``: one launch of the fused step per step, each stream on its own share
    of the CUs (1..32 streams; every stream's results bit-identical to a FUSED Runtime's)."""

    def __init__(self, model, streams: int, weight_dtype: int = 0, resident: bool = False):
        if isinstance(model, Checkpoint):
            config, tensors, mixed = model.config, model.tensors, model.mixed
        else:
            config, tensors, mixed = model
        self.config: ModelConfig = config
        self.streams = int(streams)
        cfg, keep, array = _marshal(config, tensors)
        handle = ctypes.c_void_p()
        create = library().st_batch_create_resident if resident else library().st_batch_create
        _check(create(ctypes.byref(cfg), int(bool(mixed)), array, len(array), self.streams, int(weight_dtype),
                      ctypes.byref(handle)))
        self.resident = bool(resident)
        self._h = handle
        self._scores = np.zeros(self.streams, dtype=np.float32)

    def close(self) -> None:
        if getattr(self, '_h', None):
            library().st_batch_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _handle(self):
        if not self._h:
            raise RuntimeError('BatchRuntime is closed')
        return self._h

    def step(self, events) -> np.ndarray:
        """events [streams, features] -> scores [streams]."""
        x = np.ascontiguousarray(events, dtype=np.float32)
        if x.size != self.streams * self.config.features:
            raise ValueError('events must hold streams*features floats')
        _check(library().st_batch_step(self._handle(), _fptr(x), _fptr(self._scores)))
        return self._scores.copy()

    def reset(self, stream: int = -1) -> None:
        """Zero one stream (all when -1)."""
        _check(library().st_batch_reset(self._handle(), int(stream)))

    def snapshot(self, stream: int):
        """Runtime.snapshot() of one stream."""
        c = self.config
        keys = np.empty((c.layers, c.heads, c.window, c.dim), dtype=np.float32)
        values = np.empty_like(keys)
        hidden = np.empty((c.layers, c.width), dtype=np.float32)
        pos = ctypes.c_uint64(0)
        _check(library().st_batch_snapshot(self._handle(), int(stream), ctypes.byref(pos), _fptr(keys),
                                           _fptr(values), _fptr(hidden)))
        return int(pos.value), keys, values, hidden

    def device_run(self, inputs):
        """Steps from a preloaded device copy of inputs [count, streams, features]; continues
        the current state. (mean us per step, per-step us)."""
        x = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, self.streams * self.config.features)
        per = np.empty(x.shape[0], dtype=np.float64)
        mean = ctypes.c_double(0)
        _check(library().st_batch_device_run(self._handle(), _fptr(x), x.shape[0], ctypes.byref(mean),
                                             per.ctypes.data_as(ctypes.POINTER(ctypes.c_double))))
        return float(mean.value), per

    def set_eager(self, eager: bool = True) -> None:
        """Launch each step's kernels directly instead of replaying the captured graph (the
        phase-kernel path; the same results). For kernel traces."""
        _check(library().st_batch_set_eager(self._handle(), 1 if eager else 0))

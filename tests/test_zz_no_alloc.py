"""The allocation-free device trace (st_runtime_device_trace_noalloc) against the allocating
one (st_runtime_device_trace), through the C ABI.

The caller owns the device events: this test allocates them with hipMalloc from the same HIP
runtime the library links (/opt/rocm/lib/libamdhip64.so) and passes the device address, as a C
caller would. Two calls in a row, the second with fewer events: each leaves exactly the
carried state (position, K/V rings, hidden state) that st_runtime_device_trace leaves for the
same events (bit for bit), and reports positive per-event times whose sum is the mean times
the count. A count above the fixed stamp array is rejected before any device work.
"""
import ctypes

import numpy as np
import pytest

from streamtx import Backend, ModelConfig, Runtime, RuntimeOptions, synthetic_checkpoint

pytestmark = pytest.mark.gpu

MAX_EVENTS = 1 << 20


class DeviceArray:
    """count*features float32 events in device memory, allocated and filled by the caller."""

    def __init__(self, events):
        self.hip = ctypes.CDLL('/opt/rocm/lib/libamdhip64.so')
        self.hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.hip.hipFree.argtypes = [ctypes.c_void_p]
        data = np.ascontiguousarray(events, dtype=np.float32)
        self.ptr = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(self.ptr), data.nbytes) == 0
        assert self.hip.hipMemcpy(self.ptr, data.ctypes.data, data.nbytes, 1) == 0  # host to device

    def close(self):
        if self.ptr:
            self.hip.hipFree(self.ptr)
            self.ptr = None


def _states_equal(a, b):
    assert a[0] == b[0]
    for x, y in zip(a[1:], b[1:]):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize('blocks', [0, 1])
def test_noalloc_trace_matches_allocating_trace(blocks):
    c = ModelConfig(2, 256, 4, 512, 40, 250)  # features 250: unpadded rows of 250 floats
    w = synthetic_checkpoint(c, seed=41)
    events = np.random.default_rng(41).standard_normal((300, c.features), dtype=np.float32)
    print(f'[case] noalloc trace blocks={blocks} counts=300,70', flush=True)
    dev = DeviceArray(events)
    try:
        with Runtime((c, w, False), RuntimeOptions(backend=Backend.FUSED, blocks=blocks)) as rt, \
                Runtime((c, w, False), RuntimeOptions(backend=Backend.FUSED, blocks=blocks)) as ref:
            for count in (300, 70):
                mean, per = rt.device_trace_noalloc(dev.ptr.value, count)
                got = rt.snapshot()
                ref.device_trace(events[:count])
                _states_equal(got, ref.snapshot())
                assert got[0] == count
                assert mean > 0 and per.shape == (count,) and np.all(per > 0)
                assert abs(per.sum() - mean * count) <= 1e-6 * mean * count + 1e-3
                # Stepping after the trace continues from the traced state, like the allocating call.
                assert rt.step(events[0]) == ref.step(events[0])
            with pytest.raises(RuntimeError, match='limited to'):
                rt.device_trace_noalloc(dev.ptr.value, MAX_EVENTS + 1)
            mean, per = rt.device_trace_noalloc(dev.ptr.value, 5, per_event=False)
            assert mean > 0 and per is None
    finally:
        dev.close()


def test_noalloc_trace_requires_fused_backend_and_device_memory():
    c = ModelConfig(1, 64, 4, 128, 8, 64)
    w = synthetic_checkpoint(c, seed=42)
    events = np.zeros((4, c.features), np.float32)
    with Runtime((c, w, False), RuntimeOptions(backend=Backend.GRAPH, blocks=0)) as rt:
        with pytest.raises(RuntimeError, match='fused backend'):
            rt.device_trace_noalloc(events.ctypes.data, 4)
    with Runtime((c, w, False), RuntimeOptions(backend=Backend.FUSED, blocks=0)) as rt:
        with pytest.raises(RuntimeError, match='device memory'):
            rt.device_trace_noalloc(events.ctypes.data, 4)

"""The FP32 parity bar of the GPU tests, for deep models.

Per element, |a - r| <= 1e-6 + 1e-5 |r| against the FP64-accumulating oracle r (the strict
bar). In deep models (Large: 12 layers of 1024-4096-long dot products) the reference's own FP32
algorithm, the float oracle f (a restatement of src/cpu/Cpu.cpp:59-141), misses that bar on
some elements: its worst element reaches about 3x the bar on the Large configuration. There the
GPU result passes when it is at least as accurate as the reference path on the same inputs, by
two measures against the FP64 referee:
  - its worst normalized error, max_i |a_i - r_i| / bar_i, is no larger than the float
    oracle's (or within the bar);
  - its count of elements over the bar is no larger than the float oracle's count.
Both figures, for the GPU and for the float oracle, are returned, and appended as JSON lines to
the file named by STAMD_PARITY_MARGINS when that variable is set, so that a run can record its
margins.
"""
import json
import os

import numpy as np



def bar(reference, atol=1e-6, rtol=1e-5):
    return atol + rtol * np.abs(np.asarray(reference, np.float64))


def margins(actual, reference):
    """(worst normalized error, elements over the bar): inf / all elements if a value is not
    finite."""
    a, r = np.asarray(actual, np.float64).ravel(), np.asarray(reference, np.float64).ravel()
    if not (np.isfinite(a).all() and np.isfinite(r).all()):
        return np.inf, a.size
    if not a.size:
        return 0.0, 0
    ratio = np.abs(a - r) / bar(r)
    return float(ratio.max()), int(np.count_nonzero(ratio > 1.0))


def worst(actual, reference):
    """max_i |a_i - r_i| / bar_i (inf where a value is not finite)."""
    return margins(actual, reference)[0]


def record(entry: dict) -> None:
    path = os.environ.get('STAMD_PARITY_MARGINS')
    if path:
        with open(path, 'a') as f:
            f.write(json.dumps(entry) + '\n')


def check(actual, reference64, reference32, what=''):
    """Strict bar, or no worse than the reference's FP32 algorithm by both measures (see the
    module doc). Returns the four figures."""
    got, got_n = margins(actual, reference64)
    ref, ref_n = margins(reference32, reference64)
    m = dict(what=what, elements=int(np.size(actual)), gpu_worst=got, gpu_over_bar=got_n, float_oracle_worst=ref,
             float_oracle_over_bar=ref_n)
    record(m)
    assert got <= max(1.0, ref), f'{what}: worst error {got:.3g} x the FP32 bar; the float oracle reaches {ref:.3g} x'
    assert got_n <= ref_n, f'{what}: {got_n} elements over the FP32 bar; the float oracle has {ref_n}'
    return m

"""Acceptance metrics of the reference's numerical policy ``mixed-depth-rms-v3``.

Restates include/Numerical.hpp:10-30 (residualScale, relativeL2, mixedStateScale),
reference/numerical.py:13-37 (state_errors, score_errors) and the per-element bounds of
bench/Main.cpp:57-84 as used at :354-409:
  FP32: |a - r| <= 1e-5 + 1e-4 |r| for every score, hidden coordinate and cache entry;
  mixed: |a - r| <= 0.002 (l+1) max(1, RMS(vector)) + 0.02 |r| per hidden / KV vector,
         complete per-layer state relative L2 <= 0.002; scores |a - r| <= 0.002 L + 0.02 |r|
         and RMS(score error) / max(1, RMS(scores)) <= 0.002 (docs/NumericalPolicy.md:5-20).
The tighter FP32 gate used by the GPU parity tests, |a - r| <= 1e-6 + 1e-5 |r|, is
:func:`fp32_strict_failures`.
"""
from __future__ import annotations

import numpy as np

POLICY = 'mixed-depth-rms-v3'


def residual_scale(reference) -> float:
    r = np.asarray(reference, dtype=np.float64)
    return max(1.0, float(np.sqrt(np.mean(r * r))))


def relative_l2(actual, reference) -> float:
    a, r = np.asarray(actual, np.float64), np.asarray(reference, np.float64)
    return float(np.sqrt(np.sum((a - r) ** 2) / max(1e-30, float(np.sum(r * r)))))


def mixed_state_scale(reference, layer: int) -> float:
    return (layer + 1) * residual_scale(reference)


def fp32_failures(actual, reference) -> int:
    a, r = np.asarray(actual, np.float64), np.asarray(reference, np.float64)
    bad = ~np.isfinite(a) | ~np.isfinite(r) | (np.abs(a - r) > 1e-5 + 1e-4 * np.abs(r))
    return int(np.count_nonzero(bad))


def fp32_strict_failures(actual, reference, atol: float = 1e-6, rtol: float = 1e-5) -> int:
    a, r = np.asarray(actual, np.float64), np.asarray(reference, np.float64)
    bad = ~np.isfinite(a) | ~np.isfinite(r) | (np.abs(a - r) > atol + rtol * np.abs(r))
    return int(np.count_nonzero(bad))


def state_errors(actual, reference, layer: int, mixed: bool = True) -> dict:
    """reference/numerical.py:13-26 over vectors along the last axis."""
    a, r = np.asarray(actual, np.float64), np.asarray(reference, np.float64)
    if a.shape != r.shape:
        raise ValueError('State tensor shapes differ')
    diff = np.abs(a - r)
    finite = np.isfinite(a) & np.isfinite(r)
    atol, rtol = (2e-3, 2e-2) if mixed else (1e-5, 1e-4)
    scale = ((layer + 1) * np.maximum(1, np.sqrt(np.mean(r * r, axis=-1, keepdims=True)))) if mixed else 1
    raw_failed = int(np.count_nonzero(~finite | (diff > atol + rtol * np.abs(r))))
    failed = int(np.count_nonzero(~finite | (diff > atol * scale + rtol * np.abs(r))))
    rel = float(np.linalg.norm(diff.ravel()) / max(1e-30, np.linalg.norm(r.ravel())))
    return dict(raw_failed=raw_failed, failed=failed, nonfinite=int((~finite).sum()),
                max_abs=float(diff.max()) if diff.size else 0.0, relative_l2=rel,
                passed=failed == 0 and (not mixed or rel <= .002))


def score_errors(actual, reference, layers: int) -> dict:
    """reference/numerical.py:29-37."""
    a, r = np.asarray(actual, np.float64), np.asarray(reference, np.float64)
    diff = np.abs(a - r)
    finite = np.isfinite(a) & np.isfinite(r)
    failed = int(np.count_nonzero(~finite | (diff > .002 * layers + .02 * np.abs(r))))
    rel = float(np.linalg.norm(diff) / max(1e-30, np.linalg.norm(r)))
    normalized = float(np.sqrt(np.mean(diff * diff)) / max(1., np.sqrt(np.mean(r * r))))
    return dict(failed=failed, max_abs=float(diff.max()), relative_l2=rel, normalized_rmse=normalized,
                passed=failed == 0 and normalized <= .002)


def mixed_state_passes(keys, values, hidden, ref_keys, ref_values, ref_hidden) -> dict:
    """v3 gate for one snapshot: per-layer K/V caches ([L,H,W,dh]) and hidden ([L,width])."""
    out = dict(passed=True, failures=[])
    for layer in range(ref_hidden.shape[0]):
        for name, a, r in (('keys', keys[layer], ref_keys[layer]), ('values', values[layer], ref_values[layer]),
                           ('hidden', hidden[layer], ref_hidden[layer])):
            res = state_errors(a, r, layer, mixed=True)
            if not res['passed']:
                out['passed'] = False
                out['failures'].append((name, layer, res))
    return out

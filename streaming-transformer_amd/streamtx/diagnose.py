"""Per-operation diagnosis: read, write and compare the reference's diagnostic archives.

An archive (bench/Diagnose.cpp:38-62) is a directory with
  stages.bin     float32, event-major: every event's trace entries back to back, the entries
                 in the order of their names;
  manifest.json  version 1, dtype, layout "event_major", events, event_elements, stages
                 [{name, offset_elements, elements}], backend, checkpoint_sha256, trace_sha256,
                 resets, sha256 of stages.bin (and compiler / provenance).
`stream-diagnose` writes one for the GPU's staged backend; the test oracle writes one with
the same entry names (oracle/stage_archive.py). `compare` diffs two archives operation by
operation, after scripts/diagnose_native.py:31-140:
  - per stage, the elements over the bar (FP32: 1e-5 + 1e-4|e|; mixed: 2e-3 + 2e-2|e|, and the
    v3 bar, whose absolute term scales by the depth (layer + 1 in a layer, the layer count for
    the final norm and score) times max(1, RMS of the expected vector)),
    the largest difference, relative L2 and absolute-difference quantiles;
  - the first divergence in execution order (event, stage, coordinate): the earliest cast
    boundary at which the two runs part;
  - isolated checks on the first archive's own operands, which remove upstream drift: every
    projection's pre-cast output against its FP64 product within the conservative FP32 dot
    bound gamma(2n) * sum|x w| (docs/NumericalDiagnosis.md:23), and its output against the
    cast of its own pre-cast value (in mixed mode also how often that differs from rounding
    the exact product); every norm against its FP64 value; SwiGLU and the two residual adds
    against their exact values at the cast.
Usage: python -m streamtx.diagnose ACTUAL_DIR EXPECTED_DIR --weights CHECKPOINT_DIR [--output report.json]
"""
from __future__ import annotations

import argparse
import hashlib
import json
from pathlib import Path

import numpy as np

from .model import load_checkpoint


def read_archive(directory) -> tuple[dict, dict]:
    """(manifest, {stage name: float32 array [events, elements]}), hash-checked."""
    directory = Path(directory)
    manifest = json.loads((directory / 'manifest.json').read_text())
    raw = (directory / 'stages.bin').read_bytes()
    if hashlib.sha256(raw).hexdigest() != manifest['sha256']:
        raise ValueError(f'{directory}: stages.bin does not match its manifest hash')
    if manifest.get('layout') != 'event_major' or manifest.get('dtype') != 'float32':
        raise ValueError(f'{directory}: unsupported archive layout')
    events, width = manifest['events'], manifest['event_elements']
    if len(raw) != 4 * events * width:
        raise ValueError(f'{directory}: stages.bin holds {len(raw)} bytes, expected {4 * events * width}')
    data = np.frombuffer(raw, dtype='<f4').reshape(events, width)
    stages = {s['name']: data[:, s['offset_elements']:s['offset_elements'] + s['elements']] for s in manifest['stages']}
    return manifest, stages


def write_archive(directory, events, *, backend, checkpoint_sha256, trace_sha256, resets, provenance=None) -> Path:
    """Write an archive from an iterable of per-event {name: vector} traces (all events with
    the same entries), stages in name order."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    digest = hashlib.sha256()
    layout, count, width = None, 0, 0
    with open(directory / 'stages.bin', 'wb') as out:
        for trace in events:
            names = sorted(trace)
            if layout is None:
                layout, offset = [], 0
                for n in names:
                    layout.append(dict(name=n, offset_elements=offset, elements=int(np.size(trace[n]))))
                    offset += int(np.size(trace[n]))
                width = offset
            elif [s['name'] for s in layout] != names:
                raise ValueError('trace entries changed between events')
            blob = b''.join(np.ascontiguousarray(trace[n], dtype='<f4').tobytes() for n in names)
            if len(blob) != 4 * width:
                raise ValueError('trace entry sizes changed between events')
            out.write(blob)
            digest.update(blob)
            count += 1
    manifest = dict(version=1, dtype='float32', layout='event_major', events=count, event_elements=width,
                    stages=layout or [], backend=backend, checkpoint_sha256=checkpoint_sha256,
                    trace_sha256=trace_sha256, resets=list(resets), provenance=provenance or {},
                    sha256=digest.hexdigest())
    (directory / 'manifest.json').write_text(json.dumps(manifest, indent=2) + '\n')
    return directory


def execution_order(layers: int) -> list[str]:
    """The trace entries in the order a step produces them (Cpu::step, src/cpu/Cpu.cpp:59-141)."""
    def linear(n):
        return [f'{n}.operand', f'{n}.pre_cast', f'{n}.linear']

    def norm(n):
        return [f'{n}.operand', f'{n}.pre_cast', f'{n}.norm']

    order = linear('input') + ['input']
    for l in range(layers):
        p = f'layers.{l}.'
        order += norm(p + 'norm1') + linear(p + 'q') + linear(p + 'k') + linear(p + 'v')
        order += [p + 'q', p + 'k', p + 'v', p + 'attention'] + linear(p + 'out') + [p + 'attention_residual']
        order += norm(p + 'norm2') + linear(p + 'gate') + linear(p + 'up') + [p + 'activation']
        order += linear(p + 'down') + [p + 'hidden']
    return order + norm('final_norm') + linear('score')


def _depth(name: str, layers: int) -> int:
    """The v3 policy's depth factor of a stage: layer + 1 inside layer `layer`, 1 for the input
    projection, `layers` for the final norm and the score (whose policy atol is 0.002 * layers)."""
    if name.startswith('layers.'):
        return int(name.split('.')[1]) + 1
    return 1 if name.startswith('input') else layers


def summarize(actual, expected, mixed: bool, depth: int = 1, v3: bool = False) -> dict:
    """Elements over the bar and error statistics of one stage ([events, n] arrays)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    diff = np.abs(a - e)
    atol = np.full((e.shape[0], 1), 2e-3 if mixed else 1e-5)
    if mixed and v3:
        rms = np.sqrt(np.mean(e * e, axis=1, keepdims=True))
        atol = 2e-3 * depth * np.maximum(1.0, rms)
    bound = atol + (2e-2 if mixed else 1e-4) * np.abs(e)
    finite = np.isfinite(a) & np.isfinite(e)
    bad = ~finite | (diff > bound)
    diff = np.where(finite, diff, np.inf)
    examples = [dict(event=int(i), coordinate=int(j), actual=float(a[i, j]), expected=float(e[i, j]),
                     difference=float(diff[i, j])) for i, j in np.argwhere(bad)[:8]]
    fin = diff[np.isfinite(diff)]
    return dict(elements=int(diff.size), failed=int(bad.sum()), nonfinite=int((~finite).sum()),
                max_abs=float(fin.max()) if fin.size else 0.0,
                relative_l2=float(np.linalg.norm(fin) / max(1e-30, np.linalg.norm(e[finite]))),
                absolute_quantiles=np.quantile(fin, [.5, .95, .99, .999, 1]).tolist() if fin.size else [],
                examples=examples)


def first_divergence(actual: dict, expected: dict, order: list[str]) -> dict | None:
    """Earliest (event, stage in execution order, coordinate) whose values differ at all."""
    events = next(iter(actual.values())).shape[0]
    for i in range(events):
        for name in order:
            if name not in actual or name not in expected:
                continue
            changed = np.flatnonzero(actual[name][i] != expected[name][i])
            if changed.size:
                j = int(changed[0])
                return dict(event=i, stage=name, coordinate=j, actual=float(actual[name][i, j]),
                            expected=float(expected[name][i, j]))
    return None


def _round_half(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def isolated_checks(stages: dict, weights: dict, config, mixed: bool) -> dict:
    """Each operation recomputed in FP64 from the archive's own operands (removing upstream
    drift): projections against the FP32 dot bound and their cast; norms, SwiGLU and the
    residual adds against their exact values (scripts/diagnose_native.py:86-128)."""
    u = np.finfo(np.float32).eps / 2
    linear, nonlinear = {}, {}
    for name, w in weights.items():
        w = np.asarray(w, np.float64)
        if w.ndim != 2 or name + '.operand' not in stages:
            continue
        x = stages[name + '.operand'].astype(np.float64)
        exact = x @ w.T
        n = 2 * x.shape[1]
        gamma = n * u / (1 - n * u)
        bound = gamma * (np.abs(x) @ np.abs(w).T)
        pre = stages[name + '.pre_cast'].astype(np.float64)
        diff = np.abs(pre - exact)
        out = stages[name + '.linear'].astype(np.float64)
        rounds = mixed and name != 'score'  # the score is never cast
        entry = dict(max_pre_cast_abs=float(diff.max()), fp32_dot_bound_violations=int((diff > bound).sum()),
                     max_fraction_of_dot_bound=float(np.max(diff / np.maximum(bound, 1e-30))),
                     # the cast itself: the output is the pre-cast value, rounded to FP16 in mixed mode
                     cast_mismatches=int(np.count_nonzero(out != (_round_half(pre) if rounds else pre))))
        if rounds:
            # legitimate: an FP32 sum on the other side of an FP16 rounding midpoint from the
            # exact product (docs/NumericalDiagnosis.md:9-21)
            entry['cast_differs_from_exact_rounding'] = int(np.count_nonzero(out != _round_half(exact)))
        linear[name] = entry
    for name, w in weights.items():
        w = np.asarray(w, np.float64)
        if w.ndim != 1 or name + '.operand' not in stages:
            continue
        x = stages[name + '.operand'].astype(np.float64)
        exact = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + config.epsilon) * w
        nonlinear[name] = summarize(stages[name + '.pre_cast'], exact, False)
    for layer in range(config.layers):
        p = f'layers.{layer}.'
        gate = stages[p + 'gate.linear'].astype(np.float64)
        up = stages[p + 'up.linear'].astype(np.float64)
        act = gate / (1 + np.exp(-gate)) * up
        nonlinear[p + 'activation'] = summarize(stages[p + 'activation'], _round_half(act) if mixed else act, mixed)
        prior = stages['input'] if layer == 0 else stages[f'layers.{layer - 1}.hidden']
        for target, lhs, rhs in (('attention_residual', prior, stages[p + 'out.linear']),
                                 ('hidden', stages[p + 'attention_residual'], stages[p + 'down.linear'])):
            exact = lhs.astype(np.float64) + rhs
            nonlinear[p + target] = summarize(stages[p + target], _round_half(exact) if mixed else exact, mixed)
    return dict(linear=linear, nonlinear=nonlinear)


def compare(actual_dir, expected_dir, weights_dir) -> dict:
    """Diff two archives of the same fixture operation by operation (see the module doc)."""
    ma, actual = read_archive(actual_dir)
    me, expected = read_archive(expected_dir)
    ck = load_checkpoint(weights_dir)
    for key in ('checkpoint_sha256', 'trace_sha256', 'events', 'resets'):
        if ma[key] != me[key]:
            raise ValueError(f'archives differ in {key}: {ma[key]} vs {me[key]}')
    if ma['checkpoint_sha256'] != ck.manifest['sha256']:
        raise ValueError('archives were not written from this checkpoint')
    if sorted(actual) != sorted(expected):
        raise ValueError('archives hold different stages')
    mixed = ck.mixed
    order = execution_order(ck.config.layers)
    stages = {}
    for name in order:
        if name in actual:
            stages[name] = summarize(actual[name], expected[name], mixed)
            if mixed:
                stages[name]['v3'] = summarize(actual[name], expected[name], True, _depth(name, ck.config.layers),
                                               v3=True)
    report = dict(actual=dict(backend=ma['backend'], sha256=ma['sha256']),
                  expected=dict(backend=me['backend'], sha256=me['sha256']),
                  checkpoint_sha256=ck.manifest['sha256'], mode='mixed' if mixed else 'fp32', events=ma['events'],
                  resets=ma['resets'], stages=stages, first_divergence=first_divergence(actual, expected, order),
                  isolated=isolated_checks(actual, ck.tensors, ck.config, mixed),
                  timing='diagnostic operation snapshots; excluded from performance evidence')
    failed = [n for n, s in stages.items() if (s['v3']['failed'] if mixed else s['failed'])]
    report['stages_over_bar'] = failed
    return report


def main() -> None:
    parser = argparse.ArgumentParser(description='Diff two per-operation diagnostic archives.')
    parser.add_argument('actual')
    parser.add_argument('expected')
    parser.add_argument('--weights', required=True, help='checkpoint directory both archives were written from')
    parser.add_argument('--output', help='write the report as JSON here')
    a = parser.parse_args()
    report = compare(a.actual, a.expected, a.weights)
    text = json.dumps(report, indent=2)
    if a.output:
        Path(a.output).write_text(text + '\n')
    print(json.dumps(dict(stages_over_bar=report['stages_over_bar'], first_divergence=report['first_divergence'])))


if __name__ == '__main__':
    main()

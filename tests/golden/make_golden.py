"""Copy the reference's golden fixtures into compact, verified test fixtures.

Reads the reference checkout (default /root/reference) as data only: nothing
there is imported or executed. For fixtures/small-{fp32,mixed} (the only
fixtures with expected outputs, written by reference/export.py:46-70) it keeps

  checkpoint/manifest.json + tensors.bin   the checkpoint, byte for byte
  trace.bin, resets.json                  the 201-event trace and reset schedule
  expected.npz                            scores[E], hidden[E,L,d],
                                          key_rows/value_rows[E,L,H,dh]

The reference stores the full K/V cache after every event ([E,L,H,W,dh], 6.6 MB
per fixture). Each event writes exactly one ring slot per layer and head
(src/cpu/Cpu.cpp:91-96; reference/model.py:124-125), so the full cache after
event i is determined by the rows written since the last reset. This script
keeps those rows and checks, for every event, that rebuilding the cache from
them reproduces the reference's full tensor bit for bit before writing.

For fixtures/main-{fp32,mixed} and fixtures/large-{fp32,mixed} (checkpoint and
trace, no expected outputs) only the checkpoint, trace and reset schedule are kept.

The 30 window variants fixtures/{small,main,large}-w{32,64,128,256,512}-{fp32,mixed}
hold the same weights as their base checkpoint (scripts/prepare_windows.py:20-23
refuses any other); only the config's window, the 3W+9-event trace and the reset
schedule differ. They are kept as windows/<name>/{manifest.json, trace.bin,
resets.json}, after checking that the variant's tensors.bin is the base's byte for
byte; tests/harness_layout.py rebuilds each variant from its base checkpoint.

Usage: python tests/golden/make_golden.py [--reference /root/reference]
"""
import argparse
import hashlib
import json
import shutil
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def sha256(raw):
    return hashlib.sha256(raw).hexdigest()


def read_archive(directory):
    manifest = json.loads((directory / 'manifest.json').read_text())
    raw = (directory / 'tensors.bin').read_bytes()
    if sha256(raw) != manifest['sha256']:
        raise ValueError(f'archive hash mismatch: {directory}')
    tensors = {}
    for t in manifest['tensors']:
        part = raw[t['offset']:t['offset'] + t['nbytes']]
        if sha256(part) != t['sha256']:
            raise ValueError(f'tensor hash mismatch: {directory} {t["name"]}')
        dtype = {'float32': '<f4', 'float16': '<f2'}[t['dtype']]
        tensors[t['name']] = np.frombuffer(part, dtype=dtype).reshape(t['shape'])
    return manifest, tensors


def rebuild_cache(rows, resets, window):
    """Full cache after each event from the per-event written rows."""
    events, layers, heads, dim = rows.shape
    cache = np.zeros((layers, heads, window, dim), dtype=rows.dtype)
    position = 0
    for i in range(events):
        if i in resets:
            cache[:] = 0
            position = 0
        cache[:, :, position % window] = rows[i]
        position += 1
        yield cache


def compact(source, target):
    manifest, expected = read_archive(source / 'expected')
    config = manifest['config']
    resets = set(json.loads((source / 'resets.json').read_text()))
    if sorted(resets) != manifest['resets']:
        raise ValueError('reset schedule differs from expected manifest')
    window = config['window']
    keys, values = expected['keys'], expected['values']
    events = keys.shape[0]
    key_rows = np.empty(keys.shape[:3] + keys.shape[4:], dtype=np.float32)
    value_rows = np.empty_like(key_rows)
    position = 0
    for i in range(events):
        if i in resets:
            position = 0
        key_rows[i] = keys[i][:, :, position % window]
        value_rows[i] = values[i][:, :, position % window]
        position += 1
    for name, rows, full in (('keys', key_rows, keys), ('values', value_rows, values)):
        for i, cache in enumerate(rebuild_cache(rows, resets, window)):
            if not np.array_equal(cache, full[i]):
                raise ValueError(f'{name} at event {i} is not reproduced by its written rows')
    trace = (source / 'trace.bin').read_bytes()
    events_tensor = next(t for t in manifest['tensors'] if t['name'] == 'events')
    if sha256(trace) != events_tensor['sha256']:
        raise ValueError('trace does not match expected events')
    target.mkdir(parents=True, exist_ok=True)
    np.savez(target / 'expected.npz', scores=expected['scores'].astype(np.float32),
             hidden=expected['hidden'].astype(np.float32), key_rows=key_rows, value_rows=value_rows,
             resets=np.array(sorted(resets), dtype=np.int64))
    provenance = dict(source=f'fixtures/{source.name}/expected', expected_sha256=manifest['sha256'],
                      config=config, mode=manifest['mode'], events=int(events),
                      note='key_rows/value_rows[i] = cache slot written by event i; '
                           'full cache rebuilt and compared bit for bit with the source')
    (target / 'expected.json').write_text(json.dumps(provenance, indent=2) + '\n')


def copy_checkpoint(source, target):
    read_archive(source)  # verifies every hash before copying
    (target / 'checkpoint').mkdir(parents=True, exist_ok=True)
    for name in ('manifest.json', 'tensors.bin'):
        shutil.copyfile(source / name, target / 'checkpoint' / name)
    for name in ('trace.bin', 'resets.json'):
        shutil.copyfile(source / name, target / name)


def copy_window_variant(source, base, target):
    """A window variant: its manifest, trace and resets; its tensors must be the base's."""
    manifest, _ = read_archive(source)  # verifies every hash
    base_manifest = json.loads((base / 'manifest.json').read_text())
    if (source / 'tensors.bin').read_bytes() != (base / 'tensors.bin').read_bytes() or \
            manifest['sha256'] != base_manifest['sha256']:
        raise ValueError(f'{source.name}: weights differ from {base.name}')
    config = manifest['config']
    if {k: v for k, v in config.items() if k != 'window'} != \
            {k: v for k, v in base_manifest['config'].items() if k != 'window'}:
        raise ValueError(f'{source.name}: config differs from {base.name} beyond the window')
    trace = (source / 'trace.bin').read_bytes()
    if len(trace) != 4 * config['features'] * (3 * config['window'] + 9):
        raise ValueError(f'{source.name}: trace is not 3W+9 events')
    target.mkdir(parents=True, exist_ok=True)
    for name in ('manifest.json', 'trace.bin', 'resets.json'):
        shutil.copyfile(source / name, target / name)


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument('--reference', type=Path, default=Path('/root/reference'))
    args = parser.parse_args()
    fixtures = args.reference / 'fixtures'
    for name in ('small-fp32', 'small-mixed'):
        copy_checkpoint(fixtures / name, HERE / name)
        compact(fixtures / name, HERE / name)
        print('wrote', HERE / name)
    for name in ('main-fp32', 'main-mixed', 'large-fp32', 'large-mixed'):
        copy_checkpoint(fixtures / name, HERE / name)
        print('wrote', HERE / name)
    for size in ('small', 'main', 'large'):
        for window in (32, 64, 128, 256, 512):
            for mode in ('fp32', 'mixed'):
                name = f'{size}-w{window}-{mode}'
                copy_window_variant(fixtures / name, fixtures / f'{size}-{mode}', HERE / 'windows' / name)
        print('wrote', HERE / 'windows', size)


if __name__ == '__main__':
    main()

"""The reference's fixture families, pinned on the CPU before the GPU validation matrix uses
them (tests/test_validation_matrix_gpu.py).

  - the input-family generator (tests/harness_layout.adversarial_trace, restating
    reference/export.py:12-28) reproduces, for kind 'random', the trace.bin of every one of the
    reference's 36 fixtures byte for byte, and each fixture's reset schedule is [2W + 3];
  - the other families have their defining properties (zeros, constant 0.25, impulses every
    17th event, alternating signs, a period of 7);
  - every window variant rebuilt from its base checkpoint has the checkpoint's hash, its
    config differs from the base only in the window, and its trace is 3W + 9 events;
  - the oracle steps every window variant through its fixture trace with the reset, and the
    zero-input family gives a score of exactly 0 at every event (tests/Lifecycle.cu:38,60-62).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from harness_layout import GOLDEN, adversarial_trace, window_fixture
from oracle.pyoracle import Oracle
from streamtx import load_checkpoint

SIZES = ('small', 'main', 'large')
WINDOWS = (32, 64, 128, 256, 512)
KINDS = ('zeros', 'constant', 'impulses', 'alternating', 'repeated')


def all_fixtures():
    out = []
    for size in SIZES:
        for mode in ('fp32', 'mixed'):
            out.append((GOLDEN / f'{size}-{mode}', f'{size}-{mode}', True))
            for w in WINDOWS:
                out.append((GOLDEN / 'windows' / f'{size}-w{w}-{mode}', f'{size}-w{w}-{mode}', False))
    return out


@pytest.mark.parametrize('directory,name,base', all_fixtures(), ids=lambda v: v if isinstance(v, str) else '')
def test_random_family_reproduces_every_fixture_trace(directory, name, base):
    manifest = json.loads((directory / ('checkpoint/manifest.json' if base else 'manifest.json')).read_text())
    c = manifest['config']
    raw = (directory / 'trace.bin').read_bytes()
    count = len(raw) // (4 * c['features'])
    assert count == 3 * c['window'] + 9 or name.startswith('small-') and base  # small: 201 = 3 * 64 + 9
    assert raw == adversarial_trace(count, c['features'], 'random').tobytes()
    assert json.loads((directory / 'resets.json').read_text()) == [2 * c['window'] + 3]


def test_family_properties():
    n, f = 3 * 64 + 9, 32
    assert not adversarial_trace(n, f, 'zeros').any()
    assert (adversarial_trace(n, f, 'constant') == np.float32(0.25)).all()
    imp = adversarial_trace(n, f, 'impulses')
    assert imp.sum() == len(range(0, n, 17)) and (imp[::17, 0] == 1).all()
    alt = adversarial_trace(n, f, 'alternating')
    assert (alt[0::2] == 1).all() and (alt[1::2] == -1).all()
    rep = adversarial_trace(n, f, 'repeated')
    assert (rep[7:] == rep[:-7]).all() and len({r.tobytes() for r in rep}) == 7


@pytest.mark.parametrize('size', SIZES)
def test_window_variants_share_their_base_weights(tmp_path, size):
    for mode in ('fp32', 'mixed'):
        base = load_checkpoint(GOLDEN / f'{size}-{mode}' / 'checkpoint')
        for w in WINDOWS:
            weights, config = window_fixture(f'{size}-w{w}-{mode}', tmp_path / f'{size}-w{w}-{mode}')
            ck = load_checkpoint(weights)  # verifies the archive and tensor hashes
            assert ck.manifest['sha256'] == base.manifest['sha256'] and ck.mixed == base.mixed
            assert ck.config.window == w
            assert {k: v for k, v in ck.manifest['config'].items() if k != 'window'} == \
                {k: v for k, v in base.manifest['config'].items() if k != 'window'}
            assert json.loads(config.read_text()) == ck.manifest['config']


@pytest.mark.parametrize('size', SIZES)
def test_oracle_runs_window_variants_and_zero_family(tmp_path, size):
    for w in (32, 512):
        weights, _ = window_fixture(f'{size}-w{w}-fp32', tmp_path / f'w{w}')
        ck = load_checkpoint(weights)
        c = ck.config
        events = np.fromfile(weights / 'trace.bin', dtype='<f4').reshape(-1, c.features)
        oracle = Oracle(c, ck.tensors, threads=4)
        scores = []
        for i, e in enumerate(events):
            if i == 2 * w + 3:
                oracle.reset()
                assert oracle.position == 0
            scores.append(oracle.step(e))
        assert np.isfinite(scores).all() and oracle.position == len(events) - (2 * w + 3)
        zero = Oracle(c, ck.tensors)
        assert all(zero.step(e) == 0.0 for e in adversarial_trace(3 * w + 9, c.features, 'zeros'))

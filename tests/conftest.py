import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / 'streaming-transformer_amd'):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = Path(__file__).resolve().parent / 'golden'


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) GPU and the built libstamd.so')


class Golden:
    """One of the reference's golden fixtures (compact form, see tests/golden/make_golden.py)."""

    def __init__(self, name):
        from streamtx import load_checkpoint
        self.path = GOLDEN / name
        self.checkpoint = load_checkpoint(self.path / 'checkpoint')
        self.config = self.checkpoint.config
        self.trace = np.fromfile(self.path / 'trace.bin', dtype='<f4').reshape(-1, self.config.features)
        self.resets = set(json.loads((self.path / 'resets.json').read_text()))
        exp = self.path / 'expected.npz'
        self.expected = dict(np.load(exp)) if exp.exists() else None

    def expected_state(self):
        """Yield (event, score, keys[L,H,W,dh], values, hidden[L,d]) rebuilding the full cache
        from the rows written by each event."""
        e = self.expected
        c = self.config
        keys = np.zeros((c.layers, c.heads, c.window, c.dim), dtype=np.float32)
        values = np.zeros_like(keys)
        position = 0
        for i in range(len(e['scores'])):
            if i in self.resets:
                keys[:] = 0
                values[:] = 0
                position = 0
            keys[:, :, position % c.window] = e['key_rows'][i]
            values[:, :, position % c.window] = e['value_rows'][i]
            position += 1
            yield i, e['scores'][i], keys, values, e['hidden'][i]


@pytest.fixture(scope='session')
def golden():
    cache = {}

    def get(name):
        if name not in cache:
            cache[name] = Golden(name)
        return cache[name]
    return get

"""The oracle's per-operation diagnostic archive of a fixture.

TEST INFRASTRUCTURE ONLY (like everything under oracle/): it writes, from the C oracle's trace
mode (so_step_trace, the reference's CpuTrace of src/cpu/Cpu.cpp:29-57,64-66,86-133), the same
archive that the reference's `stream-diagnose FIXTURE OUTPUT cpu` writes (bench/Diagnose.cpp:
12-68): every event of the fixture's trace.bin, resets from its resets.json, the entries of each
event in name order in stages.bin, and manifest.json. `stream-diagnose` writes the GPU's archive
of the same fixture; streamtx.diagnose compares the two.

Usage: python oracle/stage_archive.py FIXTURE OUTPUT_DIRECTORY [--accumulate float|double]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
for p in (HERE.parent, HERE.parent / 'streaming-transformer_amd'):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

from oracle.pyoracle import Oracle  # noqa: E402
from streamtx.diagnose import write_archive  # noqa: E402
from streamtx.model import load_checkpoint  # noqa: E402


def write(fixture, output, accumulate='float', events=None) -> Path:
    """Trace the fixture's events (the first `events` of them, default all) through the oracle
    and write the archive."""
    fixture = Path(fixture)
    ck = load_checkpoint(fixture)
    c = ck.config
    raw = (fixture / 'trace.bin').read_bytes()
    frames = np.frombuffer(raw, dtype='<f4').reshape(-1, c.features)
    if events is not None:
        frames = frames[:events]
    resets = json.loads((fixture / 'resets.json').read_text())
    oracle = Oracle(c, ck.tensors, mixed=ck.mixed, accumulate=accumulate)

    def traces():
        for i, event in enumerate(frames):
            if i in resets:
                oracle.reset()
            yield oracle.trace_step(event)[1]

    return write_archive(output, traces(), backend=f'oracle ({accumulate} accumulation)',
                         checkpoint_sha256=ck.manifest['sha256'], trace_sha256=hashlib.sha256(raw).hexdigest(),
                         resets=resets, provenance=dict(writer='oracle/stage_archive.py',
                                                        oracle='oracle/stream_oracle.c so_step_trace'))


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument('fixture')
    parser.add_argument('output')
    parser.add_argument('--accumulate', choices=('float', 'double'), default='float')
    a = parser.parse_args()
    print(write(a.fixture, a.output, a.accumulate))


if __name__ == '__main__':
    main()

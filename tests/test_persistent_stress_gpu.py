"""Stress of the persistent mailbox worker (the reference's 1M-command validation,
scripts/validate.py:55-74: reset every 10007 events, snapshots every 4096).

50,000 commands by default (about 40 s with the fused replay and the oracle); the full
1,000,000 when STAMD_STRESS_EVENTS is set to it (about 7 minutes on one MI355X).
Main architecture with bfloat16 weights, one stream, inputs from seed 4. Checks:
  - ordering: every score and every 4096-event snapshot of the persistent worker is
    bit-identical to the fused backend fed the same events with the same resets (a lost,
    repeated or reordered command would change the carried state);
  - the last snapshot against the FP64-accumulating oracle replayed from the last reset;
  - per-command host latency percentiles, printed.
"""
import hashlib
import os
import time

import numpy as np
import pytest

from oracle.pyoracle import Oracle
from streamtx import Backend, ModelConfig, Runtime, RuntimeOptions, WeightStorage, numerical, round_bf16, \
    synthetic_checkpoint

pytestmark = pytest.mark.gpu

EVENTS = int(os.environ.get('STAMD_STRESS_EVENTS', '50000'))
RESET_EVERY = 10007
SNAPSHOT_EVERY = 4096
CHUNK = 8192
STRICT = dict(atol=1e-6, rtol=1e-5)


def _chunks(config, total):
    """The same event sequence on every call: seed 4, CHUNK rows at a time."""
    rng = np.random.default_rng(4)
    for start in range(0, total, CHUNK):
        yield start, rng.standard_normal((min(CHUNK, total - start), config.features), dtype=np.float32)


def _digest(snapshot):
    h = hashlib.blake2b(digest_size=16)
    h.update(np.uint64(snapshot[0]).tobytes())
    for a in snapshot[1:]:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _drive(rt, config, total, latencies=None):
    scores = np.empty(total, dtype=np.float32)
    digests = []
    for start, chunk in _chunks(config, total):
        for j, e in enumerate(chunk):
            i = start + j
            if i and i % RESET_EVERY == 0:
                rt.reset()
            t0 = time.perf_counter()
            scores[i] = rt.step(e)
            if latencies is not None:
                latencies[i] = time.perf_counter() - t0
            if (i + 1) % SNAPSHOT_EVERY == 0:
                digests.append(_digest(rt.snapshot()))
        if (start // CHUNK) % 16 == 15:
            print(f'[stress] {start + len(chunk)} events', flush=True)
    return scores, digests


def test_persistent_commands_ordering():
    c = ModelConfig(8, 512, 8, 2048, 128, 512)
    w = synthetic_checkpoint(c, seed=4)
    bf16 = WeightStorage.BF16
    print(f'[case] persistent stress events={EVENTS} reset_every={RESET_EVERY}', flush=True)
    latencies = np.empty(EVENTS, dtype=np.float64)
    with Runtime((c, w, False), RuntimeOptions(backend=Backend.PERSISTENT, blocks=0, weight_dtype=bf16,
                                               idle_seconds=60.0)) as rt:
        scores, digests = _drive(rt, c, EVENTS, latencies)
        last = rt.snapshot()
        rt.stop()
    us = latencies * 1e6
    print('[stress] persistent per-command host latency us: p50 %.1f p99 %.1f p99.9 %.1f max %.1f' %
          (np.percentile(us, 50), np.percentile(us, 99), np.percentile(us, 99.9), us.max()), flush=True)

    print('[case] fused replay', flush=True)
    with Runtime((c, w, False), RuntimeOptions(backend=Backend.FUSED, blocks=0, weight_dtype=bf16)) as rt:
        ref_scores, ref_digests = _drive(rt, c, EVENTS)
        ref_last = rt.snapshot()
    mismatch = np.flatnonzero(scores.view(np.uint32) != ref_scores.view(np.uint32))
    assert mismatch.size == 0, f'first differing score at event {mismatch[0]}'
    assert digests == ref_digests
    assert _digest(last) == _digest(ref_last)

    # The oracle from the last reset to the end (the state depends only on that segment).
    reset_at = (EVENTS - 1) // RESET_EVERY * RESET_EVERY
    oracle = Oracle(c, {k: round_bf16(v) for k, v in w.items()}, accumulate='double', threads=16)
    for start, chunk in _chunks(c, EVENTS):
        for j, e in enumerate(chunk):
            if start + j >= reset_at:
                got = oracle.step(e)
                assert numerical.fp32_strict_failures([scores[start + j]], [got], **STRICT) == 0, start + j
    opos, ok, ov, oh = oracle.snapshot()
    assert last[0] == opos == EVENTS - reset_at
    for a, o in zip(last[1:], (ok, ov, oh)):
        assert numerical.fp32_strict_failures(a, o, **STRICT) == 0, float(np.abs(a - o).max())

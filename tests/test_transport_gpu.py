"""Transport microbenchmarks (Stream::transportBench, src/cuda/Runtime.cu:703-814): every mode
completes its round trips with no checksum failure and writes one CSV row per sample."""
import csv

import pytest

from streamtx import transport_bench

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('mode', ['ping-pong', 'gpu-ping', 'empty', 'empty-graph', 'copy'])
@pytest.mark.parametrize('backoff', [False, True])
def test_transport_modes(tmp_path, mode, backoff):
    print(f'[case] transport mode={mode} backoff={backoff}', flush=True)
    out = tmp_path / f'{mode}.csv'
    report = transport_bench(mode, 300, backoff, str(out))
    assert report['mode'] == mode and report['events'] == 300 and report['failed'] == 0
    assert 0 < report['p50_us'] <= report['p99_us'] <= report['worst_us']
    rows = list(csv.reader(out.open()))
    assert rows[0] == ['sequence', 'host_observation_us', 'device_round_trip_or_wait_cycles'] and len(rows) == 301
    if mode in ('ping-pong', 'gpu-ping'):
        assert all(float(r[2]) > 0 for r in rows[1:])

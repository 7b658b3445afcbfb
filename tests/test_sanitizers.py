"""Host code under the compiler's sanitizers, on the CPU (no GPU: the device side of the
persistent mailbox is a host thread that follows the worker's protocol).

  - the mailbox protocol (streaming-transformer_amd/csrc/mailbox.hpp, the runtime's own host
    half, against the host-thread worker of tests/mailbox_selftest.cpp): commands in order, STOP
    twice, a finite RUN budget, an idle exit, a worker that never answers, a launch that ends
    without answering, the watchdog word and the last sequence IDs; built plain, with
    AddressSanitizer + UndefinedBehaviorSanitizer and with ThreadSanitizer;
  - the driver's JSON parser, SHA-256 and checks (harness_selftest) and 50,000 randomly
    mutated JSON documents, under AddressSanitizer + UndefinedBehaviorSanitizer;
  - the whole benchmark driver under AddressSanitizer + UndefinedBehaviorSanitizer over the CPU
    stand-in runtime (the checkpoint reader with intact and corrupted checkpoints, the
    expected-output archives, correctness and scheduled modes), and its scheduled
    producer/consumer queue under ThreadSanitizer.
A sanitizer report makes the program exit nonzero (-fno-sanitize-recover=all, halt_on_error).
"""
import os
import subprocess
from pathlib import Path

import pytest

from harness_layout import reference_fixture

ROOT = Path(__file__).resolve().parent.parent
OUT = ROOT / 'tests' / '_build' / 'sanitizers'
INCLUDES = [f'-I{ROOT / "include"}', f'-I{ROOT / "streaming-transformer_amd" / "csrc"}',
            f'-I{ROOT / "streaming-transformer_amd" / "harness"}']
FLAVOURS = {
    'plain': [],
    'asan': ['-fsanitize=address,undefined', '-fno-sanitize-recover=all', '-fno-omit-frame-pointer'],
    'tsan': ['-fsanitize=thread'],
}
ENV = dict(os.environ, ASAN_OPTIONS='halt_on_error=1:detect_leaks=1', UBSAN_OPTIONS='halt_on_error=1:print_stacktrace=1',
           TSAN_OPTIONS='halt_on_error=1:second_deadlock_stack=1')


def build(source, flavour, name, extra=()):
    OUT.mkdir(parents=True, exist_ok=True)
    exe = OUT / f'{name}-{flavour}'
    cmd = ['g++', '-O1', '-g', '-std=c++17', '-Wall', '-Wextra', *FLAVOURS[flavour], *INCLUDES, '-o', str(exe),
           str(source), *extra, '-pthread']
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def sanitizer_runs(flavour):
    """ThreadSanitizer needs a usable address-space layout; skip (with the reason) where the
    kernel's layout makes its runtime refuse to start."""
    probe = build(ROOT / 'tests' / 'mailbox_selftest.cpp', flavour, 'probe')
    r = subprocess.run([str(probe)], capture_output=True, text=True, env=ENV, timeout=120)
    if flavour == 'tsan' and 'unexpected memory mapping' in r.stderr:
        pytest.skip('ThreadSanitizer cannot run under this kernel memory layout: ' + r.stderr.strip()[:200])
    return r


@pytest.mark.parametrize('flavour', ['plain', 'asan', 'tsan'])
def test_mailbox_protocol(flavour):
    r = sanitizer_runs(flavour)
    assert r.returncode == 0 and 'OK: 0 failure(s)' in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


def test_json_and_selftest_under_asan():
    exe = build(ROOT / 'tests' / 'harness_selftest.cpp', 'asan', 'harness_selftest')
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=ENV, timeout=120)
    assert r.returncode == 0 and 'OK: 0 failure(s)' in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]
    r = subprocess.run([str(exe), 'fuzz', '50000'], capture_output=True, text=True, env=ENV, timeout=300)
    assert r.returncode == 0 and 'fuzz: 50000 rounds' in r.stdout, r.stderr[-4000:]


@pytest.fixture(scope='module')
def stand_in():
    from harness_layout import build_stand_in
    return build_stand_in()


def driver(flavour, stand_in):
    return build(ROOT / 'streaming-transformer_amd' / 'harness' / 'stream_bench.cpp', flavour, 'stream-bench',
                 extra=[f'-L{stand_in.parent}', '-lstamd', f'-Wl,-rpath,{stand_in.parent}'])


def test_driver_under_asan(stand_in, tmp_path):
    exe = driver('asan', stand_in)
    weights, config = reference_fixture('small-mixed', tmp_path / 'small-mixed')

    def run(*args):
        return subprocess.run([str(exe), '--weights', str(weights), '--config', str(config), *map(str, args)],
                              capture_output=True, text=True, env=ENV, timeout=300)

    r = run('--mode', 'correctness', '--backend', 'fused', '--events', 201, '--output', tmp_path / 'c')
    assert r.returncode == 0, r.stderr[-4000:]
    r = run('--mode', 'scheduled', '--events', 300, '--warmup', 0, '--rate', 200000, '--bursty', 1, '--queue', 4,
            '--output', tmp_path / 's')
    assert r.returncode == 0, r.stderr[-4000:]
    # Corrupted checkpoints end in a clean error (exit 1), never a sanitizer report.
    import json
    manifest = json.loads((weights / 'manifest.json').read_text())
    raw = (weights / 'tensors.bin').read_bytes()
    cases = {
        'truncated tensors': lambda: (weights / 'tensors.bin').write_bytes(raw[:len(raw) // 2]),
        'offset past the end': lambda: (weights / 'manifest.json').write_text(json.dumps(
            dict(manifest, tensors=[dict(t, offset=t['offset'] + 10 ** 9) for t in manifest['tensors']]))),
        'huge shape': lambda: (weights / 'manifest.json').write_text(json.dumps(
            dict(manifest, tensors=[dict(t, shape=[2 ** 31 - 1, 2 ** 31 - 1]) for t in manifest['tensors']]))),
        'malformed manifest': lambda: (weights / 'manifest.json').write_text('{"version": 1, "config": {'),
    }
    for what, corrupt in cases.items():
        corrupt()
        r = run('--mode', 'service', '--events', 5, '--output', tmp_path / 'x')
        assert r.returncode == 1 and 'Sanitizer' not in r.stderr and 'runtime error' not in r.stderr, (what, r.stderr)
        (weights / 'tensors.bin').write_bytes(raw)
        (weights / 'manifest.json').write_text(json.dumps(manifest))


def test_driver_scheduled_queue_under_tsan(stand_in, tmp_path):
    sanitizer_runs('tsan')
    exe = driver('tsan', stand_in)
    weights, config = reference_fixture('small-fp32', tmp_path / 'small-fp32')
    for rate, queue, bursty in ((20000, 64, 0), (500000, 2, 1)):
        r = subprocess.run([str(exe), '--weights', str(weights), '--config', str(config), '--mode', 'scheduled',
                            '--events', '400', '--warmup', '0', '--rate', str(rate), '--queue', str(queue), '--bursty',
                            str(bursty), '--output', str(tmp_path / f's{rate}')], capture_output=True, text=True,
                           env=ENV, timeout=300)
        assert r.returncode == 0 and 'ThreadSanitizer' not in r.stderr, r.stderr[-4000:]

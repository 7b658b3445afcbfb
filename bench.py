"""Benchmark of the streaming-step hot path on one MI355X.

Headline workload: Large FP32, W=512, one stream (d_model 1024, 12 layers, 16 heads x 64,
SwiGLU FFN 4096, RMSNorm eps 1e-5, features = d_model), synthetic weights ~ N(0, 0.02^2)
and inputs ~ N(0, 1) from seed 3. A "step" is one event through the whole model: input
projection, 12 layers, final norm and score, with the K/V rings carried on the GPU.

Timing: the window is first filled (W-1 events) and warmed (--warmup events), untimed;
then exactly --steps full-window steps run through the fused backend, one fused-kernel
launch per step, with a timing-only HIP event (no system-scope fence) recorded on the
runtime's stream after each launch (st_runtime_device_run). `value` is the p50 of those
per-step device durations (inputs already resident in HBM). The library synchronizes its
stream before and after the timed launches. One JSON line is printed.

Self-check ("self_check" in the line): the state the timed launches leave (position, K/V rings,
hidden state) and the score of the next event are compared with the C oracle's after the same
events (float accumulation, the reference's arithmetic) at the reference's bar: FP32
1e-5 + 1e-4|r| element by element, mixed the policy v3. The same oracle run then gives the CPU
baseline's timing (skipped together with it by --no-cpu-baseline).

Secondary measurements (skipped with --quick) go under "extra": host-service latency through
step() (stream copies and mapped staging), Large in the mixed and bfloat16-weight modes,
scheduled arrivals at 2000 events/s, the same step in PyTorch-ROCm (eager and captured), the
device loop, the persistent worker, the transport floors (mailbox ping-pong, empty launch,
empty graph, copy), the vendor GEMV baseline (rocBLAS projections in a captured graph) on the
same workload, the Main FP32 step across backends, B independent streams over shared weights
(Main, bfloat16 weights, W=128: the phase-kernel graph at B in 1, 16, 64, 256 and the resident
fused step per stream at B in 1, 4, 16, 32; --batched runs only those), and the Main
window sweep (W in 32..512, bfloat16 weights and mixed mode).

Usage: python bench.py [--gpus 1] [--steps 1024] [--warmup 64] [--config large|main|small]
                       [--precision fp32|bf16w|mixed] [--no-cpu-baseline] [--quick]
                       [--batched [--resident | --eager [--streams 1,16,64,256]]]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / 'streaming-transformer_amd'):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

from streamtx import (Backend, BatchRuntime, ModelConfig, Runtime, RuntimeOptions, WeightStorage,  # noqa: E402
                     synthetic_checkpoint, transport_bench)

CONFIGS = {
    'small': (ModelConfig(4, 256, 4, 1024, 64, 256), 0),
    'main': (ModelConfig(8, 512, 8, 2048, 128, 512), 1),
    'large': (ModelConfig(12, 1024, 16, 4096, 512, 1024), 3),
}
HBM_PEAK_GBS = 8000.0
METRIC = 'p50 µs per streaming step + matvec achieved HBM GB/s, Main/Large fp32'


def weight_bytes_per_step(c: ModelConfig, wb: int) -> int:
    """All matvec weights, norm weights and the score row read once per step."""
    d, f, L = c.width, c.ffn, c.layers
    return wb * (c.features * d + L * (4 * d * d + 3 * d * f + 2 * d) + 2 * d)


def kv_bytes_per_step(c: ModelConfig, kvb: int, valid: int) -> int:
    """K and V rows read over the valid window plus the new row written, every layer."""
    return 2 * c.layers * c.width * valid * kvb + 2 * c.layers * c.width * kvb


def batched_streams(counts=(1, 16, 64, 256), steps=64, mode='bf16w', resident=False, eager=False):
    """B independent streams over shared weights (st_batch_*): Main architecture, W=128, as in
    the batched configuration, with bfloat16 weights and FP32 K/V (mode 'bf16w') or the
    reference's mixed mode (FP16 weights and K/V); `resident`: one launch of the fused step
    per step, each stream on its own share of the CUs (st_batch_create_resident), else the
    graph of phase kernels (`eager`: its kernels launched directly instead of the graph replay,
    for kernel traces). Each B runs a full window of events (untimed), then `steps` timed
    steps with a HIP event after each. Algorithmic bytes per step: the weights once plus every
    stream's K/V window and new rows (the resident kernel reads the weights once per stream,
    mostly from the Infinity Cache and L2)."""
    c, seed = CONFIGS['main']
    mixed = mode == 'mixed'
    weights = synthetic_checkpoint(c, seed=seed, mixed=mixed)
    out = {'workload': f'main {mode} batched streams, W={c.window}', 'steps': steps,
           'kernel': 'resident fused step per stream' if resident else
           'phase kernels, eager launches' if eager else 'phase-kernel graph'}
    for b in counts:
        rng = np.random.default_rng([seed, 2, b])
        events = rng.standard_normal((c.window + steps, b, c.features), dtype=np.float32)
        storage = WeightStorage.AS_MODEL if mixed else WeightStorage.BF16
        with BatchRuntime((c, weights, mixed), b, storage, resident=resident) as rt:
            if eager:
                rt.set_eager()
            rt.device_run(events[:c.window])
            mean, per = rt.device_run(events[c.window:])
        p50 = nearest_rank(per, 0.5)
        step_bytes = weight_bytes_per_step(c, 2) + b * kv_bytes_per_step(c, 2 if mixed else 4, c.window)
        gbs = step_bytes / (mean * 1e-6) / 1e9
        out[f'B{b}'] = {'p50_us_per_step': round(p50, 2), 'mean_us_per_step': round(mean, 2),
                        'events_per_s': round(b / (p50 * 1e-6)), 'algorithmic_bytes_per_step': step_bytes,
                        'achieved_gbs': round(gbs, 1), 'hbm_frac': round(gbs / HBM_PEAK_GBS, 4),
                        'mall_resident': step_bytes < 256e6}
    return out


def torch_baseline(c: ModelConfig, weights, events, fill: int, steps: int = 128, inductor: bool = False):
    """The same single-stream step written with PyTorch-ROCm operators in FP32 (the
    reference's bench/torch_bench.py comparison): eager, and captured once in a hipGraph with
    the position held on the device (ring slot, valid-window mask and RoPE angles computed from
    it). Returns p50 microseconds per step for both and the largest score difference from the
    HIP runtime on the same events (a sanity check, not a parity bar). With `inductor`, only
    the reference's third variant instead: the step compiled by torch.compile (Inductor,
    fullgraph), p50 per step, compile time and the largest score difference from eager."""
    import torch

    dev = torch.device('cuda')
    T = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(dev) for k, v in weights.items()}
    L, d, H, W, dh = c.layers, c.width, c.heads, c.window, c.dim
    keys = torch.zeros(L, H, W, dh, device=dev)
    values = torch.zeros_like(keys)
    pos = torch.zeros((), dtype=torch.int64, device=dev)
    inv = torch.pow(torch.tensor(10000.0, device=dev), -torch.arange(0, dh, 2, device=dev, dtype=torch.float32) / dh)
    slots = torch.arange(W, device=dev)
    event = torch.zeros(c.features, device=dev)
    score = torch.zeros(1, device=dev)

    def rms(x, g):
        return x * torch.rsqrt(x.pow(2).mean() + c.epsilon) * g

    def rope(v, cos, sin):
        v = v.view(H, dh // 2, 2)
        a, b = v[..., 0], v[..., 1]
        return torch.stack((a * cos - b * sin, a * sin + b * cos), -1).reshape(d)

    def step():
        ang = pos.to(torch.float32) * inv
        cos, sin = torch.cos(ang), torch.sin(ang)
        slot = torch.remainder(pos, W).view(1)
        mask = (slots <= pos).view(1, 1, W)
        x = T['input'] @ event
        for l in range(L):
            p = f'layers.{l}.'
            n = rms(x, T[p + 'norm1'])
            q = rope(T[p + 'q'] @ n, cos, sin)
            k = rope(T[p + 'k'] @ n, cos, sin)
            v = T[p + 'v'] @ n
            keys[l].index_copy_(1, slot, k.view(H, 1, dh))
            values[l].index_copy_(1, slot, v.view(H, 1, dh))
            logits = torch.matmul(keys[l], q.view(H, dh, 1)).view(H, 1, W) / (dh ** 0.5)
            prob = torch.softmax(logits.masked_fill(~mask, float('-inf')), -1)
            attn = torch.matmul(prob, values[l]).reshape(d)
            x = x + T[p + 'out'] @ attn
            n = rms(x, T[p + 'norm2'])
            g = T[p + 'gate'] @ n
            x = x + T[p + 'down'] @ (torch.nn.functional.silu(g) * (T[p + 'up'] @ n))
        score.copy_(T['score'] @ rms(x, T['final_norm']))
        pos.add_(1)

    timed_events = torch.from_numpy(np.ascontiguousarray(events[fill:fill + steps])).to(dev)

    def timed(run, n):
        start = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
        start[0].record()
        for i in range(n):
            event.copy_(timed_events[i])  # device-to-device: inputs resident, like the runtime's timing
            run()
            start[i + 1].record()
        torch.cuda.synchronize()
        return np.array([start[i].elapsed_time(start[i + 1]) * 1e3 for i in range(n)])

    with torch.no_grad():
        for i in range(fill):  # fill the window
            event.copy_(torch.from_numpy(events[i]).to(dev))
            step()
        state = (keys.clone(), values.clone(), pos.clone())  # the filled window
        if inductor:
            eager_scores = []
            for i in range(8):
                event.copy_(torch.from_numpy(events[fill + i]).to(dev))
                step()
                eager_scores.append(float(score))
            compiled = torch.compile(step, fullgraph=True, backend='inductor')
            keys.copy_(state[0]), values.copy_(state[1]), pos.copy_(state[2])
            t0 = time.perf_counter()
            event.copy_(torch.from_numpy(events[fill]).to(dev))
            compiled()
            torch.cuda.synchronize()
            compile_s = time.perf_counter() - t0
            diff = abs(float(score) - eager_scores[0])
            for i in range(1, 8):
                event.copy_(torch.from_numpy(events[fill + i]).to(dev))
                compiled()
                diff = max(diff, abs(float(score) - eager_scores[i]))
            keys.copy_(state[0]), values.copy_(state[1]), pos.copy_(state[2])
            per = timed(compiled, steps)
            return {'inductor_p50_us': round(float(np.median(per)), 1), 'inductor_compile_s': round(compile_s, 1),
                    'inductor_vs_eager_max_abs': diff, 'torch': torch.__version__}
        eager = timed(step, steps)
        eager_scores = []
        # Graph capture of the same step on a side stream, then replays checked against eager.
        keys.copy_(state[0]), values.copy_(state[1]), pos.copy_(state[2])
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        keys.copy_(state[0]), values.copy_(state[1]), pos.copy_(state[2])
        with torch.cuda.graph(graph):
            step()
        keys.copy_(state[0]), values.copy_(state[1]), pos.copy_(state[2])
        for i in range(8):
            event.copy_(torch.from_numpy(events[fill + i]).to(dev))
            step()
            eager_scores.append(float(score))
        keys.copy_(state[0]), values.copy_(state[1]), pos.copy_(state[2])
        replay_diff = 0.0
        for i in range(8):
            event.copy_(torch.from_numpy(events[fill + i]).to(dev))
            graph.replay()
            torch.cuda.synchronize()
            replay_diff = max(replay_diff, abs(float(score) - eager_scores[i]))
        graphed = timed(graph.replay, steps)
    # The staged backend (bit-identical to the fused one) needs no cooperative launch, which a
    # second process on the GPU may not get while the first holds the cooperative queue.
    with Runtime((c, weights, False), RuntimeOptions(backend=Backend.CUDA, blocks=0)) as rt:
        rt.device_run(events[:fill], reset=True)
        ours = [rt.step(e) for e in events[fill:fill + 8]]
    diff = max(abs(a - b) for a, b in zip(ours, eager_scores))
    return {'eager_p50_us': round(float(np.median(eager)), 1), 'graph_p50_us': round(float(np.median(graphed)), 1),
            'graph_replay_vs_eager_max_abs': replay_diff, 'score_max_abs_diff_vs_runtime': diff,
            'torch': torch.__version__}


def window_sweep(windows=(32, 64, 128, 256, 512), steps=2048):
    """Main architecture, one stream, fused backend, W in `windows`: bfloat16 weights with FP32
    K/V, and the reference's mixed mode (FP16 weights and K/V). Weights and inputs from seed 2.
    Each W fills its window (untimed), then times `steps` full-window steps. Shows how the
    attention's K/V bytes grow against the fixed weight bytes."""
    base, _ = CONFIGS['main']
    out = {'workload': 'main single-stream window sweep, fused backend', 'steps': steps}
    for mode in ('bf16w', 'mixed'):
        mixed = mode == 'mixed'
        rows = {}
        for w in windows:
            c = ModelConfig(base.layers, base.width, base.heads, base.ffn, w, base.features)
            weights = synthetic_checkpoint(c, seed=2, mixed=mixed)
            events = np.random.default_rng([2, 1]).standard_normal((w - 1 + steps, c.features), dtype=np.float32)
            opts = RuntimeOptions(backend=Backend.FUSED, blocks=0,
                                  weight_dtype=WeightStorage.AS_MODEL if mixed else WeightStorage.BF16)
            with Runtime((c, weights, mixed), opts) as rt:
                rt.device_run(events[:w - 1], reset=True)
                mean, per = rt.device_run(events[w - 1:])
            step_bytes = weight_bytes_per_step(c, 2) + kv_bytes_per_step(c, 2 if mixed else 4, w)
            gbs = step_bytes / (mean * 1e-6) / 1e9
            rows[f'W{w}'] = {'p50_us': round(nearest_rank(per, 0.5), 2), 'p99_us': round(nearest_rank(per, 0.99), 2),
                             'algorithmic_bytes_per_step': step_bytes, 'achieved_gbs': round(gbs, 1),
                             'mall_resident': step_bytes < 256e6}
        out[mode] = rows
    return out


def main_backends(steps=512):
    """Main FP32 (d 512, 8 layers, W 128; 140 MB per step, resident in the 256 MB Infinity
    Cache), one stream, seed 1, through the fused, graph and staged backends (device p50 per
    step, HIP events between launches) and the persistent worker (host service through step(),
    PCIe-inclusive)."""
    c, seed = CONFIGS['main']
    weights = synthetic_checkpoint(c, seed=seed)
    events = np.random.default_rng([seed, 1]).standard_normal((c.window - 1 + 64 + steps, c.features),
                                                               dtype=np.float32)
    fill = c.window - 1 + 64
    step_bytes = weight_bytes_per_step(c, 4) + kv_bytes_per_step(c, 4, c.window)
    out = {'workload': 'main fp32 single-stream step, W=128', 'steps': steps, 'algorithmic_bytes_per_step': step_bytes,
           'mall_resident': step_bytes < 256e6}
    for name, backend in (('fused', Backend.FUSED), ('graph', Backend.GRAPH), ('staged', Backend.CUDA)):
        with Runtime((c, weights, False), RuntimeOptions(backend=backend, blocks=0)) as rt:
            rt.device_run(events[:fill], reset=True)
            mean, per = rt.device_run(events[fill:fill + steps])
        out[name] = {'p50_us': round(nearest_rank(per, 0.5), 2), 'p99_us': round(nearest_rank(per, 0.99), 2),
                     'roofline_frac': round(step_bytes / (mean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    with Runtime((c, weights, False), RuntimeOptions(backend=Backend.PERSISTENT, blocks=0)) as rt:
        for e in events[:fill]:
            rt.step(e)
        host = []
        for e in events[fill:fill + steps]:
            s = time.perf_counter()
            rt.step(e)
            host.append((time.perf_counter() - s) * 1e6)
    out['persistent_service'] = {'p50_us': round(nearest_rank(host, 0.5), 2), 'p99_us': round(nearest_rank(host, 0.99), 2)}
    return out


def matvec_bandwidth(rt, c: ModelConfig, events, wb: int, kvb: int):
    """Achieved GB/s of each matvec kind inside the fused step, from the per-phase wall-clock
    stamps of st_runtime_phase_times over len(events) full-window steps. Bytes of a phase:
    its weight rows (QKV 3d x d, OUT d x d, GATEUP 2F x d, DOWN d x F; norm weights and padding
    excluded); ATTN: the K/V rows of the window. `phase_us` runs from one phase's start to the
    next one's (median over workgroups, layers and steps): it includes the exchange of the next
    phase's input. `compute_us` ends when this workgroup's stream waves are done with the phase.
    Recording the stamps adds a few LDS stores per phase and workgroup."""
    d, F, L = c.width, c.ffn, c.layers
    weights = {'QKV': 3 * d * d * wb, 'OUT': d * d * wb, 'GATEUP': 2 * F * d * wb, 'DOWN': d * F * wb,
               'ATTN': 2 * d * c.window * kvb}
    kinds = ['INPUT'] + [k for _ in range(L) for k in ('QKV', 'ATTN', 'OUT', 'GATEUP', 'DOWN')] + ['FINAL']
    phase, compute = {k: [] for k in weights}, {k: [] for k in weights}
    for e in events:
        st, _ = rt.phase_times(e)
        for ph, kind in enumerate(kinds[:-1]):
            if kind not in weights:
                continue
            s0 = st[ph, :, 0]
            phase[kind].append(float(np.median(st[ph + 1, :, 0] - s0)))
            compute[kind].append(float(np.median(st[ph, :, 2] - s0)))
    out = {}
    for kind, b in weights.items():
        pu, cu = float(np.median(phase[kind])), float(np.median(compute[kind]))
        out[kind] = {'bytes_per_layer': b, 'phase_us': round(pu, 2), 'compute_us': round(cu, 2),
                     'gbs_phase': round(b / (pu * 1e-6) / 1e9, 1), 'gbs_compute': round(b / (cu * 1e-6) / 1e9, 1)}
    return out


def host_cpu():
    """CPU model (lscpu's model name with family/model/stepping, else /proc/cpuinfo's), hardware
    thread count and ISA flags of this host."""
    model, threads, flags, ids = 'unknown', 0, set(), {}
    try:
        for line in Path('/proc/cpuinfo').read_text().splitlines():
            key = line.split(':', 1)[0].strip()
            if key == 'model name' and model == 'unknown':
                model = line.split(':', 1)[1].strip()
            elif key == 'processor':
                threads += 1
            elif key == 'flags' and not flags:
                flags = set(line.split(':', 1)[1].split())
            elif key in ('cpu family', 'model', 'stepping') and key not in ids:
                ids[key] = line.split(':', 1)[1].strip()
    except OSError:
        pass
    try:
        import subprocess
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith('Model name:'):
                model = line.split(':', 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if ids:
        model += f' (family {ids.get("cpu family", "?")}, model {ids.get("model", "?")}, stepping {ids.get("stepping", "?")})'
    return model, threads, flags


def nearest_rank(values, q):
    v = np.sort(np.asarray(values))
    return float(v[max(0, int(math.ceil(q * len(v))) - 1)])


def cpu_baseline(c: ModelConfig, weights, mixed, events, upto: int, sample: int, isa: str, check=None):
    """The C oracle (a restatement of the reference CPU step) on this host's cores.

    Self-check: the oracle (float accumulation, the reference's arithmetic; OpenMP over matvec
    rows on up to 16 threads) runs the same events as the GPU up to the end of its timed
    region (events[:upto]); `check` = (the GPU's snapshot there, the GPU's score of
    events[upto]) is compared with the oracle's at the reference's bar (FP32 1e-5 + 1e-4|r|;
    mixed, policy v3). Timing: then `sample` further full-window steps single-threaded (the
    reference default), and `sample` with the 16-thread split. isa: 'v3' (the AVX2 build) or
    'portable'. Returns (times by thread count, thread count, self-check report)."""
    from oracle.pyoracle import Oracle
    from streamtx import numerical
    threads_all = min(16, os.cpu_count() or 1)
    oracle = Oracle(c, weights, mixed=mixed, threads=threads_all, isa=isa)
    for e in events[:upto]:
        oracle.step(e)
    report = None
    if check is not None:
        (pos, keys, values, hidden), gpu_score = check
        opos, okeys, ovalues, ohidden = oracle.snapshot()
        ref_score = oracle.step(events[upto])
        report = {'events': upto + 1, 'position': int(pos), 'position_matches': int(pos) == int(opos),
                  'next_score': {'gpu': gpu_score, 'oracle': ref_score, 'abs_diff': abs(gpu_score - ref_score)}}
        if mixed:
            st = numerical.mixed_state_passes(keys, values, hidden, okeys, ovalues, ohidden)
            sc = numerical.score_errors([gpu_score], [ref_score], c.layers)
            report.update(bar='policy v3 (mixed)', state_failures=len(st['failures']), score_passed=sc['passed'],
                          passed=bool(st['passed'] and sc['passed'] and report['position_matches']))
        else:
            fails = {name: int(numerical.fp32_failures(a, o)) for name, a, o in
                     (('keys', keys, okeys), ('values', values, ovalues), ('hidden', hidden, ohidden))}
            fails['score'] = int(numerical.fp32_failures([gpu_score], [ref_score]))
            report.update(bar='fp32 1e-5 + 1e-4|r| against the float oracle', elements_over_bar=fails,
                          max_abs_state=float(max(np.abs(a - o).max() for a, o in
                                                  ((keys, okeys), (values, ovalues), (hidden, ohidden)))),
                          passed=bool(sum(fails.values()) == 0 and report['position_matches']))
    out = {}
    for threads in (1, threads_all):
        oracle._lib.so_set_threads(oracle._h, threads)
        times = []
        for e in events[upto - sample:upto]:
            t0 = time.perf_counter()
            oracle.step(e)
            times.append((time.perf_counter() - t0) * 1e6)
        out[threads] = times
    return out, threads_all, report


def copy_calibration(mib: int) -> None:
    """A plain copy kernel of known size: each launch reads and writes `mib` MiB. Profiling
    it with the FETCH_SIZE / WRITE_SIZE counters gives the factor between counter readings
    and HBM bytes on this device."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.empty(n, dtype=torch.float32, device='cuda').uniform_()
    dst = torch.empty_like(src)
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_calibration_bytes_per_launch': n * 4, 'launches': 8}), flush=True)


def traffic_per_launch(path: Path):
    """HBM bytes per launch from a committed counter summary (line `hbm_bytes_per_launch: N`)."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith('hbm_bytes_per_launch:'):
            return int(float(line.split(':', 1)[1]))
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=1024)
    ap.add_argument('--warmup', type=int, default=64)
    ap.add_argument('--config', choices=sorted(CONFIGS), default='large')
    ap.add_argument('--precision', choices=['fp32', 'bf16w', 'mixed'], default='fp32')
    ap.add_argument('--backend', choices=['fused', 'graph', 'cuda', 'cublas', 'cublas-graph'], default='fused')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--quick', action='store_true', help='skip the secondary measurements')
    ap.add_argument('--torch-baseline', action='store_true',
                    help='only the PyTorch comparison (FP32, eager and captured); bench.py runs it as a child')
    ap.add_argument('--inductor', action='store_true',
                    help='with --torch-baseline: the torch.compile (Inductor) variant instead')
    ap.add_argument('--batched', action='store_true',
                    help='only the batched-streams measurement (B in 1, 16, 64, 256; --steps timed steps each)')
    ap.add_argument('--resident', action='store_true',
                    help='with --batched: only the resident rows (B in 1, 4, 16, 32)')
    ap.add_argument('--eager', action='store_true',
                    help='with --batched: only the bfloat16-weight phase-kernel rows, each step\'s kernels '
                         'launched directly instead of the graph replay (for kernel traces)')
    ap.add_argument('--streams', default='1,16,64,256',
                    help='with --batched --eager: the batch sizes (comma-separated)')
    ap.add_argument('--copy-calibration', type=int, metavar='MIB', default=0,
                    help='only run 8 plain device copies of MIB MiB (reference kernel for HBM counters)')
    args = ap.parse_args()
    if args.torch_baseline:
        c, seed = CONFIGS[args.config]
        weights = synthetic_checkpoint(c, seed=seed)
        fill = c.window - 1 + args.warmup
        events = np.random.default_rng([seed, 1]).standard_normal((fill + 128, c.features), dtype=np.float32)
        print(json.dumps(torch_baseline(c, weights, events, fill, inductor=args.inductor)), flush=True)
        return
    if args.batched and args.resident:
        print(json.dumps({'resident_bf16w': batched_streams(counts=(1, 4, 16, 32), steps=args.steps, resident=True)}),
              flush=True)
        return
    if args.batched and args.eager:
        counts = tuple(int(b) for b in args.streams.split(','))
        print(json.dumps({'bf16w': batched_streams(counts=counts, steps=args.steps, eager=True)}), flush=True)
        return
    if args.batched:
        print(json.dumps({'bf16w': batched_streams(steps=args.steps),
                          'mixed': batched_streams(steps=args.steps, mode='mixed'),
                          'resident_bf16w': batched_streams(counts=(1, 4, 16, 32), steps=args.steps,
                                                            resident=True)}), flush=True)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(f'bench.py measures one GPU: the streaming step is a single ordered stream and the '
              f'runtime does not shard it (requested --gpus {args.gpus}).', file=sys.stderr)
        sys.exit(2)

    c, seed = CONFIGS[args.config]
    mixed = args.precision == 'mixed'
    weights = synthetic_checkpoint(c, seed=seed, mixed=mixed)
    fill = c.window - 1 + args.warmup
    rng = np.random.default_rng([seed, 1])  # input stream distinct from the weight stream
    events = rng.standard_normal((fill + args.steps + 1, c.features), dtype=np.float32)
    backend = {'fused': Backend.FUSED, 'graph': Backend.GRAPH, 'cuda': Backend.CUDA, 'cublas': Backend.CUBLAS,
               'cublas-graph': Backend.CUBLAS_GRAPH}[args.backend]
    opts = RuntimeOptions(backend=backend, blocks=0,
                          weight_dtype=WeightStorage.BF16 if args.precision == 'bf16w' else WeightStorage.AS_MODEL)
    wb = 4 if args.precision == 'fp32' else 2
    kvb = 2 if mixed else 4
    bytes_step = weight_bytes_per_step(c, wb) + kv_bytes_per_step(c, kvb, c.window)

    extra = {}
    with Runtime((c, weights, mixed), opts) as rt:
        info = rt.info()
        rt.device_run(events[:fill], reset=True)                      # fill + warm up, untimed
        t0 = time.perf_counter()
        mean_us, per = rt.device_run(events[fill:fill + args.steps])  # exactly --steps launches
        wall = time.perf_counter() - t0
        # What the timed launches left (position, K/V, hidden) and the next step's score, for the
        # self-check against the oracle.
        after_timed = (rt.snapshot(), rt.step(events[fill + args.steps]))
        p50 = nearest_rank(per, 0.5)
        extra['p99_us'] = nearest_rank(per, 0.99)
        extra['mean_us'] = mean_us
        extra['wall_seconds_timed_call'] = wall
        if not args.quick:
            # Host-service latency through step(): pinned H2D input, launch, D2H score, sync.
            host = []
            for e in events[fill:fill + 256]:
                s = time.perf_counter()
                rt.step(e)
                host.append((time.perf_counter() - s) * 1e6)
            extra['host_service_p50_us'] = nearest_rank(host, 0.5)
            extra['host_service_p99_us'] = nearest_rank(host, 0.99)
            # Scheduled arrivals (the reference driver's scheduled mode): the timed events offered
            # at 2000 per second into a 4096-slot queue, latency from intended arrival to completion.
            arrivals = rt.scheduled_run(events[fill:fill + args.steps], rate=2000.0, queue=4096)['summary']
            extra['scheduled_2000_per_s'] = {k: arrivals[k] for k in ('offered', 'completed', 'dropped')}
            for k in ('arrival', 'service', 'queueing'):
                extra['scheduled_2000_per_s'][k + '_p50_us'] = round(arrivals[k]['p50_us'], 1)
                extra['scheduled_2000_per_s'][k + '_p99_us'] = round(arrivals[k]['p99_us'], 1)
            if backend == Backend.FUSED:
                # Device loop inside one launch (the reference's deviceTrace).
                n = c.window - 1 + 256
                _, loop = rt.device_trace(events[:n])
                extra['device_loop_p50_us'] = nearest_rank(loop[c.window - 1:], 0.5)
                # Achieved GB/s of each matvec kind within the step (phase stamps).
                rt.device_run(events[:fill], reset=True)
                extra['matvec_gbs'] = matvec_bandwidth(rt, c, events[fill:fill + 8], wb, kvb)
    if not args.quick and backend == Backend.FUSED:
        # Same service latency through the persistent mailbox worker (no launch per step).
        popts = RuntimeOptions(backend=Backend.PERSISTENT, blocks=0, weight_dtype=opts.weight_dtype)
        with Runtime((c, weights, mixed), popts) as rt:
            for e in events[:fill]:
                rt.step(e)
            host = []
            for e in events[fill:fill + 1024]:
                s = time.perf_counter()
                rt.step(e)
                host.append((time.perf_counter() - s) * 1e6)
            extra['persistent_service_p50_us'] = nearest_rank(host, 0.5)
            extra['persistent_service_p99_us'] = nearest_rank(host, 0.99)
        # The fused backend's host service with mapped staging (RuntimeOptions.mapped: the event
        # and the score go through mapped pinned memory instead of stream copies).
        mopts = RuntimeOptions(backend=Backend.FUSED, blocks=0, weight_dtype=opts.weight_dtype, mapped=True)
        with Runtime((c, weights, mixed), mopts) as rt:
            rt.device_run(events[:fill], reset=True)
            host = []
            for e in events[fill:fill + 256]:
                s = time.perf_counter()
                rt.step(e)
                host.append((time.perf_counter() - s) * 1e6)
            extra['mapped_host_service_p50_us'] = nearest_rank(host, 0.5)
            extra['mapped_host_service_p99_us'] = nearest_rank(host, 0.99)

    if not args.quick and backend == Backend.FUSED:
        # The reference's default backend (a captured step per event): here the hipGraph holds
        # the fused kernel as one node.
        gopts = RuntimeOptions(backend=Backend.GRAPH, blocks=0, weight_dtype=opts.weight_dtype)
        with Runtime((c, weights, mixed), gopts) as rt:
            rt.device_run(events[:fill], reset=True)
            _, gper = rt.device_run(events[fill:fill + min(args.steps, 512)])
        extra['graph_p50_us'] = nearest_rank(gper, 0.5)
        extra['graph_p99_us'] = nearest_rank(gper, 0.99)
    if not args.quick and args.precision != 'bf16w':
        # The same workload through the vendor GEMV baseline (rocBLAS projections, captured).
        vopts = RuntimeOptions(backend=Backend.CUBLAS_GRAPH, blocks=0)
        with Runtime((c, weights, mixed), vopts) as rt:
            rt.device_run(events[:fill], reset=True)
            _, vper = rt.device_run(events[fill:fill + min(args.steps, 256)])
        extra['vendor_gemv_graph_p50_us'] = nearest_rank(vper, 0.5)
    if not args.quick and args.precision == 'fp32':
        # torch brings its own HIP runtime, which does not start in a process where this
        # library's runtime already runs: the comparison runs in a child process.
        import subprocess
        cmd = [sys.executable, str(Path(__file__).resolve()), '--torch-baseline', '--config', args.config,
               '--warmup', str(args.warmup)]
        def child(extra_args, timeout):
            try:
                proc = subprocess.run(cmd + extra_args, capture_output=True, text=True, timeout=timeout)
                lines = [ln for ln in proc.stdout.splitlines() if ln.startswith('{')]
                return json.loads(lines[-1]) if proc.returncode == 0 and lines else \
                    {'error': (proc.stderr or proc.stdout)[-300:]}
            except subprocess.TimeoutExpired:
                return {'error': 'timeout'}
        extra['torch_baseline'] = child([], 300)
        # The reference's third variant, torch.compile (Inductor), in a child of its own so that a
        # compiler failure leaves the other two figures.
        inductor = child(['--inductor'], 300)
        extra['torch_baseline'].update(inductor if 'error' not in inductor else {'inductor_error': inductor['error']})
    if not args.quick and args.config == 'large' and args.precision == 'fp32':
        # The same Large workload in the other storage modes: mixed (FP16 weights and K/V, the
        # reference's cast points) and bfloat16 weights with FP32 K/V.
        extra['other_precisions'] = {}
        for prec in ('mixed', 'bf16w'):
            pm = prec == 'mixed'
            pw = synthetic_checkpoint(c, seed=seed, mixed=pm)
            popts = RuntimeOptions(backend=Backend.FUSED, blocks=0,
                                   weight_dtype=WeightStorage.BF16 if prec == 'bf16w' else WeightStorage.AS_MODEL)
            with Runtime((c, pw, pm), popts) as rt:
                rt.device_run(events[:fill], reset=True)
                pmean, pper = rt.device_run(events[fill:fill + min(args.steps, 512)])
            pbytes = weight_bytes_per_step(c, 2) + kv_bytes_per_step(c, 2 if pm else 4, c.window)
            extra['other_precisions'][prec] = {
                'p50_us': round(nearest_rank(pper, 0.5), 2), 'p99_us': round(nearest_rank(pper, 0.99), 2),
                'algorithmic_bytes_per_step': pbytes,
                'roofline_frac': round(pbytes / (pmean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    if not args.quick:
        # Transport floors under a step (the reference's transportBench modes).
        extra['transport_p50_us'] = {m: round(transport_bench(m, 2000)['p50_us'], 2)
                                     for m in ('ping-pong', 'gpu-ping', 'empty', 'empty-graph', 'copy')}
        extra['batched'] = batched_streams()
        extra['batched_mixed'] = batched_streams(mode='mixed')
        extra['batched_resident'] = batched_streams(counts=(1, 4, 16, 32), resident=True)
        extra['window_sweep'] = window_sweep()
        if args.config == 'large' and args.precision == 'fp32' and backend == Backend.FUSED:
            extra['main_fp32'] = main_backends()

    achieved = bytes_step / (mean_us * 1e-6) / 1e9
    roofline = {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': None,
                'algorithmic_bytes_per_step': bytes_step,
                'roofline_us_per_step': bytes_step / (HBM_PEAK_GBS * 1e9) * 1e6,
                'kernel': {Backend.FUSED: 'fused_kernel', Backend.CUBLAS: 'rocBLAS gemv + stage kernels',
                           Backend.CUBLAS_GRAPH: 'rocBLAS gemv + stage kernels'}.get(backend, 'phase_kernel sequence')}
    if backend == Backend.GRAPH and info.get('fused_launch', '').startswith('graph node'):
        roofline['kernel'] = 'fused_kernel (graph node)'
    roofline['traffic'] = traffic_per_launch(
        ROOT / 'profiles' / f'traffic_{args.backend}_kernel_{args.config}_{args.precision}.md')
    roofline['frac_p50'] = round(bytes_step / (p50 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    extra['mall_resident'] = bytes_step < 256e6

    cpu = None
    self_check = None
    if not args.no_cpu_baseline:
        sample = min(args.steps, {'large': 24, 'main': 80, 'small': 400}[args.config])
        upto = fill + args.steps
        model, host_threads, flags = host_cpu()
        isa = 'v3' if {'avx2', 'fma', 'bmi2'} <= flags else 'portable'
        times, threads_all, self_check = cpu_baseline(
            c, weights if args.precision != 'bf16w' else
            {k: __import__('streamtx').round_bf16(v) for k, v in weights.items()},
            mixed, events, upto, sample, isa, check=after_timed)
        cpu = {'value': nearest_rank(times[1], 0.5), 'unit': 'us per step (p50)', 'cores': 1,
               'kind': 'port',
               'sample': f'{sample} full-window steps of the same {args.config} {args.precision} workload (the last '
                         f'{sample} timed events, replayed after the oracle has run all {upto + 1}); C oracle '
                         f'restating src/cpu/Cpu.cpp:59-141, 1 thread, built '
                         f'-O3 {"-march=x86-64-v3 " if isa == "v3" else ""}-ffp-contract=off',
               'cpu_model': model, 'host_threads': host_threads, 'isa': isa,
               'multithread_p50_us': nearest_rank(times[threads_all], 0.5), 'multithread_cores': threads_all}

    line = {
        'metric': METRIC, 'value': round(p50, 3), 'unit': 'us', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(mean_us / 1000.0, 6), 'higher_is_better': False,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': {'fp32': 'fp32', 'bf16w': 'bf16 weights, fp32 compute',
                                                          'mixed': 'fp16 storage, fp32 accumulate'}[args.precision],
        'data': 'synthetic (weights N(0,0.02^2), inputs N(0,1))',
        'config': {'workload': f'{args.config} {args.precision} single-stream step, W={c.window}',
                   'd_model': c.width, 'layers': c.layers, 'heads': c.heads, 'head_dim': c.dim, 'ffn': c.ffn,
                   'window': c.window, 'features': c.features, 'seed': seed, 'backend': args.backend,
                   'blocks': info['blocks'], 'threads_per_block': info['threads']},
        'roofline': roofline,
        'cpu_baseline': cpu,
        'self_check': self_check,
        'extra': extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()

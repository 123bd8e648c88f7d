"""Benchmark: train steps/sec (fwd + bwd + Adam) per config on one MI355X.

Prints ONE JSON line. `value` is the headline config's steps/s (default: the transformer,
C5, the config the north star's roofline targets are stated on) with every batch already
resident in HBM when the timed region starts (batches are staged into device slots
beforehand); each timed step still uploads the per-step optimizer scalars and PRNG seed,
replays the captured step graph and reads the 4-byte loss back (the API's semantics).
`per_config` carries the same measurement for all five configs (and the transformer with
clipGradNorm 1.0, the reference samples' setting), plus device-only replay time and
per-family kernel rates. Kernel rates come from the kernels' own durations inside eager
steps: every kernel of a step is dispatched with start / end events of its own
(tg_profile_kernels), the quantity a profiler's kernel trace reports, without the gaps
between launches. `roofline` is for the dominant kernel family of the headline config
(its f32 MFMA GEMMs), `roofline_mfma_all` for every MFMA kernel (GEMMs and fused
attention); `cpu_baseline` is the CPU oracle (a C++ restatement of the reference's CPU
evaluator, the reference itself being TypeScript that cannot run here) on this host's
cores, on a bounded number of steps of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
RING = 8


def family_rates(nodes, kms):
    """Per-family work and kernel time of one step from per-node kernel durations (ms):
    GEMMs, convolutions and attention on the f32 MFMA roofline, the rest on HBM."""
    fam = {'gemm': ('gemm',), 'conv': ('conv',), 'attention': ('attention',)}
    out = {}
    for name, kinds in fam.items():
        sel = [(n, t) for n, t in zip(nodes, kms) if n['kind'] in kinds]
        f = sum(n['flops'] for n, _ in sel)
        t = sum(t for _, t in sel)
        out[name] = {'flop_per_step': f, 'bytes_per_step': sum(n['bytes'] for n, _ in sel), 'launches': len(sel),
                     'ms': t, 'tflops': f / max(t, 1e-12) / 1e9,
                     'frac_f32_peak': f / max(t, 1e-12) / 1e9 / PEAK_F32_MFMA_TFLOPS}
    mf = out['gemm']['flop_per_step'] + out['attention']['flop_per_step'] + out['conv']['flop_per_step']
    mt = out['gemm']['ms'] + out['attention']['ms'] + out['conv']['ms']
    out['mfma_all'] = {'flop_per_step': mf, 'ms': mt, 'tflops': mf / max(mt, 1e-12) / 1e9,
                       'frac_f32_peak': mf / max(mt, 1e-12) / 1e9 / PEAK_F32_MFMA_TFLOPS}
    sel = [(n, t) for n, t in zip(nodes, kms) if n['kind'] not in ('gemm', 'conv', 'attention')]
    b = sum(n['bytes'] for n, _ in sel)
    t = sum(t for _, t in sel)
    out['non_gemm'] = {'bytes_per_step': b, 'launches': len(sel), 'ms': t, 'gbs': b / max(t, 1e-12) / 1e6,
                       'frac_hbm_peak': b / max(t, 1e-12) / 1e6 / PEAK_HBM_GBS}
    return out


def measure(key, steps, warmup, profile_iters=5, optimizer=None, label=None):
    """Steps/s of config `key` (optionally with another optimizer) from staged batches, the
    PCIe-inclusive rate, graph-replay time, and per-family kernel rates from the kernels'
    own durations in eager steps (tg_profile_kernels)."""
    from tensorgrad_amd import backend, configs
    from tensorgrad_amd.build_ir import build_training_ir
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, optimizer or cfg.optimizer)
    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(ir.initial_params(configs.INIT_SEED))
    for i, b in enumerate(configs.batches(cfg, RING)):
        rt.stage_batch(i, b)
    for i in range(warmup):
        rt.step_staged(i % RING)
    t0 = time.perf_counter()
    loss = None
    for i in range(steps):
        loss = rt.step_staged(i % RING)
    dt = time.perf_counter() - t0
    # PCIe-inclusive rate (never `value`): host-resident batches, each step copies its batch
    # host -> device through pinned staging before the replay
    host_batches = configs.batches(cfg, RING)
    host_steps = min(steps, 50)
    t1 = time.perf_counter()
    for i in range(host_steps):
        rt.step(host_batches[i % RING])
    host_dt = time.perf_counter() - t1
    replay_ms = rt.time_replays(steps) / steps
    nodes = rt.describe()['nodes']
    kms = rt.profile_kernels(profile_iters)
    rt.destroy()
    fam = family_rates(nodes, kms)
    by_kind = {}
    for n, t in zip(nodes, kms):
        k = by_kind.setdefault(n['kind'], {'launch_nodes': 0, 'ms': 0.0})
        k['launch_nodes'] += 1
        k['ms'] = round(k['ms'] + t, 4)
    top_gemm = sorted(((t, n) for n, t in zip(nodes, kms) if n['kind'] == 'gemm'), key=lambda x: -x[0])[:3]
    fam['gemm']['top'] = [{'shape': n['shape'], 'ms': round(t, 4), 'tflops': round(n['flops'] / max(t, 1e-12) / 1e9, 2)}
                          for t, n in top_gemm]
    return {
        'config': label or key,
        'title': cfg.title,
        'steps_per_s': steps / dt,
        'ms_per_step': 1e3 * dt / steps,
        'samples_per_s': cfg.samples_per_step * steps / dt,
        'sample_unit': cfg.sample_unit,
        'device_replay_ms': replay_ms,
        'kernel_ms_per_step': sum(kms),
        'host_batch_steps_per_s': host_steps / host_dt,
        'launch_nodes': len(nodes),
        'final_loss': loss,
        **fam,
        'kinds': by_kind,
    }


def kernel_events(key, iters=20, warmup=20):
    """Markdown report of one config's kernel durations from their own start / end events
    (tg_profile_kernels, `iters` eager steps after `warmup` graph replays): every launch
    node with its work and rate, then the per-family figures exactly as the bench line's
    `roofline`, `roofline_mfma_all` and `roofline_non_gemm` compute them."""
    from tensorgrad_amd import backend, configs
    from tensorgrad_amd.build_ir import build_training_ir
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(ir.initial_params(configs.INIT_SEED))
    for i, b in enumerate(configs.batches(cfg, RING)):
        rt.stage_batch(i, b)
    for i in range(warmup):
        rt.step_staged(i % RING)
    replay_ms = rt.time_replays(200) / 200
    nodes = rt.describe()['nodes']
    kms = rt.profile_kernels(iters)
    rt.destroy()
    fam = family_rates(nodes, kms)
    o = [f'# Kernel durations by launch events: {cfg.title}', '',
         f'Command: `python3 bench.py --config {key} --kernel-events`', '',
         f'Every kernel of {iters} eager steps (after {warmup} graph replays) dispatched with start / end events of '
         'its own on the runtime\'s stream (tg_profile_kernels); a node\'s time is the mean over the steps of the sum '
         'of its kernels\' durations, without the gaps between launches. These are the durations the bench line\'s '
         f'rooflines use. Sum per step: {1e3 * sum(kms):.1f} us over {len(nodes)} launch nodes; the graph replay of '
         f'the whole step takes {1e3 * replay_ms:.1f} us.', '',
         '| # | kind | shape | us | algorithmic work | rate |', '|---:|---|---|---:|---:|---:|']
    for i, (n, t) in enumerate(zip(nodes, kms)):
        if n['kind'] in ('gemm', 'conv', 'attention'):
            work = f"{n['flops'] / 1e9:.3f} GFLOP"
            rate = f"{n['flops'] / max(t, 1e-12) / 1e9:.1f} TFLOP/s"
        else:
            work = f"{n['bytes'] / 1e6:.2f} MB"
            rate = f"{n['bytes'] / max(t, 1e-12) / 1e6:.0f} GB/s"
        o.append(f"| {i} | {n['kind']} | {n['shape'][:60]} | {1e3 * t:.2f} | {work} | {rate} |")
    o += ['', '| family | launches | us / step | work / step | rate | of peak |', '|---|---:|---:|---:|---:|---:|']
    for name in ('gemm', 'attention', 'conv'):
        f = fam[name]
        if f['launches']:
            o.append(f"| {name} (f32 MFMA) | {f['launches']} | {1e3 * f['ms']:.1f} | {f['flop_per_step'] / 1e9:.3f} GFLOP | "
                     f"{f['tflops']:.1f} TFLOP/s | {100 * f['frac_f32_peak']:.1f} % |")
    m = fam['mfma_all']
    o.append(f"| all MFMA work | | {1e3 * m['ms']:.1f} | {m['flop_per_step'] / 1e9:.3f} GFLOP | {m['tflops']:.1f} TFLOP/s | "
             f"{100 * m['frac_f32_peak']:.1f} % |")
    ng = fam['non_gemm']
    o.append(f"| other launches (HBM) | {ng['launches']} | {1e3 * ng['ms']:.1f} | {ng['bytes_per_step'] / 1e6:.1f} MB | "
             f"{ng['gbs']:.0f} GB/s | {100 * ng['frac_hbm_peak']:.1f} % |")
    return '\n'.join(o) + '\n'


def copy_probe(n=16 << 20, reps=3):
    """Run a plain streaming copy of known size (y = x * 1.0 over n f32, one fused
    launch reading 4n bytes and writing 4n bytes) so that profiler byte counters can be
    scaled against known traffic. Returns the best kernel-pass time in ms."""
    import numpy as np
    from tensorgrad_amd import backend, ir as IR
    from tensorgrad_amd import ops as O
    from tensorgrad_amd.trace import tensor_input, trace_fn
    g = trace_fn(lambda: O.mul_scalar(tensor_input('x', [n]), 1.0))
    w = {'graph': IR.graph_to_wire(g), 'paramGrads': {}, 'writebacks': [], 'optimizer': None}
    rt = backend.NativeRuntime(IR.dumps(w))
    x = np.ones(n, np.float32)
    for _ in range(reps):
        rt.run({'x': x}, [n], np.float32)
    t, _ = rt.time_kinds('elementwise,fused', 10)
    rt.destroy()
    return t


def profiled_traffic(path):
    """HBM bytes per GEMM launch recorded by the committed rocprofv3 --pmc summary (the
    line 'hbm_bytes_per_launch: N'), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith('hbm_bytes_per_launch:'):
                    return float(line.split(':', 1)[1])
    except OSError:
        pass
    return None


def trace_steps(key, steps, probe):
    """Profiling driver: `steps` training steps of config `key` (staged batches) with
    every launch issued directly, optionally after the streaming-copy probe."""
    os.environ['TG_GRAPH'] = '0'
    from tensorgrad_amd import backend, configs
    from tensorgrad_amd.build_ir import build_training_ir
    if probe:
        copy_probe()
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(ir.initial_params(configs.INIT_SEED))
    for i, b in enumerate(configs.batches(cfg, 2)):
        rt.stage_batch(i, b)
    loss = None
    for i in range(steps):
        loss = rt.step_staged(i % 2)
    rt.destroy()
    print(json.dumps({'trace_steps': steps, 'config': key, 'final_loss': loss, 'copy_probe': bool(probe)}), flush=True)


def vendor_gemm(key, iters=100):
    """For every single-GEMM launch node of config `key` whose operands are 2-D after
    merging the leading dims ("[..,m,k]x[k,n]"): this backend's per-node time (HIP events
    around the node, eager passes) beside the vendor BLAS (torch.matmul in f32 with TF32
    off: hipBLASLt / rocBLAS) on the same M, N, K, the faster of its two B layouts."""
    import torch
    from tensorgrad_amd import backend, configs
    from tensorgrad_amd.build_ir import build_training_ir
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(ir.initial_params(configs.INIT_SEED))
    rt.stage_batch(0, configs.batches(cfg, 1)[0])
    rt.step_staged(0)
    nodes = rt.describe()['nodes']
    ms = rt.profile_nodes(20)
    rt.destroy()

    def lib_us(M, N, K):
        best = None
        a = torch.randn(M, K, device='cuda')
        for bt in (False, True):
            b = torch.randn(N, K, device='cuda').t() if bt else torch.randn(K, N, device='cuda')
            for _ in range(10):
                a @ b
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                a @ b
            e1.record()
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e3 / iters
            best = t if best is None else min(best, t)
        return best

    rows, seen = [], {}
    for n, t in zip(nodes, ms):
        if n['kind'] != 'gemm' or n.get('ops') or 'x[' not in n['shape']:
            continue
        left, right = n['shape'].split('x[', 1)
        right = right.split(']', 1)[0]   # drop a note after the shape (" by 2 sources", ...)
        ld = [int(v) for v in left.strip('[] ').split(',')]
        rd = [int(v) for v in right.strip('[] ').split(',')]
        if len(rd) != 2:
            continue
        M, K, N = 1, ld[-1], rd[-1]
        for v in ld[:-1]:
            M *= v
        if (M, N, K) not in seen:
            seen[(M, N, K)] = lib_us(M, N, K)
        lu = seen[(M, N, K)]
        rows.append({'shape': n['shape'], 'M': M, 'N': N, 'K': K, 'us': round(t * 1e3, 2), 'vendor_us': round(lu, 2),
                     'tflops': round(2.0 * M * N * K / (t * 1e-3) / 1e12, 1),
                     'vendor_tflops': round(2.0 * M * N * K / (lu * 1e-6) / 1e12, 1)})
    print(json.dumps({'vendor_gemm': key, 'nodes': rows}), flush=True)


def cpu_info():
    """nproc (CPUs this process may run on), os.cpu_count() and the CPU model name."""
    model = None
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count()
    return {'nproc': avail, 'cpu_count': os.cpu_count(), 'cpu_model': model}


def cpu_rate(key, threads, min_steps=3, min_seconds=10.0, exact_steps=None):
    """Steps/s of the CPU oracle (the C++ restatement of the reference's CPU evaluator) on
    config `key` with `threads` OpenMP threads: the same model, seed-42 init and batch
    ring as the GPU run. Runs `exact_steps` steps, or else until at least `min_steps`
    steps or at least `min_seconds` have passed (at least one step)."""
    sys.path.insert(0, os.path.join(ROOT, 'oracle'))
    import pyoracle
    from tensorgrad_amd import configs
    from tensorgrad_amd.build_ir import build_training_ir
    pyoracle.set_threads(threads)
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    o = pyoracle.OracleRuntime(ir.wire())
    o.upload_params(ir.initial_params(configs.INIT_SEED))
    bs = configs.batches(cfg, RING)
    n, t0 = 0, time.perf_counter()
    while True:
        o.step(bs[n % RING])
        n += 1
        dt = time.perf_counter() - t0
        if exact_steps is not None:
            if n >= exact_steps:
                break
        elif n >= min_steps or dt >= min_seconds:
            break
        if dt > 20:
            print(f'# cpu {key} threads={threads}: {n} steps, {dt:.1f}s', file=sys.stderr, flush=True)
    return {'steps_per_s': n / dt, 's_per_step': dt / n, 'steps': n, 'seconds': round(dt, 3), 'threads': threads}


def cpu_threads():
    # The GPU box allots 16 host cores per GPU (OMP_NUM_THREADS=16 there); more threads
    # than the allotment would only time oversubscription.
    info = cpu_info()
    return max(1, min(16, info['nproc'] or 1))


def cpu_baseline(key):
    """The headline config's CPU baseline in both modes: `value` from the parallel mode
    (OpenMP over output elements, `cores` threads), `single_thread` beside it."""
    info = cpu_info()
    threads = cpu_threads()
    par = cpu_rate(key, threads, exact_steps=1000 if key == 'mlp_sin' else None)
    one = cpu_rate(key, 1, exact_steps=1000 if key == 'mlp_sin' else None)
    return {'value': par['steps_per_s'], 'unit': 'steps/s', 'cores': threads, 'kind': 'port',
            'sample': f"{par['steps']} full {key} training steps (fwd+bwd+Adam) of the CPU oracle in "
                      f"{par['seconds']}s, OpenMP over output elements",
            'single_thread': {'value': one['steps_per_s'], 'steps': one['steps'], 'seconds': one['seconds']},
            **info}


def cpu_protocol():
    """Every config in both modes: C1 for 1000 steps, the others until 3 steps or 10 s."""
    from tensorgrad_amd import configs
    threads = cpu_threads()
    out = []
    for key in configs.CONFIGS:
        exact = 1000 if key == 'mlp_sin' else None
        row = {'config': key}
        for mode, th in (('parallel', threads), ('single_thread', 1)):
            r = cpu_rate(key, th, exact_steps=exact)
            row[mode] = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in r.items()}
            print(f'# cpu {key} {mode} ({th} threads): {r["s_per_step"]:.4f} s/step over {r["steps"]} steps',
                  file=sys.stderr, flush=True)
        out.append(row)
    return {'cpu_protocol': out, **cpu_info()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--config', default='transformer')
    ap.add_argument('--only', action='store_true', help='measure the headline config only')
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--trace-steps', type=int, default=0,
                    help='only run this many steps of --config with launches issued directly (TG_GRAPH=0: '
                         'profilers trace direct launches, not graph replays), then exit')
    ap.add_argument('--cpu-protocol', action='store_true',
                    help='only time the CPU oracle: every config, single-thread and parallel, then exit')
    ap.add_argument('--profile-iters', type=int, default=5,
                    help='eager steps with per-kernel start/end events for the per-family kernel rates')
    ap.add_argument('--vendor-gemm', action='store_true',
                    help='only compare every single-GEMM node of --config with the vendor BLAS, then exit')
    ap.add_argument('--probe-copy', action='store_true',
                    help='first run a 64 MiB streaming copy (profiler counter calibration)')
    ap.add_argument('--kernel-events', action='store_true',
                    help='only print a markdown report of --config\'s per-launch kernel durations (events), then exit')
    args = ap.parse_args()
    if args.kernel_events:
        print(kernel_events(args.config), end='', flush=True)
        return
    if args.cpu_protocol:
        print(json.dumps(cpu_protocol()), flush=True)
        return
    if args.trace_steps > 0:
        trace_steps(args.config, args.trace_steps, args.probe_copy)
        return
    if args.vendor_gemm:
        vendor_gemm(args.config)
        return
    if args.gpus != 1:
        print(json.dumps({'error': 'this build runs on one GPU per process; multi-GPU data parallelism is '
                                   'designed (DESIGN.md) but not built, so --gpus must be 1'}))
        sys.exit(2)
    from tensorgrad_amd import backend, configs
    if backend.device_count() < 1:
        print(json.dumps({'error': 'no HIP device visible'}))
        sys.exit(1)
    keys = [args.config] + ([] if args.only else [k for k in configs.CONFIGS if k != args.config])
    probe = None
    if args.probe_copy:
        t = copy_probe()
        probe = {'bytes': 2 * 4 * (16 << 20), 'ms': round(t, 4), 'gbs': round(2 * 4 * (16 << 20) / t / 1e6, 1)}
        print(f'# copy probe: {probe}', file=sys.stderr, flush=True)
    results = {}
    for k in keys:
        results[k] = measure(k, args.steps, args.warmup, args.profile_iters)
        print(f'# {k}: {results[k]["steps_per_s"]:.1f} steps/s, replay {results[k]["device_replay_ms"]:.3f} ms',
              file=sys.stderr, flush=True)
        if k == 'transformer' and not args.only:
            # the reference samples' optimizer setting: the same step with global clipping
            cfg5 = configs.CONFIGS[k]
            r = measure(k, args.steps, args.warmup, args.profile_iters,
                        optimizer=dict(cfg5.optimizer, clipGradNorm=1.0), label='transformer_clip')
            results['transformer_clip'] = r
            print(f'# transformer_clip: {r["steps_per_s"]:.1f} steps/s, replay {r["device_replay_ms"]:.3f} ms',
                  file=sys.stderr, flush=True)
    head = results[args.config]
    cpu = None if args.no_cpu else cpu_baseline(args.config)
    cfg = configs.CONFIGS[args.config]
    g = head['gemm']
    line = {
        'metric': 'train steps/sec (fwd+bwd+Adam) per config; % of f32 MFMA / HBM roofline',
        'value': round(head['steps_per_s'], 3),
        'unit': 'steps/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(head['ms_per_step'], 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic (mulberry32(1000+c) batches, seed-42 init); batches staged in HBM before timing',
        'config': {'workload': cfg.title, 'samples_per_step': cfg.samples_per_step, 'sample_unit': cfg.sample_unit,
                   'samples_per_s': round(head['samples_per_s'], 1),
                   'device_replay_ms_per_step': round(head['device_replay_ms'], 4)},
        'roofline': {'bound': 'mfma', 'kernel': 'k_gemm (f32 MFMA GEMM family: every matmul / matmul_batched '
                                                'launch of one step, split-K reductions included)',
                     'achieved': round(g['tflops'], 3), 'peak': PEAK_F32_MFMA_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': round(g['frac_f32_peak'], 4),
                     'traffic': profiled_traffic(os.path.join(ROOT, 'profiles', 'gemm_transformer_traffic.txt')),
                     'timing': 'kernel start/end events of each launch in eager steps (tg_profile_kernels)',
                     'launches_per_step': g['launches'],
                     'avg_launch_us': round(1e3 * g['ms'] / max(g['launches'], 1), 3),
                     'algorithmic_flop_per_launch': round(g['flop_per_step'] / max(g['launches'], 1)),
                     'algorithmic_bytes_per_launch': round(g['bytes_per_step'] / max(g['launches'], 1))},
        'roofline_mfma_all': {'bound': 'mfma', 'kernels': 'GEMMs + fused attention (+ convolutions)',
                              'achieved': round(head['mfma_all']['tflops'], 3), 'peak': PEAK_F32_MFMA_TFLOPS,
                              'unit': 'TFLOP/s', 'frac': round(head['mfma_all']['frac_f32_peak'], 4),
                              'flop_per_step': head['mfma_all']['flop_per_step']},
        'roofline_non_gemm': {'bound': 'hbm', 'achieved': round(head['non_gemm']['gbs'], 1), 'peak': PEAK_HBM_GBS,
                              'unit': 'GB/s', 'frac': round(head['non_gemm']['frac_hbm_peak'], 4),
                              'launches_per_step': head['non_gemm']['launches']},
        'copy_probe': probe,
        'cpu_baseline': None if cpu is None else {k: (round(v, 5) if isinstance(v, float) else v) for k, v in cpu.items()},
        'per_config': [{'config': r['config'], 'steps_per_s': round(r['steps_per_s'], 2),
                        'samples_per_s': round(r['samples_per_s'], 1), 'device_replay_ms': round(r['device_replay_ms'], 4),
                        'kernel_ms_per_step': round(r['kernel_ms_per_step'], 4),
                        'host_batch_steps_per_s': round(r['host_batch_steps_per_s'], 2),
                        'gemm_tflops': round(r['gemm']['tflops'], 2), 'gemm_frac_f32_peak': round(r['gemm']['frac_f32_peak'], 4),
                        'conv_tflops': round(r['conv']['tflops'], 2),
                        'attention_tflops': round(r['attention']['tflops'], 2),
                        'mfma_all_frac_f32_peak': round(r['mfma_all']['frac_f32_peak'], 4),
                        'non_gemm_gbs': round(r['non_gemm']['gbs'], 1),
                        'non_gemm_frac_hbm': round(r['non_gemm']['frac_hbm_peak'], 4),
                        'launch_nodes': r['launch_nodes'], 'kinds': r['kinds'], 'top_gemms': r['gemm']['top']}
                       for r in results.values()],
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()

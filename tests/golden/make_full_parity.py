"""Writes the full-size training fixtures for tests/test_gpu_parity.py: each benchmark
config trained for 100 optimizer steps by the CPU oracle (oracle/, the restatement of the
reference evaluator test/_eval.ts plus the Adam convention of src/codegen.ts:841-905) from
the seeded initial params on the seeded batches that the GPU test regenerates.

Stored per config in full_<key>.npz (numpy, no pickles): the loss of every step, and per
parameter tensor at step 100 either all values (every tensor of the configs in WHOLE, and
tensors up to FULL_LIMIT elements) or a fixed seeded sample of SAMPLE indices, with the
f64 norm of the whole tensor.

For the configs in NTWIN the oracle also trains NTWIN[key] twins from the same initial
parameters moved by one ulp each (a seeded random direction per element, different per
twin), the size of the rounding difference any f32 implementation that is not
bit-identical to the evaluator introduces in its first step; the twins' losses and
step-100 values (same indices) measure how far the workload itself amplifies such a
difference over 100 steps ('twin_losses' [n, steps], 'twin:<param>' [n, sample],
'twin_norm:<param>' [n]). The test bounds each tensor by its farthest twin, so that
spread is estimated from several samples: four for the eight-layer NeRF MLP, two for the
CNN. Per parameter tensor with Adam moments, 'upd:<param>' holds the oracle's own update size at
step 100 on the same indices, |lrt * m / (sqrt(v) + eps)| from its m and v (the scale of an
update gone the other way, which the test's sign-ambiguity floor uses; taken from the
oracle, not from the implementation under test).

For the configs in ARITH_TWINS more twins train from the unperturbed parameters with
another valid rounding at every step rather than once: 'f32', every matmul accumulated in
f32 (pyoracle.set_matmul_f32), as f32 GPU kernels accumulate (the reference's own WGSL
kernels among them); 'sum64', sum_to_shape (the bias and LayerNorm-parameter gradients)
accumulated in f64 and rounded once (pyoracle.set_sum_f64) instead of the evaluator's f32
running sum, as this backend's column sums do. 'twin_kinds' names each twin.

    python tests/golden/make_full_parity.py [keys...] [--threads N]
    python tests/golden/make_full_parity.py nerf --add-twins   # train only the missing twins
    python tests/golden/make_full_parity.py --add-updates      # retrain the base run, check it
                                                               # reproduces the fixture, add upd:
"""
import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, 'oracle'))

import pyoracle  # noqa: E402
from tensorgrad_amd import configs  # noqa: E402
from tensorgrad_amd.build_ir import build_training_ir  # noqa: E402

STEPS = 100
FULL_LIMIT = 16_384
SAMPLE = 4096
WHOLE = {'char_mlp'}
NTWIN = {'cnn': 2, 'nerf': 4}
ARITH_TWINS = {'nerf': ('f32', 'sum64'), 'cnn': ('f32', 'sum64')}
SWITCHES = {'f32': pyoracle.set_matmul_f32, 'sum64': pyoracle.set_sum_f64}


def sample_indices(key: str, name: str, n: int) -> np.ndarray:
    if key in WHOLE or n <= FULL_LIMIT:
        return np.arange(n, dtype=np.int64)
    seed = sum(ord(ch) * (i + 1) for i, ch in enumerate(name)) + n
    return np.sort(np.random.default_rng(seed).choice(n, SAMPLE, replace=False)).astype(np.int64)


def one_ulp(params: dict, twin: int = 0) -> dict:
    """Every element moved to its f32 neighbour, up or down by a seeded coin."""
    out = {}
    for i, (n, v) in enumerate(sorted(params.items())):
        v = np.asarray(v, np.float32)
        up = np.random.default_rng(1000 * (twin + 1) + i).random(v.shape) < 0.5
        out[n] = np.where(up, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(-np.inf))).astype(np.float32)
    return out


def train(key: str, cfg, ir, params: dict, tag: str):
    o = pyoracle.OracleRuntime(ir.wire())
    o.upload_params(params)
    losses = []
    t0 = time.time()
    for i, b in enumerate(configs.batches(cfg, STEPS)):
        losses.append(o.step(b))
        if i % 10 == 9:
            print(f'  [{key}{tag}] step {i + 1} loss {losses[-1]:.9g} ({time.time() - t0:.0f}s)', flush=True)
    return o, np.array(losses, np.float64)


def update_sizes(o, cfg, n: str, size: int, idx: np.ndarray):
    """|lrt * m / (sqrt(v) + eps)| of the oracle's state at step STEPS, or None."""
    opt = cfg.optimizer
    if opt.get('kind', 'adam') not in ('adam', 'adamw'):
        return None
    b1, b2, eps = opt.get('beta1', 0.9), opt.get('beta2', 0.999), opt.get('eps', 1e-8)
    lrt = pyoracle.resolve_lr(opt['lr'], STEPS) * np.sqrt(1 - b2 ** STEPS) / (1 - b1 ** STEPS)
    m = o.get_home(f'adam_m_{n}', size).astype(np.float64)[idx]
    v = o.get_home(f'adam_v_{n}', size).astype(np.float64)[idx]
    return np.abs(lrt * m / (np.sqrt(v) + eps))


def base_run(key: str, cfg, ir) -> dict:
    p0 = ir.initial_params(configs.INIT_SEED)
    o, losses = train(key, cfg, ir, p0, '')
    out = {'losses': losses, 'steps': np.array(STEPS)}
    shapes = ir.param_shapes()
    sizes = {n: int(np.prod(shapes[n])) if shapes[n] else 1 for n in ir.param_names}
    for n in ir.param_names:
        v = o.get_home(n, sizes[n])
        idx = sample_indices(key, n, sizes[n])
        out[f'idx:{n}'] = idx
        out[f'val:{n}'] = v[idx]
        out[f'norm:{n}'] = np.array(np.linalg.norm(v.astype(np.float64)))
        u = update_sizes(o, cfg, n, sizes[n], idx)
        if u is not None:
            out[f'upd:{n}'] = u
    return out


def make(key: str) -> str:
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    p0 = ir.initial_params(configs.INIT_SEED)
    out = base_run(key, cfg, ir)
    if key in NTWIN:
        add_twins(key, cfg, ir, p0, out, 0)
    path = os.path.join(HERE, f'full_{key}.npz')
    np.savez_compressed(path, **out)
    return path


def add_twins(key: str, cfg, ir, p0: dict, out: dict, have: int):
    """Train the one-ulp twins have .. NTWIN[key] - 1 and the ARITH_TWINS kinds the
    fixture lacks, and append them to the fixture dict `out`."""
    shapes = ir.param_shapes()
    sizes = {n: int(np.prod(shapes[n])) if shapes[n] else 1 for n in ir.param_names}
    kinds = [str(k) for k in out['twin_kinds']] if 'twin_kinds' in out else ['ulp'] * have
    runs, new_kinds = [], []
    for j in range(have, NTWIN[key]):
        runs.append(train(key, cfg, ir, one_ulp(p0, j), f' twin {j}'))
        new_kinds.append('ulp')
    for kind in ARITH_TWINS.get(key, ()):
        if kind in kinds:
            continue
        SWITCHES[kind](True)
        try:
            runs.append(train(key, cfg, ir, p0, f' {kind} twin'))
        finally:
            SWITCHES[kind](False)
        new_kinds.append(kind)
    if not runs:
        return
    new_l = np.stack([tl for _, tl in runs])
    out['twin_losses'] = np.concatenate([out['twin_losses'], new_l]) if have else new_l
    out['twin_kinds'] = np.array(kinds + new_kinds)
    for n in ir.param_names:
        vs = [t.get_home(n, sizes[n]) for t, _ in runs]
        val = np.stack([v[out[f'idx:{n}']] for v in vs])
        nrm = np.array([np.linalg.norm(v.astype(np.float64)) for v in vs])
        out[f'twin:{n}'] = np.concatenate([out[f'twin:{n}'], val]) if have else val
        out[f'twin_norm:{n}'] = np.concatenate([out[f'twin_norm:{n}'], nrm]) if have else nrm


def extend(key: str) -> str:
    """Add the missing twins to an existing fixture (its base run and twins are kept)."""
    path = os.path.join(HERE, f'full_{key}.npz')
    with np.load(path) as z:
        out = {k: z[k] for k in z.files}
    have = int(np.sum(out['twin_kinds'] == 'ulp')) if 'twin_kinds' in out else (
        out['twin_losses'].shape[0] if 'twin_losses' in out else 0)
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    add_twins(key, cfg, ir, ir.initial_params(configs.INIT_SEED), out, have)
    np.savez_compressed(path, **out)
    return path


def add_updates(key: str) -> str:
    """Train the base run again, check that it reproduces the stored losses and values
    bit for bit, and store its update sizes."""
    path = os.path.join(HERE, f'full_{key}.npz')
    with np.load(path) as z:
        out = {k: z[k] for k in z.files}
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    new = base_run(key, cfg, ir)
    for k, v in new.items():
        if k.startswith('upd:'):
            out[k] = v
        elif not np.array_equal(np.asarray(out[k]), np.asarray(v)):
            raise SystemExit(f'{key}: the base run no longer reproduces {k}')
    np.savez_compressed(path, **out)
    return path


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('keys', nargs='*', default=['char_mlp', 'cnn', 'transformer', 'nerf'])
    ap.add_argument('--threads', type=int, default=os.cpu_count() or 8)
    ap.add_argument('--add-twins', action='store_true', help='only train the twins the fixture lacks')
    ap.add_argument('--add-updates', action='store_true',
                    help='retrain the base run, check it reproduces the fixture, store the update sizes')
    a = ap.parse_args()
    pyoracle.set_threads(a.threads)
    for k in a.keys:
        if a.add_updates:
            print(k, '->', add_updates(k), flush=True)
        if a.add_twins:
            print(k, '->', extend(k), flush=True)
        if not (a.add_updates or a.add_twins):
            print(k, '->', make(k), flush=True)


if __name__ == '__main__':
    main()

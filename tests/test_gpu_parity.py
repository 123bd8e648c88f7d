"""Training parity on the GPU: each benchmark config trains through the C ABI and through
the CPU oracle from identical seeded params and batches.

Bar (the north star's): f32 losses within 1e-4 relative at every step, and every
parameter tensor within 1e-4 relative (L2 norm of the difference over the norm of the
oracle's tensor) after 100 optimizer steps. Reduced-size variants with the same topology
run the full 100 steps; the full-size configs run the steps the oracle can afford.
"""
import time

import numpy as np
import pytest

import pyoracle
from tensorgrad_amd import backend, configs
from tensorgrad_amd.build_ir import build_training_ir

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-4
PARAM_TOL = 1e-4


def _train_both(cfg, steps, seed=42, opt=None):
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, opt or cfg.optimizer)
    rt = backend.NativeRuntime(ir.wire_json())
    o = pyoracle.OracleRuntime(ir.wire())
    p0 = ir.initial_params(seed)
    rt.upload_params(p0)
    o.upload_params(p0)
    worst_loss = 0.0
    exact_losses = 0
    for i, b in enumerate(configs.batches(cfg, steps)):
        lg, lo = rt.step(b), o.step(b)
        r = abs(lg - lo) / max(abs(lo), 1e-30)
        worst_loss = max(worst_loss, r)
        exact_losses += int(np.float32(lg) == np.float32(lo))
        print(f'  [{cfg.key}] step {i + 1}: gpu {lg:.9g} oracle {lo:.9g}', flush=True) if i in (0, steps - 1) else None
    pg = rt.download_params()
    worst_param = 0.0
    for n in ir.param_names:
        po = o.get_home(n, pg[n].size).astype(np.float64)
        d = np.linalg.norm(pg[n].astype(np.float64) - po) / max(np.linalg.norm(po), 1e-30)
        worst_param = max(worst_param, d)
    rt.destroy()
    print(f'  [{cfg.key}] {steps} steps: worst loss rel {worst_loss:.2e} ({exact_losses} bit-exact), '
          f'worst param rel {worst_param:.2e}', flush=True)
    return worst_loss, worst_param


@pytest.mark.parametrize('key', ['mlp_sin', 'char_mlp', 'cnn', 'nerf', 'transformer'])
def test_small_variant_100_steps(key):
    wl, wp = _train_both(configs.small_variant(key), 100)
    assert wl <= LOSS_TOL and wp <= PARAM_TOL


@pytest.mark.parametrize('key,steps', [('mlp_sin', 100), ('char_mlp', 10), ('cnn', 3), ('transformer', 2), ('nerf', 1)])
def test_full_config_parity(key, steps):
    pyoracle.set_threads(16)
    t0 = time.time()
    wl, wp = _train_both(configs.CONFIGS[key], steps)
    print(f'  [{key}] {time.time() - t0:.1f}s', flush=True)
    assert wl <= LOSS_TOL and wp <= PARAM_TOL


def test_sgd_momentum_nesterov_and_scheduled_adamw():
    cfg = configs.small_variant('mlp_sin')
    wl, wp = _train_both(cfg, 40, opt={'kind': 'sgd', 'lr': 0.01, 'momentum': 0.9, 'nesterov': True,
                                       'weightDecay': 1e-3})
    assert wl <= LOSS_TOL and wp <= PARAM_TOL
    sched = {'kind': 'warmup', 'peak': 3e-3, 'steps': 5, 'after': {'kind': 'cosineAnnealing', 'peak': 3e-3,
                                                                   'final': 1e-4, 'steps': 30}}
    wl, wp = _train_both(configs.small_variant('char_mlp'), 40,
                         opt={'kind': 'adamw', 'lr': sched, 'weightDecay': 0.05, 'clipGradNorm': 0.5})
    assert wl <= LOSS_TOL and wp <= PARAM_TOL
    wl, wp = _train_both(configs.small_variant('nerf'), 30, opt={'kind': 'adam', 'lr': 1e-3, 'normalizeGrads': True})
    assert wl <= LOSS_TOL and wp <= PARAM_TOL

"""Training parity on the GPU: each benchmark config trains through the C ABI and through
the CPU oracle from identical seeded params and batches.

Bar (the north star's): f32 losses within 1e-4 relative at every step, and every
parameter tensor within 1e-4 relative (L2 norm of the difference over the norm of the
oracle's tensor) after 100 optimizer steps. Reduced-size variants with the same topology
run the full 100 steps; the full-size configs run the steps the oracle can afford.
"""
import os
import time

import numpy as np
import pytest

import pyoracle
from _helpers import rel_err, sign_ambiguous
from tensorgrad_amd import backend, configs
from tensorgrad_amd.build_ir import build_training_ir

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-4
PARAM_TOL = 1e-4
GRAD_TOL = 1e-4


def _train_both(cfg, steps, seed=42, opt=None, flip_step=None):
    """Train the GPU runtime and the oracle side by side; return (worst loss rel error,
    worst per-tensor param rel error, number of sign-ambiguous elements).

    With `flip_step` set, parameter elements that differ by at least flip_step / 4 are
    counted as sign-ambiguous and left out of the parameter error (see
    test_full_config_parity)."""
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
        worst_loss = max(worst_loss, rel_err(lg, lo, f'[{cfg.key}] step {i + 1} loss'))
        exact_losses += int(np.float32(lg) == np.float32(lo))
        print(f'  [{cfg.key}] step {i + 1}: gpu {lg:.9g} oracle {lo:.9g}', flush=True) if i in (0, steps - 1) else None
    pg = rt.download_params()
    worst_param, worst_name, worst_max = 0.0, '', 0.0
    flips = 0
    for n in ir.param_names:
        po = o.get_home(n, pg[n].size).astype(np.float64)
        diff = pg[n].astype(np.float64) - po
        if not np.all(np.isfinite(diff)):
            raise AssertionError(f'[{cfg.key}] {n}: non-finite parameters')
        if flip_step is not None:
            amb = sign_ambiguous(diff, flip_step, steps)
            flips += int(amb.sum())
            if amb.any():
                print(f'  [{cfg.key}] {n}: sign-ambiguous at {np.flatnonzero(amb)[:16].tolist()}', flush=True)
            diff = np.where(amb, 0.0, diff)
        d = rel_err(po + diff, po, f'[{cfg.key}] {n}')
        if d > worst_param:
            worst_param, worst_name, worst_max = d, n, float(np.max(np.abs(diff)))
    rt.destroy()
    print(f'  [{cfg.key}] {steps} steps: worst loss rel {worst_loss:.2e} ({exact_losses} bit-exact), '
          f'worst param rel {worst_param:.2e} ({worst_name}, max |diff| {worst_max:.2e})'
          + (f', {flips} sign-ambiguous elements' if flip_step else ''), flush=True)
    return worst_loss, worst_param, flips


def _update_error(cfg, seed=42, opt=None, want_ops=None):
    """One plain SGD step (no momentum) from identical params and batch on both sides: the
    update p1 - p0 = -lr * g, so its per-tensor relative error is the gradient's. lr is a
    large power of two so that |lr * g| dwarfs |p0| and the f32 rounding of p1 does not
    hide the gradient's low digits. `opt` replaces the optimizer; `want_ops` names a launch
    the plan must contain."""
    opt = opt or {'kind': 'sgd', 'lr': float(2 ** 24)}
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, opt)
    rt = backend.NativeRuntime(ir.wire_json())
    if want_ops:
        assert want_ops in [n.get('ops', '') for n in rt.describe()['nodes']]
    o = pyoracle.OracleRuntime(ir.wire())
    p0 = ir.initial_params(seed)
    rt.upload_params(p0)
    o.upload_params(p0)
    b = configs.batches(cfg, 1)[0]
    rt.step(b)
    o.step(b)
    pg = rt.download_params()
    worst = 0.0
    for n in ir.param_names:
        start = np.asarray(p0[n], np.float64).reshape(-1)
        ug = pg[n].astype(np.float64) - start
        uo = o.get_home(n, pg[n].size).astype(np.float64) - start
        worst = max(worst, rel_err(ug, uo, f'[{cfg.key}] {n} update'))
    rt.destroy()
    print(f'  [{cfg.key}] gradient (SGD update) worst rel {worst:.2e}', flush=True)
    return worst


@pytest.mark.parametrize('key', ['transformer'])
def test_grouped_weight_gradients(key):
    """Weight gradients that only Adam reads run as one grouped GEMM launch (whole-K tiles)
    just before it. Adam's first update is lr * g / (|g| + eps); with eps = 2^20 far above
    every |g| it is (lr / eps) * g to a relative 1e-6 or better, the same on both sides, so
    lr = 2^44 turns it into the SGD gradient check above."""
    w = _update_error(configs.CONFIGS[key], opt={'kind': 'adam', 'lr': float(2 ** 44), 'eps': float(2 ** 20)},
                      want_ops='gemm_group')
    assert w <= GRAD_TOL


def test_recomputed_values_are_bit_identical():
    """Element groups that evaluate another group's pointwise chain again (the GELU
    backward recomputing the pre-activation and exp terms from the GEMM output) run the
    same per-element code as the group that used to store them: two training steps give
    the same parameters bit for bit with recomputation off (TG_REMAT=0) and on."""
    cfg = configs.small_variant('transformer')
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    p0 = ir.initial_params(3)
    batches = configs.batches(cfg, 2)
    out = {}
    for remat in ('0', '1'):
        old = os.environ.get('TG_REMAT')
        os.environ['TG_REMAT'] = remat
        try:
            rt = backend.NativeRuntime(ir.wire_json())
        finally:
            if old is None:
                os.environ.pop('TG_REMAT', None)
            else:
                os.environ['TG_REMAT'] = old
        shapes = [n['shape'] for n in rt.describe()['nodes']]
        assert any('recomputed' in s for s in shapes) == (remat == '1'), shapes
        rt.upload_params(p0)
        for b in batches:
            rt.step(b)
        out[remat] = rt.download_params()
        rt.destroy()
    for n in ir.param_names:
        assert np.array_equal(out['0'][n].view(np.uint32), out['1'][n].view(np.uint32)), n


@pytest.mark.parametrize('key', ['mlp_sin', 'char_mlp', 'cnn', 'nerf', 'transformer'])
def test_small_variant_100_steps(key):
    wl, wp, _ = _train_both(configs.small_variant(key), 100)
    assert wl <= LOSS_TOL and wp <= PARAM_TOL


@pytest.mark.parametrize('key,steps', [('mlp_sin', 100), ('char_mlp', 10), ('cnn', 3), ('transformer', 2), ('nerf', 1)])
def test_full_config_parity(key, steps):
    """Full-size configs with their own optimizer, for as many steps as the oracle affords.

    Adam's first updates are lr * g / (|g| + eps), about lr * sign(g): a gradient entry
    whose exact value lies inside the f32 rounding noise of its GEMM (the GPU accumulates
    in f32, the evaluator in f64) can move either way by lr. One such entry among the cnn's
    1.2M fc weights moves that tensor's relative error by ~2e-4 after 3 steps, so after a
    few steps at full size those elements (|diff| >= lr / 4; ordinary differences are
    ~1e-7) are counted, bounded, and left out of the 1e-4 parameter bar. The reduced
    variants above apply the bar to every element after 100 steps, and
    test_full_config_gradients checks the full-size gradients directly."""
    pyoracle.set_threads(16)
    t0 = time.time()
    cfg = configs.CONFIGS[key]
    lr = cfg.optimizer['lr']
    wl, wp, flips = _train_both(cfg, steps, flip_step=None if steps >= 100 else lr)
    print(f'  [{key}] {time.time() - t0:.1f}s', flush=True)
    assert wl <= LOSS_TOL and wp <= PARAM_TOL
    n_params = sum(int(np.prod(s)) for s in build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs,
                                                                cfg.optimizer).param_shapes().values())
    assert flips <= max(4, 1e-5 * n_params * steps)


@pytest.mark.parametrize('key', ['char_mlp', 'cnn', 'transformer', 'nerf'])
def test_full_config_gradients(key):
    pyoracle.set_threads(16)
    assert _update_error(configs.CONFIGS[key]) <= GRAD_TOL


def test_sgd_momentum_nesterov_and_scheduled_adamw():
    cfg = configs.small_variant('mlp_sin')
    wl, wp, _ = _train_both(cfg, 40, opt={'kind': 'sgd', 'lr': 0.01, 'momentum': 0.9, 'nesterov': True,
                                       'weightDecay': 1e-3})
    assert wl <= LOSS_TOL and wp <= PARAM_TOL
    sched = {'kind': 'warmup', 'peak': 3e-3, 'steps': 5, 'after': {'kind': 'cosineAnnealing', 'peak': 3e-3,
                                                                   'final': 1e-4, 'steps': 30}}
    wl, wp, _ = _train_both(configs.small_variant('char_mlp'), 40,
                         opt={'kind': 'adamw', 'lr': sched, 'weightDecay': 0.05, 'clipGradNorm': 0.5})
    assert wl <= LOSS_TOL and wp <= PARAM_TOL
    wl, wp, _ = _train_both(configs.small_variant('nerf'), 30, opt={'kind': 'adam', 'lr': 1e-3, 'normalizeGrads': True})
    assert wl <= LOSS_TOL and wp <= PARAM_TOL

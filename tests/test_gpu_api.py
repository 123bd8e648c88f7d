"""The compile / step API on the GPU (reference surface of src/compile.ts:198-319 and the
worker handlers of src/worker.ts): step results, strict parameter upload, reset, setLR,
attach (forward siblings sharing parameters, polymorphic batch), captures,
replaceModel, destroy -> aborted."""
import numpy as np
import pytest

import pyoracle
from tensorgrad_amd import configs, nn
from tensorgrad_amd import ops as O
from tensorgrad_amd.backend import BackendError
from tensorgrad_amd.build_ir import build_training_ir
from tensorgrad_amd.compile import compile as tg_compile
from tensorgrad_amd.module import Module
from tensorgrad_amd.trace import capture

pytestmark = pytest.mark.gpu


def _close(got, want):
    # GEMMs accumulate in f32 on the matrix cores where the evaluator accumulates in f64,
    # so losses agree to f32 rounding noise, not bit for bit.
    assert abs(got - want) <= 1e-5 * abs(want), (got, want)


def _c1():
    cfg = configs.CONFIGS['mlp_sin']
    return cfg, tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=42)


def test_step_matches_oracle_and_returns_completed():
    cfg, t = _c1()
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    o = pyoracle.OracleRuntime(ir.wire())
    o.upload_params(ir.initial_params(42))
    for b in configs.batches(cfg, 5):
        r = t.step(b)
        assert r.kind == 'completed'
        _close(r.loss, o.step(b))
    assert t.param_names == ['l1.W', 'l1.b', 'l2.W', 'l2.b', 'l3.W', 'l3.b']
    t.destroy()


def test_upload_download_roundtrip_and_strictness():
    cfg, t = _c1()
    p = t.download_params()
    p2 = {k: (v + 1).astype(np.float32) for k, v in p.items()}
    t.upload_params(p2)
    back = t.download_params()
    assert all(np.array_equal(back[k], p2[k]) for k in p)
    missing = dict(p2)
    missing.pop('l1.W')
    with pytest.raises(BackendError, match='missing'):
        t.upload_params(missing)
    with pytest.raises(BackendError, match='unknown'):
        t.upload_params(dict(p2, bogus=np.zeros(3, np.float32)))
    with pytest.raises(BackendError):
        t.upload_params(dict(p2, **{'l1.b': np.zeros(3, np.float32)}))
    t.destroy()


def test_step_input_validation_fails_not_raises():
    cfg, t = _c1()
    r = t.step({'x': np.zeros((255, 1), np.float32), 'y': np.zeros((256, 1), np.float32)})
    assert r.kind == 'failed' and 'bytes' in str(r.error)
    r = t.step({'x': np.zeros((256, 1), np.float32)})
    assert r.kind == 'failed' and 'missing' in str(r.error)
    t.destroy()


def test_failed_step_still_consumes_t_and_seed():
    """The worker bumps the optimizer step and the PRNG counter before the runtime checks
    the inputs (src/worker.ts:225), so after a rejected step the next good step runs at
    t = 2 with seed 2 on both sides. The transformer variant uses dropout, so a seed that
    did not advance changes the loss."""
    cfg = configs.small_variant('transformer')
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    t = tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=7)
    o = pyoracle.OracleRuntime(ir.wire())
    o.upload_params(ir.initial_params(7))
    b = configs.batches(cfg, 1)[0]
    bad = {k: v for k, v in b.items() if k != next(iter(b))}
    r = t.step(bad)
    assert r.kind == 'failed' and 'missing' in str(r.error)
    with pytest.raises(RuntimeError, match='missing'):
        o.step(bad)
    _close(t.step(b).loss, o.step(b))
    p = t.download_params()
    for n in ir.param_names:
        po = o.get_home(n, p[n].size)
        assert np.linalg.norm(p[n].reshape(-1) - po) <= 1e-5 * max(np.linalg.norm(po), 1e-30), n
    t.destroy()


def test_run_on_a_training_graph_is_rejected():
    """`run` injects only the PRNG seed (src/worker.ts:242-250): on a training graph the
    optimizer's per-step scalar is a missing input, so nothing trains."""
    from tensorgrad_amd.backend import NativeRuntime
    cfg = configs.CONFIGS['mlp_sin']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    rt = NativeRuntime(ir.wire_json())
    p0 = ir.initial_params(42)
    rt.upload_params(p0)
    with pytest.raises(BackendError, match='missing input'):
        rt.run(configs.batches(cfg, 1)[0], (), np.float32)
    after = rt.download_params()
    assert all(np.array_equal(after[k].reshape(-1), np.asarray(p0[k], np.float32).reshape(-1)) for k in p0)
    rt.destroy()


def test_reset_restores_initial_state():
    cfg, t = _c1()
    bs = configs.batches(cfg, 3)
    first = [t.step(b).loss for b in bs]
    t.reset()
    again = [t.step(b).loss for b in bs]
    assert first == again
    t.reset(params=False, optimizer=True)
    t.destroy()


def test_set_lr_rebases_like_the_oracle():
    cfg = configs.CONFIGS['mlp_sin']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    t = tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=42)
    o = pyoracle.OracleRuntime(ir.wire())
    o.upload_params(ir.initial_params(42))
    bs = configs.batches(cfg, 12)
    sched = {'kind': 'linear', 'peak': 0.01, 'final': 0.001, 'steps': 5}
    for i, b in enumerate(bs):
        if i == 4:
            t.set_lr(sched)
            o.set_lr(sched)
        _close(t.step(b).loss, o.step(b))
    t.destroy()


def test_attach_shares_params_and_caches_shapes():
    cfg, t = _c1()

    def predict(m, inp):
        return m.l3.fwd(O.relu(m.l2.fwd(O.relu(m.l1.fwd(inp['x'])))))
    f = t.attach(predict, {'x': [None, 1]}, max_cached_shapes=2)
    x = np.linspace(-3, 3, 10, dtype=np.float32).reshape(10, 1)
    r1 = f.run({'x': x})
    assert r1.kind == 'completed' and r1.output.shape == (10, 1)
    t.step(configs.batches(cfg, 1)[0])      # training updates are visible to the sibling
    r2 = f.run({'x': x})
    assert not np.array_equal(r1.output, r2.output)
    # same params on the host side give the same prediction through the oracle
    g = f.graph_for({'x': x})
    o = pyoracle.OracleRuntime({'graph': __import__('tensorgrad_amd').ir.graph_to_wire(g.graph), 'paramGrads': {},
                                'writebacks': [], 'optimizer': None})
    o.upload_params(t.download_params())
    o.run({'x': x})
    np.testing.assert_allclose(r2.output, o.output(), rtol=2e-6, atol=1e-7)
    for n in (1, 3, 7):
        assert f.run({'x': np.zeros((n, 1), np.float32)}).output.shape == (n, 1)
    assert len(f._cache) == 2
    t.destroy()
    assert f.run({'x': x}).kind == 'aborted'


def test_captures_and_replace_model():
    class Cap(Module):
        def __init__(self):
            self.l1 = nn.Linear(1, 8)
            self.l2 = nn.Linear(8, 1)

    def loss(m, inp):
        h = capture('hidden', O.relu(m.l1.fwd(inp['x'])))
        return O.mean(O.square(O.sub(m.l2.fwd(h), inp['y'])))
    inputs = {'x': [16, 1], 'y': [16, 1]}
    t = tg_compile(Cap(), loss, inputs, {'kind': 'adam', 'lr': 1e-2}, seed=3)
    x = np.linspace(-1, 1, 16, dtype=np.float32).reshape(16, 1)
    r = t.step({'x': x, 'y': np.sin(x)})
    h = r.captures.get('hidden')
    assert h.shape == (16, 8) and np.all(h >= 0)
    assert r.captures.shape('hidden') == (16, 8)
    t.replace_model(configs.SinMLP(hidden=4), seed=1)
    assert 'l3.W' in t.param_names and t.download_params()['l1.W'].size == 4
    with pytest.raises(ValueError):
        t.replace_model(Cap(), optimizer={'kind': 'sgd', 'lr': 0.1})
    t.destroy()
    assert t.step({'x': x, 'y': x}).kind == 'aborted'


def _predict(m, inp):
    return m.l3.fwd(O.relu(m.l2.fwd(O.relu(m.l1.fwd(inp['x'])))))


def _oracle_forward(ir, params, inputs):
    from tensorgrad_amd import ir as IR
    o = pyoracle.OracleRuntime({'graph': IR.graph_to_wire(ir.graph), 'paramGrads': {}, 'writebacks': [],
                                'optimizer': None})
    o.upload_params(params)
    o.run(inputs)
    return o.output()


def test_compile_forward_owns_its_params():
    """compileForward (compile.ts:424-452, :895-1018): concrete shapes create the owner
    eagerly with params from mulberry32(seed); run matches the oracle."""
    from tensorgrad_amd.build_ir import build_forward_ir
    from tensorgrad_amd.compile import compile_forward
    f = compile_forward(configs.SinMLP(), _predict, {'x': [10, 1]}, seed=5)
    assert f.param_names == ['l1.W', 'l1.b', 'l2.W', 'l2.b', 'l3.W', 'l3.b']
    ir = build_forward_ir(configs.SinMLP(), _predict, {'x': [10, 1]})
    p0 = ir.initial_params(5)
    got = f.download_params()
    assert all(np.array_equal(got[k], np.asarray(p0[k], np.float32).reshape(-1)) for k in p0)
    x = np.linspace(-3, 3, 10, dtype=np.float32).reshape(10, 1)
    r = f.run({'x': x})
    assert r.kind == 'completed'
    np.testing.assert_allclose(r.output, _oracle_forward(ir, p0, {'x': x}), rtol=2e-6, atol=1e-7)
    f.destroy()
    assert f.run({'x': x}).kind == 'aborted'


def test_compile_forward_parametric_shapes_and_buffered_upload():
    from tensorgrad_amd.build_ir import build_forward_ir
    from tensorgrad_amd.compile import compile_forward
    f = compile_forward(configs.SinMLP(), _predict, {'x': [None, 1]}, max_cached_shapes=2, seed=9)
    with pytest.raises(RuntimeError, match='before any params exist'):
        f.download_params()
    rng = np.random.default_rng(3)
    ir = build_forward_ir(configs.SinMLP(), _predict, {'x': [4, 1]})
    mine = {k: rng.standard_normal(np.shape(v)).astype(np.float32) for k, v in ir.initial_params(0).items()}
    f.upload_params(dict(list(mine.items())[:3]))
    f.upload_params(dict(list(mine.items())[3:]))          # merged with the first call
    for n in (4, 7, 1, 7):
        x = rng.standard_normal((n, 1)).astype(np.float32)
        r = f.run({'x': x})
        assert r.kind == 'completed' and r.output.shape == (n, 1)
        irn = build_forward_ir(configs.SinMLP(), _predict, {'x': [n, 1]})
        np.testing.assert_allclose(r.output, _oracle_forward(irn, mine, {'x': x}), rtol=2e-6, atol=1e-7)
    assert len(f._cache) == 2          # 7 and 1; the owner (4) is held apart, never evicted
    back = f.download_params()
    assert all(np.array_equal(back[k], mine[k].reshape(-1)) for k in mine)
    f.destroy()


def test_checkpoint_resume_is_bit_identical():
    """50 steps, save, a fresh compile (other init seed) loads the file, 50 more steps:
    losses and params equal 100 straight steps bit for bit. The transformer variant
    uses dropout, so the restored seed counter matters, and AdamW's t feeds lrt."""
    import os
    import tempfile
    from tensorgrad_amd.safetensors import load_safetensors
    cfg = configs.small_variant('transformer')
    bs = configs.batches(cfg, 100)
    a = tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=11)
    straight = [a.step(b).loss for b in bs]
    want = a.download_params()
    want_state, want_t, want_c = a.download_optimizer_state()
    a.destroy()
    b1 = tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=11)
    first = [b1.step(b).loss for b in bs[:50]]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, 'ckpt.safetensors')
        b1.save_checkpoint(path)
        b1.destroy()
        with open(path, 'rb') as fh:
            saved = load_safetensors(fh.read())
        assert saved.metadata['tensorgrad.step'] == '50' and saved.metadata['tensorgrad.prngCounter'] == '50'
        assert set(saved.tensors) == set(want) | set(want_state)
        b2 = tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=12345)
        b2.load_checkpoint(path)
    second = [b2.step(b).loss for b in bs[50:]]
    assert first + second == straight
    got = b2.download_params()
    for k in want:
        assert np.array_equal(got[k].view(np.uint32), want[k].view(np.uint32)), k
    st, t, c = b2.download_optimizer_state()
    assert (t, c) == (want_t, want_c) == (100, 100)
    for k in want_state:
        assert np.array_equal(st[k].view(np.uint32), want_state[k].view(np.uint32)), k
    b2.destroy()


def test_optimizer_state_upload_is_strict_and_resumes():
    cfg, t = _c1()
    bs = configs.batches(cfg, 6)
    for b in bs[:3]:
        t.step(b)
    p, (st, step_t, cnt) = t.download_params(), t.download_optimizer_state()
    rest = [t.step(b).loss for b in bs[3:]]
    u = tg_compile(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer, seed=1)
    missing = dict(st)
    missing.pop(next(iter(missing)))
    with pytest.raises(BackendError, match='missing'):
        u.upload_optimizer_state(missing, step_t, cnt)
    u.upload_params(p)
    u.upload_optimizer_state(st, step_t, cnt)
    assert [u.step(b).loss for b in bs[3:]] == rest
    t.destroy()
    u.destroy()

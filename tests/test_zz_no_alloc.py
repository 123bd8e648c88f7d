"""tg_step_noalloc through the C ABI: the scratch-only step gives the same losses and
parameters, bit for bit, as tg_step_device on a twin runtime, on two calls in a row
(the full CNN, then its reduced variant: a smaller input and a smaller scratch footprint
of convolution weight-gradient partials, so stale scratch contents from the first call
would show), and rejects a graph whose scratch need exceeds the static array."""
import numpy as np
import pytest

from _helpers import HipBuffers
from tensorgrad_amd import backend, configs, nn
from tensorgrad_amd import ops as O
from tensorgrad_amd.backend import BackendError
from tensorgrad_amd.build_ir import build_training_ir
from tensorgrad_amd.module import Module

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20   # TG_SCRATCH_BYTES in include/tg.h


def _twin_steps(cfg, steps):
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    plan = backend.plan(ir.wire_json())
    print(f'  [{cfg.key}] workspace {plan["workspace_bytes"]} bytes', flush=True)
    ref = backend.NativeRuntime(ir.wire_json())
    na = backend.NativeRuntime(ir.wire_json())
    p0 = ir.initial_params(42)
    ref.upload_params(p0)
    na.upload_params(p0)
    for b in configs.batches(cfg, steps):
        d = HipBuffers(b)
        lr = ref.step_device(d.names, d.ptrs, d.nbytes)
        ln = na.step_noalloc(d.names, d.ptrs, d.nbytes)
        d.free()
        assert np.float32(lr).view(np.uint32) == np.float32(ln).view(np.uint32), (lr, ln)
    pr, pn = ref.download_params(), na.download_params()
    for k in pr:
        assert np.array_equal(pr[k].view(np.uint32), pn[k].view(np.uint32)), k
    sr, tr, cr = ref.download_state()
    sn, tn, cn = na.download_state()
    assert (tr, cr) == (tn, cn)
    for k in sr:
        assert np.array_equal(sr[k].view(np.uint32), sn[k].view(np.uint32)), k
    ref.destroy()
    na.destroy()
    return plan['workspace_bytes']


def test_step_noalloc_matches_step_device_twice():
    big = _twin_steps(configs.CONFIGS['cnn'], 3)
    small = _twin_steps(configs.small_variant('cnn'), 3)
    assert 0 < small < big <= SCRATCH_BYTES


def test_step_noalloc_rejects_graphs_beyond_the_scratch():
    class E(Module):
        def __init__(self):
            self.emb = nn.Embedding(10, 32)

    def loss(m, inp):
        return O.mean(O.square(m.emb.fwd(inp['tok'])))
    inputs = {'tok': {'shape': [1 << 20], 'dtype': 'i32'}}
    ir = build_training_ir(E(), loss, inputs, {'kind': 'adam', 'lr': 1e-3})
    assert backend.plan(ir.wire_json())['workspace_bytes'] > SCRATCH_BYTES
    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(ir.initial_params(1))
    tok = np.zeros(1 << 20, np.int32)
    d = HipBuffers({'tok': tok})
    with pytest.raises(BackendError, match='bytes of scratch'):
        rt.step_noalloc(d.names, d.ptrs, d.nbytes)
    rt.step_device(d.names, d.ptrs, d.nbytes)     # the regular entry point still works
    d.free()
    rt.destroy()

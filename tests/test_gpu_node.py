"""Training driven from Node through the N-API addon and the WorkerProxy shim, on the
GPU: createRuntime with a reference-shaped payload, steps, downloadParams, a
compileForward sibling's run and destroy -> AbortError, compared bit for bit with the
same calls made through ctypes."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from _refplan import reference_payload
from tensorgrad_amd import backend, configs
from tensorgrad_amd import ops as O
from tensorgrad_amd.build_ir import build_forward_ir, build_training_ir

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which('node')

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(NODE is None, reason='node is not installed')]


def _rec(d):
    return {k: {'dtype': 'i32' if np.asarray(v).dtype == np.int32 else 'f32',
                'data': np.asarray(v).reshape(-1).tolist()} for k, v in d.items()}


def _predict(m, inp):
    return m.l3.fwd(O.relu(m.l2.fwd(O.relu(m.l1.fwd(inp['x'])))))


@pytest.mark.parametrize('key', ['mlp_sin', 'transformer'])
def test_node_shim_trains_like_ctypes(tmp_path, key):
    cfg = configs.CONFIGS['mlp_sin'] if key == 'mlp_sin' else configs.small_variant(key)
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    p0 = ir.initial_params(42)
    bs = configs.batches(cfg, 4)
    payload = reference_payload(ir)
    payload['initialParams'] = _rec({k: np.asarray(v, np.float32) for k, v in p0.items()})
    if key == 'mlp_sin':
        fwd_ir = build_forward_ir(cfg.make_model(), _predict, {'x': [5, 1]})
        x = np.linspace(-1, 1, 5, dtype=np.float32).reshape(5, 1)
    else:
        fwd_ir = build_forward_ir(cfg.make_model(), lambda m, inp: cfg.loss(m, inp), cfg.inputs)
        x = None
    fwd_inputs = {'x': x} if x is not None else bs[0]
    spec = {'payload': payload, 'steps': [_rec(b) for b in bs],
            'forward': {'ir': reference_payload(fwd_ir)['ir'], 'inputs': _rec(fwd_inputs)}}
    f = tmp_path / 'spec.json'
    f.write_text(json.dumps(spec))
    r = subprocess.run([NODE, os.path.join(ROOT, 'tests', 'node', 'train_check.js'), str(f)], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    got = json.loads(r.stdout)

    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(p0)
    losses = [rt.step(b) for b in bs]
    params = rt.download_params()
    sib = backend.NativeRuntime(fwd_ir.wire_json(), parent=rt)
    out_t = fwd_ir.graph.tensors[fwd_ir.graph.outputs[0]]
    out = sib.run(fwd_inputs, out_t.shape, np.float32)
    rt.destroy()

    assert got['paramNames'] == list(params)
    assert [np.float32(v) for v in got['losses']] == [np.float32(v) for v in losses]
    for k in params:
        assert np.array_equal(np.asarray(got['params'][k], np.float32), params[k]), k
    assert np.array_equal(np.asarray(got['forward'], np.float32), out.reshape(-1))
    assert got['abortedAfterDestroy'] == 'AbortError'


def test_node_requests_run_off_the_event_loop(tmp_path):
    """The addon works off the JS thread, as the reference's Web Worker does: a 1 ms
    setInterval keeps ticking through the full transformer's createRuntime (lowering,
    kernel compilation, allocation, upload) and through 20 training steps, and the
    losses are bit-identical to the same steps through ctypes. Four more steps issued
    without awaiting run in arrival order (the family's queue)."""
    cfg = configs.CONFIGS['transformer']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    p0 = ir.initial_params(42)
    bs = configs.batches(cfg, 20)
    payload = reference_payload(ir)
    payload['initialParams'] = _rec({k: np.asarray(v, np.float32) for k, v in p0.items()})
    f = tmp_path / 'spec.json'
    f.write_text(json.dumps({'payload': payload, 'steps': [_rec(b) for b in bs]}))
    r = subprocess.run([NODE, os.path.join(ROOT, 'tests', 'node', 'async_check.js'), str(f)], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    got = json.loads(r.stdout)
    print(f"  create {got['createMs']} ms / {got['createTicks']} ticks, 20 steps {got['stepMs']} ms / "
          f"{got['stepTicks']} ticks, 4 queued steps {got['concurrentMs']} ms / {got['concurrentTicks']} ticks",
          flush=True)
    # a blocked event loop would count no ticks at all; a free one counts about one per ms
    assert got['createTicks'] >= max(3, got['createMs'] // 4)
    assert got['stepTicks'] >= max(2, got['stepMs'] // 4)

    rt = backend.NativeRuntime(ir.wire_json())
    rt.upload_params(p0)
    losses = [rt.step(b) for b in bs]
    more = [rt.step(b) for b in bs[:4]]
    rt.destroy()
    assert [np.float32(v) for v in got['losses']] == [np.float32(v) for v in losses]
    assert [np.float32(v) for v in got['more']] == [np.float32(v) for v in more]

"""The N-API addon and the JS WorkerProxy shim on the CPU (Node 12, no device): the
addon exports the binding, its host-only lowering returns the same bytes as the ctypes
path, its safetensors index agrees, and `toWire` recovers the parameter-gradient and
writeback tensor ids from a reference-shaped createRuntime payload (pooled buffers
included)."""
import ctypes
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from _refplan import reference_payload
from tensorgrad_amd import backend, configs
from tensorgrad_amd.build_ir import build_training_ir
from tensorgrad_amd.safetensors import save_safetensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, 'tensorgrad_amd', 'node', 'tg_napi.node')
NODE = shutil.which('node')

pytestmark = pytest.mark.skipif(NODE is None, reason='node is not installed')


def _node(script, *args):
    r = subprocess.run([NODE, os.path.join(ROOT, 'tests', 'node', script), *args], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr
    return r.stdout.splitlines()


def _plan_raw(ir_json: str) -> str:
    buf = ctypes.create_string_buffer(1 << 24)
    rc = backend.lib().tg_plan(ir_json.encode(), buf, len(buf))
    assert rc == 0, backend.lib().tg_last_error()
    return buf.value.decode()


def test_addon_is_built_and_exports_the_binding():
    assert os.path.exists(ADDON), 'tg_napi.node is not built (run __graft_entry__.build())'
    r = subprocess.run([NODE, '-e', f"const a=require({json.dumps(ADDON)});"
                                    "console.log(JSON.stringify(Object.keys(a)))"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    keys = set(json.loads(r.stdout))
    assert {'plan', 'create', 'createSibling', 'destroy', 'step', 'run', 'uploadParams', 'downloadParams',
            'resetOptimizer', 'setLR', 'saveCheckpoint', 'loadCheckpoint', 'downloadState',
            'uploadState', 'safetensorsIndex'} <= keys


def test_plan_from_node_is_byte_identical_to_ctypes(tmp_path):
    files, want = [], []
    for key in ('mlp_sin', 'char_mlp', 'cnn', 'nerf', 'transformer'):
        cfg = configs.CONFIGS[key]
        ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
        f = tmp_path / f'{key}.json'
        f.write_text(ir.wire_json())
        files.append(str(f))
        want.append(_plan_raw(ir.wire_json()))
    got = _node('plan_check.js', *files)
    assert got == want


@pytest.mark.parametrize('key', ['mlp_sin', 'char_mlp', 'transformer'])
def test_to_wire_recovers_the_c_abi_document(tmp_path, key):
    """toWire maps the reference payload's buffer-level plan back to the tensor-level
    document tg_runtime_create takes; the plan pools intermediates, so only the dedicated
    buffers (gradients, writeback sources) are invertible, which is all it needs."""
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    payload = reference_payload(ir)
    assert payload['ir']['plan']['n_buffers'] < payload['ir']['plan']['n_tensors']   # pooling happened
    f = tmp_path / 'payload.json'
    f.write_text(json.dumps(payload))
    got = json.loads(_node('to_wire_check.js', str(f))[0])
    want = ir.wire()
    assert got['paramGrads'] == want['paramGrads']
    assert got['writebacks'] == want['writebacks']
    assert got['optimizer'] == want['optimizer']
    assert got['graph']['ops'] == want['graph']['ops']
    assert got['graph']['outputs'] == want['graph']['outputs']
    assert [(t['id'], t['shape'], t['dtype']) for t in got['graph']['tensors']] == \
        [(t['id'], t['shape'], t['dtype']) for t in want['graph']['tensors']]
    # the recovered document lowers to the same schedule
    assert _plan_raw(json.dumps(got)) == _plan_raw(ir.wire_json())


def test_safetensors_index_from_node_matches_ctypes(tmp_path):
    buf = save_safetensors({'a': np.arange(6, dtype=np.float32).reshape(2, 3), 'b': np.ones(1, np.float32)},
                           {'format': 'pt'})
    f = tmp_path / 'x.safetensors'
    f.write_bytes(buf)
    r = subprocess.run([NODE, '-e', f"const a=require({json.dumps(ADDON)});const fs=require('fs');"
                                    f"console.log(a.safetensorsIndex(fs.readFileSync({json.dumps(str(f))})))"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout) == backend.safetensors_index(buf)
    bad = subprocess.run([NODE, '-e', f"const a=require({json.dumps(ADDON)});"
                                      "try{a.safetensorsIndex(new Uint8Array(4))}catch(e){console.log(e.message,e.tgStatus)}"],
                         capture_output=True, text=True)
    assert 'too small' in bad.stdout and bad.stdout.strip().endswith('2')


def test_device_calls_return_promises():
    """Calls that touch the device run as asynchronous work and return Promises: without a
    device (or with an invalid document) create rejects with the library's status and the
    message read on the worker thread; argument errors throw synchronously before any
    work is queued."""
    script = (f"const a=require({json.dumps(ADDON)});"
              "const p=a.create('{}');"
              "console.log(p instanceof Promise);"
              "p.then(()=>console.log('resolved'),e=>console.log('rejected',e.tgStatus,JSON.stringify(e.message)));"
              "try{a.step(null,{},null)}catch(e){console.log('throws',e.name)}")
    r = subprocess.run([NODE, '-e', script], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = r.stdout.strip().split('\n')
    assert out[0] == 'true' and out[1] == 'throws TypeError', out
    assert out[2].startswith('rejected 2 ') and 'graph' in out[2], out   # TG_INVALID_ARGUMENT

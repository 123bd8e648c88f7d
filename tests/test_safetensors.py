"""safetensors loader (the reference's test/safetensors.ts:51-147, restated) and writer.
CPU only: the container is indexed by the native library's host code."""
import json

import numpy as np
import pytest

from tensorgrad_amd.backend import BackendError
from tensorgrad_amd.safetensors import load_safetensors, save_safetensors


def build(entries, metadata=None):
    """A container laid out like the reference test's builder: 8-byte LE header length,
    JSON header, then the blob with no padding (so the blob is not 4-byte aligned)."""
    header = {}
    if metadata:
        header['__metadata__'] = metadata
    off = 0
    for name, shape, data in entries:
        header[name] = {'dtype': 'F32', 'shape': shape, 'data_offsets': [off, off + data.nbytes]}
        off += data.nbytes
    hj = json.dumps(header).encode()
    return len(hj).to_bytes(8, 'little') + hj + b''.join(np.asarray(d, '<f4').tobytes() for _, _, d in entries)


def raw(header, blob_len):
    hj = json.dumps(header).encode()
    return len(hj).to_bytes(8, 'little') + hj + bytes(blob_len)


def test_round_trip():
    w = np.array([1, 2, 3, 4, 5, 6], np.float32)
    b = np.array([0.5, -0.5], np.float32)
    d = load_safetensors(build([('l1.W', [3, 2], w), ('l1.b', [2], b)]))
    np.testing.assert_array_equal(d.tensors['l1.W'], w)
    np.testing.assert_array_equal(d.tensors['l1.b'], b)
    assert d.shapes == {'l1.W': [3, 2], 'l1.b': [2]}
    assert len(d.tensors) == 2 and d.skipped == {}


def test_metadata_is_not_a_tensor():
    d = load_safetensors(build([('w', [2], np.array([7, 8], np.float32))], {'format': 'pt', 'note': 'hello'}))
    assert '__metadata__' not in d.tensors and list(d.tensors) == ['w']
    assert d.metadata == {'format': 'pt', 'note': 'hello'}


def test_scalar_shape():
    d = load_safetensors(build([('s', [], np.array([42], np.float32))]))
    assert d.tensors['s'].tolist() == [42.0] and d.shapes['s'] == []


def test_non_f32_float_rejected():
    with pytest.raises(BackendError, match='f32-only'):
        load_safetensors(raw({'x': {'dtype': 'F16', 'shape': [2], 'data_offsets': [0, 4]}}, 4))


def test_integer_tensors_skipped_and_reported():
    w = np.array([1.5, -2.5], np.float32)
    header = {'bn.weight': {'dtype': 'F32', 'shape': [2], 'data_offsets': [0, 8]},
              'bn.num_batches_tracked': {'dtype': 'I64', 'shape': [], 'data_offsets': [8, 16]}}
    hj = json.dumps(header).encode()
    buf = len(hj).to_bytes(8, 'little') + hj + w.tobytes() + bytes(8)
    d = load_safetensors(buf)
    np.testing.assert_array_equal(d.tensors['bn.weight'], w)
    assert 'bn.num_batches_tracked' not in d.tensors
    assert d.skipped == {'bn.num_batches_tracked': 'I64'}
    assert d.shapes['bn.num_batches_tracked'] == []


def test_malformed_buffers():
    with pytest.raises(BackendError, match='too small'):
        load_safetensors(bytes(4))
    with pytest.raises(BackendError, match='exceeds buffer'):
        load_safetensors((9999).to_bytes(8, 'little'))
    with pytest.raises(BackendError, match='not valid JSON'):
        load_safetensors((3).to_bytes(8, 'little') + b'{x}')
    with pytest.raises(BackendError, match='out of range'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [4], 'data_offsets': [0, 16]}}, 8))


def test_offset_shape_mismatch():
    with pytest.raises(BackendError, match='byte length'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [4], 'data_offsets': [0, 8]}}, 8))


def test_writer_round_trip_aligned_and_order_preserved():
    rng = np.random.default_rng(1)
    ts = {'b': rng.standard_normal((3, 5)).astype(np.float32), 'a': rng.standard_normal(7).astype(np.float32),
          'c': np.array([3.0], np.float32)}
    buf = save_safetensors(ts, {'k': 'v'}, shapes={'c': []})
    hlen = int.from_bytes(buf[:8], 'little')
    assert (8 + hlen) % 8 == 0
    assert list(json.loads(buf[8:8 + hlen])) == ['__metadata__', 'b', 'a', 'c']
    d = load_safetensors(buf)
    for k, v in ts.items():
        np.testing.assert_array_equal(d.tensors[k], v.reshape(-1))
    assert d.shapes == {'b': [3, 5], 'a': [7], 'c': []} and d.metadata == {'k': 'v'}
    with pytest.raises(ValueError):
        save_safetensors({'x': np.zeros(3, np.float32)}, shapes={'x': [2]})


def test_dimensions_beyond_exact_doubles_are_rejected():
    """A dimension or offset of 2^53 or more cannot be read exactly from a JSON number: it
    is refused before any integer conversion."""
    with pytest.raises(BackendError, match='malformed shape'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [2 ** 63], 'data_offsets': [0, 0]}}, 0))
    with pytest.raises(BackendError, match='malformed shape'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [2 ** 53], 'data_offsets': [0, 0]}}, 0))
    with pytest.raises(BackendError, match='malformed data_offsets'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [1], 'data_offsets': [0, 2 ** 64]}}, 4))


def test_element_count_that_wraps_is_rejected():
    """[2^31, 2^31, 4] has 2^64 elements: a product in 64-bit arithmetic wraps to 0 and would
    match an empty byte range; the parser detects the overflow instead."""
    with pytest.raises(BackendError, match='overflows'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [2 ** 31, 2 ** 31, 4], 'data_offsets': [0, 0]}}, 0))
    with pytest.raises(BackendError, match='overflows'):
        load_safetensors(raw({'x': {'dtype': 'F32', 'shape': [2 ** 40, 2 ** 23], 'data_offsets': [0, 0]}}, 0))


# ---- checkpoint checks against a graph (tg_check_checkpoint: the validation of
# ---- tg_load_checkpoint, without a device) ------------------------------------------------

def _mlp_ir():
    from tensorgrad_amd import configs
    from tensorgrad_amd.build_ir import build_training_ir
    cfg = configs.small_variant('mlp_sin')
    return build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)


def _checkpoint(ir, with_state=True, meta=None, extra=None):
    """A container shaped like tg_save_checkpoint's output: params, then Adam's m and v."""
    p0 = ir.initial_params(1)
    tensors = {n: np.asarray(p0[n], np.float32) for n in ir.param_names}
    if with_state:
        for n in ir.param_names:
            tensors[f'adam_m_{n}'] = np.zeros_like(tensors[n])
            tensors[f'adam_v_{n}'] = np.zeros_like(tensors[n])
    shp = {n: list(s) for n, s in ir.param_shapes().items()}
    for n in ir.param_names:
        shp[f'adam_m_{n}'] = shp[f'adam_v_{n}'] = shp[n]
    m = {'format': 'tensorgrad', 'tensorgrad.optimizer': 'adam', 'tensorgrad.step': '12',
         'tensorgrad.prngCounter': '34'}
    m.update(meta or {})
    buf = save_safetensors(tensors, m, shapes=shp)
    if extra is not None:
        # append one integer tensor after the f32 ones (rebuild the header)
        hlen = int.from_bytes(buf[:8], 'little')
        header = json.loads(buf[8:8 + hlen])
        blob = buf[8 + hlen:]
        header[extra] = {'dtype': 'I64', 'shape': [], 'data_offsets': [len(blob), len(blob) + 8]}
        hj = json.dumps(header).encode()
        buf = len(hj).to_bytes(8, 'little') + hj + blob + bytes(8)
    return buf


def test_checkpoint_check_full_and_params_only(tmp_path):
    from tensorgrad_amd import backend
    ir = _mlp_ir()
    path = tmp_path / 'full.safetensors'
    path.write_bytes(_checkpoint(ir))
    r = backend.check_checkpoint(ir.wire_json(), path)
    assert r == {'params': len(ir.param_names), 'state': 2 * len(ir.param_names), 'restoresCounters': True,
                 'step': 12, 'prngCounter': 34}
    # a params-only file (e.g. converted pretrained weights) leaves t and the seed counter
    # alone, whatever its metadata says
    path.write_bytes(_checkpoint(ir, with_state=False))
    r = backend.check_checkpoint(ir.wire_json(), path)
    assert r['state'] == 0 and not r['restoresCounters'] and r['step'] == 0 and r['prngCounter'] == 0


def test_checkpoint_check_rejects_integer_tensors_and_bad_counters(tmp_path):
    from tensorgrad_amd import backend
    ir = _mlp_ir()
    path = tmp_path / 'x.safetensors'
    path.write_bytes(_checkpoint(ir, extra='bn.num_batches_tracked'))
    with pytest.raises(BackendError, match="unknown tensor 'bn.num_batches_tracked'"):
        backend.check_checkpoint(ir.wire_json(), path)
    for bad in ('12x', '-3', '', '1e3', '99999999999999999999'):
        path.write_bytes(_checkpoint(ir, meta={'tensorgrad.step': bad}))
        with pytest.raises(BackendError, match='tensorgrad.step') as ei:
            backend.check_checkpoint(ir.wire_json(), path)
        assert ei.value.status == backend.TG_INVALID_ARGUMENT
    path.write_bytes(_checkpoint(ir, meta={'tensorgrad.prngCounter': 'seven'}))
    with pytest.raises(BackendError, match='tensorgrad.prngCounter'):
        backend.check_checkpoint(ir.wire_json(), path)

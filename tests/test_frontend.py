"""Front-end structure (restating test/smoke.ts and test/ops.ts checks): IR shapes, param
grads, capture registry rules, optimizer pass structure, error attribution."""
import numpy as np
import pytest

from tensorgrad_amd import configs, nn
from tensorgrad_amd import ops as O
from tensorgrad_amd.build_ir import build_forward_ir, build_training_ir
from tensorgrad_amd.grad import append_grad
from tensorgrad_amd.ir import get_op_inputs, OP_KINDS
from tensorgrad_amd.module import Module
from tensorgrad_amd.shape import ShapeError
from tensorgrad_amd.trace import capture, param_input, tensor_input, trace_fn, trace_into


@pytest.mark.parametrize('key', list(configs.CONFIGS))
def test_config_param_counts_and_grad_shapes(key):
    want = {'mlp_sin': 4353, 'char_mlp': 113315, 'cnn': 1199882, 'nerf': 494084, 'transformer': 3221569}[key]
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    shapes = ir.param_shapes()
    assert sum(int(np.prod(s)) for s in shapes.values()) == want
    for n, t in ir.param_grads.items():
        assert t.shape == shapes[n]
    # one adam_update_p per param (test/smoke.ts:572-585), three writebacks each
    assert sum(op['kind'] == 'adam_update_p' for op in ir.graph.ops) == len(shapes)
    assert len(ir.opt.writebacks) == 3 * len(shapes)
    # topological order: every input defined before use
    for i, op in enumerate(ir.graph.ops):
        for t in get_op_inputs(op):
            assert ir.graph.tensors[t].source < i


def test_gemm_flops_match_the_survey_counts():
    def flops(g):
        tot = 0
        for op in g.ops:
            if op['kind'] in ('matmul', 'matmul_batched'):
                a, b = g.tensors[op['a']].shape, g.tensors[op['b']].shape
                tot += 2 * int(np.prod(a[:-1])) * a[-1] * b[-1]
        return tot
    want = {'mlp_sin': 6455296, 'nerf': 191360925696}
    for k, v in want.items():
        cfg = configs.CONFIGS[k]
        assert flops(build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer).graph) == v


def test_adamw_decay_defaults_and_literal_shrink():
    cfg = configs.CONFIGS['transformer']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    by_p = {}
    for op in ir.graph.ops:
        if op['kind'] == 'adam_update_p':
            name = ir.graph.ops[ir.graph.tensors[op['p']].source]['name']
            by_p[name] = op
    assert by_p['layers.0.attn.q.W']['decayShrink'] == 1 - 3e-4 * 0.01
    assert by_p['layers.0.ln1.g']['decayShrink'] == 1 and by_p['head.b']['decayShrink'] == 1
    assert all(op['decayShrinkTensor'] is None for op in by_p.values())


def test_scheduled_lr_routes_decay_shrink_through_an_input():
    cfg = configs.CONFIGS['mlp_sin']
    opt = {'kind': 'adamw', 'lr': {'kind': 'linear', 'peak': 0.01, 'final': 0.001, 'steps': 10}, 'weightDecay': 0.1}
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, opt)
    names = [op['name'] for op in ir.graph.ops if op['kind'] == 'tensor_input']
    assert '_adam_decay_shrink' in names and '_adam_lrt' in names
    assert ir.opt.wire_config['decayShrinkInputName'] == '_adam_decay_shrink'


def test_sgd_writeback_structure():
    cfg = configs.CONFIGS['mlp_sin']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, {'kind': 'sgd', 'lr': 0.1, 'momentum': 0.9})
    kinds = [(w.dest_kind, w.dest_name) for w in ir.opt.writebacks]
    n = len(ir.param_names)
    assert sum(k == 'state' for k, _ in kinds) == n and sum(k == 'param' for k, _ in kinds) == n
    with pytest.raises(ValueError):
        build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, {'kind': 'sgd', 'lr': 0.1, 'nesterov': True})


def test_capture_rules():
    def body():
        x = tensor_input('x', [4])
        capture('a', O.relu(x))
        with pytest.raises(ValueError):
            capture('a', x)
        return O.mean(x)
    g = trace_fn(body)
    assert list(g.captures) == ['a']

    def inner():
        capture('b', g.tensors[0])
    trace_into(g, inner)
    assert 'b' not in g.captures


def test_shape_errors_name_the_op():
    with pytest.raises(ShapeError, match='matmul'):
        trace_fn(lambda: O.matmul(tensor_input('a', [2, 3]), tensor_input('b', [4, 5])))
    with pytest.raises(ShapeError, match='add'):
        trace_fn(lambda: O.add(tensor_input('a', [2, 3]), tensor_input('b', [4])))
    with pytest.raises(ValueError):
        trace_fn(lambda: O.add(tensor_input('a', [2]), tensor_input('a', [2])))


def test_forward_ir_and_embedding_decomposition():
    cfg = configs.CONFIGS['char_mlp']
    ir = build_forward_ir(cfg.make_model(), lambda m, inp: O.argmax(m.l2.fwd(O.tanh(m.l1.fwd(
        O.reshape(m.emb.fwd(inp['tokens']), [4, 192])))), -1), {'tokens': {'shape': [4, 8], 'dtype': 'i32'}})
    out = ir.graph.tensors[ir.graph.outputs[0]]
    assert out.dtype == 'i32' and out.shape == (4,)
    kinds = [op['kind'] for op in ir.graph.ops]
    assert 'one_hot' in kinds and 'matmul' in kinds


def test_op_kind_table_covers_the_ir():
    # 58 kinds in src/ir.ts:74-271
    assert len(OP_KINDS) == 58

"""Reverse-mode autograd and gradient transforms (reference `src/grad.ts`).

`append_grad` (grad.ts:46-93) walks the forward ops in reverse and appends adjoint ops
through the public op functions; one rule per kind (grad.ts:194-557), with the same
emission order, so the appended IR matches the reference op for op.
`append_grad_clip` (grad.ts:110-130) and `append_grad_normalize` (grad.ts:148-172) are
the post-grad transforms the optimizer passes share.
"""
from __future__ import annotations

import math
from typing import Callable, Dict, Optional

from . import ops as O
from .ir import Graph, Tensor
from .shape import shapes_equal
from .trace import trace_into


class GradResult:
    def __init__(self, graph: Graph, param_grads: Dict[str, Tensor], loss: Tensor):
        self.graph = graph
        self.param_grads = param_grads
        self.loss = loss


def append_grad(graph: Graph) -> GradResult:
    if len(graph.outputs) != 1:
        raise ValueError(f'autograd: expected graph with exactly 1 output (the loss); got {len(graph.outputs)}')
    loss_id = graph.outputs[0]
    loss_t = graph.tensors[loss_id]
    if len(loss_t.shape) != 0:
        raise ValueError(f'autograd: loss must be a rank-0 scalar; got shape {list(loss_t.shape)}. '
                         'Reduce with sum / mulScalar to a scalar before calling appendGrad.')
    forward_ops = list(graph.ops)
    cot: Dict[int, Tensor] = {}

    def body():
        cot[loss_id] = O.const_scalar(1.0, 'f32')
        for op in reversed(forward_ops):
            oc = cot.get(op['out'])
            if oc is None:
                continue
            _adjoint(op, oc, graph, cot)
        param_grads: Dict[str, Tensor] = {}
        for op in forward_ops:
            if op['kind'] != 'param_input':
                continue
            c = cot.get(op['out'])
            if c is None:
                t = graph.tensors[op['out']]
                param_grads[op['name']] = O.broadcast_to(O.const_scalar(0.0, t.dtype), t.shape)
            else:
                param_grads[op['name']] = c
        return GradResult(graph, param_grads, loss_t)
    return trace_into(graph, body)


def append_grad_clip(graph: Graph, param_grads: Dict[str, Tensor], max_norm: float) -> Dict[str, Tensor]:
    def body():
        entries = list(param_grads.items())
        if not entries:
            return param_grads
        sum_sq = O.sum_(O.mul(entries[0][1], entries[0][1]))
        for _, g in entries[1:]:
            sum_sq = O.add(sum_sq, O.sum_(O.mul(g, g)))
        scale = O.minimum(O.div(O.const_scalar(max_norm, 'f32'), O.add(O.sqrt(sum_sq), 1e-6)), 1)
        return {name: O.mul(g, O.broadcast_to(scale, g.shape)) for name, g in entries}
    return trace_into(graph, body)


def append_grad_normalize(graph: Graph, param_grads: Dict[str, Tensor],
                          filt: Optional[Callable[[str], bool]] = None) -> Dict[str, Tensor]:
    def body():
        out: Dict[str, Tensor] = {}
        matched = 0
        for name, g in param_grads.items():
            if filt is not None and not filt(name):
                out[name] = g
                continue
            matched += 1
            norm = O.add(O.sqrt(O.sum_(O.mul(g, g))), 1e-8)
            out[name] = O.div(g, O.broadcast_to(norm, g.shape))
        if filt is not None and matched == 0 and len(param_grads) > 0:
            raise ValueError("normalizeGrads: the filter matched no parameters. Param names are property paths "
                             f"like 'w1.W' — available: {', '.join(param_grads.keys())}")
        return out
    return trace_into(graph, body)


def _accumulate(cot: Dict[int, Tensor], input_id: int, contribution: Tensor) -> None:
    existing = cot.get(input_id)
    cot[input_id] = O.add(existing, contribution) if existing is not None else contribution


def _unbroadcast(c: Tensor, to_shape) -> Tensor:
    if shapes_equal(c.shape, to_shape):
        return c
    return O.sum_to_shape(c, to_shape)


def _invert_perm(perm):
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return inv


def _adjoint(op: dict, oc: Tensor, graph: Graph, cot: Dict[int, Tensor]) -> None:
    k = op['kind']
    T = lambda i: graph.tensors[i]  # noqa: E731
    acc = lambda i, c: _accumulate(cot, i, c)  # noqa: E731

    if k in ('param_input', 'tensor_input', 'state_input', 'arange', 'const_scalar', 'const_fill'):
        return
    if k == 'add':
        a, b = T(op['a']), T(op['b'])
        acc(op['a'], _unbroadcast(oc, a.shape))
        acc(op['b'], _unbroadcast(oc, b.shape))
    elif k == 'sub':
        a, b = T(op['a']), T(op['b'])
        acc(op['a'], _unbroadcast(oc, a.shape))
        acc(op['b'], _unbroadcast(O.mul_scalar(oc, -1), b.shape))
    elif k == 'mul':
        a, b = T(op['a']), T(op['b'])
        acc(op['a'], _unbroadcast(O.mul(oc, b), a.shape))
        acc(op['b'], _unbroadcast(O.mul(oc, a), b.shape))
    elif k == 'div':
        a, b = T(op['a']), T(op['b'])
        acc(op['a'], _unbroadcast(O.div(oc, b), a.shape))
        numer = O.mul(oc, a)
        b_sq = O.mul(b, b)
        acc(op['b'], _unbroadcast(O.mul_scalar(O.div(numer, b_sq), -1), b.shape))
    elif k == 'mul_scalar':
        acc(op['a'], O.mul_scalar(oc, op['scalar']))
    elif k == 'add_scalar':
        acc(op['a'], oc)
    elif k == 'sqrt':
        c = T(op['out'])
        acc(op['a'], O.mul_scalar(O.div(oc, c), 0.5))
    elif k == 'rsqrt':
        c = T(op['out'])
        c3 = O.mul(O.mul(c, c), c)
        acc(op['a'], O.mul_scalar(O.mul(oc, c3), -0.5))
    elif k == 'log':
        acc(op['a'], O.div(oc, T(op['a'])))
    elif k == 'exp':
        acc(op['a'], O.mul(oc, T(op['out'])))
    elif k == 'relu':
        acc(op['a'], O.relu_grad(T(op['a']), oc))
    elif k == 'neg':
        acc(op['a'], O.mul_scalar(oc, -1))
    elif k == 'abs':
        a = T(op['a'])
        acc(op['a'], O.where(O.less(a, O.const_scalar(0, 'f32')), O.mul_scalar(oc, -1), oc))
    elif k == 'tanh':
        c = T(op['out'])
        acc(op['a'], O.mul(oc, O.sub(O.const_scalar(1, 'f32'), O.mul(c, c))))
    elif k == 'sigmoid':
        c = T(op['out'])
        acc(op['a'], O.mul(oc, O.sub(c, O.mul(c, c))))
    elif k == 'erf':
        a = T(op['a'])
        d = O.mul_scalar(O.exp(O.mul_scalar(O.mul(a, a), -1)), 2 / math.sqrt(math.pi))
        acc(op['a'], O.mul(oc, d))
    elif k == 'sin':
        acc(op['a'], O.mul(oc, O.cos(T(op['a']))))
    elif k == 'cos':
        acc(op['a'], O.mul(oc, O.mul_scalar(O.sin(T(op['a'])), -1)))
    elif k == 'dropout':
        acc(op['a'], O.dropout_with_salt(oc, op['p'], op['salt'], op['seed']))
    elif k in ('randn', 'stop_gradient'):
        return
    elif k == 'concat':
        cursor = 0
        for iid in op['inputs']:
            size = T(iid).shape[op['axis']]
            acc(iid, O.narrow(oc, op['axis'], cursor, size))
            cursor += size
    elif k == 'slice_range':
        a = T(op['a'])
        acc(op['a'], O.scatter_axis(oc, a.shape, op['axis'], op['start'], op['end']))
    elif k in ('min', 'max'):
        a, b = T(op['a']), T(op['b'])
        zero = O.const_scalar(0, 'f32')
        a_wins = O.less(a, b) if k == 'min' else O.greater(a, b)
        acc(op['a'], _unbroadcast(O.where(a_wins, oc, O.broadcast_to(zero, oc.shape)), a.shape))
        acc(op['b'], _unbroadcast(O.where(a_wins, O.broadcast_to(zero, oc.shape), oc), b.shape))
    elif k == 'mean_last':
        a = T(op['a'])
        D = a.shape[-1]
        acc(op['a'], O.mul_scalar(O.broadcast_to(oc, a.shape), 1 / D))
    elif k == 'sum_last':
        a = T(op['a'])
        with_keep = O.reshape(oc, list(oc.shape) + [1])
        acc(op['a'], O.broadcast_to(with_keep, a.shape))
    elif k == 'reshape':
        acc(op['a'], O.reshape(oc, T(op['a']).shape))
    elif k == 'permute':
        acc(op['a'], O.permute(oc, _invert_perm(op['perm'])))
    elif k == 'matmul':
        # dA = dC @ B^T; dB = [K, rows] @ [rows, N] over flattened leading dims (grad.ts:407-427).
        a, b = T(op['a']), T(op['b'])
        acc(op['a'], O.matmul(oc, O.swap_axes(b, -1, -2)))
        K, N = a.shape[-1], b.shape[-1]
        rows = 1
        for d in a.shape[:-1]:
            rows *= d
        a2 = O.reshape(a, [rows, K])
        oc2 = O.reshape(oc, [rows, N])
        acc(op['b'], O.sum_to_shape(O.matmul(O.swap_axes(a2, -1, -2), oc2), b.shape))
    elif k == 'matmul_batched':
        a, b = T(op['a']), T(op['b'])
        acc(op['a'], O.matmul(oc, O.swap_axes(b, -1, -2)))
        acc(op['b'], O.matmul(O.swap_axes(a, -1, -2), oc))
    elif k == 'one_hot':
        return
    elif k == 'broadcast_to':
        acc(op['a'], O.sum_to_shape(oc, T(op['a']).shape))
    elif k == 'sum_to_shape':
        acc(op['a'], O.broadcast_to(oc, T(op['a']).shape))
    elif k == 'log_softmax_last':
        c = T(op['out'])
        sm = O.exp(c)
        s_keep = O.sum_(oc, -1, keep_dims=True)
        term = O.mul(sm, O.broadcast_to(s_keep, c.shape))
        acc(op['a'], O.sub(oc, term))
    elif k == 'softmax_causal_last':
        c = T(op['out'])
        dcxc = O.mul(oc, c)
        s_keep = O.sum_(dcxc, -1, keep_dims=True)
        inner = O.sub(oc, O.broadcast_to(s_keep, c.shape))
        acc(op['a'], O.mul(inner, c))
    elif k in ('less', 'greater', 'argmax_last', 'categorical_last'):
        return
    elif k == 'where':
        a, b = T(op['a']), T(op['b'])
        zero_a = O.broadcast_to(O.const_scalar(0, a.dtype), oc.shape)
        zero_b = O.broadcast_to(O.const_scalar(0, b.dtype), oc.shape)
        acc(op['a'], _unbroadcast(O.where(T(op['cond']), oc, zero_a), a.shape))
        acc(op['b'], _unbroadcast(O.where(T(op['cond']), zero_b, oc), b.shape))
    elif k == 'where_causal':
        acc(op['a'], O.where_causal(oc, 0))
    elif k in ('adam_update_m', 'adam_update_v', 'adam_update_p'):
        raise ValueError(f'autograd: cannot differentiate through {k}')
    elif k == 'conv2d':
        x, w = T(op['input']), T(op['weight'])
        acc(op['input'], O.conv2d_input_grad(w, oc, x.shape[2], x.shape[3], op['strideH'], op['strideW'],
                                             op['padH'], op['padW'], op['groups']))
        acc(op['weight'], O.conv2d_weight_grad(x, oc, w.shape[2], w.shape[3], op['strideH'], op['strideW'],
                                               op['padH'], op['padW'], op['groups']))
    elif k == 'max_pool_2d':
        x = T(op['input'])
        acc(op['input'], O.max_pool2d_grad(x, oc, op['kH'], op['kW'], op['strideH'], op['strideW'],
                                           op['padH'], op['padW']))
    elif k in ('conv2d_input_grad', 'conv2d_weight_grad', 'max_pool_2d_grad', 'scatter_axis'):
        raise ValueError(f"autograd: cannot differentiate through {k} (it's a backward op)")
    elif k == 'relu_grad':
        raise ValueError('autograd: cannot take second-order gradient through relu_grad — '
                         'tensorgrad does not support higher-order autodiff.')
    else:
        raise ValueError(f'autograd: unhandled op kind {k}')

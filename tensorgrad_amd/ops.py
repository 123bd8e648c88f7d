"""User-facing op surface: each call validates shapes and appends IR (reference
`src/ops.ts`). Composite ops decompose into the same primitive kinds, in the same
emission order, as the reference — the IR this produces is what the backend executes
and what the oracle evaluates, so the order of `add_op` calls below is load-bearing
(salts, tensor ids, DCE renumbering).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple, Union

from . import shape as S
from .ir import Graph, Tensor, add_op
from .shape import ShapeError
from .trace import current_graph, tensor_input

Number = Union[int, float]

PRNG_SEED_INPUT = '__prngSeed'   # ops.ts:191


def _num(x) -> bool:
    return isinstance(x, (int, float)) and not isinstance(x, bool)


# ---- Element-wise binops (ops.ts:21-101) -------------------------------------------

def _binop(name: str, kind: str, a: Tensor, b: Tensor, out_dtype: Optional[str] = None) -> Tensor:
    if a.dtype != b.dtype:
        raise ShapeError(f'{name}: dtype mismatch ({a.dtype} vs {b.dtype})', name)
    out_shape = S.infer_elementwise_binop(name, a.shape, b.shape, name)
    return add_op(current_graph(), kind, out_shape, out_dtype or a.dtype, name, {'a': a.id, 'b': b.id})


def add(a, b) -> Tensor:
    if _num(a):
        return add_scalar(b, a)
    if _num(b):
        return add_scalar(a, b)
    return _binop('add', 'add', a, b)


def sub(a, b) -> Tensor:
    if _num(b):
        return add_scalar(a, -b)
    if _num(a):
        return _binop('sub', 'sub', const_scalar(a, b.dtype), b)
    return _binop('sub', 'sub', a, b)


def mul(a, b) -> Tensor:
    if _num(a):
        return mul_scalar(b, a)
    if _num(b):
        return mul_scalar(a, b)
    return _binop('mul', 'mul', a, b)


def div(a, b) -> Tensor:
    if _num(b):
        if b == 0:
            raise ShapeError('div: scalar divisor cannot be zero', 'div')
        return mul_scalar(a, 1 / b)
    if _num(a):
        return _binop('div', 'div', const_scalar(a, b.dtype), b)
    return _binop('div', 'div', a, b)


def minimum(a, b) -> Tensor:
    if _num(a):
        return minimum(b, a)
    rhs = const_scalar(b, a.dtype) if _num(b) else b
    return _binop('min', 'min', a, rhs)


def maximum(a, b) -> Tensor:
    if _num(a):
        return maximum(b, a)
    rhs = const_scalar(b, a.dtype) if _num(b) else b
    return _binop('max', 'max', a, rhs)


def clamp(a: Tensor, lo: Number, hi: Number) -> Tensor:
    return minimum(maximum(a, lo), hi)


def mul_scalar(a: Tensor, scalar: Number) -> Tensor:
    return add_op(current_graph(), 'mul_scalar', a.shape, a.dtype, 'mulScalar', {'a': a.id, 'scalar': scalar})


def add_scalar(a: Tensor, scalar: Number) -> Tensor:
    return add_op(current_graph(), 'add_scalar', a.shape, a.dtype, 'addScalar', {'a': a.id, 'scalar': scalar})


# ---- Unary (ops.ts:121-184) ----------------------------------------------------------

def _unary(name: str, a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'{name}: requires f32, got {a.dtype}', name)
    return add_op(current_graph(), name, a.shape, 'f32', name, {'a': a.id})


def sqrt(a): return _unary('sqrt', a)
def rsqrt(a): return _unary('rsqrt', a)
def log(a): return _unary('log', a)
def exp(a): return _unary('exp', a)
def relu(a): return _unary('relu', a)
def neg(a): return _unary('neg', a)
def abs_(a): return _unary('abs', a)
def tanh(a): return _unary('tanh', a)
def sigmoid(a): return _unary('sigmoid', a)
def erf(a): return _unary('erf', a)
def sin(a): return _unary('sin', a)
def cos(a): return _unary('cos', a)


def square(a: Tensor) -> Tensor:
    return mul(a, a)


def stop_gradient(a: Tensor) -> Tensor:
    return add_op(current_graph(), 'stop_gradient', a.shape, a.dtype, 'stopGradient', {'a': a.id})


def silu(a: Tensor) -> Tensor:
    return mul(a, sigmoid(a))


# ---- Stochastic ops (ops.ts:193-310) ---------------------------------------------------

def _find_or_create_prng_seed(g: Graph) -> Tensor:
    for op in g.ops:
        if op['kind'] == 'tensor_input' and op['name'] == PRNG_SEED_INPUT:
            return g.tensors[op['out']]
    return tensor_input(PRNG_SEED_INPUT, [], 'i32')


def _count_stochastic_ops(g: Graph) -> int:
    return sum(1 for op in g.ops if op['kind'] in ('dropout', 'randn', 'categorical_last'))


def dropout(x: Tensor, p: float) -> Tensor:
    if p == 0:
        return x
    if p < 0 or p >= 1:
        raise ShapeError(f'dropout: p must be in [0, 1), got {p}', 'dropout')
    if x.dtype != 'f32':
        raise ShapeError(f'dropout: requires f32, got {x.dtype}', 'dropout')
    g = current_graph()
    seed = _find_or_create_prng_seed(g)
    salt = _count_stochastic_ops(g)
    return add_op(g, 'dropout', x.shape, 'f32', 'dropout', {'a': x.id, 'seed': seed.id, 'p': p, 'salt': salt})


def randn(shape: Sequence[int]) -> Tensor:
    for d in shape:
        if not isinstance(d, int) or d <= 0:
            raise ShapeError(f'randn: shape must be positive integers, got {S.show(shape)}', 'randn')
    g = current_graph()
    seed = _find_or_create_prng_seed(g)
    salt = _count_stochastic_ops(g)
    return add_op(g, 'randn', shape, 'f32', 'randn', {'seed': seed.id, 'salt': salt, 'shape': list(shape)})


def dropout_with_salt(dy: Tensor, p: float, salt: int, seed_id: int) -> Tensor:
    """Backward dropout sharing the forward's (seed, salt, p) (ops.ts:255-258)."""
    return add_op(current_graph(), 'dropout', dy.shape, 'f32', 'dropout', {'a': dy.id, 'seed': seed_id, 'p': p, 'salt': salt})


def _categorical_last(a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'categorical: requires f32 logits, got {a.dtype}', 'categorical')
    out_shape = S.infer_sum_last('categorical', a.shape, 'categorical')
    g = current_graph()
    seed = _find_or_create_prng_seed(g)
    salt = _count_stochastic_ops(g)
    return add_op(g, 'categorical_last', out_shape, 'i32', 'categorical', {'a': a.id, 'seed': seed.id, 'salt': salt})


def categorical(logits: Tensor, axis: int = -1) -> Tensor:
    return _axis_reducing(logits, axis, 'categorical', _categorical_last)


def gelu(a: Tensor, approximate: str = 'none') -> Tensor:
    """Exact GELU `0.5*x*(1+erf(x/sqrt2))`, or the tanh form (ops.ts:319-327)."""
    if approximate == 'tanh':
        c = 0.7978845608028654
        x3 = mul(mul(a, a), a)
        inner = mul(add(a, mul(x3, 0.044715)), c)
        return mul(mul(a, 0.5), add(tanh(inner), 1))
    return mul(mul(a, 0.5), add(erf(mul(a, 1 / math.sqrt(2))), 1))


def leaky_relu(a: Tensor, alpha: float = 0.01) -> Tensor:
    return where(greater(a, 0), a, mul(a, alpha))


def softplus(a: Tensor) -> Tensor:
    return add(maximum(a, 0), log(add(exp(neg(abs_(a))), 1)))


# ---- Reductions (ops.ts:358-457) ---------------------------------------------------------

def _mean_last(a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'mean: requires f32, got {a.dtype}', 'mean')
    return add_op(current_graph(), 'mean_last', S.infer_mean_last('mean', a.shape, 'mean'), a.dtype, 'mean', {'a': a.id})


def _sum_last(a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'sum: requires f32, got {a.dtype}', 'sum')
    return add_op(current_graph(), 'sum_last', S.infer_sum_last('sum', a.shape, 'sum'), a.dtype, 'sum', {'a': a.id})


def _argmax_last(a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'argmax: requires f32, got {a.dtype}', 'argmax')
    return add_op(current_graph(), 'argmax_last', S.infer_sum_last('argmax', a.shape, 'argmax'), 'i32', 'argmax', {'a': a.id})


def argmax(a: Tensor, axis: Optional[int] = None) -> Tensor:
    if axis is None:
        return _argmax_last(reshape(a, [-1]))
    return _axis_reducing(a, axis, 'argmax', _argmax_last)


def argmin(a: Tensor, axis: Optional[int] = None) -> Tensor:
    return argmax(neg(a), axis)


def mean(a: Tensor, axis: Optional[int] = None, keep_dims: bool = False) -> Tensor:
    if axis is None:
        n = S.shape_size(a.shape)
        if n == 0:
            raise ShapeError('mean: cannot mean over zero elements', 'mean')
        return mul_scalar(_sum_last(reshape(a, [-1])), 1 / n)
    return _reduce_axis(a, axis, keep_dims, 'mean')


def sum_(a: Tensor, axis: Optional[int] = None, keep_dims: bool = False) -> Tensor:
    if axis is None:
        return _sum_last(reshape(a, [-1]))
    return _reduce_axis(a, axis, keep_dims, 'sum')


def _reduce_axis(a: Tensor, axis_arg: int, keep_dims: bool, kind: str) -> Tensor:
    r = len(a.shape)
    k = r + axis_arg if axis_arg < 0 else axis_arg
    if k < 0 or k >= r:
        raise ShapeError(f"{kind}: axis {axis_arg} out of range for shape [{','.join(map(str, a.shape))}]", kind)
    is_last = k == r - 1
    inp = a if is_last else permute(a, [i for i in range(r) if i != k] + [k])
    if kind == 'mean':
        reduced = _mean_last(inp)
        if is_last:
            return reduced if keep_dims else reshape(reduced, reduced.shape[:-1])
        if not keep_dims:
            return reshape(reduced, reduced.shape[:-1])
        return permute(reduced, _back_perm(k, r))
    dropped = _sum_last(inp)
    if is_last:
        return reshape(dropped, list(dropped.shape) + [1]) if keep_dims else dropped
    if not keep_dims:
        return dropped
    return permute(reshape(dropped, list(dropped.shape) + [1]), _back_perm(k, r))


def _back_perm(k: int, r: int) -> List[int]:
    return list(range(k)) + [r - 1] + list(range(k, r - 1))


# ---- Shape ops (ops.ts:468-502) -----------------------------------------------------------

def reshape(a: Tensor, new_shape: Sequence[int]) -> Tensor:
    out = S.infer_reshape('reshape', a.shape, list(new_shape), 'reshape')
    return add_op(current_graph(), 'reshape', out, a.dtype, 'reshape', {'a': a.id, 'newShape': list(out)})


def permute(a: Tensor, perm: Sequence[int]) -> Tensor:
    out = S.infer_permute('permute', a.shape, perm, 'permute')
    return add_op(current_graph(), 'permute', out, a.dtype, 'permute', {'a': a.id, 'perm': list(perm)})


def swap_axes(a: Tensor, axis1: int, axis2: int) -> Tensor:
    r = len(a.shape)
    i1 = r + axis1 if axis1 < 0 else axis1
    i2 = r + axis2 if axis2 < 0 else axis2
    if i1 < 0 or i1 >= r or i2 < 0 or i2 >= r:
        raise ShapeError(f'swapAxes: axis out of range — got ({axis1}, {axis2}) for rank-{r} tensor', 'swapAxes')
    if i1 == i2:
        return a
    perm = list(range(r))
    perm[i1], perm[i2] = i2, i1
    return permute(a, perm)


# ---- Linear algebra (ops.ts:513-538) ----------------------------------------------------------

def matmul(a: Tensor, b: Tensor) -> Tensor:
    if a.dtype != 'f32' or b.dtype != 'f32':
        raise ShapeError(f'matmul: requires f32, got {a.dtype} and {b.dtype}', 'matmul')
    if len(a.shape) < 2:
        raise ShapeError(f'matmul: lhs must have rank >= 2, got {S.show(a.shape)}', 'matmul')
    if len(b.shape) < 2:
        raise ShapeError(f'matmul: rhs must have rank >= 2, got {S.show(b.shape)}', 'matmul')
    if len(b.shape) == 2:
        out = S.infer_matmul('matmul', a.shape, b.shape, 'matmul')
        return add_op(current_graph(), 'matmul', out, 'f32', 'matmul', {'a': a.id, 'b': b.id})
    if len(a.shape) != len(b.shape):
        raise ShapeError(f'matmul: rank mismatch — lhs {S.show(a.shape)} vs rhs {S.show(b.shape)}. When rhs is '
                         f'batched (rank > 2), lhs must have the same rank. Reshape explicitly if needed.', 'matmul')
    out = S.infer_matmul_batched('matmul', a.shape, b.shape, 'matmul')
    return add_op(current_graph(), 'matmul_batched', out, 'f32', 'matmul', {'a': a.id, 'b': b.id})


# ---- Indexing / casting (ops.ts:545-671) ---------------------------------------------------------

def one_hot(indices: Tensor, depth: int, dtype: str = 'f32') -> Tensor:
    if indices.dtype != 'i32':
        raise ShapeError(f'oneHot: indices must be i32, got {indices.dtype}', 'oneHot')
    out = S.infer_one_hot('oneHot', indices.shape, depth, 'oneHot')
    return add_op(current_graph(), 'one_hot', out, dtype, 'oneHot', {'indices': indices.id, 'depth': depth, 'dtype': dtype})


def take_along_axis(inp: Tensor, indices: Tensor, axis: int) -> Tensor:
    if inp.dtype != 'f32':
        raise ShapeError(f'takeAlongAxis: input must be f32, got {inp.dtype}', 'takeAlongAxis')
    if indices.dtype != 'i32':
        raise ShapeError(f'takeAlongAxis: indices must be i32, got {indices.dtype}', 'takeAlongAxis')
    N = len(inp.shape)
    if len(indices.shape) != N:
        raise ShapeError('takeAlongAxis: input and indices must have the same rank', 'takeAlongAxis')
    k = N + axis if axis < 0 else axis
    if k < 0 or k >= N:
        raise ShapeError(f'takeAlongAxis: axis {axis} out of range for rank-{N} input', 'takeAlongAxis')
    for i in range(N):
        if i != k and inp.shape[i] != indices.shape[i]:
            raise ShapeError(f'takeAlongAxis: input and indices must match on every axis except {k}', 'takeAlongAxis')
    permuted = permute(inp, [i for i in range(N) if i != k] + [k])
    sA = inp.shape[k]
    expanded = reshape(permuted, [1 if i == k else inp.shape[i] for i in range(N)] + [sA])
    oh = one_hot(indices, sA, 'f32')
    return sum_(mul(expanded, oh), -1)


def embedding(table: Tensor, indices: Tensor) -> Tensor:
    """`matmul(oneHot(indices, V), table)` (ops.ts:626-635). The backend recognises this
    pattern and runs a gather forward / segmented scatter-add backward."""
    if len(table.shape) != 2:
        raise ShapeError(f'embedding: table must be 2-d [vocab, dim], got {S.show(table.shape)}', 'embedding')
    if indices.dtype != 'i32':
        raise ShapeError(f'embedding: indices must be i32, got {indices.dtype}', 'embedding')
    return matmul(one_hot(indices, table.shape[0], 'f32'), table)


def arange(n: int, dtype: str = 'i32') -> Tensor:
    if not isinstance(n, int) or n <= 0:
        raise ShapeError(f'arange: n must be a positive integer, got {n}', 'arange')
    return add_op(current_graph(), 'arange', [n], dtype, 'arange', {'n': n, 'dtype': dtype})


def _const_fill(name: str, shape: Sequence[int], dtype: str, value: Number) -> Tensor:
    for d in shape:
        if not isinstance(d, int) or d <= 0:
            raise ShapeError(f'{name}: shape must be positive integers, got {S.show(shape)}', name)
    return add_op(current_graph(), 'const_fill', shape, dtype, name, {'value': value, 'dtype': dtype})


def zeros(shape, dtype='f32'): return _const_fill('zeros', shape, dtype, 0)
def ones(shape, dtype='f32'): return _const_fill('ones', shape, dtype, 1)


# ---- ML primitives (ops.ts:675-760) ----------------------------------------------------------------

def _softmax_causal_last(a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'softmaxCausal: requires f32, got {a.dtype}', 'softmaxCausal')
    S.infer_where_causal('softmaxCausal', a.shape, 'softmaxCausal')
    return add_op(current_graph(), 'softmax_causal_last', a.shape, 'f32', 'softmaxCausal', {'a': a.id})


def softmax_causal(a: Tensor, axis: int = -1) -> Tensor:
    return _axis_preserving(a, axis, 'softmaxCausal', _softmax_causal_last)


def _log_softmax_last(a: Tensor) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'logSoftmax: requires f32, got {a.dtype}', 'logSoftmax')
    return add_op(current_graph(), 'log_softmax_last', a.shape, 'f32', 'logSoftmax', {'a': a.id})


def log_softmax(a: Tensor, axis: int = -1) -> Tensor:
    return _axis_preserving(a, axis, 'logSoftmax', _log_softmax_last)


def softmax(a: Tensor, axis: int = -1) -> Tensor:
    return exp(log_softmax(a, axis))


def _axis_preserving(a: Tensor, axis_arg: int, name: str, apply_last) -> Tensor:
    r = len(a.shape)
    if r == 0:
        raise ShapeError(f'{name}: cannot apply to 0-d tensor', name)
    k = r + axis_arg if axis_arg < 0 else axis_arg
    if k < 0 or k >= r:
        raise ShapeError(f'{name}: axis {axis_arg} out of range', name)
    if k == r - 1:
        return apply_last(a)
    perm = [i for i in range(r) if i != k] + [k]
    return permute(apply_last(permute(a, perm)), _back_perm(k, r))


def _axis_reducing(a: Tensor, axis_arg: int, name: str, apply_last) -> Tensor:
    r = len(a.shape)
    if r == 0:
        raise ShapeError(f'{name}: cannot reduce a 0-d tensor', name)
    k = r + axis_arg if axis_arg < 0 else axis_arg
    if k < 0 or k >= r:
        raise ShapeError(f'{name}: axis {axis_arg} out of range', name)
    if k == r - 1:
        return apply_last(a)
    return apply_last(permute(a, [i for i in range(r) if i != k] + [k]))


def where_causal(a: Tensor, fill_value: Number) -> Tensor:
    if a.dtype != 'f32':
        raise ShapeError(f'whereCausal: requires f32, got {a.dtype}', 'whereCausal')
    S.infer_where_causal('whereCausal', a.shape, 'whereCausal')
    return add_op(current_graph(), 'where_causal', a.shape, 'f32', 'whereCausal', {'a': a.id, 'fillValue': fill_value})


# ---- Slicing / concat (ops.ts:766-857) -------------------------------------------------------------

def narrow(a: Tensor, axis: int, start: int, length: int) -> Tensor:
    ax = len(a.shape) + axis if axis < 0 else axis
    end = start + length
    out = S.infer_slice_range('narrow', a.shape, ax, start, end, 'narrow')
    return add_op(current_graph(), 'slice_range', out, a.dtype, 'narrow', {'a': a.id, 'axis': ax, 'start': start, 'end': end})


def scatter_axis(a: Tensor, out_shape: Sequence[int], axis: int, start: int, end: int) -> Tensor:
    out = S.infer_scatter_axis('scatterAxis', a.shape, out_shape, axis, start, end, 'scatterAxis')
    return add_op(current_graph(), 'scatter_axis', out, a.dtype, 'scatterAxis',
                  {'a': a.id, 'outShape': list(out_shape), 'axis': axis, 'start': start, 'end': end})


CONCAT_INPUT_CAP = 7   # ops.ts:788 (kept: it shapes the emitted IR)


def concat(tensors: Sequence[Tensor], axis: int) -> Tensor:
    if len(tensors) == 0:
        raise ShapeError('concat: needs at least one input', 'concat')
    if len(tensors) == 1:
        return tensors[0]
    dtype = tensors[0].dtype
    for t in tensors:
        if t.dtype != dtype:
            raise ShapeError(f'concat: dtype mismatch ({dtype} vs {t.dtype})', 'concat')
    ax = len(tensors[0].shape) + axis if axis < 0 else axis
    layer = list(tensors)
    while len(layer) > CONCAT_INPUT_CAP:
        nxt = []
        for i in range(0, len(layer), CONCAT_INPUT_CAP):
            chunk = layer[i:i + CONCAT_INPUT_CAP]
            nxt.append(chunk[0] if len(chunk) == 1 else _concat_one(chunk, ax))
        layer = nxt
    return _concat_one(layer, ax)


def _concat_one(tensors: Sequence[Tensor], ax: int) -> Tensor:
    out = S.infer_concat('concat', [t.shape for t in tensors], ax, 'concat')
    return add_op(current_graph(), 'concat', out, tensors[0].dtype, 'concat', {'inputs': [t.id for t in tensors], 'axis': ax})


def stack(tensors: Sequence[Tensor], axis: int) -> Tensor:
    if len(tensors) == 0:
        raise ShapeError('stack: needs at least one input', 'stack')
    t0 = tensors[0]
    ax = len(t0.shape) + 1 + axis if axis < 0 else axis
    new_shape = list(t0.shape[:ax]) + [1] + list(t0.shape[ax:])
    return concat([reshape(t, new_shape) for t in tensors], ax)


def split_heads(x: Tensor, n_heads: int) -> Tensor:
    r = len(x.shape)
    if r < 2:
        raise ShapeError(f'splitHeads: requires rank >= 2, got {r}', 'splitHeads')
    T, D = x.shape[r - 2], x.shape[r - 1]
    if D % n_heads != 0:
        raise ShapeError(f'splitHeads: last dim {D} not divisible by nHeads {n_heads}', 'splitHeads')
    lead = list(x.shape[:r - 2])
    reshaped = reshape(x, lead + [T, n_heads, D // n_heads])
    return swap_axes(reshaped, len(lead), len(lead) + 1)


def merge_heads(x: Tensor) -> Tensor:
    r = len(x.shape)
    if r < 3:
        raise ShapeError(f'mergeHeads: requires rank >= 3, got {r}', 'mergeHeads')
    H, T, d = x.shape[r - 3], x.shape[r - 2], x.shape[r - 1]
    lead = list(x.shape[:r - 3])
    swapped = swap_axes(x, r - 3, r - 2)
    return reshape(swapped, lead + [T, H * d])


def split(t: Tensor, sizes: Sequence[int], axis: int) -> List[Tensor]:
    ax = len(t.shape) + axis if axis < 0 else axis
    if ax < 0 or ax >= len(t.shape):
        raise ShapeError(f'split: axis {axis} out of range', 'split')
    if sum(sizes) != t.shape[ax]:
        raise ShapeError(f'split: sizes sum to {sum(sizes)}, but axis {ax} has size {t.shape[ax]}', 'split')
    out, cursor = [], 0
    for s in sizes:
        out.append(narrow(t, ax, cursor, s))
        cursor += s
    return out


def rope(q: Tensor, k: Tensor, base: float = 10000) -> Tuple[Tensor, Tensor]:
    """Rotary embedding, rotate-half convention (ops.ts:878-919)."""
    if q.dtype != 'f32' or k.dtype != 'f32':
        raise ShapeError('rope: q and k must be f32', 'rope')
    T, D = q.shape[-2], q.shape[-1]
    if k.shape[-2] != T or k.shape[-1] != D:
        raise ShapeError('rope: q and k must share sequence and feature dims', 'rope')
    if D % 2 != 0:
        raise ShapeError(f'rope: rotation dim must be even (rotates pairs), got {D}', 'rope')
    half = D // 2
    idx = arange(half, 'f32')
    freqs = exp(mul(idx, -math.log(base) / half))
    positions = arange(T, 'f32')
    angles = mul(reshape(positions, [T, 1]), reshape(freqs, [1, half]))
    cos_half, sin_half = cos(angles), sin(angles)
    cos_full = concat([cos_half, cos_half], -1)
    sin_full = concat([sin_half, sin_half], -1)

    def apply_rot(x: Tensor) -> Tensor:
        x1, x2 = split(x, [half, half], -1)
        rotated = concat([neg(x2), x1], -1)
        return add(mul(x, cos_full), mul(rotated, sin_full))
    return apply_rot(q), apply_rot(k)


# ---- Broadcast / constants / comparisons (ops.ts:943-1008) -----------------------------------------

def broadcast_to(a: Tensor, target: Sequence[int]) -> Tensor:
    S.infer_broadcast_to('broadcastTo', a.shape, target, 'broadcastTo')
    return add_op(current_graph(), 'broadcast_to', target, a.dtype, 'broadcastTo', {'a': a.id, 'targetShape': list(target)})


def sum_to_shape(a: Tensor, target: Sequence[int]) -> Tensor:
    S.infer_sum_to_shape('sumToShape', a.shape, target, 'sumToShape')
    return add_op(current_graph(), 'sum_to_shape', target, a.dtype, 'sumToShape', {'a': a.id, 'targetShape': list(target)})


def const_scalar(value: Number, dtype: str = 'f32') -> Tensor:
    return add_op(current_graph(), 'const_scalar', [], dtype, 'constScalar', {'value': value, 'dtype': dtype})


def less(a, b) -> Tensor:
    if _num(a):
        return greater(b, a)
    rhs = const_scalar(b, a.dtype) if _num(b) else b
    return _binop('less', 'less', a, rhs, 'bool')


def greater(a, b) -> Tensor:
    if _num(a):
        return less(b, a)
    rhs = const_scalar(b, a.dtype) if _num(b) else b
    return _binop('greater', 'greater', a, rhs, 'bool')


def where(cond: Tensor, a: Tensor, b: Tensor) -> Tensor:
    if cond.dtype != 'bool':
        raise ShapeError(f'where: cond must be bool, got {cond.dtype}', 'where')
    if a.dtype != b.dtype:
        raise ShapeError(f'where: a/b dtype mismatch ({a.dtype} vs {b.dtype})', 'where')
    out = S.infer_where('where', cond.shape, a.shape, b.shape, 'where')
    return add_op(current_graph(), 'where', out, a.dtype, 'where', {'cond': cond.id, 'a': a.id, 'b': b.id})


def relu_grad(x: Tensor, dy: Tensor) -> Tensor:
    if x.dtype != 'f32' or dy.dtype != 'f32':
        raise ShapeError(f'reluGrad: requires f32, got {x.dtype} and {dy.dtype}', 'reluGrad')
    out = S.infer_relu_grad('reluGrad', x.shape, dy.shape, 'reluGrad')
    return add_op(current_graph(), 'relu_grad', out, 'f32', 'reluGrad', {'x': x.id, 'dy': dy.id})


# ---- Adam-fused ops (ops.ts:1014-1065) -----------------------------------------------------------------

def adam_update_m(m: Tensor, g: Tensor, beta1: float) -> Tensor:
    if m.dtype != 'f32' or g.dtype != 'f32':
        raise ShapeError('adamUpdateM: requires f32', 'adamUpdateM')
    if m.shape != g.shape:
        raise ShapeError('adamUpdateM: shape mismatch', 'adamUpdateM')
    return add_op(current_graph(), 'adam_update_m', m.shape, 'f32', 'adamUpdateM', {'m': m.id, 'g': g.id, 'beta1': beta1})


def adam_update_v(v: Tensor, g: Tensor, beta2: float) -> Tensor:
    if v.dtype != 'f32' or g.dtype != 'f32':
        raise ShapeError('adamUpdateV: requires f32', 'adamUpdateV')
    if v.shape != g.shape:
        raise ShapeError('adamUpdateV: shape mismatch', 'adamUpdateV')
    return add_op(current_graph(), 'adam_update_v', v.shape, 'f32', 'adamUpdateV', {'v': v.id, 'g': g.id, 'beta2': beta2})


def adam_update_p(p: Tensor, m_new: Tensor, v_new: Tensor, lrt: Tensor, eps: float, decay_shrink=1) -> Tensor:
    if p.dtype != 'f32':
        raise ShapeError('adamUpdateP: requires f32', 'adamUpdateP')
    if lrt.dtype != 'f32' or len(lrt.shape) != 0:
        raise ShapeError('adamUpdateP: lrt must be a 0-d f32 scalar', 'adamUpdateP')
    if p.shape != m_new.shape:
        raise ShapeError('adamUpdateP: p/mNew shape mismatch', 'adamUpdateP')
    is_tensor = isinstance(decay_shrink, Tensor)
    if is_tensor and (decay_shrink.dtype != 'f32' or len(decay_shrink.shape) != 0):
        raise ShapeError('adamUpdateP: decayShrink tensor must be a 0-d f32 scalar', 'adamUpdateP')
    return add_op(current_graph(), 'adam_update_p', p.shape, 'f32', 'adamUpdateP', {
        'p': p.id, 'mNew': m_new.id, 'vNew': v_new.id, 'lrt': lrt.id, 'eps': eps,
        'decayShrink': 1 if is_tensor else decay_shrink,
        'decayShrinkTensor': decay_shrink.id if is_tensor else None,
    })


# ---- Conv / pool (ops.ts:1084-1197) ----------------------------------------------------------------------

def pair_opt(v, default: int) -> Tuple[int, int]:
    if v is None:
        return (default, default)
    if isinstance(v, int):
        return (v, v)
    return (v[0], v[1])


def conv2d(inp: Tensor, weight: Tensor, stride=None, padding=None, groups: int = 1) -> Tensor:
    if inp.dtype != 'f32':
        raise ShapeError(f'conv2d: input must be f32, got {inp.dtype}', 'conv2d')
    if weight.dtype != 'f32':
        raise ShapeError(f'conv2d: weight must be f32, got {weight.dtype}', 'conv2d')
    sH, sW = pair_opt(stride, 1)
    pH, pW = pair_opt(padding, 0)
    out = S.infer_conv2d('conv2d', inp.shape, weight.shape, sH, sW, pH, pW, groups, 'conv2d')
    return add_op(current_graph(), 'conv2d', out, 'f32', 'conv2d', {
        'input': inp.id, 'weight': weight.id, 'strideH': sH, 'strideW': sW, 'padH': pH, 'padW': pW, 'groups': groups})


def conv2d_input_grad(weight: Tensor, dy: Tensor, inH, inW, strideH, strideW, padH, padW, groups) -> Tensor:
    cOut, wInC = weight.shape[0], weight.shape[1]
    B = dy.shape[0]
    if dy.shape[1] != cOut:
        raise ShapeError(f"conv2dInputGrad: dy's C={dy.shape[1]} doesn't match weight C_out={cOut}", 'conv2dInputGrad')
    return add_op(current_graph(), 'conv2d_input_grad', [B, wInC * groups, inH, inW], 'f32', 'conv2dInputGrad', {
        'weight': weight.id, 'dy': dy.id, 'inH': inH, 'inW': inW, 'strideH': strideH, 'strideW': strideW,
        'padH': padH, 'padW': padW, 'groups': groups})


def conv2d_weight_grad(inp: Tensor, dy: Tensor, kH, kW, strideH, strideW, padH, padW, groups) -> Tensor:
    cIn, cOut = inp.shape[1], dy.shape[1]
    return add_op(current_graph(), 'conv2d_weight_grad', [cOut, cIn // groups, kH, kW], 'f32', 'conv2dWeightGrad', {
        'input': inp.id, 'dy': dy.id, 'kH': kH, 'kW': kW, 'strideH': strideH, 'strideW': strideW,
        'padH': padH, 'padW': padW, 'groups': groups})


def max_pool2d(inp: Tensor, kernel_size, stride=None, padding=None) -> Tensor:
    if inp.dtype != 'f32':
        raise ShapeError(f'maxPool2d: input must be f32, got {inp.dtype}', 'maxPool2d')
    kH, kW = (kernel_size, kernel_size) if isinstance(kernel_size, int) else (kernel_size[0], kernel_size[1])
    if stride is None:
        sH, sW = kH, kW
    elif isinstance(stride, int):
        sH, sW = stride, stride
    else:
        sH, sW = stride[0], stride[1]
    pH, pW = pair_opt(padding, 0)
    out = S.infer_max_pool2d('maxPool2d', inp.shape, kH, kW, sH, sW, pH, pW, 'maxPool2d')
    return add_op(current_graph(), 'max_pool_2d', out, 'f32', 'maxPool2d', {
        'input': inp.id, 'kH': kH, 'kW': kW, 'strideH': sH, 'strideW': sW, 'padH': pH, 'padW': pW})


def max_pool2d_grad(inp: Tensor, dy: Tensor, kH, kW, strideH, strideW, padH, padW) -> Tensor:
    return add_op(current_graph(), 'max_pool_2d_grad', inp.shape, 'f32', 'maxPool2dGrad', {
        'input': inp.id, 'dy': dy.id, 'kH': kH, 'kW': kW, 'strideH': strideH, 'strideW': strideW,
        'padH': padH, 'padW': padW})


def nearest_upsample2d(x: Tensor, factor: int) -> Tensor:
    if len(x.shape) != 4:
        raise ShapeError('nearestUpsample2d: input must be rank-4 [B, C, H, W]', 'nearestUpsample2d')
    if factor == 1:
        return x
    B, C, H, W = x.shape
    expanded = broadcast_to(reshape(x, [B, C, H, 1, W, 1]), [B, C, H, factor, W, factor])
    return reshape(expanded, [B, C, H * factor, W * factor])

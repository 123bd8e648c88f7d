"""Kernel-level parity on the GPU: every IR op kind, run as a one-op forward graph through
the C ABI (tg_run), against the CPU oracle on the same inputs.

Bar: element-wise, data-movement, stochastic, softmax, pooling, embedding and i32 ops are
bit-exact; row sums / un-broadcast sums accumulate in f64 in a different order and must
match to 1 ulp of f32; GEMMs and the implicit-GEMM convolutions accumulate in f32 on the
matrix cores and must match to 2e-6 relative (norm-wise)."""
import os

import numpy as np
import pytest

import pyoracle
from _helpers import make_range, wire
from tensorgrad_amd import backend
from tensorgrad_amd import ir as IR
from tensorgrad_amd import nn
from tensorgrad_amd import ops as O
from tensorgrad_amd.grad import append_grad
from tensorgrad_amd.trace import param_input, tensor_input, trace_fn

pytestmark = pytest.mark.gpu


def _rand(shape, seed, lo=-1.0, hi=1.0):
    r = np.random.default_rng(seed)
    return r.uniform(lo, hi, size=shape).astype(np.float32)


def run_both(build, inputs):
    g = trace_fn(build)
    w = wire(g)
    rt = backend.NativeRuntime(IR.dumps(w))
    out_t = g.tensors[g.outputs[0]]
    dt = np.int32 if out_t.dtype in ('i32', 'bool') else np.float32
    got = rt.run(inputs, out_t.shape, dt)
    rt.destroy()
    o = pyoracle.OracleRuntime(w)
    o.run(inputs)
    want = o.output()
    return got, want


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return int(np.max(np.abs(a - b))) if a.size else 0


def exact(got, want):
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.int32), want.view(np.int32)) or np.array_equal(got, want), \
        f'max |diff| {np.max(np.abs(got.astype(np.float64) - want))}'


def near(got, want, ulps=1):
    assert got.shape == want.shape
    assert ulp_diff(got, want) <= ulps


def gemm_close(got, want, tol=2e-6):
    err = np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want.astype(np.float64)), 1e-30)
    assert err <= tol, f'rel err {err:.2e}'


BIN_CASES = [([3, 5], [5]), ([2, 1, 4], [3, 1]), ([6, 7], [6, 7]), ([1000], []), ([4, 1], [1, 9])]


@pytest.mark.parametrize('kind', ['add', 'sub', 'mul', 'div', 'min', 'max'])
@pytest.mark.parametrize('shapes', BIN_CASES)
def test_binary_broadcast(kind, shapes):
    sa, sb = shapes
    fn = {'add': O.add, 'sub': O.sub, 'mul': O.mul, 'div': O.div, 'min': O.minimum, 'max': O.maximum}[kind]
    a, b = _rand(sa, 1), _rand(sb, 2, 0.5, 2.0)
    got, want = run_both(lambda: fn(tensor_input('a', sa), tensor_input('b', sb)), {'a': a, 'b': b})
    exact(got, want)


@pytest.mark.parametrize('R,C', [(12, 8), (9, 6), (5, 20)])
def test_fused_chain_operand_layouts(R, C):
    """A fused pointwise chain reading a transposed view (inner stride != 1), a row vector
    and a column vector broadcast, and a contiguous operand; C % 4 == 0 takes the
    four-elements-per-thread path."""
    x, y, z, w = _rand([C, R], 40), _rand([R, C], 41), _rand([C], 42), _rand([R, 1], 43)

    def body():
        t = O.mul(O.permute(tensor_input('x', [C, R]), [1, 0]), tensor_input('y', [R, C]))
        t = O.add(t, tensor_input('z', [C]))
        t = O.sub(O.relu(t), tensor_input('w', [R, 1]))
        return O.mul(O.dropout(t, 0.25), 3.0)
    got, want = run_both(body, {'x': x, 'y': y, 'z': z, 'w': w})
    exact(got, want)


def test_compare_and_where():
    a, b = _rand([4, 6], 3), _rand([6], 4)
    got, want = run_both(lambda: O.less(tensor_input('a', [4, 6]), tensor_input('b', [6])), {'a': a, 'b': b})
    exact(got, want)

    def body():
        x = tensor_input('a', [4, 6])
        return O.where(O.greater(x, tensor_input('b', [6])), x, O.mul(x, 0.25))
    got, want = run_both(body, {'a': a, 'b': b})
    exact(got, want)
    got, want = run_both(lambda: O.leaky_relu(tensor_input('a', [4, 6]), 2), {'a': a})
    exact(got, want)


@pytest.mark.parametrize('kind', ['sqrt', 'rsqrt', 'log', 'exp', 'relu', 'neg', 'abs', 'tanh', 'sigmoid', 'erf', 'sin',
                                  'cos'])
def test_unary(kind):
    x = _rand([3001], 5, -3, 3)
    if kind in ('sqrt', 'rsqrt', 'log'):
        x = np.abs(x) + np.float32(0.05)
    fn = getattr(O, kind if kind != 'abs' else 'abs_')
    got, want = run_both(lambda: fn(tensor_input('x', [3001])), {'x': x})
    exact(got, want)


def test_scalar_ops_and_gelu():
    x = _rand([257, 3], 6, -4, 4)
    got, want = run_both(lambda: O.gelu(tensor_input('x', [257, 3])), {'x': x})
    exact(got, want)
    got, want = run_both(lambda: O.add(O.mul(tensor_input('x', [257, 3]), 1 / 3), 0.1), {'x': x})
    exact(got, want)


@pytest.mark.parametrize('shape', [[7, 33], [3, 300], [2, 1], [1, 5000], [4096, 256]])
def test_row_reductions(shape):
    x = _rand(shape, 7)
    got, want = run_both(lambda: O.mean(tensor_input('x', shape), -1, keep_dims=True), {'x': x})
    near(got, want)
    got, want = run_both(lambda: O.sum_(tensor_input('x', shape), -1), {'x': x})
    near(got, want)
    got, want = run_both(lambda: O.argmax(tensor_input('x', shape), -1), {'x': x})
    exact(got, want)


def test_argmax_ties_and_nan_semantics():
    x = np.array([[1, 3, 3, 2], [np.nan, 5, 6, 1], [1, np.nan, 5, 5], [-0.0, 0.0, -1, -2], [2, 2, 2, 2]], np.float32)
    x = np.concatenate([x, np.tile(np.array([[0.5, 7, 7, np.nan]], np.float32), (3, 1))])
    got, want = run_both(lambda: O.argmax(tensor_input('x', [8, 4]), -1), {'x': x})
    exact(got, want)
    wide = np.full((3, 200), 1.0, np.float32)
    wide[0, 150] = 2.0
    wide[1, 77] = 2.0
    wide[1, 140] = 2.0
    wide[2, 0] = np.nan
    wide[2, 99] = 5.0
    got, want = run_both(lambda: O.argmax(tensor_input('x', [3, 200]), -1), {'x': wide})
    exact(got, want)


@pytest.mark.parametrize('cells', [([4, 3, 5], [3, 1]), ([6, 5], [5]), ([2, 3, 4, 5], [1, 3, 1, 1]),
                                   ([65536, 4], [4]), ([1000], []), ([128, 64, 24, 24], [1, 64, 1, 1]),
                                   ([4096, 256], [256]), ([3000, 70], [70]), ([32, 128, 256], [128, 256])])
def test_sum_to_shape(cells):
    src, dst = cells
    x = _rand(src, 8)
    got, want = run_both(lambda: O.sum_to_shape(tensor_input('x', src), dst), {'x': x})
    # The GPU sums in f64, so it must equal the f64 sum rounded once (to 1 ulp); the
    # evaluator's f32 running sum differs from that by its own rounding error, bounded by
    # n * eps * max|running sum|.
    xs = x.astype(np.float64).reshape(src)
    keep = tuple(i for i in range(len(src)) if i >= len(src) - len(dst) and dst[i - len(src) + len(dst)] != 1)
    axes = tuple(i for i in range(len(src)) if i not in keep)
    exact64 = xs.sum(axis=axes).reshape(got.shape).astype(np.float32)
    near(got, exact64)
    n = np.prod(src) // max(1, np.prod(dst))
    bound = n * 6e-8 * np.max(np.abs(np.cumsum(np.moveaxis(xs, axes, range(len(axes))).reshape(n, -1), 0)))
    assert np.max(np.abs(got.astype(np.float64) - want)) <= bound + 1e-7


def test_column_sums_repeat_bit_identical():
    """Multi-block column sums count their blocks on device counters that each launch
    leaves at zero: repeated runs of one runtime (two reductions per run) give the same
    bits, equal to the f64 sums rounded once."""
    x = _rand([4096, 256], 21)
    y = _rand([1000, 1030], 22)

    def build():
        a = O.sum_to_shape(tensor_input('x', [4096, 256]), [256])
        b = O.sum_to_shape(tensor_input('y', [1000, 1030]), [1030])
        return O.add(O.sum_(a), O.sum_(b))

    g = trace_fn(build)
    rt = backend.NativeRuntime(IR.dumps(wire(g)))
    outs = [rt.run({'x': x, 'y': y}, [], np.float32) for _ in range(3)]
    rt.destroy()
    for r in outs[1:]:
        exact(r, outs[0])
    want = np.float32(x.astype(np.float64).sum(0).astype(np.float32).astype(np.float64).sum()
                      + y.astype(np.float64).sum(0).astype(np.float32).astype(np.float64).sum())
    assert abs(float(outs[0]) - float(want)) <= 1e-6 * abs(float(want)) + 1e-6


def test_column_sums_of_products_batched():
    """A single-use f32 product feeding a column sum is multiplied inside the sum kernel,
    and two same-shape column sums share one launch: each result equals the f64 sum of the
    f32-rounded products (or values), rounded once."""
    x, y = _rand([3000, 70], 23), _rand([3000, 70], 24)

    def build():
        ty = tensor_input('y', [3000, 70])
        a = O.sum_to_shape(O.mul(tensor_input('x', [3000, 70]), ty), [70])
        b = O.sum_to_shape(ty, [70])
        return O.sub(a, O.mul(b, 0.5))

    g = trace_fn(build)
    rt = backend.NativeRuntime(IR.dumps(wire(g)))
    kinds = [(n['kind'], n.get('ops', '')) for n in rt.describe()['nodes']]
    got = rt.run({'x': x, 'y': y}, [70], np.float32)
    rt.destroy()
    assert ('reduce', 'mul,sum_to_shape,sum_to_shape') in kinds, kinds
    a = (x * y).astype(np.float64).sum(0).astype(np.float32)
    b = y.astype(np.float64).sum(0).astype(np.float32)
    want = (a.astype(np.float64) - (b.astype(np.float64) * 0.5).astype(np.float32)).astype(np.float32)
    near(got, want, 2)


def test_broadcast_permute_slice_concat_scatter():
    x = _rand([2, 3, 4], 9)
    got, want = run_both(lambda: O.permute(tensor_input('x', [2, 3, 4]), [2, 0, 1]), {'x': x})
    exact(got, want)
    got, want = run_both(lambda: O.reshape(O.permute(tensor_input('x', [2, 3, 4]), [1, 2, 0]), [12, 2]), {'x': x})
    exact(got, want)
    got, want = run_both(lambda: O.broadcast_to(tensor_input('x', [2, 3, 4]), [5, 2, 3, 4]), {'x': x})
    exact(got, want)
    got, want = run_both(lambda: O.narrow(tensor_input('x', [2, 3, 4]), 1, 1, 2), {'x': x})
    exact(got, want)
    y, z = _rand([2, 5, 4], 10), _rand([2, 1, 4], 11)
    got, want = run_both(lambda: O.concat([tensor_input('x', [2, 3, 4]), tensor_input('y', [2, 5, 4]),
                                           tensor_input('z', [2, 1, 4])], 1), {'x': x, 'y': y, 'z': z})
    exact(got, want)
    # along the last axis (one launch writing whole rows): C4's encoding [x, sin, cos] and
    # skip [h, pe] at 1000 rows, a 3-d case with a one-wide input
    for shapes in ([[1000, 3], [1000, 30], [1000, 30]], [[1000, 256], [1000, 63]], [[2, 5, 3], [2, 5, 7], [2, 5, 1]]):
        ins = {f'i{j}': _rand(s, 20 + j) for j, s in enumerate(shapes)}
        got, want = run_both(lambda: O.concat([tensor_input(f'i{j}', s) for j, s in enumerate(shapes)], -1), ins)
        exact(got, want)
    got, want = run_both(lambda: O.scatter_axis(tensor_input('x', [2, 3, 4]), [2, 7, 4], 1, 2, 5), {'x': x})
    exact(got, want)
    got, want = run_both(lambda: O.add(O.zeros([3, 4]), O.arange(4, 'f32')), {})
    exact(got, want)


@pytest.mark.parametrize('T', [128, 300])
def test_row_groups_wide_rows(T):
    """Row-fused groups with two or four columns per lane access (D = 128, and 300 with a
    partly live last chunk): causal softmax with dropout, and a row chain reading one
    operand through a transposed view (scalar accesses at vector-layout columns)."""
    x = _rand([2, T, T], 51, -4, 4)
    got, want = run_both(lambda: O.dropout(O.softmax_causal(O.mul(tensor_input('x', [2, T, T]), 0.125)), 0.1),
                         {'x': x})
    exact(got, want)
    a, bt = _rand([7, T], 52), _rand([T, 7], 53)

    def chain():
        t = O.mul(tensor_input('a', [7, T]), O.permute(tensor_input('b', [T, 7]), [1, 0]))
        return O.sub(t, O.mean(t, -1, keep_dims=True))
    got, want = run_both(chain, {'a': a, 'b': bt})
    near(got, want)


def test_softmaxes_and_causal_mask():
    x = _rand([3, 2, 17, 17], 12, -5, 5)
    got, want = run_both(lambda: O.softmax_causal(tensor_input('x', [3, 2, 17, 17])), {'x': x})
    exact(got, want)
    got, want = run_both(lambda: O.where_causal(tensor_input('x', [3, 2, 17, 17]), -1e30), {'x': x})
    exact(got, want)
    y = _rand([50, 65], 13, -8, 8)
    got, want = run_both(lambda: O.log_softmax(tensor_input('x', [50, 65])), {'x': y})
    exact(got, want)
    got, want = run_both(lambda: O.softmax(tensor_input('x', [50, 65]), 0), {'x': y})
    exact(got, want)


CE_SHAPES = [(64, 27), (128, 10), (50, 65), (7, 130), (4096, 65)]


@pytest.mark.parametrize('R,D', CE_SHAPES)
def test_cross_entropy_row_chains(R, D):
    """The row groups of a cross-entropy forward (bias add, log-softmax, exp) and backward
    (one-hot scaling, row sum, softmax correction), one elements per lane (D <= 64) and
    several, against the oracle bit for bit."""
    x = _rand([R, D], 31, -6, 6)
    b = _rand([D], 32)
    t = np.random.default_rng(33).integers(0, D, size=[R]).astype(np.int32)
    g = _rand([R, 1], 34)
    ins = {'x': x, 'b': b, 't': t, 'g': g}

    def lsm():
        return O.log_softmax(O.add(tensor_input('x', [R, D]), tensor_input('b', [D])))

    got, want = run_both(lsm, ins)
    exact(got, want)
    got, want = run_both(lambda: O.exp(lsm()), ins)
    exact(got, want)

    def backward(e):
        oh = O.one_hot(tensor_input('t', [R], 'i32'), D, 'f32')
        d = O.mul(O.broadcast_to(tensor_input('g', [R, 1]), [R, D]), oh)
        s = O.reshape(O.sum_(d, -1), [R, 1])
        return O.sub(d, O.mul(O.broadcast_to(s, [R, D]), e))

    got, want = run_both(lambda: backward(tensor_input('x', [R, D])), ins)
    exact(got, want)
    got, want = run_both(lambda: backward(O.exp(lsm())), ins)
    exact(got, want)
    # The loss itself: the target pick (one_hot evaluated inside the row group from the
    # targets) and the batch mean (one wide single-row group when R > 1024), f64 row sums
    # in lane order: within one f32 ulp of the evaluator's sequential sum.
    got, want = run_both(lambda: nn.cross_entropy(O.add(tensor_input('x', [R, D]), tensor_input('b', [D])),
                                                  tensor_input('t', [R], 'i32')), ins)
    near(got, want)


def _attention_graph(B, H, T, dh, what):
    def body():
        q, k, v = (tensor_input(n, [B, H, T, dh]) for n in ('q', 'k', 'v'))
        s = O.matmul(q, O.permute(k, [0, 1, 3, 2]))
        p = O.softmax_causal(O.mul(s, 0.125))
        pd = O.dropout(p, 0.1)
        o = O.matmul(pd, v)
        return {'o': o, 'p': p, 'pd': pd}[what]
    return body


def _node_ops(g, env):
    """The launch list ('ops' of each node) of a runtime created under `env`."""
    import os
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        rt = backend.NativeRuntime(IR.dumps(wire(g)))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    ops = [n.get('ops', '') for n in rt.describe()['nodes']]
    rt.destroy()
    return ops


def _run_native(g, inputs, env=None):
    import os
    old = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        rt = backend.NativeRuntime(IR.dumps(wire(g)))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    out_t = g.tensors[g.outputs[0]]
    kinds = [n['kind'] for n in rt.describe()['nodes']]
    got = rt.run(inputs, out_t.shape, np.float32)
    rt.destroy()
    return got, kinds


# (B, H, T, dh): the matrix-core kernels (dh = 64, T = 64 / 128) and the one-workgroup-per-
# head kernels for smaller heads, at the reference samples' shapes (T = 8 and 16 with
# dh = 16), odd sizes, one token, and T = 64 with a head below 64
ATTN_SHAPES = [(2, 3, 64, 64), (2, 3, 128, 64), (32, 4, 128, 64), (128, 4, 8, 16), (32, 4, 16, 16), (3, 2, 5, 12),
               (2, 2, 1, 8), (2, 3, 32, 64), (2, 2, 64, 32), (1, 2, 48, 20)]


@pytest.mark.parametrize('B,H,T,dh', ATTN_SHAPES)
@pytest.mark.parametrize('what', ['o', 'p', 'pd'])
def test_fused_attention(B, H, T, dh, what):
    """The fused attention kernel (Q K^T, scale, causal softmax, dropout, P V in one
    launch) against the oracle (GEMM tolerance: the products run on f32 matrix cores, or
    for small heads accumulate in f64 as the oracle does; the softmax takes f32 exp with
    an f64 row sum), and against the unfused kernels (TG_ATTN=0) within the same
    tolerance. P and Pd hold exact zeros past the diagonal and the same dropout mask as
    the oracle (the reference's hash on the flat index)."""
    ins = {n: _rand([B, H, T, dh], s, -2, 2) for n, s in (('q', 61), ('k', 62), ('v', 63))}
    g = trace_fn(_attention_graph(B, H, T, dh, what))
    got, kinds = _run_native(g, ins)
    assert 'attention' in kinds
    ref, kinds0 = _run_native(g, ins, {'TG_ATTN': '0'})
    assert 'attention' not in kinds0
    o = pyoracle.OracleRuntime(wire(g))
    o.run(ins)
    want = o.output()
    if what == 'o':
        gemm_close(got, want)
        gemm_close(got, ref)
    else:
        for r in (want, ref):
            assert np.allclose(got, r, rtol=1e-5, atol=1e-7), np.max(np.abs(got.astype(np.float64) - r))
        g4 = got.reshape(B, H, T, T)
        assert np.all(g4[..., np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0)
        assert np.array_equal(got.reshape(-1) == 0, np.asarray(want).reshape(-1) == 0)


def _attention_grad(B, H, T, dh, which, params, g_in, env=None):
    """d(sum(attention(q, k, v) * g)) / d`which` on the native runtime, with the graph."""
    def body():
        q, k, v = (param_input(n, [B, H, T, dh]) for n in ('q', 'k', 'v'))
        s = O.matmul(q, O.permute(k, [0, 1, 3, 2]))
        p = O.softmax_causal(O.mul(s, 0.125))
        o = O.matmul(O.dropout(p, 0.1), v)
        return O.sum_(O.mul(o, tensor_input('g', [B, H, T, dh])))
    g = trace_fn(body)
    gr = append_grad(g)
    g.outputs = [gr.param_grads[which].id]
    w = wire(g, gr.param_grads)
    import os
    old = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        rt = backend.NativeRuntime(IR.dumps(w))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    ops = [n.get('ops', '') for n in rt.describe()['nodes']]
    rt.upload_params(params)
    got = rt.run({'g': g_in}, [B, H, T, dh], np.float32)
    rt.destroy()
    return got, ops, w


@pytest.mark.parametrize('B,H,T,dh', ATTN_SHAPES)
def test_fused_attention_backward(B, H, T, dh):
    """The fused attention backward (dPd = dO V^T, dropout and softmax backward row math,
    dQ = dS K, dK = dS^T Q, dV = Pd^T dO; two launches for dh = 64, one for small heads)
    for the gradients of q, k and v, against the oracle and the unfused kernels
    (TG_ATTN=0), GEMM tolerance."""
    params = {n: _rand([B, H, T, dh], s, -2, 2) for n, s in (('q', 71), ('k', 72), ('v', 73))}
    g_in = _rand([B, H, T, dh], 74)
    for which in ('q', 'k', 'v'):
        got, ops, w = _attention_grad(B, H, T, dh, which, params, g_in)
        assert 'attention_backward' in ops
        ref, ops0, _ = _attention_grad(B, H, T, dh, which, params, g_in, {'TG_ATTN': '0'})
        assert 'attention_backward' not in ops0
        gemm_close(got, ref, 1e-5)
        o = pyoracle.OracleRuntime(w)
        for k, v in params.items():
            o.set_home(k, v)
        o.run({'g': g_in})
        gemm_close(got, o.output(), 1e-5)


@pytest.mark.parametrize('M,N,K,act', [(512, 256, 256, 'relu'), (4096, 1024, 256, 'gelu'), (300, 64, 128, 'gelu'),
                                       (1000, 256, 512, 'dropout'), (20000, 256, 4, 'relu'), (3001, 100, 9, 'gelu'),
                                       (1000, 256, 63, 'relu'), (700, 128, 45, 'gelu'), (130, 64, 10, 'relu'),
                                       (256, 64, 1, 'relu'), (300, 1, 64, 'gelu'), (1, 200, 77, 'relu')])
def test_gemm_epilogue(M, N, K, act):
    """With TG_GEMM_EPI=1, a product read only by one pointwise group runs that group in
    the GEMM's epilogue (a kernel generated per group): bit-identical to the GEMM and the
    group run apart (TG_GEMM_EPI=0), and within GEMM tolerance of the oracle. By default
    only groups of inexpensive ops (the relu case) run in the epilogue. K <= 16 takes the
    small-K kernel (one thread per column, FMA chains) with the epilogue in it; K not a
    multiple of 32 the element-wise tile (a partial last k stage); one of M, N, K equal to
    1 the tiny kernel (lanes per output and a butterfly)."""
    ins = {'a': _rand([M, K], 101), 'b': _rand([K, N], 102), 'c': _rand([N], 103), 'r': _rand([M, N], 104)}

    def body():
        h = O.add(O.matmul(tensor_input('a', [M, K]), tensor_input('b', [K, N])), tensor_input('c', [N]))
        if act == 'relu':
            y = O.relu(h)
        elif act == 'gelu':
            y = O.mul(O.mul(h, 0.5), O.add(O.erf(O.mul(h, 0.7071067811865476)), 1.0))
        else:
            y = O.dropout(O.mul(h, tensor_input('r', [M, N])), 0.25)
        return O.mul(y, 2.0)
    g = trace_fn(body)
    got, _ = _run_native(g, ins, {'TG_GEMM_EPI': '1'})
    ref, _ = _run_native(g, ins, {'TG_GEMM_EPI': '0'})
    ops = _node_ops(g, {'TG_GEMM_EPI': '1'})
    assert any(o.startswith('gemm+') for o in ops), ops
    assert not any(o.startswith('gemm+') for o in _node_ops(g, {'TG_GEMM_EPI': '0'}))
    assert any(o.startswith('gemm+') for o in _node_ops(g, {})) == (act == 'relu')
    auto, _ = _run_native(g, ins)
    exact(auto, ref)
    exact(got, ref)
    o = pyoracle.OracleRuntime(wire(g))
    o.run(ins)
    gemm_close(got, o.output(), 1e-5)


@pytest.mark.parametrize('terms,K', [(2, 256), (3, 256), (3, 128)])
def test_sum_of_products(terms, K):
    """add(matmul, matmul[, matmul]) with single-use products runs as one GEMM over the
    concatenated k segments (each segment read through its own operand bases): against the
    oracle with GEMM tolerance, and against the unfused products and adds (TG_GEMM_GROUP=0)
    within f32 rounding."""
    M, N = 512, 256
    ins = {}
    for q in range(terms):
        ins[f'a{q}'] = _rand([M, K], 80 + q)
        ins[f'b{q}'] = _rand([N, K], 90 + q)

    def body():
        acc = None
        for q in range(terms):
            p = O.matmul(tensor_input(f'a{q}', [M, K]), O.swap_axes(tensor_input(f'b{q}', [N, K]), -1, -2))
            acc = p if acc is None else O.add(acc, p)
        return O.relu(acc)
    g = trace_fn(body)
    got, kinds = _run_native(g, ins)
    ref, _ = _run_native(g, ins, {'TG_GEMM_GROUP': '0'})
    rt = backend.NativeRuntime(IR.dumps(wire(g)))
    ops = [n.get('ops', '') for n in rt.describe()['nodes']]
    rt.destroy()
    assert 'gemm_sum' in ops
    o = pyoracle.OracleRuntime(wire(g))
    o.run(ins)
    gemm_close(got, o.output())
    gemm_close(got, ref)


@pytest.mark.parametrize('M,k0,k1,N,epi', [(1000, 32, 63, 256, False), (700, 256, 63, 256, True),
                                            (513, 64, 1, 100, False), (2048, 128, 32, 64, True),
                                            (300, 32, 100, 36, False), (4096, 256, 63, 256, True)])
def test_concat_product(M, k0, k1, N, epi):
    """matmul(concat([S0, S1], -1), W), C4's skip layer: one GEMM reading both sources in
    place (S0's 32-k stages sixteen bytes per lane, S1's one element per lane, a partial
    last stage zeroed in LDS), with the bias + ReLU group in its epilogue when present;
    the concatenation itself is not materialised. Against the oracle with GEMM tolerance
    and against the concatenation copied and multiplied (TG_GEMM_GROUP=0)."""
    ins = {'s0': _rand([M, k0], 111), 's1': _rand([M, k1], 112), 'w': _rand([k0 + k1, N], 113),
           'c': _rand([N], 114)}

    def body():
        x = O.concat([tensor_input('s0', [M, k0]), tensor_input('s1', [M, k1])], -1)
        h = O.matmul(x, tensor_input('w', [k0 + k1, N]))
        return O.relu(O.add(h, tensor_input('c', [N]))) if epi else h
    g = trace_fn(body)
    ops = _node_ops(g, {})
    assert ('gemm_cat+add,relu' if epi else 'gemm_cat') in ops, ops
    got, kinds = _run_native(g, ins)
    assert 'copy' not in kinds, kinds
    ref, _ = _run_native(g, ins, {'TG_GEMM_GROUP': '0'})
    o = pyoracle.OracleRuntime(wire(g))
    o.run(ins)
    gemm_close(got, o.output())
    gemm_close(got, ref)


def test_sliced_products():
    """A product read only by a slice keeping its first columns computes just those columns
    (B read through the same view, narrowed); an embedding product (one_hot @ table, the
    row gather) is gathered whole and then sliced, since the gather reads whole table rows.
    Against the oracle: GEMM tolerance for the product, bit-exact for the gather."""
    M, K, N, w = 300, 64, 96, 40
    ins = {'a': _rand([M, K], 131), 'b': _rand([N, K], 132)}

    def prod():
        p = O.matmul(tensor_input('a', [M, K]), O.swap_axes(tensor_input('b', [N, K]), -1, -2))
        return O.relu(O.narrow(p, -1, 0, w))
    g = trace_fn(prod)
    rt = backend.NativeRuntime(IR.dumps(wire(g)))
    shapes = [n['shape'] for n in rt.describe()['nodes']]
    rt.destroy()
    assert not any('[300,40]' == s for s in shapes if s), shapes   # no slice copy
    got, want = run_both(prod, ins)
    gemm_close(got, want)

    idx = np.random.default_rng(133).integers(0, 10, 64).astype(np.int32)
    tab = _rand([10, 32], 134)

    def emb():
        e = O.matmul(O.one_hot(tensor_input('i', [64], 'i32'), 10), tensor_input('t', [10, 32]))
        return O.narrow(e, -1, 0, 16)
    got, want = run_both(emb, {'i': idx, 't': tab})
    exact(got, want)
    assert np.array_equal(got, tab[idx, :16])


def test_concat_forward_and_transposed_readers():
    """A concatenation read by a product (the forward) and, transposed, by another (the
    weight gradient): the first runs over the sources in place, the second as one GEMM per
    source writing its own rows, and the concatenation is never written. Both products
    (stacked into one output) against the oracle."""
    M, k0, k1, N = 2000, 64, 40, 96
    ins = {'s0': _rand([M, k0], 121), 's1': _rand([M, k1], 122), 'w': _rand([k0 + k1, N], 123),
           'd': _rand([M, N], 124)}

    def body():
        x = O.concat([tensor_input('s0', [M, k0]), tensor_input('s1', [M, k1])], -1)
        y = O.matmul(x, tensor_input('w', [k0 + k1, N]))
        gw = O.matmul(O.swap_axes(x, -1, -2), tensor_input('d', [M, N]))
        return O.concat([y, gw], 0)
    g = trace_fn(body)
    rt = backend.NativeRuntime(IR.dumps(wire(g)))
    nodes = rt.describe()['nodes']
    rt.destroy()
    shapes = [n['shape'] for n in nodes]
    assert f'[{k0 + k1},{M}]x[{M},{N}] by 2 sources' in shapes, shapes
    assert 'gemm_cat' in [n.get('ops') for n in nodes], nodes
    assert not [n for n in nodes if n['kind'] == 'copy' and n['shape'] == f'[{M},{k0 + k1}]'], shapes
    got, _ = _run_native(g, ins)
    o = pyoracle.OracleRuntime(wire(g))
    o.run(ins)
    gemm_close(got, o.output())


GEMMS = [([5, 7], [7, 3], False, False), ([2, 33, 65], [65, 17], False, False), ([129, 64], [64, 300], False, False),
         ([70, 40], [50, 40], False, True), ([40, 70], [40, 50], True, False), ([4096, 256], [4096, 256], True, False),
         ([300, 4096], [4096, 64], False, False),
         # rows of B not 16-byte aligned (65 / 67 wide): the direct-to-LDS tile moving B one
         # element per lane, a partial last column tile, and split-K for a long K
         ([4096, 256], [256, 65], False, False), ([4096, 256], [4096, 65], True, False),
         ([200, 128], [128, 67], False, False),
         # neither operand 16-byte aligned and K not a multiple of 32 (C4's 63- and 319-wide
         # inputs): both operands one element per lane, a partial last k stage zeroed in LDS
         ([1000, 63], [63, 256], False, False), ([700, 319], [319, 256], False, False),
         ([2000, 319], [2000, 256], True, False), ([4096, 4], [4, 256], False, False),
         ([9000, 63], [9000, 64], True, False), ([3, 33, 17], [17, 9], False, False),
         ([130, 45], [70, 45], False, True), ([8192, 319], [319, 512], False, False),
         # skinny products (16-wide column tiles, N padded to a multiple of 16 only): the LM
         # head forward, input gradient (K = 65) and weight gradient (split-K), C2's and C3's
         # heads, 100- and 112-wide products, short k with 256 columns
         ([4096, 65], [256, 65], False, True), ([1024, 512], [512, 27], False, False),
         ([1024, 512], [1024, 27], True, False), ([128, 128], [128, 10], False, False),
         ([128, 10], [128, 10], False, True), ([128, 128], [128, 10], True, False),
         ([512, 96], [96, 100], False, False), ([333, 200], [200, 112], False, False),
         ([300, 27], [27, 256], False, False), ([2048, 300], [2048, 65], True, False),
         # short products (K <= 16, at least 64K outputs: the small-K kernel, also taking
         # [4096, 4] x [4, 256] above): batched with a shared B, B transposed, 33 columns of
         # a 256-column block, C4's head input gradient, K = 1 beyond the tiny kernel's size
         ([3, 700, 13], [13, 300], False, False), ([5000, 9], [300, 9], False, True),
         ([20000, 7], [7, 33], False, False), ([65536, 4], [4, 256], False, False),
         ([3000, 1], [1, 1000], False, False), ([40, 50, 16], [40, 16, 70], False, False)]


@pytest.mark.parametrize('case', GEMMS)
def test_matmul(case):
    sa, sb, ta, tb = case
    a, b = _rand(sa, 14), _rand(sb, 15)

    def body():
        A = tensor_input('a', sa)
        B = tensor_input('b', sb)
        if ta:
            A = O.swap_axes(A, -1, -2)
        if tb:
            B = O.swap_axes(B, -1, -2)
        return O.matmul(A, B)
    got, want = run_both(body, {'a': a, 'b': b})
    gemm_close(got, want)


@pytest.mark.parametrize('sa,sb,ta', [([256, 1], [1, 64], False), ([256, 64], [64, 1], False),
                                      ([1, 256], [256, 64], False), ([64, 4096], [4096, 1], False),
                                      ([3, 1], [1, 5], False), ([256, 1], [64, 1], True),
                                      ([2, 7, 1], [2, 1, 9], False), ([5, 1, 300], [5, 300, 33], False)])
def test_degenerate_products(sa, sb, ta):
    """Products with one of M, N, K equal to 1 (outer products, matrix-vector products,
    batched too) run on the lane-group kernel: within GEMM tolerance of the oracle, and
    bit for bit with K = 1, where each output is the single product rounded once."""
    a, b = _rand(sa, 31), _rand(sb, 32)

    def body():
        B = tensor_input('b', sb)
        if ta:
            B = O.swap_axes(B, -1, -2)
        return O.matmul(tensor_input('a', sa), B)
    got, want = run_both(body, {'a': a, 'b': b})
    if sa[-1] == 1:
        exact(got, want)
    else:
        gemm_close(got, want)


def test_matmul_batched_head_views():
    # q @ k^T on split-head views: [B,T,D] -> [B,H,T,d] permutes read in place.
    B, T, H, d = 3, 20, 4, 8
    x, y = _rand([B, T, H * d], 16), _rand([B, T, H * d], 17)

    def body():
        q = O.split_heads(tensor_input('x', [B, T, H * d]), H)
        k = O.split_heads(tensor_input('y', [B, T, H * d]), H)
        return O.merge_heads(O.matmul(O.softmax_causal(O.mul(O.matmul(q, O.swap_axes(k, -1, -2)), 0.3)), k))
    got, want = run_both(body, {'x': x, 'y': y})
    gemm_close(got, want, 5e-6)


@pytest.mark.parametrize('V,N,rows,skew', [
    (65, 48, 300, False),      # per-wave histograms, token stash in LDS
    (3000, 40, 2000, False),   # V > 1024: one wavefront places all rows
    (50, 300, 20000, False),   # too many rows for the LDS stash; N > 256 columns
    (7, 33, 5000, True),       # one token owns most rows: long buckets cut into many items
    (2, 8, 64, False),
])
def test_embedding_gather_and_scatter(V, N, rows, skew):
    rng = np.random.default_rng(18)
    idx = rng.integers(-2, V + 2, size=rows).astype(np.int32)   # includes out-of-range ids
    if skew:
        idx[rng.random(rows) < 0.9] = V // 2
    table, dy = _rand([V, N], 19), _rand([rows, N], 20)
    got, want = run_both(lambda: O.embedding(tensor_input('t', [V, N]), tensor_input('i', [rows], 'i32')),
                         {'t': table, 'i': idx})
    exact(got, want)

    def grad_body():
        oh = O.reshape(O.one_hot(tensor_input('i', [rows], 'i32'), V), [rows, V])
        return O.matmul(O.swap_axes(oh, -1, -2), tensor_input('d', [rows, N]))
    got, want = run_both(grad_body, {'i': idx, 'd': dy})
    # f64 sums in row order (small vocabularies sequentially, large ones in runs of 16
    # rows): equal to the evaluator's sequential f64 sum up to f64 rounding, so at most
    # one f32 ulp apart.
    near(got, want)
    got, want = run_both(lambda: O.one_hot(tensor_input('i', [rows], 'i32'), V), {'i': idx})
    exact(got, want)


def _conv_env(impl):
    """TG_CONV is read when a runtime is created: 'direct' selects the f64 direct kernels."""
    import os
    old = os.environ.get('TG_CONV')
    if impl == 'direct':
        os.environ['TG_CONV'] = 'direct'
    else:
        os.environ.pop('TG_CONV', None)
    return old


CONV_CASES = [
    # B, Ci, H, W, Co, G, k, stride, pad
    (2, 4, 9, 8, 6, 2, 3, 2, 1),
    (128, 1, 28, 28, 32, 1, 3, 1, 0),      # the CNN config's first layer
    (128, 32, 26, 26, 64, 1, 3, 1, 0),     # its second layer (split-K weight gradient)
    (3, 5, 11, 7, 130, 1, 5, 1, 2),        # 5x5, padding, Cout above one tile
    (4, 2, 10, 9, 6, 2, 3, 2, 1),          # 9 taps per output (vector-ALU forward / weight
    (5, 2, 7, 7, 5, 1, 2, 1, 0),           # gradient): groups, stride, padding, partial chunks
    (2, 64, 9, 10, 40, 2, 3, 2, 1),        # direct-to-LDS conv2d: 32 channels per group, stride,
    (3, 40, 7, 9, 64, 2, 3, 1, 1),         # padding, partial tiles; direct-to-LDS input gradient
    (2, 8, 12, 11, 32, 1, 5, 1, 2),        # (32 output channels per group), 3x3 and 5x5, padded
]


@pytest.mark.parametrize('impl', ['gemm', 'direct'])
@pytest.mark.parametrize('case', CONV_CASES)
def test_conv_kernels(impl, case):
    """Implicit-GEMM convolutions (default) accumulate in f32 on the matrix cores (layers
    with at most 16 taps per output: forward and weight gradient on the vector ALU): within
    2e-6 relative (norm-wise) of the evaluator, like the GEMMs. The direct kernels
    (TG_CONV=direct) reproduce the evaluator's f64 loops: forward and input gradient bit
    for bit, the weight gradient (different f64 summation order) within 1 ulp."""
    B, Ci, H, W, Co, G, k, s, pd = case
    if impl == 'direct' and B > 8:
        pytest.skip('the direct kernels are checked at small sizes')
    old = _conv_env(impl)
    try:
        x, w = _rand([B, Ci, H, W], 21), _rand([Co, Ci // G, k, k], 22)
        got, want = run_both(lambda: O.conv2d(tensor_input('x', [B, Ci, H, W]), tensor_input('w', [Co, Ci // G, k, k]),
                                              stride=s, padding=pd, groups=G), {'x': x, 'w': w})
        exact(got, want) if impl == 'direct' else gemm_close(got, want)
        yshape = list(want.shape)
        dy = _rand(yshape, 23)
        got, want = run_both(lambda: O.conv2d_input_grad(tensor_input('w', [Co, Ci // G, k, k]),
                                                         tensor_input('d', yshape), H, W, s, s, pd, pd, G),
                             {'w': w, 'd': dy})
        exact(got, want) if impl == 'direct' else gemm_close(got, want)
        got, want = run_both(lambda: O.conv2d_weight_grad(tensor_input('x', [B, Ci, H, W]), tensor_input('d', yshape),
                                                          k, k, s, s, pd, pd, G), {'x': x, 'd': dy})
        near(got, want) if impl == 'direct' else gemm_close(got, want)
    finally:
        if old is None:
            os.environ.pop('TG_CONV', None)
        else:
            os.environ['TG_CONV'] = old


@pytest.mark.parametrize('B,Ci,H,Co,k,pd', [(4, 3, 12, 16, 3, 1), (8, 1, 28, 32, 3, 0), (2, 8, 9, 40, 5, 2)])
def test_conv_epilogues(B, Ci, H, Co, k, pd):
    """A convolution whose output only its layer's pointwise step reads applies that step
    at the store: relu(conv2d(x, w) + b) in the forward (the implicit GEMM, or the few-taps
    kernel for a 1-channel input) and relu_grad(m, conv2d_input_grad(w, dy)) in the input
    gradient. Against the oracle with the convolutions' GEMM tolerance; masks with ties at
    zero and negative values."""
    Ho = H + 2 * pd - k + 1
    x, w, b = _rand([B, Ci, H, H], 31), _rand([Co, Ci, k, k], 32), _rand([Co], 33)
    dy = _rand([B, Co, Ho, Ho], 34)
    m = np.round(_rand([B, Ci, H, H], 35) * 2) / 2   # zeros, negatives and positives

    def fwd():
        y = O.conv2d(tensor_input('x', [B, Ci, H, H]), tensor_input('w', [Co, Ci, k, k]), padding=pd)
        return O.relu(O.add(y, O.reshape(tensor_input('b', [Co]), [1, Co, 1, 1])))
    assert 'conv2d,add,relu' in _node_ops(trace_fn(fwd), {})
    got, want = run_both(fwd, {'x': x, 'w': w, 'b': b})
    gemm_close(got, want)
    assert np.array_equal(got > 0, want > 0) or np.mean((got > 0) != (want > 0)) < 1e-3

    def dgrad():
        g = O.conv2d_input_grad(tensor_input('w', [Co, Ci, k, k]), tensor_input('d', [B, Co, Ho, Ho]), H, H, 1, 1,
                                pd, pd, 1)
        return O.relu_grad(tensor_input('m', [B, Ci, H, H]), g)
    assert 'conv2d_input_grad,relu_grad' in _node_ops(trace_fn(dgrad), {})
    got, want = run_both(dgrad, {'w': w, 'd': dy, 'm': m})
    gemm_close(got, want)
    assert np.all(got[m <= 0] == 0) and not np.any(np.signbit(got[m <= 0]))


@pytest.mark.parametrize('k,s,pd', [(3, 2, 1), (2, 2, 0), (3, 3, 0)])
def test_pool_kernels(k, s, pd):
    """Overlapping / padded windows use the gather adjoint; windows that tile the input
    (2x2 and 3x3 with stride = window on 12x12) use the scatter adjoint. Both bit-exact,
    ties resolving to the first element scanned."""
    H = 12
    Ho = (H + 2 * pd - k) // s + 1
    p = np.round(_rand([2, 3, H, H], 24) * 4) / 4   # ties inside windows
    got, want = run_both(lambda: O.max_pool2d(tensor_input('x', [2, 3, H, H]), k, stride=s, padding=pd), {'x': p})
    exact(got, want)
    assert got.shape == (2, 3, Ho, Ho)
    d = _rand([2, 3, Ho, Ho], 25)
    got, want = run_both(lambda: O.max_pool2d_grad(tensor_input('x', [2, 3, H, H]), tensor_input('d', [2, 3, Ho, Ho]),
                                                    k, k, s, s, pd, pd), {'x': p, 'd': d})
    exact(got, want)


@pytest.mark.parametrize('k,s,pd', [(3, 2, 1), (2, 2, 0), (3, 3, 0)])
def test_pool_grad_with_relu_grad(k, s, pd):
    """relu_grad(x, max_pool2d_grad(relu(x), d)) (the CNN's pooled ReLU layer): the pool
    gradient launch applies the ReLU mask of its own input and writes the relu_grad's
    output, for the gather and the scatter adjoints. Bit-exact against the oracle, with
    ties, zeros, negative maxima and whole non-positive windows."""
    H = 12
    Ho = (H + 2 * pd - k) // s + 1
    x = np.round(_rand([2, 3, H, H], 28) * 4) / 4 - 0.25
    x[0, 0, :4, :4] = -1.0    # windows with no positive element
    d = _rand([2, 3, Ho, Ho], 29)

    def body():
        xi = tensor_input('x', [2, 3, H, H])
        g = O.max_pool2d_grad(O.relu(xi), tensor_input('d', [2, 3, Ho, Ho]), k, k, s, s, pd, pd)
        return O.relu_grad(xi, g)
    g = trace_fn(body)
    assert 'max_pool_2d_grad,relu_grad' in _node_ops(g, {})
    got, want = run_both(body, {'x': x, 'd': d})
    exact(got, want)


def test_relu_grad():
    x, dy = _rand([1000], 26), _rand([1000], 27)
    got, want = run_both(lambda: O.relu_grad(tensor_input('x', [1000]), tensor_input('d', [1000])), {'x': x, 'd': dy})
    exact(got, want)


@pytest.mark.parametrize('cols', [257, 256])   # one element per thread / four per thread
def test_stochastic_ops_bit_exact(cols):
    x = _rand([64, cols], 28)
    got, want = run_both(lambda: O.dropout(tensor_input('x', [64, cols]), 0.1), {'x': x})
    exact(got, want)
    zeros = np.mean(got == 0)
    assert 0.07 < zeros < 0.13
    got, want = run_both(lambda: O.randn([300, 7]), {})
    exact(got, want)
    got, want = run_both(lambda: O.categorical(tensor_input('x', [40, 65])), {'x': _rand([40, 65], 29)})
    exact(got, want)

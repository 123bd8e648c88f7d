"""Independent pins for the oracle's op kinds that the configs' torch checks do not reach.

Each test evaluates one op kind on the CPU oracle and compares it with a formulation that
shares no code with it: numpy / math in f64 rounded to f32, numpy slicing, the textbook
definition of the op (the evaluator's own definitions are test/_eval.ts:133-236, 316-459,
536-607), or a statistical property of the distribution the op samples. Each check is
chosen so that a plausible slip in the restatement (a transposed triangle, "last max
wins", a dropped sign of zero, the wrong hash input, a swapped Box-Muller pair) fails it.
"""
import math

import numpy as np
import pytest

import pyoracle
from _helpers import wire
from tensorgrad_amd import ir as IR
from tensorgrad_amd import ops as O
from tensorgrad_amd.trace import tensor_input, trace_fn


def _dt(a):
    return 'i32' if a.dtype == np.int32 else 'f32'


def ev(build, runs=1, **arrays):
    """Trace build(**tensor inputs) and evaluate it on the oracle; returns the output of
    each of `runs` consecutive runs (the worker's seed counter gives run k seed k)."""
    def body():
        return build(**{k: tensor_input(k, list(v.shape), _dt(v)) for k, v in arrays.items()})
    g = trace_fn(body)
    o = pyoracle.OracleRuntime(wire(g))
    outs = []
    for _ in range(runs):
        o.run(arrays)
        outs.append(o.output().copy())
    return outs[0] if runs == 1 else outs


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def _ulps(got, want):
    """Distance in units in the last place between two f32 arrays of finite values."""
    def key(a):
        i = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(key(got) - key(want))


RNG = np.random.default_rng(20261202)


# ---- argmax_last (_eval.ts:221-236) ---------------------------------------------------

def test_argmax_first_max_wins_on_tie_heavy_rows():
    a = RNG.integers(-3, 4, size=(257, 19)).astype(np.float32)   # many ties per row
    got = ev(lambda a: O.argmax(a, -1), a=a)
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, np.argmax(a, axis=-1))
    # an explicit check of the tie rule: every row [1, 5, 5, 5]
    t = np.tile(np.array([1, 5, 5, 5], np.float32), (4, 1))
    np.testing.assert_array_equal(ev(lambda a: O.argmax(a, -1), a=t), [1, 1, 1, 1])


def test_argmax_nan_rule():
    """x > best is false for NaN: a NaN at index 0 wins the row, NaN elsewhere never does."""
    a = np.array([[np.nan, 1, 2], [0, np.nan, -1], [-np.inf, np.nan, -np.inf], [3, 2, np.nan]], np.float32)
    np.testing.assert_array_equal(ev(lambda a: O.argmax(a, -1), a=a), [0, 0, 0, 0])


# ---- min / max (_eval.ts:133-153: Math.min / Math.max) ----------------------------------

def _js_minmax(a, b, is_min):
    """ECMAScript Math.min / Math.max: NaN if either operand is NaN; -0 is smaller than +0."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    out = np.where(a < b, a, b) if is_min else np.where(a > b, a, b)
    zeros = (a == 0) & (b == 0)
    neg = np.signbit(a) | np.signbit(b) if is_min else np.signbit(a) & np.signbit(b)
    out = np.where(zeros, np.where(neg, -0.0, 0.0), out)
    return np.where(np.isnan(a) | np.isnan(b), np.nan, out).astype(np.float32)


@pytest.mark.parametrize('kind', ['min', 'max'])
def test_min_max_js_semantics_with_broadcast(kind):
    special = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1.5, -1.5], np.float32)
    a = np.concatenate([RNG.standard_normal(41).astype(np.float32), special]).reshape(48, 1)
    a = np.tile(a, (1, 7))                                   # [48, 7]
    b = special.reshape(1, 7)                                # broadcast over rows
    fn = O.minimum if kind == 'min' else O.maximum
    got = ev(lambda a, b: fn(a, b), a=a, b=b)
    want = _js_minmax(a, np.broadcast_to(b, a.shape), kind == 'min')
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(_bits(got)[ok], _bits(want)[ok])   # sign of zero included


# ---- less / greater / where (_eval.ts:328-356) ------------------------------------------

@pytest.mark.parametrize('kind', ['less', 'greater'])
def test_comparisons_against_numpy(kind):
    a = RNG.integers(-2, 3, size=(6, 5, 4)).astype(np.float32)
    a[0, 0, :] = [np.nan, 0.0, -0.0, np.inf]
    b = RNG.integers(-2, 3, size=(5, 1)).astype(np.float32)
    b[0, 0] = 0.0
    fn = O.less if kind == 'less' else O.greater
    got = ev(lambda a, b: fn(a, b), a=a, b=b)
    want = (a < b) if kind == 'less' else (a > b)
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, want.astype(np.int32))


def test_where_selects_with_broadcast_condition():
    a = RNG.standard_normal((4, 3, 5)).astype(np.float32)
    b = RNG.standard_normal((1, 5)).astype(np.float32)
    c = RNG.standard_normal((3, 1)).astype(np.float32)
    got = ev(lambda a, b, c: O.where(O.greater(c, O.const_scalar(0.0)), a, b), a=a, b=b, c=c)
    np.testing.assert_array_equal(_bits(got), _bits(np.where(c > 0, a, b)))


# ---- where_causal (_eval.ts:406-420) ----------------------------------------------------

def test_where_causal_is_the_lower_triangle():
    a = RNG.standard_normal((2, 3, 6, 6)).astype(np.float32)
    got = ev(lambda a: O.where_causal(a, -1e9), a=a)
    keep = np.tril(np.ones((6, 6), bool))          # j <= i kept, strictly upper filled
    want = np.where(keep, a, np.float32(-1e9))
    np.testing.assert_array_equal(_bits(got), _bits(want))
    assert got[0, 0, 0, 1] == np.float32(-1e9) and got[0, 0, 1, 0] == a[0, 0, 1, 0]


def test_softmax_causal_masks_the_upper_triangle_and_rows_sum_to_one():
    a = RNG.standard_normal((3, 7, 7)).astype(np.float32)
    got = ev(lambda a: O.softmax_causal(a), a=a).astype(np.float64)
    assert np.all(got[:, ~np.tril(np.ones((7, 7), bool))] == 0)
    np.testing.assert_allclose(got.sum(-1), 1.0, rtol=0, atol=4e-7)
    e = np.where(np.tril(np.ones((7, 7), bool)), np.exp(a.astype(np.float64) - a.max()), 0)
    np.testing.assert_allclose(got, e / e.sum(-1, keepdims=True), rtol=2e-7, atol=1e-9)


# ---- slice_range / scatter_axis / concat (_eval.ts:423-480) -----------------------------

@pytest.mark.parametrize('axis', [0, 1, 2])
def test_slice_range_is_numpy_slicing(axis):
    a = RNG.standard_normal((5, 6, 7)).astype(np.float32)
    start, length = 1, 3
    got = ev(lambda a: O.narrow(a, axis, start, length), a=a)
    np.testing.assert_array_equal(got, np.take(a, np.arange(start, start + length), axis=axis))


@pytest.mark.parametrize('axis', [0, 1, 2])
def test_scatter_axis_inverts_slicing(axis):
    """scatter(slice(x)) puts the slice back and zeros the rest; the three pieces of a
    partition add up to x exactly."""
    x = RNG.standard_normal((4, 5, 6)).astype(np.float32)
    n = x.shape[axis]
    cuts = [(0, 2), (2, n - 1), (n - 1, n)]
    total = np.zeros_like(x)
    for s, e in cuts:
        piece = np.take(x, np.arange(s, e), axis=axis)
        got = ev(lambda p: O.scatter_axis(p, list(x.shape), axis, s, e), p=piece)
        want = np.zeros_like(x)
        idx = [slice(None)] * 3
        idx[axis] = slice(s, e)
        want[tuple(idx)] = piece
        np.testing.assert_array_equal(_bits(got), _bits(want))
        total += got
    np.testing.assert_array_equal(total, x)


def test_concat_is_numpy_concatenate():
    parts = [RNG.standard_normal((3, k, 2)).astype(np.float32) for k in (1, 4, 2)]
    got = ev(lambda a, b, c: O.concat([a, b, c], 1), a=parts[0], b=parts[1], c=parts[2])
    np.testing.assert_array_equal(got, np.concatenate(parts, axis=1))
    ints = [RNG.integers(-9, 9, (2, 3)).astype(np.int32) for _ in range(2)]
    np.testing.assert_array_equal(ev(lambda a, b: O.concat([a, b], 0), a=ints[0], b=ints[1]),
                                  np.concatenate(ints, 0))


# ---- unary ops (_eval.ts:166-203) -------------------------------------------------------

def _unary_input(positive=False):
    x = np.concatenate([RNG.standard_normal(2000) * 4, RNG.standard_normal(500) * 1e-3,
                        np.array([0.5, 1.0, 2.0, 1e-30, 3e4])]).astype(np.float32)
    return np.abs(x) + np.float32(1e-6) if positive else x


UNARY = {
    # kind: (op, input domain, f64 definition, ulp bound)
    'sigmoid': (O.sigmoid, False, lambda x: 1.0 / (1.0 + np.exp(-x)), 1),
    'rsqrt': (O.rsqrt, True, lambda x: 1.0 / np.sqrt(x), 1),
    'sqrt': (O.sqrt, True, np.sqrt, 0),
    'log': (O.log, True, np.log, 1),
    'exp': (O.exp, False, np.exp, 1),
    'tanh': (O.tanh, False, np.tanh, 1),
    'sin': (O.sin, False, np.sin, 1),
    'cos': (O.cos, False, np.cos, 1),
    'abs': (O.abs_, False, np.abs, 0),
    'neg': (O.neg, False, np.negative, 0),
    'relu': (O.relu, False, lambda x: np.maximum(x, 0.0), 0),
}


@pytest.mark.parametrize('kind', sorted(UNARY))
def test_unary_against_f64_definition(kind):
    fn, positive, ref, bound = UNARY[kind]
    x = _unary_input(positive)
    got = ev(lambda a: fn(a), a=x)
    with np.errstate(over='ignore'):
        want = ref(x.astype(np.float64)).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    assert _ulps(got[fin], want[fin]).max() <= bound, kind


def test_neg_and_abs_signs_of_zero():
    x = np.array([0.0, -0.0, np.inf, -np.inf], np.float32)
    np.testing.assert_array_equal(_bits(ev(lambda a: O.neg(a), a=x)), _bits(-x))
    np.testing.assert_array_equal(_bits(ev(lambda a: O.abs_(a), a=x)), _bits(np.abs(x)))


def test_erf_is_abramowitz_stegun_within_its_error_bound():
    """A&S 7.1.26 has |error| <= 1.5e-7 against the true erf; the f32 store adds half an
    ulp. A wrong constant or a dropped sign(x) breaks the bound."""
    x = np.concatenate([np.linspace(-4, 4, 4001), RNG.standard_normal(1000)]).astype(np.float32)
    got = ev(lambda a: O.erf(a), a=x).astype(np.float64)
    want = np.array([math.erf(float(v)) for v in x])
    assert np.max(np.abs(got - want)) <= 1.5e-7 + 6e-8
    assert np.all(np.sign(got[x != 0]) == np.sign(x[x != 0]))


# ---- randn / categorical_last (_eval.ts:536-607) ----------------------------------------

def _pcg_wrap(h):
    """One PCG output step on uint32 arrays with wrapping (Math.imul) products."""
    h = h.astype(np.uint64)
    m = np.uint64(0xFFFFFFFF)
    h = (h * np.uint64(747796405) + np.uint64(2891336453)) & m
    h = ((h ^ (h >> ((h >> np.uint64(28)) + np.uint64(4)))) * np.uint64(277803737)) & m
    return (h ^ (h >> np.uint64(22))) & m


def _pcg_f64(h):
    """The same step with the products done as correctly rounded f64 (JS `*` on numbers)
    and ToUint32 of the result."""
    h = h.astype(np.uint64)
    t = np.fmod(h.astype(np.float64) * 747796405.0 + 2891336453.0, 2.0 ** 32).astype(np.uint64)
    x = (t ^ (t >> ((t >> np.uint64(28)) + np.uint64(4)))) & np.uint64(0xFFFFFFFF)
    t = np.fmod(x.astype(np.float64) * 277803737.0, 2.0 ** 32).astype(np.uint64)
    return (t ^ (t >> np.uint64(22))) & np.uint64(0xFFFFFFFF)


def _stoch_op(g, kind):
    return next(op for op in g.ops if op['kind'] == kind)


def test_randn_is_box_muller_of_two_chained_hashes():
    shape = (64, 33)
    g = trace_fn(lambda: O.randn(list(shape)))
    salt = _stoch_op(g, 'randn')['salt']
    o = pyoracle.OracleRuntime(wire(g))
    for seed in (1, 2, 3):
        o.run({})
        got = o.output()
        i = np.arange(np.prod(shape), dtype=np.uint64)
        sc = np.uint64((salt * 0x9E3779B1) & 0xFFFFFFFF)
        h1 = _pcg_wrap(np.uint64(seed) ^ sc ^ i)
        h2 = _pcg_wrap(h1)
        u1 = np.maximum(1e-10, h1.astype(np.float64) / 2 ** 32)
        u2 = h2.astype(np.float64) / 2 ** 32
        want = (np.sqrt(-2 * np.log(u1)) * np.cos(2 * np.pi * u2)).astype(np.float32).reshape(shape)
        assert _ulps(got, want).max() <= 1, seed


def test_randn_is_standard_normal():
    """Mean, variance and a Kolmogorov-Smirnov distance over 2^17 draws of one run."""
    n = 1 << 17
    z = np.sort(ev(lambda: O.randn([n])).astype(np.float64))
    assert abs(z.mean()) < 5 / math.sqrt(n)
    assert abs(z.var() - 1) < 6 * math.sqrt(2 / n)
    cdf = 0.5 * (1 + np.array([math.erf(v / math.sqrt(2)) for v in z]))
    ks = max(np.max(np.arange(1, n + 1) / n - cdf), np.max(cdf - np.arange(n) / n))
    assert ks < 1.95 / math.sqrt(n)     # 0.1% critical value


def test_categorical_is_gumbel_max_of_the_f64_hash():
    logits = RNG.standard_normal((300, 9)).astype(np.float32)
    g = trace_fn(lambda: O.categorical(tensor_input('a', [300, 9])))
    salt = _stoch_op(g, 'categorical_last')['salt']
    o = pyoracle.OracleRuntime(wire(g))
    for seed in (1, 2):
        o.run({'a': logits})
        got = o.output()
        i = np.arange(logits.size, dtype=np.uint64)
        sc = np.uint64((salt * 0x9E3779B1) & 0xFFFFFFFF)
        u = np.maximum(1e-10, _pcg_f64(np.uint64(seed) ^ sc ^ i).astype(np.float64) / 2 ** 32)
        val = logits.astype(np.float64).reshape(-1) + -np.log(-np.log(u))
        np.testing.assert_array_equal(got, np.argmax(val.reshape(logits.shape), axis=-1))


def test_categorical_frequencies_follow_softmax():
    """Gumbel-max samples row j with probability softmax(logits)_j."""
    base = np.array([0.0, 1.0, 2.0, -1.0, 0.5], np.float32)
    rows = 40000
    draws = ev(lambda a: O.categorical(a), a=np.tile(base, (rows, 1)))
    p = np.exp(base.astype(np.float64))
    p /= p.sum()
    freq = np.bincount(draws, minlength=5) / rows
    sigma = np.sqrt(p * (1 - p) / rows)
    assert np.all(np.abs(freq - p) < 5 * sigma), (freq, p)


def test_dropout_keeps_with_probability_one_minus_p():
    n = 1 << 16
    x = np.ones(n, np.float32)
    y = ev(lambda a: O.dropout(a, 0.25), a=x)
    kept = y != 0
    assert np.all(y[kept] == np.float32(1 / 0.75))
    assert abs(kept.mean() - 0.75) < 5 * math.sqrt(0.75 * 0.25 / n)


# ---- leaves: const_fill / const_scalar / arange / one_hot -------------------------------

def test_leaves_and_one_hot():
    np.testing.assert_array_equal(ev(lambda: O.ones([2, 3])), np.ones((2, 3), np.float32))
    np.testing.assert_array_equal(ev(lambda: O.zeros([4], 'i32')), np.zeros(4, np.int32))
    np.testing.assert_array_equal(ev(lambda: O.arange(7)), np.arange(7, dtype=np.int32))
    idx = np.array([[0, 3, -1], [4, 2, 9]], np.int32)
    got = ev(lambda i: O.one_hot(i, 5), i=idx)
    want = np.zeros((2, 3, 5), np.float32)
    for r in range(2):
        for c in range(3):
            if 0 <= idx[r, c] < 5:
                want[r, c, idx[r, c]] = 1
    np.testing.assert_array_equal(got, want)
    assert np.all(got.sum(-1) == ((idx >= 0) & (idx < 5)))


# ---- coverage: every op kind has a pin somewhere ----------------------------------------

PINNED_ELSEWHERE = {
    # kind: where its independent check lives
    'param_input': 'every test', 'tensor_input': 'every test', 'state_input': 'test_oracle_vs_torch (Adam state)',
    'const_scalar': 'test_where_selects_with_broadcast_condition',
    'add': 'test_oracle_vs_torch', 'sub': 'test_oracle_vs_torch', 'mul': 'test_oracle_vs_torch',
    'div': 'test_oracle_vs_torch', 'matmul': 'test_oracle_vs_torch', 'matmul_batched': 'test_oracle_vs_torch',
    'mul_scalar': 'test_oracle_vs_torch', 'add_scalar': 'test_oracle_vs_torch', 'erf': 'test_erf_*',
    'mean_last': 'test_oracle_vs_torch', 'sum_last': 'test_oracle_vs_torch', 'reshape': 'test_oracle_vs_torch',
    'permute': 'test_oracle_vs_torch', 'log_softmax_last': 'test_oracle_vs_torch',
    'stop_gradient': 'test_reference_kats (exact 1/N)', 'broadcast_to': 'test_oracle_vs_torch',
    'sum_to_shape': 'test_oracle_vs_torch', 'dropout': 'test_prng + test_dropout_keeps_*',
    'relu_grad': 'test_oracle_vs_torch', 'adam_update_m': 'test_oracle_vs_torch (torch.optim)',
    'adam_update_v': 'test_oracle_vs_torch (torch.optim)', 'adam_update_p': 'test_oracle_vs_torch (torch.optim)',
    'conv2d': 'test_reference_kats (torch conv2d)', 'conv2d_input_grad': 'test_oracle_vs_torch (cnn)',
    'conv2d_weight_grad': 'test_oracle_vs_torch (cnn)', 'max_pool_2d': 'test_oracle_vs_torch (cnn)',
    'max_pool_2d_grad': 'test_oracle_vs_torch (cnn)',
}
PINNED_HERE = {
    'argmax_last', 'min', 'max', 'less', 'greater', 'where', 'where_causal', 'softmax_causal_last',
    'slice_range', 'scatter_axis', 'concat', 'sigmoid', 'rsqrt', 'sqrt', 'log', 'exp', 'tanh', 'sin', 'cos',
    'abs', 'neg', 'relu', 'randn', 'categorical_last', 'const_fill', 'arange', 'one_hot',
}


def test_every_op_kind_is_pinned():
    assert set(IR.OP_KINDS) == set(PINNED_ELSEWHERE) | PINNED_HERE

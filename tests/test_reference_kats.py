"""The reference's own numeric tests, restated against this build's front end + CPU oracle:
test/grad.ts (finite differences per derivative class, stopGradient, grouped conv,
normalizeGrads), test/ops.ts (leakyRelu KAT, dropout salts), test/smoke.ts (LR KATs),
test/dce.ts (DCE invariants)."""
import math

import numpy as np
import pytest

import pyoracle
from _helpers import fd_check, make_range, oracle_eval, random_buf, wire
from tensorgrad_amd import ops as O
from tensorgrad_amd import lr
from tensorgrad_amd.dce import eliminate_dead_code
from tensorgrad_amd.grad import append_grad, append_grad_normalize
from tensorgrad_amd.trace import param_input, tensor_input, trace_fn


# ---- FD vs autograd, one exemplar per derivative class (test/grad.ts:35-146) --------------

def test_fd_mul():
    fd_check('mul', [4, 8], lambda p: O.mean(O.mul(p, p)))


def test_fd_mean_keepdims():
    fd_check('mean', [4, 8], lambda p: O.mean(O.mean(p, -1, keep_dims=True)))


def test_fd_matmul():
    fd_check('matmul', [4, 8], lambda p: O.mean(O.matmul(p, tensor_input('x', [8, 16]))),
             extra={'x': make_range([8, 16])})


def test_fd_embedding():
    fd_check('embedding', [10, 4], lambda p: O.mean(O.embedding(p, tensor_input('idx', [3], 'i32'))),
             extra={'idx': np.array([2, 5, 7], np.int32)})


def test_fd_softmax_causal():
    fd_check('softmaxCausal', [4, 4], lambda p: O.mean(O.softmax_causal(p)))


def test_fd_dropout_seed42():
    fd_check('dropout', [4, 8], lambda p: O.mean(O.dropout(p, 0.1)), extra={'__prngSeed': np.array([42], np.int32)})


def test_fd_concat():
    fd_check('concat', [3, 4], lambda p: O.mean(O.concat([p, tensor_input('q', [3, 5])], 1)),
             extra={'q': make_range([3, 5])})


def test_fd_erf_and_gelu():
    fd_check('erf', [5], lambda p: O.mean(O.erf(p)))
    fd_check('gelu exact', [5], lambda p: O.mean(O.gelu(p)))
    fd_check('gelu tanh', [4], lambda p: O.mean(O.gelu(p, approximate='tanh')))


@pytest.mark.parametrize('case', ['input', 'weight_s2p1', 'groups_input', 'groups_weight', 'depthwise'])
def test_fd_conv2d(case):
    if case == 'input':
        fd_check('conv2d dx', [1, 2, 4, 4], lambda p: O.mean(O.conv2d(p, tensor_input('k', [3, 2, 2, 2]))),
                 extra={'k': make_range([3, 2, 2, 2])})
    elif case == 'weight_s2p1':
        fd_check('conv2d dw', [3, 2, 2, 2],
                 lambda p: O.mean(O.conv2d(tensor_input('x', [1, 2, 4, 4]), p, stride=2, padding=1)),
                 extra={'x': make_range([1, 2, 4, 4])})
    elif case == 'groups_input':
        fd_check('conv2d g2 dx', [1, 4, 4, 4],
                 lambda p: O.mean(O.conv2d(p, tensor_input('k', [6, 2, 2, 2]), groups=2)),
                 extra={'k': make_range([6, 2, 2, 2])})
    elif case == 'groups_weight':
        fd_check('conv2d g2 dw', [6, 2, 2, 2],
                 lambda p: O.mean(O.conv2d(tensor_input('x', [1, 4, 4, 4]), p, stride=2, padding=1, groups=2)),
                 extra={'x': make_range([1, 4, 4, 4])})
    else:
        fd_check('conv2d depthwise', [1, 3, 4, 4],
                 lambda p: O.mean(O.conv2d(p, tensor_input('k', [3, 1, 3, 3]), padding=1, groups=3)),
                 extra={'k': make_range([3, 1, 3, 3])})


def test_fd_narrow_split_where_causal_maxpool():
    fd_check('narrow', [4, 6], lambda p: O.mean(O.narrow(p, 1, 1, 3)))

    def split_loss(p):
        a, b = O.split(p, [2, 4], 1)
        return O.add(O.mean(O.mul(a, a)), O.mean(O.mul(b, b)))
    fd_check('split', [4, 6], split_loss)
    fd_check('whereCausal', [4, 4], lambda p: O.mean(O.where_causal(p, 0)))
    fd_check('maxPool2d', [1, 2, 4, 4], lambda p: O.mean(O.max_pool2d(p, 2)), init=make_range([1, 2, 4, 4]))


def test_fd_remaining_unary_and_binary_classes():
    # Derivative classes the configs use beyond the reference's exemplars.
    fd_check('tanh', [6], lambda p: O.mean(O.tanh(p)))
    fd_check('sqrt', [6], lambda p: O.mean(O.sqrt(O.add(p, 1.0))))
    fd_check('div', [6], lambda p: O.mean(O.div(O.add(p, 2.0), O.add(O.mul(p, p), 1.0))))
    fd_check('sin/cos', [6], lambda p: O.mean(O.mul(O.sin(p), O.cos(p))))
    fd_check('log_softmax', [3, 5], lambda p: O.mean(O.mul(O.log_softmax(p), tensor_input('t', [3, 5]))),
             extra={'t': make_range([3, 5])})
    fd_check('relu', [8], lambda p: O.mean(O.mul(O.relu(p), O.relu(p))))
    fd_check('broadcast add', [4], lambda p: O.mean(O.square(O.add(tensor_input('x', [3, 4]), p))),
             extra={'x': make_range([3, 4])})


# ---- stopGradient: autograd gives exactly 1/N on the undetached path (test/grad.ts:153-170) --

def test_stop_gradient_exact_one_over_n():
    N = 6
    init = (np.arange(N) * 0.1 - 0.3).astype(np.float32)
    g = trace_fn(lambda: O.mean(O.add(O.stop_gradient(p := param_input('w', [N])), p)))
    gr = append_grad(g)
    vals = oracle_eval(g, {'w': init}, {}, gr.param_grads)
    got = vals[gr.param_grads['w'].id]
    assert np.all(np.abs(got - 1 / N) <= 1e-5)


# ---- grouped conv == dense conv with a block-diagonal weight (test/grad.ts:176-206) ---------

def test_grouped_conv_equals_block_diagonal_dense():
    B, cIn, cOut, G, K, H, W = 2, 4, 6, 2, 3, 5, 5
    cInPG, cOutPG = cIn // G, cOut // G
    x = make_range([B, cIn, H, W])
    wg = make_range([cOut, cInPG, K, K]).reshape(cOut, cInPG, K, K)
    wd = np.zeros((cOut, cIn, K, K), np.float32)
    for co in range(cOut):
        g = co // cOutPG
        wd[co, g * cInPG:(g + 1) * cInPG] = wg[co]
    gg = trace_fn(lambda: O.conv2d(tensor_input('x', [B, cIn, H, W]), tensor_input('w', [cOut, cInPG, K, K]),
                                   padding=1, groups=G))
    gd = trace_fn(lambda: O.conv2d(tensor_input('x', [B, cIn, H, W]), tensor_input('w', [cOut, cIn, K, K]), padding=1))
    og = oracle_eval(gg, None, {'x': x, 'w': wg.reshape(-1)})[gg.outputs[0]]
    od = oracle_eval(gd, None, {'x': x, 'w': wd.reshape(-1)})[gd.outputs[0]]
    assert np.max(np.abs(og - od)) <= 1e-5


def test_grouped_conv_matches_torch():
    torch = pytest.importorskip('torch')
    B, cIn, cOut, G, K, H, W = 2, 4, 6, 2, 3, 5, 5
    x = make_range([B, cIn, H, W])
    w = make_range([cOut, cIn // G, K, K])
    g = trace_fn(lambda: O.conv2d(tensor_input('x', [B, cIn, H, W]), tensor_input('w', [cOut, cIn // G, K, K]),
                                  stride=2, padding=1, groups=G))
    got = oracle_eval(g, None, {'x': x, 'w': w})[g.outputs[0]]
    ref = torch.nn.functional.conv2d(torch.tensor(x, dtype=torch.float64).reshape(B, cIn, H, W),
                                     torch.tensor(w, dtype=torch.float64).reshape(cOut, cIn // G, K, K),
                                     stride=2, padding=1, groups=G).numpy()
    np.testing.assert_allclose(got, ref.astype(np.float32), rtol=1e-6, atol=1e-7)


# ---- normalizeGrads (test/grad.ts:211-250) -------------------------------------------------------

def test_normalize_grads_unit_norm_and_filter():
    N = 6
    init = make_range([N])
    holder = {}

    def body():
        p = param_input('w', [N])
        q = param_input('v', [N])
        return O.add(O.mean(O.mul(p, p)), O.mean(O.mul(q, q)))
    g = trace_fn(body)
    gr = append_grad(g)
    normed = append_grad_normalize(g, gr.param_grads, lambda n: n == 'w')
    assert normed['v'] is gr.param_grads['v']
    vals = oracle_eval(g, {'w': init, 'v': init})
    raw = vals[gr.param_grads['w'].id].astype(np.float64)
    got = vals[normed['w'].id].astype(np.float64)
    assert abs(np.linalg.norm(got) - 1) <= 1e-4
    np.testing.assert_allclose(got, raw / (np.linalg.norm(raw) + 1e-8), atol=1e-5)


def test_normalize_grads_zero_match_filter_throws():
    g = trace_fn(lambda: O.mean(O.mul(p := param_input('w', [4]), p)))
    gr = append_grad(g)
    with pytest.raises(ValueError):
        append_grad_normalize(g, gr.param_grads, lambda n: n == 'typo.W')


# ---- leakyRelu KAT, alpha >= 1 (test/ops.ts:49-58) ---------------------------------------------

def test_leaky_relu_alpha2_kat():
    g = trace_fn(lambda: O.leaky_relu(tensor_input('x', [4]), 2))
    out = oracle_eval(g, None, {'x': np.array([-1, -0.5, 0.5, 1], np.float32)})[g.outputs[0]]
    np.testing.assert_allclose(out, [-2, -1, 0.5, 1], atol=1e-6)


def test_dropout_p0_is_identity_and_salts_unique():
    g = trace_fn(lambda: O.dropout(tensor_input('x', [4]), 0))
    assert not any(op['kind'] == 'dropout' for op in g.ops)

    def body():
        x = tensor_input('x', [4])
        return O.add(O.dropout(x, 0.1), O.add(O.dropout(x, 0.2), O.dropout(x, 0.3)))
    g = trace_fn(body)
    seeds = [op for op in g.ops if op['kind'] == 'tensor_input' and op['name'] == '__prngSeed']
    salts = [op['salt'] for op in g.ops if op['kind'] == 'dropout']
    assert len(seeds) == 1 and len(set(salts)) == len(salts) == 3


# ---- LR schedule KATs (test/smoke.ts:411-470), on both the Python and the C++ oracle copy ----

@pytest.mark.parametrize('impl', ['python', 'oracle'])
def test_lr_kats(impl):
    resolve = lr.resolve_lr if impl == 'python' else pyoracle.resolve_lr
    s = lr.staircase(1.0, 1, 0.7)
    for step, want in [(1, 1.0), (2, 0.7), (3, 0.49), (10, math.pow(0.7, 9))]:
        assert abs(resolve(s, step) - want) < 1e-7
    s = lr.staircase(0.1, 3, 0.5)
    for step, want in [(1, 0.1), (3, 0.1), (4, 0.05), (6, 0.05), (7, 0.025)]:
        assert abs(resolve(s, step) - want) < 1e-9
    s = lr.multi_step(1.0, [3, 7], 0.1)
    for step, want in [(1, 1.0), (2, 1.0), (3, 0.1), (4, 0.1), (6, 0.1), (7, 0.01), (10, 0.01)]:
        assert abs(resolve(s, step) - want) < 1e-9


def test_lr_closed_forms_and_rebase():
    # linear: peak at intrinsic step 1 .. final at `steps`; cosine endpoints; warmup ramp.
    s = lr.linear(0.005, 0.0005, 1500)
    assert lr.resolve_lr(s, 1500) == pytest.approx(0.0005) and lr.resolve_lr(s, 10 ** 6) == pytest.approx(0.0005)
    c = lr.cosine_annealing(1.0, 0.0, 10)
    assert lr.resolve_lr(c, 10) == pytest.approx(0.0, abs=1e-12) and lr.resolve_lr(c, 5) == pytest.approx(0.5)
    w = lr.warmup(1.0, 4, 0.5)
    assert [lr.resolve_lr(w, t) for t in (1, 2, 4, 5, 9)] == [0.25, 0.5, 1.0, 0.5, 0.5]
    r = lr.rebase_lr(s, 11)
    assert r['startStep'] == 10 and lr.resolve_lr(r, 11) == lr.resolve_lr(s, 1)
    assert lr.rebase_lr(0.1, 5) == 0.1
    for sched in (s, c, w, r, lr.multi_step(1.0, [2], 0.5)):
        for t in (1, 2, 3, 7, 50):
            assert pyoracle.resolve_lr(sched, t) == lr.resolve_lr(sched, t)


# ---- DCE invariants (test/dce.ts:33-120) ----------------------------------------------------------

def _frozen_conv():
    return trace_fn(lambda: O.mean(O.conv2d(param_input('img', [1, 2, 4, 4]), tensor_input('k', [3, 2, 2, 2]))))


def test_dce_frozen_conv_weight_grad_pruned_values_bit_identical():
    inputs = {'k': make_range([3, 2, 2, 2])}
    params = {'img': make_range([1, 2, 4, 4])}
    g_ref = _frozen_conv()
    gr_ref = append_grad(g_ref)
    ref = oracle_eval(g_ref, params, inputs, gr_ref.param_grads)
    g = _frozen_conv()
    gr = append_grad(g)
    assert any(op['kind'] == 'conv2d_weight_grad' for op in g.ops)
    id_map = eliminate_dead_code(g, [t.id for t in gr.param_grads.values()])
    assert not any(op['kind'] == 'conv2d_weight_grad' for op in g.ops)
    assert any(op['kind'] == 'conv2d_input_grad' for op in g.ops)
    assert len(g.ops) == len(g.tensors)
    for i, op in enumerate(g.ops):
        assert g.tensors[op['out']].source == i
    vals = oracle_eval(g, params, inputs)
    assert np.array_equal(vals[g.outputs[0]], ref[g_ref.outputs[0]])
    assert np.array_equal(vals[id_map[gr.param_grads['img'].id].id], ref[gr_ref.param_grads['img'].id])


def test_dce_captures_are_roots_and_named_leaves_survive():
    from tensorgrad_amd.trace import capture

    def body():
        p = param_input('w', [4])
        x = tensor_input('x', [4])
        capture('kept', O.mul(p, p))
        O.relu(O.sub(x, 1))
        return O.mean(O.mul(p, x))
    g = trace_fn(body)
    gr = append_grad(g)
    eliminate_dead_code(g, [t.id for t in gr.param_grads.values()])
    assert 'kept' in g.captures and g.captures['kept'] < len(g.tensors)
    assert not any(op['kind'] == 'relu' for op in g.ops)

    def body2():
        p = param_input('w', [4])
        tensor_input('unused', [4])
        return O.mean(p)
    g2 = trace_fn(body2)
    append_grad(g2)
    eliminate_dead_code(g2)
    assert any(op['kind'] == 'tensor_input' and op['name'] == 'unused' for op in g2.ops)

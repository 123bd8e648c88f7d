"""The C-ABI library on a machine without a GPU: it loads, exports every entry point
include/tg.h declares, and lowers every config's IR (including the host-side bounds
proof of every launch) without touching a device."""
import ctypes
import os
import re

import pytest

from tensorgrad_amd import backend, configs
from tensorgrad_amd.build_ir import build_forward_ir, build_training_ir

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'include', 'tg.h')


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(tg_[a-z_]+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(backend.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(lib, s), f'libtg.so does not export {s}'
    assert sorted(backend.EXPORTED) == syms


@pytest.mark.parametrize('key', list(configs.CONFIGS))
def test_plan_lowers_every_config(key):
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    p = backend.plan(ir.wire_json())
    kinds = [n['kind'] for n in p['nodes']]
    assert kinds.count('adam_multi') == 1 and kinds[-1] == 'adam_multi'
    gemm_flops = sum(n['flops'] for n in p['nodes'] if n['kind'] == 'gemm')
    assert gemm_flops > 0
    if key in ('char_mlp', 'transformer'):
        # embeddings become a gather forward and a segmented scatter-add backward; the
        # scatter, read only by Adam, runs inside the deferred column-sum launch
        assert 'gather' in kinds
        merged = [n for n in p['nodes'] if n['kind'] == 'reduce' and '+ scatter' in n['shape']]
        assert kinds.count('scatter') + len(merged) == 1, kinds
        assert sum(1 for n in p['nodes'] if n['kind'] == 'gemm' and n['shape'].endswith('x[27,24]')) == 0


def test_embedding_gradient_joins_the_column_sums(monkeypatch):
    """The transformer's embedding gradient (read only by Adam) is planned into the launch of
    the deferred column sums, with its operands among the node's reads and its output among
    the writes; TG_COLSUM_SCATTER=0 keeps it a launch of its own."""
    cfg = configs.CONFIGS['transformer']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    merged = [n for n in nodes if n['kind'] == 'reduce' and '+ scatter' in n['shape']]
    assert len(merged) == 1 and 'scatter' not in [n['kind'] for n in nodes]
    assert merged[0]['ops'].endswith(',scatter')
    monkeypatch.setenv('TG_COLSUM_SCATTER', '0')
    nodes = backend.plan(ir.wire_json())['nodes']
    assert [n['kind'] for n in nodes].count('scatter') == 1
    assert not any('+ scatter' in n['shape'] for n in nodes)


@pytest.mark.parametrize('key', ['mlp_sin', 'char_mlp', 'cnn', 'transformer'])
def test_loss_mean_joins_the_column_sums(monkeypatch, key):
    """The loss mean (a row group reducing the per-sample losses to the output scalar) runs
    as a one-column sum in the deferred column-sum launch: one launch fewer per step;
    TG_COLSUM_LOSS=0 keeps its own row-group launch."""
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    merged = [n for n in nodes if n['kind'] == 'reduce' and ' + loss [' in n['shape']]
    assert len(merged) == 1, [n['shape'] for n in nodes if n['kind'] == 'reduce']
    monkeypatch.setenv('TG_COLSUM_LOSS', '0')
    apart = backend.plan(ir.wire_json())['nodes']
    assert not any(' + loss [' in n['shape'] for n in apart)
    assert len(apart) == len(nodes) + 1


def test_bias_sums_join_the_column_sums(monkeypatch):
    """The CNN's convolution bias gradients (sums over images and positions of [B, C, H, W],
    read only by Adam) run as blocks of the deferred column-sum launch; TG_COLSUM_MID=0
    keeps them as reductions of their own."""
    cfg = configs.CONFIGS['cnn']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    tail = [n for n in nodes if n['kind'] == 'reduce']
    assert len(tail) == 1 and tail[0]['shape'].count('] sum') == 2, [n['shape'] for n in tail]
    monkeypatch.setenv('TG_COLSUM_MID', '0')
    apart = backend.plan(ir.wire_json())['nodes']
    assert sum(1 for n in apart if n['kind'] == 'reduce') == 3
    assert len(apart) == len(nodes) + 2


def test_plan_with_gemm_epilogues(monkeypatch):
    """TG_GEMM_EPI=1 (pointwise groups in GEMM epilogues) lowers every config, also where a
    backward group recomputes from a GEMM's product (that product keeps its own store)."""
    monkeypatch.setenv('TG_GEMM_EPI', '1')
    fused = 0
    for key in configs.CONFIGS:
        cfg = configs.CONFIGS[key]
        ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
        nodes = backend.plan(ir.wire_json())['nodes']
        fused += sum(1 for n in nodes if n.get('ops', '').startswith('gemm+'))
    assert fused > 0


def test_gelu_backward_recomputes_instead_of_reading():
    """The transformer's GELU backward group evaluates the pre-activation and exp terms
    again from the FC1 GEMM output (the erf term stays stored: its f64 evaluation costs
    more than reading it), so per layer the forward group reads 1 and writes 2 full
    [B, T, 4d] tensors and the backward group reads 3 and writes 1, instead of 1 + 4 and
    4 + 1."""
    cfg = configs.CONFIGS['transformer']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    full = 4 * 32 * 128 * 1024
    fwd = [n for n in nodes if n['kind'] == 'fused' and 'erf' in n.get('ops', '')]
    bwd = [n for n in nodes if n['kind'] == 'fused' and 'recomputed' in n['shape']]
    assert len(fwd) == 4 and len(bwd) == 4
    for n in fwd:
        assert full * 3 <= n['bytes'] < full * 3 + 65536, n
    for n in bwd:
        assert full * 4 <= n['bytes'] < full * 4 + 65536, n


def test_plan_forward_graph_and_small_variants():
    for key in configs.CONFIGS:
        cfg = configs.small_variant(key)
        ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
        backend.plan(ir.wire_json())
    cfg = configs.CONFIGS['mlp_sin']
    from tensorgrad_amd import ops as O
    fir = build_forward_ir(cfg.make_model(), lambda m, i: m.l3.fwd(O.relu(m.l2.fwd(O.relu(m.l1.fwd(i['x']))))),
                           {'x': [7, 1]})
    p = backend.plan(fir.wire_json())
    assert not any(n['kind'] == 'adam_multi' for n in p['nodes'])


@pytest.mark.parametrize('vocab,seq,d,layers', [(12, 8, 64, 3), (27, 16, 64, 2), (65, 128, 256, 4)])
def test_attention_fuses_at_the_reference_samples_shapes(vocab, seq, d, layers):
    """Every attention of a training step lowers to one fused forward and one fused
    backward node: the reference's addition transformer (samples/transformer/spec.ts:12-19:
    T = 8, 4 heads of 16) and Pokeformer (samples/pokeformer/spec.ts:20-25: T = 16, 4
    heads of 16) take the small-head kernels, C5 (T = 128, heads of 64) the matrix-core
    ones."""
    ir = build_training_ir(configs.Transformer(vocab=vocab, seq=seq, d=d, n_layers=layers, hidden=4 * d),
                           configs.transformer_loss,
                           {'tokens': {'shape': [4, seq], 'dtype': 'i32'}, 'targets': {'shape': [4, seq], 'dtype': 'i32'}},
                           {'kind': 'adamw', 'lr': 1e-3, 'weightDecay': 0.01})
    nodes = backend.plan(ir.wire_json())['nodes']
    fwd = [n for n in nodes if n['kind'] == 'attention' and not n['shape'].endswith('backward')]
    bwd = [n for n in nodes if n['kind'] == 'attention' and n['shape'].endswith('backward')]
    assert len(fwd) == layers and len(bwd) == layers, [n['shape'] for n in nodes if n['kind'] == 'attention']


def test_malformed_ir_is_rejected_with_a_message():
    with pytest.raises(backend.BackendError) as e:
        backend.plan('{"graph": ')
    assert e.value.status == backend.TG_INVALID_ARGUMENT
    bad = '{"graph":{"ops":[{"kind":"nonsense","out":0,"a":0}],"tensors":[{"id":0,"shape":[1],"dtype":"f32"}],' \
          '"outputs":[0],"captures":{}},"paramGrads":{},"writebacks":[],"optimizer":null}'
    with pytest.raises(backend.BackendError):
        backend.plan(bad)


def test_device_count_is_callable():
    assert backend.device_count() >= 0


def test_parity_helpers_reject_non_finite_and_bound_the_exclusion():
    """The comparison helpers of the GPU parity tests fail on NaN / infinity instead of
    letting a comparison with NaN read as 'within tolerance', and the sign-ambiguous
    exclusion never covers a difference larger than two opposite updates per step."""
    import numpy as np
    import pytest
    from _helpers import rel_err, sign_ambiguous
    assert rel_err(1.0, 1.0) == 0.0
    assert abs(rel_err([1.0, 2.0], [1.0, 2.0 + 1e-6]) - 1e-6 / np.sqrt(5)) < 1e-12
    for bad in (float('nan'), float('inf')):
        with pytest.raises(AssertionError, match='non-finite'):
            rel_err(bad, 1.0)
        with pytest.raises(AssertionError, match='non-finite'):
            rel_err([0.5, bad], [0.5, 0.5])
        with pytest.raises(AssertionError, match='non-finite'):
            rel_err(1.0, bad)
    lr, steps = 1e-3, 3
    d = np.array([1e-7, lr / 4, 2 * lr, 2.5 * lr * steps, 2.5 * lr * steps * 1.01, 1.0])
    assert sign_ambiguous(d, lr, steps).tolist() == [False, True, True, True, False, False]
    assert sign_ambiguous(-d, lr, steps).tolist() == [False, True, True, True, False, False]
    # with the elements' own update sizes the floor is half an update, within [lr/16, lr/4];
    # the ceiling does not move
    upd = np.full(d.shape, lr / 5)
    assert sign_ambiguous(np.full(6, lr / 10), lr, steps, upd).all()
    assert not sign_ambiguous(np.full(6, lr / 11), lr, steps, upd).any()
    assert not sign_ambiguous(np.full(6, lr / 17), lr, steps, np.zeros(6)).any()
    assert sign_ambiguous(np.full(6, lr / 16), lr, steps, np.zeros(6)).all()
    assert sign_ambiguous(d, lr, steps, np.full(6, 4 * lr)).tolist() == [False, True, True, True, False, False]


def test_full_fixtures_carry_the_oracles_update_sizes():
    """The full-size fixtures hold, for every stored parameter element, the oracle's own
    Adam update size at step 100 (the sign-ambiguity floor of the 100-step test comes from
    the oracle, not from the runtime under test), and the twin configs their arithmetic
    twins."""
    import numpy as np
    root = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')
    for key in ('char_mlp', 'cnn', 'nerf', 'transformer'):
        g = np.load(os.path.join(root, f'full_{key}.npz'), allow_pickle=False)
        names = [f[4:] for f in g.files if f.startswith('idx:')]
        assert names
        for n in names:
            u = g[f'upd:{n}']
            assert u.shape == g[f'idx:{n}'].shape and np.all(np.isfinite(u)) and np.all(u >= 0), (key, n)
        if key in ('cnn', 'nerf'):
            kinds = [str(k) for k in g['twin_kinds']]
            assert 'f32' in kinds and 'sum64' in kinds and kinds.count('ulp') >= 2, (key, kinds)


def test_several_streams_are_rejected(monkeypatch):
    """TG_STREAMS other than 1 is an error at runtime creation (the several-stream
    schedule is removed), checked through the host-only lowering."""
    cfg = configs.CONFIGS['mlp_sin']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    monkeypatch.setenv('TG_STREAMS', '1')
    backend.plan(ir.wire_json())
    monkeypatch.setenv('TG_STREAMS', '2')
    with pytest.raises(backend.BackendError, match='TG_STREAMS'):
        backend.plan(ir.wire_json())


def test_relu_grad_reads_the_relu_output():
    """An add + relu layer whose backward takes relu_grad of the pre-activation stores only
    the relu output: the gradient reads that instead (relu(x) > 0 exactly when x > 0)."""
    cfg = configs.CONFIGS['nerf']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    relu_groups = [n for n in nodes if n.get('ops') in ('add,relu', 'gemm+add,relu', 'gemm_cat+add,relu')]
    assert len(relu_groups) == 8, [n.get('ops') for n in nodes]
    M, N = 65536, 256
    for n in relu_groups:
        if n['kind'] == 'gemm':   # a GEMM epilogue: operands in, the group's outputs out
            K = n['flops'] / (2 * M * N)
            out_bytes = n['bytes'] - 4 * (M * K + K * N + N)
        else:                     # reads the product (bias aside)
            out_bytes = n['bytes'] - 4 * (M * N + N)
        assert out_bytes < 1.05 * 4 * M * N, n   # one [65536, 256] tensor written


def test_skip_concatenation_gradients_lower_without_copies():
    """C4's skip connection (samples/nerf: the hidden state concatenated with the encoding,
    [65536, 256 + 63]): the input gradient's product computes only the 256 columns its
    slice keeps and takes the ReLU gradient in its epilogue (no [65536, 319] product, no
    slice copy, no separate relu_grad launch), and the weight gradient runs one GEMM per
    concatenation source instead of one over the concatenation's unaligned rows."""
    cfg = configs.CONFIGS['nerf']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    shapes = [(n['kind'], n['shape']) for n in nodes]
    assert ('copy', '[65536,256]') not in shapes
    assert not [s for k, s in shapes if k == 'gemm' and s.startswith('[65536,256]x[256,319]')]
    assert shapes.count(('gemm', '[319,65536]x[65536,256] by 2 sources')) == 1
    # the encoding's own concatenation has 3- and 30-wide sources: one GEMM over its 63 rows
    assert shapes.count(('gemm', '[63,65536]x[65536,256]')) == 1
    assert not [n for n in nodes if n.get('ops') == 'relu_grad']
    # seven hidden layers' and the head's ([65536, 4] x [4, 256], the small-K kernel)
    assert len([n for n in nodes if (n.get('ops') or '').startswith('gemm+relu_grad')]) == 8


def test_embedding_products_are_not_narrowed():
    """A slice of one_hot(idx) @ table keeps the whole-row gather (which reads table rows of
    the table's width) and slices after it; a plain product is narrowed to the kept columns."""
    import sys
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from _helpers import wire
    from tensorgrad_amd import ir as IR
    from tensorgrad_amd import ops as O
    from tensorgrad_amd.trace import tensor_input, trace_fn

    def emb():
        e = O.matmul(O.one_hot(tensor_input('i', [64], 'i32'), 10), tensor_input('t', [10, 32]))
        return O.narrow(e, -1, 0, 16)

    def prod():
        return O.narrow(O.matmul(tensor_input('a', [64, 10]), tensor_input('t', [10, 32])), -1, 0, 16)
    ne = backend.plan(IR.dumps(wire(trace_fn(emb))))['nodes']
    assert [(n['kind'], n['shape']) for n in ne] == [('gather', '[64,10]x[10,32]'), ('copy', '[64,16]')], ne
    npr = backend.plan(IR.dumps(wire(trace_fn(prod))))['nodes']
    assert [n['shape'] for n in npr] == ['[64,10]x[10,32] first 16 columns'], npr


def test_bias_sums_come_from_gemm_epilogues(monkeypatch):
    """C4's hidden-layer bias gradients are column sums of the ReLU-gradient outputs of
    GEMM epilogues: those epilogues write f64 column partials (one row per tile row slot of
    wavefronts, or per row block of the small-K kernel) and the deferred column-sum launch
    adds the partials instead of reading the [65536, 256] gradients back. TG_COLSUM_EPI=0
    restores the reads."""
    cfg = configs.CONFIGS['nerf']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    epi = [n for n in nodes if (n.get('ops') or '').endswith(',colsum')]
    assert len(epi) == 8, [n.get('ops') for n in nodes]   # seven on the tiles, the head's small-K product
    red = [n for n in nodes if n['kind'] == 'reduce' and 'sum_partials' in (n.get('ops') or '')]
    assert len(red) == 1 and red[0]['ops'].split(',').count('sum_partials') == 8
    assert red[0]['bytes'] < 30e6   # the head's [65536, 4] read whole, f64 partials for the rest
    monkeypatch.setenv('TG_COLSUM_EPI', '0')
    plain = backend.plan(ir.wire_json())['nodes']
    assert not [n for n in plain if 'colsum' in (n.get('ops') or '') or 'partials' in (n.get('ops') or '')]


@pytest.mark.parametrize('n', [1, 3, 10])
def test_forward_of_one_row_lowers_with_epilogues(n):
    """C1's forward at batch n (compileForward's shapes): every product is tiny and takes
    its bias (+ ReLU) group as an epilogue, the last one a single element at n = 1 (which
    merges to no dimension; the host-side binding accepts it)."""
    from tensorgrad_amd import ops as O
    cfg = configs.CONFIGS['mlp_sin']

    def predict(m, inp):
        return m.l3.fwd(O.relu(m.l2.fwd(O.relu(m.l1.fwd(inp['x'])))))
    ir = build_forward_ir(cfg.make_model(), predict, {'x': {'shape': [n, 1], 'dtype': 'f32'}})
    ops = [x.get('ops') for x in backend.plan(ir.wire_json())['nodes']]
    assert ops == ['gemm+add,relu', 'gemm+add,relu', 'gemm+add'], ops


def test_sums_of_products_lower_to_one_gemm(monkeypatch):
    """The transformer's Q/K/V input gradient dX = dQ Wq^T + dK Wk^T + dV Wv^T is one GEMM
    over three k segments, each with its own base pointer; the host-only lowering runs the
    bounds proof of every segment against the real memory plan. TG_GEMM_SUM=0 keeps the
    products and the adds apart."""
    cfg = configs.CONFIGS['transformer']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    sums = [n for n in nodes if n.get('ops') == 'gemm_sum']
    assert len(sums) == 4   # one per layer
    for n in sums:
        assert n['shape'] == '[32,128,256] sum of 3 products'
        assert n['flops'] == 3 * 2 * 4096 * 256 * 256
    monkeypatch.setenv('TG_GEMM_SUM', '0')
    plain = backend.plan(ir.wire_json())['nodes']
    assert not [n for n in plain if n.get('ops') == 'gemm_sum']
    assert sum(n['flops'] for n in plain if n['kind'] == 'gemm') == sum(n['flops'] for n in nodes if n['kind'] == 'gemm')


def test_loss_gradient_rows_join_the_loss_rows():
    """The cross-entropy gradient rows (softmax minus one-hot, scaled by a constant) read the
    log-softmax rows' exp; they start from a constant broadcast, so only the merge pass puts
    them in the forward row group: one launch for the loss rows and their gradient, the exp
    kept in registers. The MSE forward and backward element groups merge the same way, and
    the merged group runs in the product's epilogue (its scale constant lowered ahead)."""
    for key, n_rows in (('char_mlp', 1), ('transformer', 1)):
        cfg = configs.CONFIGS[key]
        ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
        nodes = backend.plan(ir.wire_json())['nodes']
        ce = [n for n in nodes if 'log_softmax_last' in n.get('ops', '')]
        assert len(ce) == n_rows and ce[0]['ops'].endswith('exp,sum_last,broadcast_to,mul,sub'), ce
    cfg = configs.CONFIGS['mlp_sin']
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, cfg.optimizer)
    nodes = backend.plan(ir.wire_json())['nodes']
    assert [n['ops'] for n in nodes if n['shape'].startswith('[256,1]')] == ['gemm+add,sub,mul,mul,mul,add']


def test_groups_merge_only_where_their_inputs_exist():
    """A later group joins an earlier one of the same shape only when everything it reads
    exists where the earlier group runs: reading the earlier group's result and constants
    merges; reading a product computed after the earlier group does not."""
    import sys
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from _helpers import wire
    from tensorgrad_amd import ir as IR
    from tensorgrad_amd import ops as O
    from tensorgrad_amd.trace import tensor_input, trace_fn

    def plan_groups(body):
        nodes = backend.plan(IR.dumps(wire(trace_fn(body))))['nodes']
        return [(n['kind'], n.get('ops', '')) for n in nodes]

    def merges():   # b = 2 h + 3 reads only h and constants
        h = O.relu(O.add_scalar(tensor_input('x', [64, 32]), 1.0))
        g = O.matmul(h, tensor_input('w', [32, 32]))
        return [g, O.add_scalar(O.mul_scalar(h, 2.0), 3.0)]

    def stays_apart():  # b = 2 g + h reads the product g, computed after h's group
        h = O.relu(O.add_scalar(tensor_input('x', [64, 32]), 1.0))
        g = O.matmul(h, tensor_input('w', [32, 32]))
        return O.add(O.mul_scalar(g, 2.0), h)

    fused = [k for k in plan_groups(merges) if k[0] in ('fused', 'elementwise')]
    assert len(fused) == 1 and fused[0][1] == 'add_scalar,relu,mul_scalar,add_scalar', fused
    kinds = plan_groups(stays_apart)
    # the later group runs after the product: as its epilogue (the default for cheap groups)
    assert kinds == [('fused', 'add_scalar,relu'), ('gemm', 'gemm+mul_scalar,add')], kinds


def _plan(key, opt):
    cfg = configs.CONFIGS[key]
    ir = build_training_ir(cfg.make_model(), cfg.loss, cfg.inputs, opt)
    return backend.plan(ir.wire_json())['nodes']


def test_clip_normalize_and_sgd_lower_to_the_fused_optimizer(monkeypatch):
    """clipGradNorm (grad.ts:110-130), normalizeGrads (grad.ts:148-172) and SGD's update
    chain (sgd.ts:155-170) run in the fused optimizer: one sum-of-squares launch per
    transform stage (its scalar chain evaluated in its last block) and one update launch,
    so the transformer keeps the launch count of plain AdamW and its deferred grouped
    weight-gradient GEMMs (the norm now reads the gradients inside the optimizer).
    TG_OPT_FUSED=0 lowers the same IR op by op."""
    cfg = configs.CONFIGS['transformer']
    plain = _plan('transformer', cfg.optimizer)
    clip = _plan('transformer', dict(cfg.optimizer, clipGradNorm=1.0))
    kinds = [n['kind'] for n in clip]
    assert len(clip) == len(plain) + 1 and len(clip) <= 77, len(clip)
    assert kinds.count('gemm') == 36 and kinds.count('grad_norm') == 1 and kinds[-1] == 'adam_multi'
    assert kinds[-2] == 'grad_norm'
    assert 'gemm_group' in [n.get('ops', '') for n in clip]
    norm = clip[-2]
    # the scalar chain of appendGradClip: chained adds, sqrt, + 1e-6, maxNorm / ., min(., 1)
    assert norm['ops'].count('add') >= 40 and 'sqrt' in norm['ops'] and 'div' in norm['ops'] and 'min' in norm['ops']
    assert norm['bytes'] == 4 * sum(n['bytes'] / 28 for n in clip if n['kind'] == 'adam_multi')
    both = _plan('transformer', dict(cfg.optimizer, clipGradNorm=1.0, normalizeGrads=True))
    assert [n['kind'] for n in both].count('grad_norm') == 2 and len(both) == len(plain) + 2
    for opt in ({'kind': 'sgd', 'lr': 0.01}, {'kind': 'sgd', 'lr': 0.01, 'momentum': 0.9},
                {'kind': 'sgd', 'lr': 0.01, 'momentum': 0.9, 'nesterov': True, 'weightDecay': 1e-3}):
        sgd = _plan('transformer', opt)
        k = [n['kind'] for n in sgd]
        assert len(sgd) <= 76 and k[-1] == 'sgd_multi' and k.count('sgd_multi') == 1 and 'adam_multi' not in k, k
        assert k.count('gemm') == 36
    monkeypatch.setenv('TG_OPT_FUSED', '0')
    apart = _plan('transformer', dict(cfg.optimizer, clipGradNorm=1.0))
    assert 'grad_norm' not in [n['kind'] for n in apart] and len(apart) > 150
    sgd = _plan('transformer', {'kind': 'sgd', 'lr': 0.01})
    assert 'sgd_multi' not in [n['kind'] for n in sgd]


@pytest.mark.parametrize('key', list(configs.CONFIGS))
def test_fused_optimizer_lowers_every_config(key):
    cfg = configs.CONFIGS[key]
    for opt in (dict(cfg.optimizer, clipGradNorm=0.5), dict(cfg.optimizer, normalizeGrads=True),
                {'kind': 'sgd', 'lr': 0.01, 'momentum': 0.9, 'clipGradNorm': 1.0}):
        nodes = _plan(key, opt)
        kinds = [n['kind'] for n in nodes]
        assert kinds[-1] in ('adam_multi', 'sgd_multi') and kinds.count('grad_norm') == 1, kinds

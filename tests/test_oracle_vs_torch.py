"""Pins the CPU oracle (and the front end's IR for each config) against a library routine:
PyTorch float64 autograd of the same five models, on the same params and inputs.
Loss and every parameter gradient must agree to f32-storage precision, and one
Adam / AdamW step must agree with torch.optim (eps rescaled per step so that torch's
bias-corrected form equals the reference's lrt form, src/adam.ts:134-143)."""
import math

import numpy as np
import pytest

torch = pytest.importorskip('torch')
F = torch.nn.functional

import pyoracle  # noqa: E402
from tensorgrad_amd import configs  # noqa: E402
from tensorgrad_amd.build_ir import build_training_ir  # noqa: E402


def _t(a):
    return torch.tensor(np.asarray(a, dtype=np.float64), dtype=torch.float64, requires_grad=True)


def _ln(x, g, b, eps=1e-5):
    m = x.mean(-1, keepdim=True)
    c = x - m
    v = (c * c).mean(-1, keepdim=True)
    return c / torch.sqrt(v + eps) * g + b


def torch_loss(key, P, batch, model):
    if key == 'mlp_sin':
        x, y = torch.tensor(batch['x'], dtype=torch.float64), torch.tensor(batch['y'], dtype=torch.float64)
        h = F.relu(x @ P['l1.W'].reshape(1, -1) + P['l1.b'])
        h = F.relu(h @ P['l2.W'].reshape(64, 64) + P['l2.b'])
        out = h @ P['l3.W'].reshape(64, 1) + P['l3.b']
        return ((out - y) ** 2).mean()
    if key == 'char_mlp':
        V, E, Hd = 27, model.emb_dim, model.l1.outDim
        tok = torch.tensor(batch['tokens'], dtype=torch.long)
        e = P['emb.W'].reshape(V, E)[tok].reshape(tok.shape[0], -1)
        h = torch.tanh(e @ P['l1.W'].reshape(-1, Hd) + P['l1.b'])
        logits = h @ P['l2.W'].reshape(Hd, V) + P['l2.b']
        return F.cross_entropy(logits, torch.tensor(batch['targets'], dtype=torch.long))
    if key == 'cnn':
        m = model
        x = torch.tensor(batch['x'], dtype=torch.float64)
        c1, c2 = m.conv1.outC, m.conv2.outC
        h = F.relu(F.conv2d(x, P['conv1.W'].reshape(c1, 1, 3, 3)) + P['conv1.b'].reshape(1, c1, 1, 1))
        h = F.relu(F.conv2d(h, P['conv2.W'].reshape(c2, c1, 3, 3)) + P['conv2.b'].reshape(1, c2, 1, 1))
        h = F.max_pool2d(h, 2).reshape(x.shape[0], -1)
        h = F.relu(h @ P['fc1.W'].reshape(h.shape[1], -1) + P['fc1.b'])
        logits = h @ P['fc2.W'].reshape(h.shape[1], 10) + P['fc2.b']
        return F.cross_entropy(logits, torch.tensor(batch['y'], dtype=torch.long))
    if key == 'nerf':
        x = torch.tensor(batch['x'], dtype=torch.float64)
        fr = torch.tensor(batch['freqs'], dtype=torch.float64)
        n = x.shape[0]
        s = x.reshape(n, 3, 1) * fr.reshape(1, 1, -1)
        pe = torch.cat([x, torch.sin(s).reshape(n, -1), torch.cos(s).reshape(n, -1)], 1)
        h = pe
        for i in range(len(model.layers)):
            if i == model.skip:
                h = torch.cat([h, pe], 1)
            h = F.relu(h @ P[f'layers.{i}.W'].reshape(h.shape[1], -1) + P[f'layers.{i}.b'])
        out = h @ P['head.W'].reshape(h.shape[1], 4) + P['head.b']
        return ((out - torch.tensor(batch['target'], dtype=torch.float64)) ** 2).mean()
    if key == 'transformer':
        m = model
        d = P['tok_emb'].shape[0] // 65
        T = m.seq
        tok = torch.tensor(batch['tokens'], dtype=torch.long)
        B = tok.shape[0]
        x = P['tok_emb'].reshape(65, d)[tok] + P['pos_emb'].reshape(T, d)
        H = m.n_heads
        dh = d // H
        for i in range(len(m.layers)):
            p = lambda n: P[f'layers.{i}.{n}']  # noqa: E731
            h = _ln(x, p('ln1.g'), p('ln1.b'))
            q = (h @ p('attn.q.W').reshape(d, d)).reshape(B, T, H, dh).transpose(1, 2)
            k = (h @ p('attn.k.W').reshape(d, d)).reshape(B, T, H, dh).transpose(1, 2)
            v = (h @ p('attn.v.W').reshape(d, d)).reshape(B, T, H, dh).transpose(1, 2)
            sc = (q @ k.transpose(-1, -2)) * (1 / math.sqrt(dh))
            mask = torch.ones(T, T, dtype=torch.bool).tril()
            att = torch.softmax(sc.masked_fill(~mask, float('-inf')), -1)
            o = (att @ v).transpose(1, 2).reshape(B, T, d) @ p('attn.o.W').reshape(d, d)
            x1 = x + o
            h2 = _ln(x1, p('ln2.g'), p('ln2.b'))
            u = h2 @ p('mlp.up.W').reshape(d, -1) + p('mlp.up.b')
            u = 0.5 * u * (1 + torch.erf(u / math.sqrt(2)))
            x = x1 + u @ p('mlp.down.W').reshape(-1, d) + p('mlp.down.b')
        logits = _ln(x, P['lnf.g'], P['lnf.b']) @ P['head.W'].reshape(d, 65) + P['head.b']
        return F.cross_entropy(logits.reshape(-1, 65), torch.tensor(batch['targets'], dtype=torch.long).reshape(-1))
    raise KeyError(key)


def _small(key):
    cfg = configs.small_variant(key)
    if key == 'transformer':
        # dropout off: torch has no equivalent of the reference's PCG mask
        cfg.make_model = lambda: configs.Transformer(seq=16, d=32, n_layers=2, hidden=64, p_drop=0.0)
    return cfg


@pytest.mark.parametrize('key', ['mlp_sin', 'char_mlp', 'cnn', 'nerf', 'transformer'])
def test_oracle_matches_torch_f64(key):
    cfg = _small(key)
    model = cfg.make_model()
    ir = build_training_ir(model, cfg.loss, cfg.inputs, cfg.optimizer)
    params = ir.initial_params(42)
    batch = configs.batches(cfg, 1)[0]
    o = pyoracle.OracleRuntime(ir.wire())
    o.upload_params(params)
    o.retain_all(True)
    loss = o.step(batch)
    grads = {n: o.tensor(t.id).reshape(-1) for n, t in ir.param_grads.items()}
    new_params = {n: o.get_home(n, params[n].size) for n in params}

    P = {n: _t(v) for n, v in params.items()}
    tl = torch_loss(key, P, batch, model)
    tl.backward()
    assert abs(loss - tl.item()) <= 2e-6 * max(1.0, abs(tl.item()))
    for n in params:
        tg = P[n].grad.numpy()
        err = np.linalg.norm(grads[n] - tg) / max(np.linalg.norm(tg), 1e-30)
        assert err <= 2e-5 or np.max(np.abs(grads[n] - tg)) <= 1e-9, f'{key} grad {n}: rel {err:.2e}'

    # One optimizer step, from the oracle's own gradients, through torch.optim.
    opt = cfg.optimizer
    b1, b2, eps = 0.9, 0.999, 1e-8
    tp = {n: torch.tensor(params[n].astype(np.float64)) for n in params}
    decay = ir.materialized.decay_flags
    for n in params:
        wd = opt.get('weightDecay', 0) if decay.get(n, True) else 0.0
        cls = torch.optim.AdamW if opt['kind'] == 'adamw' else torch.optim.Adam
        kw = dict(lr=opt['lr'], betas=(b1, b2), eps=eps / math.sqrt(1 - b2))
        if opt['kind'] == 'adamw':
            kw['weight_decay'] = wd
        t = tp[n].clone().requires_grad_(True)
        t.grad = torch.tensor(grads[n].astype(np.float64))
        cls([t], **kw).step()
        got = new_params[n].astype(np.float64)
        want = t.detach().numpy()
        assert np.max(np.abs(got - want)) <= 1e-6 * max(1.0, np.max(np.abs(want))) + 1e-9, f'{key} adam {n}'

"""The five benchmark configurations (C1-C5), written against this package's
reference-mirroring API the way the reference's samples are written
(samples/mlp-sin/spec.ts, samples/makemore/spec.ts, samples/mnist-cnn/spec.ts,
samples/nerf-tiny/spec.ts, samples/transformer/spec.ts).

Model decisions fixed here: C3 uses padding 0 (28->26->24->pool 12, fc 9216); C4 feeds
`[x, sin(2^k pi x), cos(2^k pi x)]`, k=0..9, with the frequencies as a `[10]` tensor
input, skip-concat of the encoding before layer 5 (319 inputs) and a raw 4-wide head; C5
is pre-LN with bias-free q/k/v/o, learned position embedding through `arange`, exact
GELU, an untied 256->65 head with bias, and dropout 0.1 after the attention
probabilities, after the output projection and after the MLP down-projection.

Synthetic data: uniform draws from `mulberry32(1000 + c)`; parameter init seed 42.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Dict

import numpy as np

from . import nn
from . import ops as O
from .module import Module, Mulberry32

INIT_SEED = 42


# ---- C1: MLP 1 -> 64 -> 64 -> 1 fitting sin(x) -------------------------------------------

class SinMLP(Module):
    def __init__(self, hidden=64):
        self.l1 = nn.Linear(1, hidden)
        self.l2 = nn.Linear(hidden, hidden)
        self.l3 = nn.Linear(hidden, 1)


def sin_mlp_loss(p: SinMLP, inp):
    out = p.l3.fwd(O.relu(p.l2.fwd(O.relu(p.l1.fwd(inp['x'])))))
    diff = O.sub(out, inp['y'])
    return O.mean(O.mul(diff, diff))


# ---- C2: char-level MLP language model ------------------------------------------------------

class CharMLP(Module):
    def __init__(self, vocab=27, ctx=8, emb=24, hidden=512):
        self.ctx = ctx
        self.emb_dim = emb
        self.emb = nn.Embedding(vocab, emb)
        self.l1 = nn.Linear(ctx * emb, hidden)
        self.l2 = nn.Linear(hidden, vocab)


def char_mlp_loss(p: CharMLP, inp):
    tokens = inp['tokens']
    e = p.emb.fwd(tokens)
    h = O.reshape(e, [tokens.shape[0], p.ctx * p.emb_dim])
    h = O.tanh(p.l1.fwd(h))
    return nn.cross_entropy(p.l2.fwd(h), inp['targets'])


# ---- C3: small CNN -----------------------------------------------------------------------

class CNN(Module):
    def __init__(self):
        self.conv1 = nn.Conv2d(1, 32, 3)
        self.conv2 = nn.Conv2d(32, 64, 3)
        self.fc1 = nn.Linear(64 * 12 * 12, 128)
        self.fc2 = nn.Linear(128, 10)


def cnn_loss(m: CNN, inp):
    x = inp['x']
    h = O.relu(m.conv1.fwd(x))
    h = O.relu(m.conv2.fwd(h))
    h = O.max_pool2d(h, 2)
    h = O.reshape(h, [x.shape[0], -1])
    h = O.relu(m.fc1.fwd(h))
    return nn.cross_entropy(m.fc2.fwd(h), inp['y'])


# ---- C4: NeRF-style coordinate MLP ---------------------------------------------------------

N_FREQS = 10


class NeRF(Module):
    def __init__(self, width=256, depth=8, skip=4, in_dim=3 + 3 * 2 * N_FREQS, out_dim=4):
        self.skip = skip
        self.layers = []
        for i in range(depth):
            fan_in = in_dim if i == 0 else (width + in_dim if i == skip else width)
            self.layers.append(nn.Linear(fan_in, width))
        self.head = nn.Linear(width, out_dim)


def nerf_pos_enc(x, freqs):
    n = x.shape[0]
    scaled = O.mul(O.reshape(x, [n, 3, 1]), O.reshape(freqs, [1, 1, N_FREQS]))
    sin_f = O.reshape(O.sin(scaled), [n, 3 * N_FREQS])
    cos_f = O.reshape(O.cos(scaled), [n, 3 * N_FREQS])
    return O.concat([x, sin_f, cos_f], 1)


def nerf_loss(m: NeRF, inp):
    pe = nerf_pos_enc(inp['x'], inp['freqs'])
    h = pe
    for i, layer in enumerate(m.layers):
        if i == m.skip:
            h = O.concat([h, pe], 1)
        h = O.relu(layer.fwd(h))
    out = m.head.fwd(h)
    return O.mean(O.square(O.sub(out, inp['target'])))


# ---- C5: decoder-only transformer ------------------------------------------------------------

class Attention(Module):
    def __init__(self, d):
        self.q = nn.Linear(d, d, bias=False)
        self.k = nn.Linear(d, d, bias=False)
        self.v = nn.Linear(d, d, bias=False)
        self.o = nn.Linear(d, d, bias=False)


class MLP(Module):
    def __init__(self, d, hidden):
        self.up = nn.Linear(d, hidden)
        self.down = nn.Linear(hidden, d)


class Block(Module):
    def __init__(self, d, hidden):
        self.ln1 = nn.LayerNorm(d)
        self.attn = Attention(d)
        self.ln2 = nn.LayerNorm(d)
        self.mlp = MLP(d, hidden)


class Transformer(Module):
    def __init__(self, vocab=65, seq=128, d=256, n_layers=4, n_heads=4, hidden=1024, p_drop=0.1):
        self.n_heads = n_heads
        self.seq = seq
        self.p_drop = p_drop
        self.tok_emb = self.param([vocab, d])
        self.pos_emb = self.param([seq, d])
        self.layers = [Block(d, hidden) for _ in range(n_layers)]
        self.lnf = nn.LayerNorm(d)
        self.head = nn.Linear(d, vocab)


def _attention(p: Attention, x, n_heads, p_drop):
    q = O.split_heads(p.q.fwd(x), n_heads)
    k = O.split_heads(p.k.fwd(x), n_heads)
    v = O.split_heads(p.v.fwd(x), n_heads)
    scale = 1 / math.sqrt(q.shape[-1])
    scores = O.mul(O.matmul(q, O.swap_axes(k, -1, -2)), scale)
    attn = O.dropout(O.softmax_causal(scores), p_drop)
    return O.dropout(p.o.fwd(O.merge_heads(O.matmul(attn, v))), p_drop)


def transformer_logits(p: Transformer, tokens):
    x = O.add(O.embedding(p.tok_emb, tokens), O.embedding(p.pos_emb, O.arange(p.seq)))
    for blk in p.layers:
        a = _attention(blk.attn, blk.ln1.fwd(x), p.n_heads, p.p_drop)
        x1 = O.add(x, a)
        m = O.dropout(blk.mlp.down.fwd(O.gelu(blk.mlp.up.fwd(blk.ln2.fwd(x1)))), p.p_drop)
        x = O.add(x1, m)
    return p.head.fwd(p.lnf.fwd(x))


def transformer_loss(p: Transformer, inp):
    return nn.cross_entropy(transformer_logits(p, inp['tokens']), inp['targets'])


# ---- registry -------------------------------------------------------------------------------------

@dataclass
class Config:
    key: str
    index: int               # c in mulberry32(1000 + c)
    title: str
    make_model: Callable[[], Module]
    loss: Callable
    inputs: Dict
    optimizer: dict
    samples_per_step: int
    sample_unit: str
    make_batch: Callable[[Mulberry32], Dict[str, np.ndarray]]


def _uniform(rng: Mulberry32, n: int, lo: float, hi: float) -> np.ndarray:
    return (lo + (hi - lo) * rng.take(n)).astype(np.float32)


def _ints(rng: Mulberry32, n: int, k: int) -> np.ndarray:
    return np.floor(rng.take(n) * k).astype(np.int32)


def _c1_batch(rng):
    x = _uniform(rng, 256, -math.pi, math.pi).reshape(256, 1)
    return {'x': x, 'y': np.sin(x.astype(np.float64)).astype(np.float32)}


def _c2_batch(rng):
    return {'tokens': _ints(rng, 1024 * 8, 27).reshape(1024, 8), 'targets': _ints(rng, 1024, 27)}


def _c3_batch(rng):
    return {'x': _uniform(rng, 128 * 28 * 28, 0.0, 1.0).reshape(128, 1, 28, 28), 'y': _ints(rng, 128, 10)}


NERF_FREQS = np.array([(2.0 ** k) * math.pi for k in range(N_FREQS)], dtype=np.float32)


def _c4_batch(rng, n=65536):
    return {'x': _uniform(rng, n * 3, -1.0, 1.0).reshape(n, 3), 'freqs': NERF_FREQS.copy(),
            'target': _uniform(rng, n * 4, 0.0, 1.0).reshape(n, 4)}


def _c5_batch(rng, b=32, t=128, v=65):
    return {'tokens': _ints(rng, b * t, v).reshape(b, t), 'targets': _ints(rng, b * t, v).reshape(b, t)}


CONFIGS: Dict[str, Config] = {
    'mlp_sin': Config('mlp_sin', 1, 'C1 MLP 1-64-64-1 sin(x), B=256, Adam 5e-3', SinMLP, sin_mlp_loss,
                      {'x': [256, 1], 'y': [256, 1]}, {'kind': 'adam', 'lr': 0.005}, 256, 'samples', _c1_batch),
    'char_mlp': Config('char_mlp', 2, 'C2 char-MLP LM, B=1024 ctx 8, AdamW 1e-3', CharMLP, char_mlp_loss,
                       {'tokens': {'shape': [1024, 8], 'dtype': 'i32'}, 'targets': {'shape': [1024], 'dtype': 'i32'}},
                       {'kind': 'adamw', 'lr': 1e-3, 'weightDecay': 0.01}, 1024, 'samples', _c2_batch),
    'cnn': Config('cnn', 3, 'C3 CNN, B=128 28x28, Adam 1e-3', CNN, cnn_loss,
                  {'x': [128, 1, 28, 28], 'y': {'shape': [128], 'dtype': 'i32'}},
                  {'kind': 'adam', 'lr': 1e-3}, 128, 'samples', _c3_batch),
    'nerf': Config('nerf', 4, 'C4 NeRF MLP, N=65536, Adam 5e-4', NeRF, nerf_loss,
                   {'x': [65536, 3], 'freqs': [N_FREQS], 'target': [65536, 4]},
                   {'kind': 'adam', 'lr': 5e-4}, 65536, 'samples', _c4_batch),
    'transformer': Config('transformer', 5, 'C5 transformer B=32 T=128 d=256 L=4 H=4, AdamW 3e-4', Transformer,
                          transformer_loss,
                          {'tokens': {'shape': [32, 128], 'dtype': 'i32'}, 'targets': {'shape': [32, 128], 'dtype': 'i32'}},
                          {'kind': 'adamw', 'lr': 3e-4, 'weightDecay': 0.01}, 4096, 'tokens', _c5_batch),
}


def batches(cfg: Config, n: int):
    """n synthetic batches from mulberry32(1000 + c), generated in order."""
    rng = Mulberry32(1000 + cfg.index)
    return [cfg.make_batch(rng) for _ in range(n)]


def small_variant(key: str):
    """Reduced-size variants of each config with the same topology, for CPU-oracle-bound
    parity tests (the oracle evaluates the full configs in minutes, not seconds)."""
    if key == 'mlp_sin':
        return CONFIGS['mlp_sin']
    if key == 'char_mlp':
        return Config('char_mlp_small', 2, 'C2 small', lambda: CharMLP(hidden=64), char_mlp_loss,
                      {'tokens': {'shape': [64, 8], 'dtype': 'i32'}, 'targets': {'shape': [64], 'dtype': 'i32'}},
                      {'kind': 'adamw', 'lr': 1e-3, 'weightDecay': 0.01}, 64, 'samples',
                      lambda rng: {'tokens': _ints(rng, 64 * 8, 27).reshape(64, 8), 'targets': _ints(rng, 64, 27)})
    if key == 'cnn':
        class SmallCNN(Module):
            def __init__(self):
                self.conv1 = nn.Conv2d(1, 4, 3)
                self.conv2 = nn.Conv2d(4, 8, 3)
                self.fc1 = nn.Linear(8 * 12 * 12, 16)
                self.fc2 = nn.Linear(16, 10)
        return Config('cnn_small', 3, 'C3 small', SmallCNN, cnn_loss,
                      {'x': [4, 1, 28, 28], 'y': {'shape': [4], 'dtype': 'i32'}},
                      {'kind': 'adam', 'lr': 1e-3}, 4, 'samples',
                      lambda rng: {'x': _uniform(rng, 4 * 784, 0.0, 1.0).reshape(4, 1, 28, 28), 'y': _ints(rng, 4, 10)})
    if key == 'nerf':
        return Config('nerf_small', 4, 'C4 small', lambda: NeRF(width=32), nerf_loss,
                      {'x': [256, 3], 'freqs': [N_FREQS], 'target': [256, 4]},
                      {'kind': 'adam', 'lr': 5e-4}, 256, 'samples', lambda rng: _c4_batch(rng, 256))
    if key == 'transformer':
        return Config('transformer_small', 5, 'C5 small', lambda: Transformer(seq=16, d=32, n_layers=2, hidden=64),
                      transformer_loss,
                      {'tokens': {'shape': [2, 16], 'dtype': 'i32'}, 'targets': {'shape': [2, 16], 'dtype': 'i32'}},
                      {'kind': 'adamw', 'lr': 3e-4, 'weightDecay': 0.01}, 32, 'tokens',
                      lambda rng: _c5_batch(rng, 2, 16, 65))
    raise KeyError(key)

"""Layers and losses (reference `src/nn.ts`): Linear with W `[in, out]` (nn.ts:109-126),
composed LayerNorm (nn.ts:142-164), RMSNorm, Embedding, Conv2d, nllLoss / crossEntropy
(nn.ts:234-262). Attribute assignment order fixes the parameter order, as in the
reference's class-field order."""
from __future__ import annotations

from typing import Optional

from . import ops as O
from .ir import Tensor
from .module import Module, init
from .shape import ShapeError


class Linear(Module):
    def __init__(self, in_dim: int, out_dim: int, bias: bool = True, init_spec: Optional[dict] = None,
                 decay: Optional[bool] = None):
        self.inDim = in_dim
        self.outDim = out_dim
        self.W = self.param([in_dim, out_dim], init=init_spec, decay=decay)
        self.b = self.param([out_dim], init=init.zeros()) if bias else None

    def fwd(self, x: Tensor) -> Tensor:
        out = O.matmul(x, self.W)
        return O.add(out, self.b) if self.b is not None else out


class LayerNorm(Module):
    def __init__(self, d: int, eps: float = 1e-5, bias: bool = True, decay: bool = False):
        self.d = d
        self.eps = eps
        self.g = self.param([d], init=init.ones(), decay=decay)
        self.b = self.param([d], init=init.zeros(), decay=decay) if bias else None

    def fwd(self, x: Tensor) -> Tensor:
        m = O.mean(x, -1, keep_dims=True)
        c = O.sub(x, m)
        v = O.mean(O.mul(c, c), -1, keep_dims=True)
        stdev = O.sqrt(O.add(v, self.eps))
        scaled = O.mul(O.div(c, stdev), self.g)
        return O.add(scaled, self.b) if self.b is not None else scaled


class RMSNorm(Module):
    def __init__(self, d: int, eps: float = 1e-6, decay: bool = False):
        self.d = d
        self.eps = eps
        self.g = self.param([d], init=init.ones(), decay=decay)

    def fwd(self, x: Tensor) -> Tensor:
        ms = O.mean(O.mul(x, x), -1, keep_dims=True)
        rstd = O.sqrt(O.add(ms, self.eps))
        return O.mul(O.div(x, rstd), self.g)


class Embedding(Module):
    def __init__(self, vocab: int, dim: int, init_spec: Optional[dict] = None, decay: Optional[bool] = None):
        self.vocab = vocab
        self.dim = dim
        self.W = self.param([vocab, dim], init=init_spec, decay=decay)

    def fwd(self, idx: Tensor) -> Tensor:
        return O.embedding(self.W, idx)


class Conv2d(Module):
    def __init__(self, in_c: int, out_c: int, kernel_size, stride=None, padding=None, groups: int = 1,
                 bias: bool = True, init_spec: Optional[dict] = None, decay: Optional[bool] = None):
        self.inC = in_c
        self.outC = out_c
        kH, kW = O.pair_opt(kernel_size, 1)
        sH, sW = O.pair_opt(stride, 1)
        pH, pW = O.pair_opt(padding, 0)
        self.strideH, self.strideW = sH, sW
        self.padH, self.padW = pH, pW
        if not isinstance(groups, int) or groups < 1:
            raise ShapeError(f'Conv2d: groups must be a positive integer, got {groups}', 'Conv2d')
        if in_c % groups != 0 or out_c % groups != 0:
            raise ShapeError(f'Conv2d: inC={in_c} and outC={out_c} must both be divisible by groups={groups}', 'Conv2d')
        self.groups = groups
        self.W = self.param([out_c, in_c // groups, kH, kW], init=init_spec, decay=decay)
        self.b = self.param([out_c], init=init.zeros()) if bias else None

    def fwd(self, x: Tensor) -> Tensor:
        y = O.conv2d(x, self.W, stride=(self.strideH, self.strideW), padding=(self.padH, self.padW),
                     groups=self.groups)
        if self.b is None:
            return y
        return O.add(y, O.reshape(self.b, [1, self.outC, 1, 1]))


def _reduce_loss(t: Tensor, reduction: str) -> Tensor:
    if reduction == 'none':
        return t
    return O.mean(t) if reduction == 'mean' else O.sum_(t)


def nll_loss(log_probs: Tensor, targets: Tensor, reduction: str = 'mean') -> Tensor:
    if targets.dtype != 'i32':
        raise ShapeError(f'nllLoss: targets must be i32, got {targets.dtype}', 'nllLoss')
    vocab = log_probs.shape[-1]
    target_lp = O.sum_(O.mul(log_probs, O.one_hot(targets, vocab, 'f32')), -1)
    per_pos = O.mul(target_lp, -1)
    return _reduce_loss(per_pos, reduction)


def cross_entropy(logits: Tensor, targets: Tensor, reduction: str = 'mean') -> Tensor:
    if targets.dtype != 'i32':
        raise ShapeError(f'crossEntropy: targets must be i32, got {targets.dtype}', 'crossEntropy')
    return nll_loss(O.log_softmax(logits), targets, reduction)

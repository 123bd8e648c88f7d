"""Module tree, parameter placeholders and initialisation (reference `src/module.ts`).

Parameter names are dotted property paths in attribute-definition order
(module.ts:224-238, `Object.keys` order); one `mulberry32` stream (module.ts:72-81) is
shared by all params in plan order; `randn` draws Box-Muller pairs, first uniform into
the log, second into the cos (module.ts:88-90); weight-shaped inits decay by default
(module.ts:134-138).
"""
from __future__ import annotations

import math
from typing import Callable, Dict, List, Optional, Sequence

import numpy as np

from .ir import Tensor
from .trace import param_input


# ---- init specs (module.ts:22-48) ------------------------------------------------

class init:
    @staticmethod
    def randn(scale: float = 0.02) -> dict:
        return {'kind': 'randn', 'scale': scale}

    @staticmethod
    def zeros() -> dict:
        return {'kind': 'zeros'}

    @staticmethod
    def ones() -> dict:
        return {'kind': 'ones'}

    @staticmethod
    def kaiming(gain: Optional[float] = None) -> dict:
        return {'kind': 'kaiming'} if gain is None else {'kind': 'kaiming', 'gain': gain}

    @staticmethod
    def literal(data) -> dict:
        return {'kind': 'literal', 'data': np.asarray(data, dtype=np.float32)}


class Mulberry32:
    """`mulberry32(seed)` (module.ts:72-81). The generator state after k draws is
    `seed + k*0x6D2B79F5 (mod 2^32)`, so a block of draws is computed vectorised; each
    output is exactly the reference's `((t ^ t>>>14) >>> 0) / 2^32` double."""

    def __init__(self, seed: int):
        self.s = int(seed) & 0xFFFFFFFF

    def take(self, n: int) -> np.ndarray:
        k = np.arange(1, n + 1, dtype=np.uint64)
        s = ((np.uint64(self.s) + k * np.uint64(0x6D2B79F5)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        self.s = (self.s + n * 0x6D2B79F5) & 0xFFFFFFFF
        t = s
        t = (t ^ (t >> np.uint32(15))) * (t | np.uint32(1))
        t = t ^ (t + (t ^ (t >> np.uint32(7))) * (t | np.uint32(61)))
        out = t ^ (t >> np.uint32(14))
        return out.astype(np.float64) / 4294967296.0

    def __call__(self) -> float:
        return float(self.take(1)[0])


def box_muller_block(rng: Mulberry32, n: int) -> np.ndarray:
    """n standard normals as f64, element i from draws (2i, 2i+1): `sqrt(-2 log(max(1e-10,
    u1))) * cos(2*pi*u2)`. log/cos go through libm one value at a time (`math`), matching a
    scalar JS evaluation rather than a vector approximation."""
    u = rng.take(2 * n)
    u1 = np.maximum(1e-10, u[0::2])
    u2 = u[1::2]
    lg = np.fromiter(map(math.log, u1.tolist()), dtype=np.float64, count=n)
    cs = np.fromiter(map(math.cos, ((2 * math.pi) * u2).tolist()), dtype=np.float64, count=n)
    return np.sqrt(-2 * lg) * cs


def resolve_init(spec: Optional[dict]) -> Callable[[int, Sequence[int], Mulberry32], np.ndarray]:
    if spec is None:
        spec = init.randn()
    kind = spec['kind']
    if kind == 'randn':
        scale = spec['scale']
        return lambda size, shape, rng: (box_muller_block(rng, size) * scale).astype(np.float32)
    if kind == 'zeros':
        return lambda size, shape, rng: np.zeros(size, np.float32)
    if kind == 'ones':
        return lambda size, shape, rng: np.ones(size, np.float32)
    if kind == 'kaiming':
        gain = spec.get('gain', math.sqrt(2))

        def kaiming(size, shape, rng):
            fan_in = shape[0] if len(shape) > 0 else size
            std = gain / math.sqrt(fan_in)
            return (box_muller_block(rng, size) * std).astype(np.float32)
        return kaiming
    if kind == 'literal':
        data = spec['data']

        def lit(size, shape, rng):
            if data.size != size:
                raise ValueError(f"init.literal: data length {data.size} doesn't match param size {size}")
            return np.array(data, dtype=np.float32).reshape(-1)
        return lit
    raise ValueError(f'unknown init kind {kind!r}')


def resolve_decay(opts: Optional[dict]) -> bool:
    if opts and opts.get('decay') is not None:
        return bool(opts['decay'])
    kind = (opts or {}).get('init', {}) or {}
    kind = kind.get('kind') if isinstance(kind, dict) else None
    return kind not in ('zeros', 'ones')


class Param:
    """Frozen placeholder from `Module.param` (module.ts:408-417)."""
    __slots__ = ('shape', 'dtype', 'init_fn', 'decay')

    def __init__(self, shape, dtype, init_fn, decay):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.init_fn = init_fn
        self.decay = decay


class Module:
    """Base class for parameter trees (module.ts:446-463). Declare params with
    `self.x = self.param(shape, init=..., decay=...)` and child modules / lists of modules
    as plain attributes; names are the dotted attribute paths."""

    def param(self, shape: Sequence[int], init: Optional[dict] = None, decay: Optional[bool] = None,
              dtype: str = 'f32') -> Tensor:
        opts = {'init': init, 'decay': decay}
        return Param(shape, dtype, resolve_init(init), resolve_decay(opts))  # type: ignore[return-value]


class MaterializedParams:
    def __init__(self):
        self.tensors: Dict[str, Tensor] = {}
        self.init_fns: Dict[str, Callable] = {}
        self.decay_flags: Dict[str, bool] = {}


def _visit(node, path: str, visitor) -> None:
    if node is None:
        return
    if isinstance(node, Module):
        for key in list(vars(node).keys()):
            child = getattr(node, key)
            cp = f'{path}.{key}' if path else key
            _visit_child(child, cp, node, key, visitor)
    elif isinstance(node, list):
        for i, item in enumerate(node):
            cp = f'{path}.{i}' if path else str(i)
            _visit_child(item, cp, node, i, visitor)


def _visit_child(child, path, owner, key, visitor) -> None:
    if isinstance(child, (Module, list)):
        _visit(child, path, visitor)
    else:
        visitor(path, child, owner, key)


def materialize_params(root: Module) -> MaterializedParams:
    """Replace every Param placeholder with a `param_input` (module.ts:486-500)."""
    m = MaterializedParams()

    def visitor(path, val, owner, key):
        if isinstance(val, Param):
            t = param_input(path, val.shape, val.dtype)
            if isinstance(owner, list):
                owner[key] = t
            else:
                setattr(owner, key, t)
            m.tensors[path] = t
            m.init_fns[path] = val.init_fn
            m.decay_flags[path] = val.decay
    _visit(root, '', visitor)
    return m


def clone_module(m):
    """Deep-clone the Module tree, sharing Params and plain values (module.ts:513-532)."""
    if isinstance(m, Module):
        out = object.__new__(type(m))
        for k, v in vars(m).items():
            setattr(out, k, clone_module(v))
        return out
    if isinstance(m, list):
        return [clone_module(x) for x in m]
    return m


def build_initial_params(param_shapes: Dict[str, Sequence[int]], init_fns: Dict[str, Callable],
                         seed: int) -> Dict[str, np.ndarray]:
    """One mulberry32(seed) stream over params in plan order (compile.ts:1173-1187)."""
    rng = Mulberry32(seed)
    out = {}
    for name, shape in param_shapes.items():
        size = 1
        for d in shape:
            size *= d
        fn = init_fns.get(name)
        if fn is None:
            raise ValueError(f"compile: no init for param '{name}'")
        out[name] = fn(size, shape, rng)
    return out

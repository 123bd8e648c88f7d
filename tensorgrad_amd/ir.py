"""Intermediate representation: the drop-in boundary between tensorgrad's front end and
this backend.

Restates the reference's `src/ir.ts`: `Tensor` (ir.ts:35-45), the 58-kind `OpNode`
union (ir.ts:74-271) with its field names kept verbatim, `Graph` (ir.ts:284-296),
`addOp` (ir.ts:311-324) and the canonical op->inputs table `remapOpInputs`/`getOpInputs`
(ir.ts:342-395). Ops are plain dicts so the JSON wire form (`graph_to_wire`) carries
exactly the reference's field names and the C++ runtime / C++ oracle read one schema.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

Shape = Tuple[int, ...]

DTYPES = ('f32', 'i32', 'bool')


@dataclass(frozen=True)
class Tensor:
    """Metadata-only tensor handle (ir.ts:35-45). `source` is the producing op index or
    None for leaves; `site` is the op name that created it (error attribution)."""
    id: int
    shape: Shape
    dtype: str
    source: Optional[int]
    site: Optional[str] = None

    @property
    def size(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


@dataclass
class Graph:
    """Ops in topological (= dispatch) order plus the tensors they produce (ir.ts:284-296)."""
    ops: List[dict] = field(default_factory=list)
    tensors: List[Tensor] = field(default_factory=list)
    outputs: List[int] = field(default_factory=list)
    captures: Dict[str, int] = field(default_factory=dict)


def make_graph() -> Graph:
    return Graph()


def add_tensor(g: Graph, shape: Sequence[int], dtype: str, source: Optional[int], site: Optional[str]) -> Tensor:
    t = Tensor(len(g.tensors), tuple(int(d) for d in shape), dtype, source, site)
    g.tensors.append(t)
    return t


def add_op(g: Graph, kind: str, shape: Sequence[int], dtype: str, site: Optional[str], fields: dict) -> Tensor:
    """Append one op and its output tensor (ir.ts:311-324). Field order: kind, out, then
    the op's own fields, as the reference's object literal `{ kind, out, ...fields }`."""
    op_index = len(g.ops)
    out = add_tensor(g, shape, dtype, op_index, site)
    node = {'kind': kind, 'out': out.id}
    node.update(fields)
    g.ops.append(node)
    return out


# Which fields of each kind are tensor ids, in canonical reading order (ir.ts:356-395).
_LEAF_KINDS = ('param_input', 'tensor_input', 'state_input', 'arange', 'const_scalar', 'const_fill')
_AB_KINDS = ('add', 'sub', 'mul', 'div', 'min', 'max', 'less', 'greater', 'matmul', 'matmul_batched')
_A_KINDS = ('mul_scalar', 'add_scalar', 'sqrt', 'rsqrt', 'log', 'exp', 'relu', 'neg', 'abs', 'tanh',
            'sigmoid', 'erf', 'sin', 'cos', 'mean_last', 'sum_last', 'argmax_last', 'reshape', 'permute',
            'softmax_causal_last', 'log_softmax_last', 'where_causal', 'stop_gradient', 'slice_range',
            'scatter_axis', 'broadcast_to', 'sum_to_shape')
_INPUT_FIELDS: Dict[str, Tuple[str, ...]] = {}
for _k in _LEAF_KINDS:
    _INPUT_FIELDS[_k] = ()
for _k in _AB_KINDS:
    _INPUT_FIELDS[_k] = ('a', 'b')
for _k in _A_KINDS:
    _INPUT_FIELDS[_k] = ('a',)
_INPUT_FIELDS.update({
    'randn': ('seed',),
    'dropout': ('a', 'seed'),
    'categorical_last': ('a', 'seed'),
    'one_hot': ('indices',),
    'where': ('cond', 'a', 'b'),
    'concat': ('inputs',),
    'relu_grad': ('x', 'dy'),
    'adam_update_m': ('m', 'g'),
    'adam_update_v': ('v', 'g'),
    'adam_update_p': ('p', 'mNew', 'vNew', 'lrt', 'decayShrinkTensor'),
    'conv2d': ('input', 'weight'),
    'conv2d_input_grad': ('weight', 'dy'),
    'conv2d_weight_grad': ('input', 'dy'),
    'max_pool_2d': ('input',),
    'max_pool_2d_grad': ('input', 'dy'),
})

OP_KINDS = tuple(_INPUT_FIELDS.keys())


def input_fields(kind: str) -> Tuple[str, ...]:
    try:
        return _INPUT_FIELDS[kind]
    except KeyError:
        raise ValueError(f'unknown op kind {kind!r}') from None


def remap_op_inputs(op: dict, f: Callable[[int], int]) -> dict:
    """Copy of `op` with every input tensor id passed through `f` (ir.ts:356-395).
    `decayShrinkTensor` may be None (literal decayShrink) and is then left alone."""
    out = dict(op)
    for name in input_fields(op['kind']):
        v = op[name]
        if name == 'inputs':
            out[name] = [f(i) for i in v]
        elif v is None:
            out[name] = None
        else:
            out[name] = f(v)
    return out


def get_op_inputs(op: dict) -> List[int]:
    """Tensor ids an op reads, canonical order (ir.ts:342-346)."""
    ids: List[int] = []

    def collect(i: int) -> int:
        ids.append(i)
        return i
    remap_op_inputs(op, collect)
    return ids


def graph_to_wire(g: Graph) -> dict:
    """JSON-ready form of a Graph: ops verbatim, tensors as {id, shape, dtype, source}."""
    return {
        'ops': [dict(op) for op in g.ops],
        'tensors': [{'id': t.id, 'shape': list(t.shape), 'dtype': t.dtype, 'source': t.source}
                    for t in g.tensors],
        'outputs': list(g.outputs),
        'captures': dict(g.captures),
    }


def dumps(obj) -> str:
    """Compact JSON. Python's float repr is the shortest round-trip form, so every f64
    scalar baked into an op (scalar, p, eps, decayShrink, ...) arrives bit-identical
    in the C++ runtime and oracle (glibc strtod is correctly rounded)."""
    return json.dumps(obj, separators=(',', ':'), allow_nan=False)

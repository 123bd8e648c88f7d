"""Dead-code elimination (reference `src/dce.ts:33-76`): mark from outputs, captures and
extra roots (the param grads); keep every named leaf; rebuild ops/tensors densely in
construction order and return old-id -> new Tensor."""
from __future__ import annotations

from typing import Dict, Iterable

from .ir import Graph, Tensor, get_op_inputs, remap_op_inputs


def eliminate_dead_code(graph: Graph, extra_roots: Iterable[int] = ()) -> Dict[int, Tensor]:
    live = set()
    stack = list(graph.outputs) + list(graph.captures.values()) + list(extra_roots)
    while stack:
        tid = stack.pop()
        if tid in live:
            continue
        live.add(tid)
        src = graph.tensors[tid].source
        if src is None:
            continue
        stack.extend(get_op_inputs(graph.ops[src]))

    id_map: Dict[int, Tensor] = {}

    def map_id(old: int) -> int:
        t = id_map.get(old)
        if t is None:
            raise RuntimeError(f'dce: op input references tensor #{old} that was eliminated (internal ordering bug)')
        return t.id

    new_ops, new_tensors = [], []
    for op in graph.ops:
        named_leaf = op['kind'] in ('param_input', 'tensor_input', 'state_input')
        if not named_leaf and op['out'] not in live:
            continue
        old = graph.tensors[op['out']]
        remapped = remap_op_inputs(op, map_id)
        t = Tensor(len(new_tensors), old.shape, old.dtype, len(new_ops), old.site)
        remapped['out'] = t.id
        new_ops.append(remapped)
        new_tensors.append(t)
        id_map[op['out']] = t

    new_outputs = [map_id(i) for i in graph.outputs]
    graph.ops[:] = new_ops
    graph.tensors[:] = new_tensors
    graph.outputs[:] = new_outputs
    for name in list(graph.captures.keys()):
        graph.captures[name] = map_id(graph.captures[name])
    return id_map

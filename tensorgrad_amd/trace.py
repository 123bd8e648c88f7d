"""Trace context: the module-global current graph (reference `src/trace.ts`).

`trace_fn` (trace.ts:39-57) opens a fresh graph with capture enabled; `trace_into`
(trace.ts:66-76) re-enters an existing graph for autograd / optimizer passes with
capture disabled; `param_input` / `tensor_input` / `state_input` (trace.ts:88-117)
create the named leaves. `capture` restates `src/capture.ts:15-26`.
"""
from __future__ import annotations

from typing import Callable, List, Optional, Sequence, TypeVar, Union

from .ir import Graph, Tensor, add_op, make_graph

_current: Optional[Graph] = None
_capture_enabled = False

T = TypeVar('T')


def current_graph() -> Graph:
    if _current is None:
        raise RuntimeError('tensorgrad: ops can only be called inside traceFn(). '
                           'Did you forget to wrap your forward pass?')
    return _current


def is_capture_enabled() -> bool:
    return _capture_enabled


def trace_fn(fn: Callable[[], Union[Tensor, List[Tensor]]]) -> Graph:
    global _current, _capture_enabled
    if _current is not None:
        raise RuntimeError('tensorgrad: nested traceFn() is not supported')
    g = make_graph()
    _current = g
    _capture_enabled = True
    try:
        result = fn()
        outputs = result if isinstance(result, (list, tuple)) else [result]
        for t in outputs:
            g.outputs.append(t.id)
    finally:
        _current = None
        _capture_enabled = False
    return g


def trace_into(g: Graph, fn: Callable[[], T]) -> T:
    global _current
    if _current is not None:
        raise RuntimeError('tensorgrad: traceInto() called while another traceFn is active')
    _current = g
    try:
        return fn()
    finally:
        _current = None


def _assert_name_unused(g: Graph, name: str, kinds: Sequence[str], label: str) -> None:
    for op in g.ops:
        if op['kind'] in kinds and op.get('name') == name:
            raise ValueError(f"tensorgrad: {label} name '{name}' already used in this trace")


def param_input(name: str, shape: Sequence[int], dtype: str = 'f32') -> Tensor:
    g = current_graph()
    _assert_name_unused(g, name, ('param_input', 'tensor_input'), 'input')
    return add_op(g, 'param_input', shape, dtype, 'paramInput', {'name': name})


def tensor_input(name: str, shape: Sequence[int], dtype: str = 'f32') -> Tensor:
    g = current_graph()
    _assert_name_unused(g, name, ('param_input', 'tensor_input'), 'input')
    return add_op(g, 'tensor_input', shape, dtype, 'tensorInput', {'name': name})


def state_input(name: str, shape: Sequence[int], dtype: str = 'f32', init_value: float = 0) -> Tensor:
    g = current_graph()
    _assert_name_unused(g, name, ('state_input',), 'state')
    return add_op(g, 'state_input', shape, dtype, 'stateInput', {'name': name, 'initValue': init_value})


def capture(name: str, t: Tensor) -> Tensor:
    """Register `t` for readback under `name`; no-op outside the user's forward trace."""
    if not _capture_enabled:
        return t
    g = current_graph()
    if name in g.captures:
        raise ValueError(f"capture: name '{name}' already registered. Use unique names "
                         f"(e.g. `attn.${{layerIdx}}`) when capturing across a loop.")
    g.captures[name] = t.id
    return t

"""Public compile / step API mirroring the reference's `src/compile.ts`, served by the
gfx950 backend through the C ABI.

`compile(...)` (compile.ts:334-348) traces, differentiates, prunes and appends the
optimizer (build_ir.py), builds the initial params from `mulberry32(seed)`
(compile.ts:1173-1187) and creates the native runtime. The returned `CompiledTraining`
has the reference's surface: `step`, `upload_params`, `download_params`, `reset`,
`set_lr`, `attach`, `replace_model`, `destroy` (compile.ts:198-285). `step` / `run`
return discriminated results (`completed` / `aborted` / `failed`, compile.ts:97-110,
1201-1208) instead of raising. Calls are synchronous: the host blocks on the step's
4-byte loss read, as the reference's promise resolves after `mapAsync`.
"""
from __future__ import annotations

import random
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Callable, Dict, Optional

import numpy as np

from .backend import AbortError, NativeRuntime
from .build_ir import TrainingIR, build_forward_ir, build_training_ir, normalize_decl
from .module import Module

_DT = {'f32': np.float32, 'i32': np.int32, 'bool': np.int32}


class Captures:
    """Activation readbacks of one step/run (src/runtime.ts:26-75)."""

    def __init__(self, shapes: Dict[str, tuple], data: Dict[str, np.ndarray]):
        self._shapes = shapes
        self._data = data

    def get(self, name: str) -> np.ndarray:
        if name not in self._data:
            known = ', '.join(sorted(self._data)) or '(none registered)'
            raise KeyError(f"Captures.get: '{name}' not present. Known: {known}")
        return self._data[name]

    def shape(self, name: str):
        if name not in self._shapes:
            known = ', '.join(sorted(self._shapes)) or '(none registered)'
            raise KeyError(f"Captures.shape: '{name}' not registered. Known: {known}")
        return self._shapes[name]

    def has(self, name: str) -> bool:
        return name in self._data

    def names(self):
        return sorted(self._data)


@dataclass
class StepResult:
    kind: str                       # 'completed' | 'aborted' | 'failed'
    loss: Optional[float] = None
    captures: Optional[Captures] = None
    error: Optional[Exception] = None


@dataclass
class RunResult:
    kind: str
    output: Optional[np.ndarray] = None
    captures: Optional[Captures] = None
    error: Optional[Exception] = None


def _guarded(body, cls):
    try:
        return body()
    except AbortError:
        return cls('aborted')
    except Exception as e:  # the reference maps every other failure to 'failed'
        return cls('failed', error=e)


def _capture_meta(ir: TrainingIR):
    g = ir.graph
    return {name: (g.tensors[tid].shape, _DT[g.tensors[tid].dtype]) for name, tid in g.captures.items()}


def _read_captures(rt: NativeRuntime, meta) -> Captures:
    data = {name: rt.capture(name, shape, dt) for name, (shape, dt) in meta.items()}
    return Captures({k: v[0] for k, v in meta.items()}, data)


class CompiledForward:
    """A forward sibling sharing the training graph's parameter buffers
    (`attach`, compile.ts:665-681; LRU shape cache, compile.ts:728-891). Input dims given
    as None are resolved per call from the array lengths (compile.ts:1106-1163)."""

    def __init__(self, parent: 'CompiledTraining', forward: Callable, inputs: Dict, output: str = 'f32',
                 max_cached_shapes: int = 8):
        self.parent = parent
        self.forward = forward
        self.decls = {k: normalize_decl(v) for k, v in inputs.items()}
        self.output = output
        self.max_cached = max_cached_shapes
        self._cache: 'OrderedDict[str, tuple]' = OrderedDict()

    @property
    def param_names(self):
        return self.parent.param_names

    def _sibling(self, inputs):
        resolved = _resolve_decls(self.decls, inputs)
        key = _shape_key(resolved)
        if key in self._cache:
            self._cache.move_to_end(key)
            return self._cache[key]
        ir = build_forward_ir(self.parent.model, self.forward, resolved)
        out_t = ir.graph.tensors[ir.graph.outputs[0]]
        if out_t.dtype != self.output and not (self.output == 'f32' and out_t.dtype == 'f32'):
            raise ValueError(f"attach: declared output '{self.output}' but the forward returns '{out_t.dtype}'")
        rt = NativeRuntime(ir.wire_json(), parent=self.parent._rt)
        entry = (rt, ir, out_t.shape, _DT[out_t.dtype], _capture_meta(ir))
        self._cache[key] = entry
        while len(self._cache) > self.max_cached:
            _, old = self._cache.popitem(last=False)
            old[0].destroy()
        return entry

    def run(self, inputs: Dict[str, np.ndarray]) -> RunResult:
        def body():
            if not self.parent._rt.alive:
                raise AbortError('run aborted: graph destroyed')
            rt, ir, shape, dt, meta = self._sibling(inputs)
            out = rt.run(inputs, shape, dt)
            return RunResult('completed', output=out, captures=_read_captures(rt, meta))
        return _guarded(body, RunResult)

    def graph_for(self, inputs) -> TrainingIR:
        return self._sibling(inputs)[1]

    def upload_params(self, params):
        self.parent.upload_params(params)

    def download_params(self):
        return self.parent.download_params()

    def _invalidate(self):
        for entry in self._cache.values():
            entry[0].destroy()
        self._cache.clear()

    def destroy(self):
        self._invalidate()
        self.parent._children.discard(self)


class CompiledTraining:
    def __init__(self, model: Module, loss: Callable, inputs: Dict, optimizer: dict, seed: Optional[int] = None):
        self.model = model
        self.loss = loss
        self.inputs = inputs
        self.optimizer = optimizer
        self.seed = seed if seed is not None else random.getrandbits(32)
        self._children = set()
        self._build()

    def _build(self):
        self.ir = build_training_ir(self.model, self.loss, self.inputs, self.optimizer)
        self._rt = NativeRuntime(self.ir.wire_json())
        self._rt.upload_params(self.ir.initial_params(self.seed))
        self._capture_meta = _capture_meta(self.ir)

    @property
    def graph(self):
        return self.ir.graph

    @property
    def param_names(self):
        return list(self._rt.param_names)

    @property
    def output_shape(self):
        return list(self.ir.graph.tensors[self.ir.graph.outputs[0]].shape)

    def step(self, inputs: Dict[str, np.ndarray]) -> StepResult:
        def body():
            loss = self._rt.step(inputs)
            return StepResult('completed', loss=loss, captures=_read_captures(self._rt, self._capture_meta))
        return _guarded(body, StepResult)

    def upload_params(self, params: Dict[str, np.ndarray]) -> None:
        self._rt.upload_params(params)

    def download_params(self) -> Dict[str, np.ndarray]:
        return self._rt.download_params()

    def reset(self, params: bool = True, optimizer: bool = True) -> None:
        if params:
            self._rt.upload_params(self.ir.initial_params(self.seed))
        if optimizer:
            self._rt.reset_optimizer()

    def set_lr(self, lr) -> None:
        self._rt.set_lr(lr)

    # ---- checkpoints (no reference counterpart: the reference cannot resume) ----------

    def download_optimizer_state(self):
        """({state tensor name: flat values}, optimizer step t, PRNG seed counter)."""
        return self._rt.download_state()

    def upload_optimizer_state(self, state: Dict[str, np.ndarray], t: int, prng_counter: int) -> None:
        self._rt.upload_state(state, t, prng_counter)

    def save_checkpoint(self, path: str) -> None:
        """Params, optimizer state, t, seed counter and LR schedule to a safetensors file."""
        self._rt.save_checkpoint(path)

    def load_checkpoint(self, path: str) -> None:
        """Restore a checkpoint written by `save_checkpoint` (or load a params-only file);
        training then continues exactly as it would have from the saved step."""
        self._rt.load_checkpoint(path)

    def attach(self, forward: Callable, inputs: Dict, output: str = 'f32', max_cached_shapes: int = 8) -> CompiledForward:
        child = CompiledForward(self, forward, inputs, output, max_cached_shapes)
        self._children.add(child)
        return child

    def replace_model(self, new_model: Module, seed: Optional[int] = None, optimizer: Optional[dict] = None) -> None:
        if optimizer is not None and optimizer['kind'] != self.optimizer['kind']:
            raise ValueError(f"replaceModel: optimizer kind cannot change ('{self.optimizer['kind']}' → "
                             f"'{optimizer['kind']}'). State buffers are kind-specific — destroy and recompile.")
        for c in self._children:
            c._invalidate()
        self._rt.destroy()
        self.model = new_model
        self.seed = seed if seed is not None else random.getrandbits(32)
        if optimizer is not None:
            self.optimizer = optimizer
        self._build()

    def destroy(self) -> None:
        for c in list(self._children):
            c._invalidate()
        self._children.clear()
        self._rt.destroy()


class CompiledForwardExecutor:
    """Standalone forward-only executor (`compileForward`, compile.ts:424-452; proxy
    compile.ts:895-1018). It owns its parameters: the owner graph is a runtime created
    with no optimizer, compiled eagerly when every input dim is concrete, else at the
    first `run`; other resolved shapes are siblings sharing the owner's parameters,
    cached LRU. `upload_params` before the owner exists is buffered (merged, later keys
    win) and applied, strictly, when it is created."""

    def __init__(self, model: Module, forward: Callable, inputs: Dict, output: str = 'f32',
                 max_cached_shapes: int = 8, seed: Optional[int] = None):
        self.model = model
        self.forward = forward
        self.decls = {k: normalize_decl(v) for k, v in inputs.items()}
        self.output = output
        self.max_cached = max_cached_shapes
        self.seed = seed if seed is not None else random.getrandbits(32)
        self._owner = None            # (runtime, ir, shape, dtype, capture meta)
        self._owner_key = None
        self._cache: 'OrderedDict[str, tuple]' = OrderedDict()
        self._pending: Optional[Dict[str, np.ndarray]] = None
        self._destroyed = False
        # metadata trace: parametric dims as 1 (param shapes do not depend on them)
        meta = {k: {'shape': [1 if d is None else d for d in s], 'dtype': dt} for k, (s, dt) in self.decls.items()}
        ir = build_forward_ir(self.model, self.forward, meta)
        self._param_names = ir.param_names
        if all(d is not None for s, _ in self.decls.values() for d in s):
            self._create_owner(meta, ir)

    @property
    def param_names(self):
        return list(self._param_names)

    def _entry(self, rt, ir):
        out_t = ir.graph.tensors[ir.graph.outputs[0]]
        if out_t.dtype != self.output:
            rt.destroy()
            raise ValueError(f"compileForward: forward declares output: '{self.output}' but the traced graph's "
                             f"output tensor is '{out_t.dtype}'.")
        return (rt, ir, out_t.shape, _DT[out_t.dtype], _capture_meta(ir))

    def _create_owner(self, resolved, ir=None):
        ir = ir or build_forward_ir(self.model, self.forward, resolved)
        rt = NativeRuntime(ir.wire_json())
        rt.upload_params(ir.initial_params(self.seed))
        self._owner = self._entry(rt, ir)
        self._owner_key = _shape_key(resolved)
        self._param_names = list(rt.param_names)
        if self._pending is not None:
            pending, self._pending = self._pending, None
            rt.upload_params(pending)
        return self._owner

    def _sibling(self, inputs):
        resolved = _resolve_decls(self.decls, inputs)
        key = _shape_key(resolved)
        if self._owner is None:
            return self._create_owner(resolved)
        if key == self._owner_key:
            return self._owner
        if key in self._cache:
            self._cache.move_to_end(key)
            return self._cache[key]
        ir = build_forward_ir(self.model, self.forward, resolved)
        entry = self._entry(NativeRuntime(ir.wire_json(), parent=self._owner[0]), ir)
        self._cache[key] = entry
        while len(self._cache) > self.max_cached:
            _, old = self._cache.popitem(last=False)
            old[0].destroy()
        return entry

    def run(self, inputs: Dict[str, np.ndarray]) -> RunResult:
        def body():
            if self._destroyed:
                raise AbortError('run aborted: executor destroyed')
            rt, ir, shape, dt, meta = self._sibling(inputs)
            out = rt.run(inputs, shape, dt)
            return RunResult('completed', output=out, captures=_read_captures(rt, meta))
        return _guarded(body, RunResult)

    def graph_for(self, inputs) -> TrainingIR:
        return self._sibling(inputs)[1]

    def upload_params(self, params: Dict[str, np.ndarray]) -> None:
        if self._owner is None:
            self._pending = dict(self._pending or {}, **params)
            return
        self._owner[0].upload_params(params)

    def download_params(self) -> Dict[str, np.ndarray]:
        if self._owner is None:
            raise RuntimeError('compileForward: downloadParams() before any params exist on the GPU. With a '
                               'parametric (null-wildcard) input shape the param buffers are allocated on the first '
                               'run(); call run() once (or declare fully concrete input shapes) before downloadParams().')
        return self._owner[0].download_params()

    def load_checkpoint(self, path: str) -> None:
        """Load parameters from a safetensors file holding exactly this model's params."""
        if self._owner is None:
            from .safetensors import load_safetensors
            with open(path, 'rb') as f:
                self.upload_params(load_safetensors(f.read()).tensors)
            return
        self._owner[0].load_checkpoint(path)

    def destroy(self) -> None:
        self._destroyed = True
        self._cache.clear()          # siblings go with the owner (destroy cascades)
        if self._owner is not None:
            self._owner[0].destroy()


def _resolve_decls(decls, inputs: Dict[str, np.ndarray]) -> Dict:
    """Resolve one `None` wildcard per input from the given arrays' lengths; every input
    must agree on the resolved value (compile.ts:1106-1163)."""
    agreed, out = None, {}
    for name, (shape, dtype) in decls.items():
        nulls = [i for i, d in enumerate(shape) if d is None]
        if not nulls:
            out[name] = {'shape': list(shape), 'dtype': dtype}
            continue
        if len(nulls) > 1:
            raise ValueError(f"run: input '{name}' has {len(nulls)} parametric dims; only one is supported.")
        if name not in inputs:
            raise ValueError(f"run: missing input '{name}'")
        concrete = 1
        for d in shape:
            if d is not None:
                concrete *= d
        n = np.asarray(inputs[name]).size
        if n % concrete != 0:
            raise ValueError(f"run: input '{name}' length {n} is not divisible by {concrete}")
        dim = n // concrete
        if agreed is not None and dim != agreed:
            raise ValueError('run: parametric dim resolved inconsistently across inputs')
        agreed = dim
        s = list(shape)
        s[nulls[0]] = dim
        out[name] = {'shape': s, 'dtype': dtype}
    return out


def _shape_key(resolved: Dict) -> str:
    return '|'.join(f"{n}:{'x'.join(map(str, resolved[n]['shape']))}:{resolved[n]['dtype']}" for n in sorted(resolved))


def compile_forward(model: Module, forward: Callable, inputs: Dict, output: str = 'f32',
                    max_cached_shapes: int = 8, seed: Optional[int] = None) -> CompiledForwardExecutor:
    """`compileForward` (compile.ts:424-452): a forward-only graph with its own params."""
    return CompiledForwardExecutor(model, forward, inputs, output, max_cached_shapes, seed)


def compile(model: Module, loss: Callable, inputs: Dict, optimizer: dict, seed: Optional[int] = None) -> CompiledTraining:
    return CompiledTraining(model, loss, inputs, optimizer, seed)


def trace(model: Module, loss: Callable, inputs: Dict, optimizer: dict) -> TrainingIR:
    return build_training_ir(model, loss, inputs, optimizer)


def trace_forward(model: Module, forward: Callable, inputs: Dict) -> TrainingIR:
    return build_forward_ir(model, forward, inputs)

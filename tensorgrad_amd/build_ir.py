"""Training / forward IR construction (reference `src/compile.ts:473-538`, `:1058-1080`).

`build_training_ir` = traceModule -> appendGrad -> eliminateDeadCode (roots: loss,
captures, param grads) -> appendAdam | appendSGD. What the reference then hands to
`planBuffers`/`emitKernels`/`createRuntime` is replaced here by `TrainingIR.wire()`:
the JSON document the C-ABI runtime (`tg_runtime_create`) consumes.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional

from . import ir as IR
from .adam import OptimizerResult, append_adam, append_sgd
from .dce import eliminate_dead_code
from .grad import append_grad
from .ir import Graph, Tensor
from .module import MaterializedParams, Module, build_initial_params, clone_module, materialize_params
from .trace import tensor_input, trace_fn


def normalize_decl(d):
    if isinstance(d, dict):
        return list(d['shape']), d['dtype']
    return list(d), 'f32'


def trace_module(model: Module, forward: Callable, input_decls: Dict) -> tuple:
    cloned = clone_module(model)
    holder = {}

    def body():
        holder['m'] = materialize_params(cloned)
        tensors = {}
        for name, decl in input_decls.items():
            shape, dtype = normalize_decl(decl)
            if any(d is None for d in shape):
                raise ValueError(f"compile: input '{name}' has an unresolved parametric dim; training specs "
                                 'require fully concrete shapes.')
            tensors[name] = tensor_input(name, shape, dtype)
        return forward(cloned, tensors)
    g = trace_fn(body)
    return g, holder['m']


class TrainingIR:
    def __init__(self, graph: Graph, param_grads: Dict[str, Tensor], loss: Tensor,
                 materialized: MaterializedParams, opt: Optional[OptimizerResult]):
        self.graph = graph
        self.param_grads = param_grads
        self.loss = loss
        self.materialized = materialized
        self.opt = opt

    @property
    def param_names(self):
        return [op['name'] for op in self.graph.ops if op['kind'] == 'param_input']

    def param_shapes(self) -> Dict[str, tuple]:
        return {op['name']: self.graph.tensors[op['out']].shape for op in self.graph.ops if op['kind'] == 'param_input'}

    def initial_params(self, seed: int):
        return build_initial_params(self.param_shapes(), self.materialized.init_fns, seed)

    def wire(self) -> dict:
        return {
            'graph': IR.graph_to_wire(self.graph),
            'paramGrads': {n: t.id for n, t in self.param_grads.items()},
            'writebacks': [w.wire() for w in (self.opt.writebacks if self.opt else [])],
            'optimizer': ({'kind': self.opt.kind, 'config': self.opt.wire_config} if self.opt else None),
        }

    def wire_json(self) -> str:
        return IR.dumps(self.wire())


def _remap(rec: Dict[str, Tensor], id_map) -> Dict[str, Tensor]:
    out = {}
    for name, t in rec.items():
        m = id_map.get(t.id)
        if m is None:
            raise RuntimeError(f"dce: tensor '{name}' (#{t.id}) did not survive dead-code elimination")
        out[name] = m
    return out


def build_training_ir(model: Module, loss: Callable, inputs: Dict, optimizer: dict) -> TrainingIR:
    graph, materialized = trace_module(model, loss, inputs)
    gr = append_grad(graph)
    id_map = eliminate_dead_code(graph, [t.id for t in gr.param_grads.values()])
    param_grads = _remap(gr.param_grads, id_map)
    param_tensors = _remap(materialized.tensors, id_map)
    loss_t = id_map[gr.loss.id]
    kind = optimizer['kind']
    if kind in ('adam', 'adamw'):
        opt = append_adam(graph, param_grads, param_tensors, optimizer, materialized.decay_flags)
    elif kind == 'sgd':
        opt = append_sgd(graph, param_grads, param_tensors, optimizer, materialized.decay_flags)
    else:
        raise ValueError(f'unknown optimizer kind {kind!r}')
    return TrainingIR(graph, param_grads, loss_t, materialized, opt)


def build_forward_ir(model: Module, forward: Callable, inputs: Dict) -> TrainingIR:
    graph, materialized = trace_module(model, forward, inputs)
    eliminate_dead_code(graph)
    out = graph.tensors[graph.outputs[0]]
    return TrainingIR(graph, {}, out, materialized, None)

"""In-graph Adam / AdamW pass (reference `src/adam.ts`) and SGD pass (`src/sgd.ts`).

`append_adam` restates adam.ts:157-240: optional normalize then clip, one `_adam_lrt`
scalar input, `_adam_decay_shrink` only for scheduled lr with decayed params, per param
two state inputs and `adam_update_{m,v,p}` plus three writebacks. `adam_step_scalars`
restates adam.ts:134-143. `append_sgd` restates sgd.ts:102-175.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

from . import ops as O
from .grad import append_grad_clip, append_grad_normalize
from .ir import Graph, Tensor
from .lr import is_lr_dynamic, resolve_lr
from .trace import state_input, tensor_input, trace_into


class Writeback:
    def __init__(self, source: Tensor, dest_name: str, dest_kind: str):
        self.source = source
        self.dest_name = dest_name
        self.dest_kind = dest_kind

    def wire(self) -> dict:
        return {'source': self.source.id, 'destName': self.dest_name, 'destKind': self.dest_kind}


class OptimizerResult:
    def __init__(self, kind: str, writebacks: List[Writeback], wire_config: dict):
        self.kind = kind
        self.writebacks = writebacks
        self.wire_config = wire_config   # WireAdamConfig / WireSGDConfig (worker-protocol.ts:14-37)


def adam_step_scalars(c: dict, t: int):
    lr_now = resolve_lr(c['lr'], t)
    lrt = lr_now * math.sqrt(1 - math.pow(c['beta2'], t)) / (1 - math.pow(c['beta1'], t))
    return lrt, 1 - lr_now * c['weightDecay']


def append_adam(graph: Graph, param_grads: Dict[str, Tensor], param_tensors: Dict[str, Tensor], config: dict,
                decay_flags: Optional[Dict[str, bool]] = None) -> OptimizerResult:
    if config.get('normalizeGrads'):
        ng = config['normalizeGrads']
        param_grads = append_grad_normalize(graph, param_grads, ng if callable(ng) else None)
    if config.get('clipGradNorm') is not None and config['clipGradNorm'] > 0:
        param_grads = append_grad_clip(graph, param_grads, config['clipGradNorm'])
    lr_sched = is_lr_dynamic(config['lr'])
    initial_lr = resolve_lr(config['lr'], 1)
    # adam.ts:75-77 reads `weightDecay` whenever the config object carries one.
    wd = config['weightDecay'] if config.get('weightDecay', 0) > 0 else 0
    decay_filter = config.get('decayFilter') or (lambda name: True)
    full = {'lr': config['lr'], 'beta1': config.get('beta1', 0.9), 'beta2': config.get('beta2', 0.999),
            'eps': config.get('eps', 1e-8), 'weightDecay': wd, 'lrIsScheduled': lr_sched}
    writebacks: List[Writeback] = []
    lrt_name = '_adam_lrt'
    state = {'decay_name': None}

    def body():
        lrt = tensor_input(lrt_name, [], 'f32')
        decayed = set()
        if wd > 0:
            for name in param_grads:
                flag = decay_flags[name] if (decay_flags is not None and name in decay_flags) else decay_filter(name)
                if flag:
                    decayed.add(name)
        decay_scalar = None
        if lr_sched and decayed:
            state['decay_name'] = '_adam_decay_shrink'
            decay_scalar = tensor_input(state['decay_name'], [], 'f32')
        for name in param_grads:
            p = param_tensors.get(name)
            g = param_grads.get(name)
            if p is None:
                raise ValueError(f"appendAdam: missing param tensor for '{name}'")
            m_state = state_input(f'adam_m_{name}', p.shape, 'f32', 0)
            v_state = state_input(f'adam_v_{name}', p.shape, 'f32', 0)
            if name not in decayed:
                shrink = 1
            elif decay_scalar is not None:
                shrink = decay_scalar
            else:
                shrink = 1 - initial_lr * wd
            new_m = O.adam_update_m(m_state, g, full['beta1'])
            new_v = O.adam_update_v(v_state, g, full['beta2'])
            new_p = O.adam_update_p(p, new_m, new_v, lrt, full['eps'], shrink)
            writebacks.append(Writeback(new_m, f'adam_m_{name}', 'state'))
            writebacks.append(Writeback(new_v, f'adam_v_{name}', 'state'))
            writebacks.append(Writeback(new_p, name, 'param'))
    trace_into(graph, body)
    wire = dict(full, lrtInputName=lrt_name, decayShrinkInputName=state['decay_name'])
    return OptimizerResult('adam', writebacks, wire)


def append_sgd(graph: Graph, param_grads: Dict[str, Tensor], param_tensors: Dict[str, Tensor], config: dict,
               decay_flags: Optional[Dict[str, bool]] = None) -> OptimizerResult:
    if config.get('normalizeGrads'):
        ng = config['normalizeGrads']
        param_grads = append_grad_normalize(graph, param_grads, ng if callable(ng) else None)
    if config.get('clipGradNorm') is not None and config['clipGradNorm'] > 0:
        param_grads = append_grad_clip(graph, param_grads, config['clipGradNorm'])
    momentum = config.get('momentum', 0)
    nesterov = config.get('nesterov', False)
    if nesterov and momentum <= 0:
        raise ValueError(f'appendSGD: nesterov requires momentum > 0 (got momentum={momentum})')
    wd = config.get('weightDecay', 0)
    decay_filter = config.get('decayFilter') or (lambda name: True)
    writebacks: List[Writeback] = []
    lr_name = '_sgd_lr'

    def body():
        lr_t = tensor_input(lr_name, [], 'f32')
        decayed = set()
        if wd > 0:
            for name in param_grads:
                flag = decay_flags[name] if (decay_flags is not None and name in decay_flags) else decay_filter(name)
                if flag:
                    decayed.add(name)
        for name in param_grads:
            p, g = param_tensors[name], param_grads[name]
            g_eff = O.add(g, O.mul_scalar(p, wd)) if name in decayed else g
            if momentum > 0:
                v_state = state_input(f'sgd_v_{name}', p.shape, 'f32', 0)
                v_new = O.add(O.mul_scalar(v_state, momentum), g_eff)
                update = O.add(g_eff, O.mul_scalar(v_new, momentum)) if nesterov else v_new
                writebacks.append(Writeback(v_new, f'sgd_v_{name}', 'state'))
            else:
                update = g_eff
            p_new = O.sub(p, O.mul(O.broadcast_to(lr_t, p.shape), update))
            writebacks.append(Writeback(p_new, name, 'param'))
    trace_into(graph, body)
    wire = {'lr': config['lr'], 'momentum': momentum, 'nesterov': nesterov, 'weightDecay': wd,
            'lrIsScheduled': is_lr_dynamic(config['lr']), 'lrInputName': lr_name}
    return OptimizerResult('sgd', writebacks, wire)

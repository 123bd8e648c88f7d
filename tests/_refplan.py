"""Reference-shaped createRuntime payloads for the Node shim's tests.

`reference_plan` builds the fields of the reference's BufferPlan that `toWire` reads
(src/buffers.ts:54-88): tensorToBuffer with dedicated buffers for params, inputs,
state, parameter gradients, outputs, captures and writeback sources (src/buffers.ts:
142-145) and best-fit pooled buffers for every other intermediate (liveness over op
order), plus paramsByName / statesByName / paramGradsByName and writebacks by buffer id.
"""
from tensorgrad_amd import ir as IR


def reference_plan(ir) -> dict:
    g = ir.graph
    grads = {t.id: name for name, t in ir.param_grads.items()}
    wb_src = {w.source.id for w in (ir.opt.writebacks if ir.opt else [])}
    caps = set(g.captures.values())
    outs = set(g.outputs)
    last = {}
    for i, op in enumerate(g.ops):
        for t in IR.get_op_inputs(op):
            last[t] = i
    buffers, t2b, free = [], {}, []
    params, inputs, states, pgrads = {}, {}, {}, {}

    def alloc(n):
        buffers.append(n)
        return len(buffers) - 1
    for i, op in enumerate(g.ops):
        t = g.tensors[op['out']]
        need = max(4, t.size * 4)
        kind = op['kind']
        poolable = (kind not in ('param_input', 'tensor_input', 'state_input') and t.id not in grads
                    and t.id not in outs and t.id not in caps and t.id not in wb_src)
        if poolable:
            fit = [k for k in range(len(free)) if buffers[free[k]] >= need]
            if fit:
                k = min(fit, key=lambda q: buffers[free[q]])
                b = free.pop(k)
            else:
                b = alloc(need)
        else:
            b = alloc(need)
            if kind == 'param_input':
                params[op['name']] = b
            elif kind == 'tensor_input':
                inputs[op['name']] = b
            elif kind == 'state_input':
                states[op['name']] = b
            elif t.id in grads:
                pgrads[grads[t.id]] = b
        t2b[t.id] = b
        freed = set()
        for x in IR.get_op_inputs(op):
            xt = g.tensors[x]
            src = g.ops[xt.source]['kind'] if xt.source is not None else 'leaf'
            pool_x = (src not in ('param_input', 'tensor_input', 'state_input', 'leaf') and x not in grads
                      and x not in outs and x not in caps and x not in wb_src)
            if x in freed or not pool_x or last.get(x) != i:
                continue
            freed.add(x)
            free.append(t2b[x])
        if poolable and op['out'] not in last:
            free.append(b)
    wbs = []
    for w in (ir.opt.writebacks if ir.opt else []):
        dest = params[w.dest_name] if w.dest_kind == 'param' else states[w.dest_name]
        wbs.append({'source': t2b[w.source.id], 'dest': dest, 'bytes': buffers[dest]})
    return {'tensorToBuffer': {str(k): v for k, v in t2b.items()}, 'paramsByName': params, 'inputsByName': inputs,
            'statesByName': states, 'paramGradsByName': pgrads, 'writebacks': wbs,
            'n_buffers': len(buffers), 'n_tensors': len(g.tensors)}


def reference_payload(ir) -> dict:
    w = ir.wire()
    return {'ir': {'graph': w['graph'], 'plan': reference_plan(ir), 'kernels': []}, 'optimizer': w['optimizer']}

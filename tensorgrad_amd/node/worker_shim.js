'use strict'
// In-process replacement for the reference's WorkerProxy (src/worker-proxy.ts:16-73),
// serving the worker protocol's requests (src/worker-protocol.ts:54-63) with the
// handler semantics of src/worker.ts:86-334 on the MI355X backend through the N-API
// addon (tg_napi.node -> libtg.so). compile.ts keeps calling request / send /
// terminate; only the object it constructs changes (see INTEGRATION.md).
//
// What the C ABI takes instead of the WebGPU plan: `toWire` recovers, from the
// createRuntime / compileForward payload's `ir: {graph, plan, kernels}`, the tensor ids
// of the parameter gradients and of the writeback sources. planBuffers gives both a
// dedicated (never pooled) buffer (src/buffers.ts:142-145), so inverting
// plan.tensorToBuffer on those buffers is exact. `kernels` (the WGSL) is not used.
//
// Written for Node >= 12 (no optional chaining / nullish coalescing).

const path = require('path')

let addon = null
function native() {
  if (!addon) addon = require(path.join(__dirname, 'tg_napi.node'))
  return addon
}

function entries(m) {
  if (m == null) return []
  if (typeof m.entries === 'function' && !Array.isArray(m)) return Array.from(m.entries())
  return Object.keys(m).map(k => [k, m[k]])
}

function numKey(k) { return typeof k === 'string' ? Number(k) : k }

/** createRuntime / compileForward payload -> the C ABI's IR document (include/tg.h). */
function toWire(ir, optimizer) {
  const g = ir.graph
  const plan = ir.plan
  const owner = new Map()     // buffer id -> the one tensor id it holds, or -1 if pooled
  for (const [tid, bid] of entries(plan.tensorToBuffer)) {
    const b = numKey(bid)
    owner.set(b, owner.has(b) ? -1 : numKey(tid))
  }
  const dedicated = (bid, what) => {
    const t = owner.get(bid)
    if (t === undefined || t < 0) throw new Error(`toWire: ${what} buffer ${bid} is not a dedicated buffer`)
    return t
  }
  const paramGrads = {}
  for (const [name, bid] of entries(plan.paramGradsByName)) paramGrads[name] = dedicated(bid, `param grad '${name}'`)
  const homes = new Map()
  for (const [name, bid] of entries(plan.paramsByName)) homes.set(bid, { destName: name, destKind: 'param' })
  for (const [name, bid] of entries(plan.statesByName)) homes.set(bid, { destName: name, destKind: 'state' })
  const writebacks = (plan.writebacks || []).map(w => {
    const h = homes.get(w.dest)
    if (!h) throw new Error(`toWire: writeback destination buffer ${w.dest} is not a param or state`)
    return { source: dedicated(w.source, 'writeback source'), destName: h.destName, destKind: h.destKind }
  })
  const captures = {}
  for (const [name, tid] of entries(g.captures)) captures[name] = tid
  return {
    graph: {
      ops: g.ops,
      tensors: g.tensors.map(t => ({ id: t.id, shape: Array.from(t.shape), dtype: t.dtype })),
      outputs: Array.from(g.outputs),
      captures,
    },
    paramGrads,
    writebacks,
    optimizer: optimizer || null,
  }
}

function abortErr(msg) {
  const e = new Error(msg)
  e.name = 'AbortError'
  return e
}

function countOf(shape) { return shape.reduce((a, b) => a * b, 1) }

class NativeWorkerProxy {
  constructor() {
    this.graphs = new Map()     // graphId -> slot
    this.family = new Map()     // graphId -> id of its runtime family (the graph owning the params)
    this.queues = new Map()     // family id -> tail of its request chain
    this.terminated = false
  }

  async _slotMeta(handle, wire) {
    const g = wire.graph
    const out = g.tensors[g.outputs[0]]
    const captureShapes = {}
    const captureDtypes = {}
    for (const name of Object.keys(g.captures)) {
      const t = g.tensors[g.captures[name]]
      captureShapes[name] = t.shape
      captureDtypes[name] = t.dtype
    }
    const nodes = JSON.parse(native().describe(handle)).nodes
    return {
      handle,
      outputShape: out.shape,
      outputInt: out.dtype !== 'f32',
      captureShapes,
      captureDtypes,
      kernelCount: nodes.length,
      paramNames: native().paramNames(handle),
    }
  }

  _compileResult(slot) {
    return {
      paramNames: slot.paramNames.slice(),
      outputShape: slot.outputShape.slice(),
      kernelCount: slot.kernelCount,
      captureShapes: Object.assign({}, slot.captureShapes),
    }
  }

  // [[name, element count, isInt]] for the addon, which reads the captures back on its
  // worker thread right after the step / run
  _captureSpec(slot) {
    return Object.keys(slot.captureShapes).map(n =>
      [n, countOf(slot.captureShapes[n]), slot.captureDtypes[n] !== 'f32'])
  }

  _mustGet(graphId) {
    const slot = this.graphs.get(graphId)
    if (!slot) throw new Error(`tensorgrad worker: graph ${graphId} not found`)
    return slot
  }

  async _handle(req) {
    const p = req.payload
    const A = native()
    switch (req.kind) {
      case 'createRuntime': {
        const wire = toWire(p.ir, p.optimizer)
        const h = await A.create(JSON.stringify(wire))
        try {
          if (Object.keys(p.initialParams || {}).length > 0) await A.uploadParams(h, p.initialParams)
        } catch (e) {
          await A.destroy(h)
          throw e
        }
        const slot = Object.assign(await this._slotMeta(h, wire), { parentGraphId: null })
        this.graphs.set(p.graphId, slot)
        return this._compileResult(slot)
      }
      case 'compileForward': {
        const parent = this.graphs.get(p.parentGraphId)
        if (!parent) throw new Error(`compileForward: parent graph ${p.parentGraphId} not found`)
        const wire = toWire(p.ir, null)
        const h = await A.createSibling(parent.handle, JSON.stringify(wire))
        const slot = Object.assign(await this._slotMeta(h, wire), { parentGraphId: p.parentGraphId })
        this.graphs.set(p.graphId, slot)
        return this._compileResult(slot)
      }
      case 'step': {
        const slot = this.graphs.get(p.graphId)
        if (!slot) throw abortErr('step aborted: graph replaced mid-flight')
        const r = await A.step(slot.handle, p.inputs, this._captureSpec(slot))
        return { loss: r.loss, captures: r.captures }
      }
      case 'run': {
        const slot = this.graphs.get(p.graphId)
        if (!slot) throw abortErr('run aborted: graph replaced mid-flight')
        const r = await A.run(slot.handle, p.inputs, countOf(slot.outputShape), slot.outputInt, this._captureSpec(slot))
        return { output: r.output, captures: r.captures }
      }
      case 'uploadParams':
        await A.uploadParams(this._mustGet(p.graphId).handle, p.params)
        return null
      case 'downloadParams':
        return { params: await A.downloadParams(this._mustGet(p.graphId).handle) }
      case 'resetOptimizer':
        await A.resetOptimizer(this._mustGet(p.graphId).handle)
        return null
      case 'setLR':
        await A.setLR(this._mustGet(p.graphId).handle, JSON.stringify(p.lr))
        return null
      case 'destroy': {
        for (const [id, slot] of Array.from(this.graphs.entries()))
          if (slot.parentGraphId === p.graphId) this.graphs.delete(id)
        const slot = this.graphs.get(p.graphId)
        if (!slot) return null
        this.graphs.delete(p.graphId)
        await A.destroy(slot.handle)  // cascades to the siblings in the library
        return null
      }
      default:
        throw new Error(`unknown request kind: ${req.kind}`)
    }
  }

  // The family a request belongs to, fixed when the request is made: a forward sibling
  // (compileForward) joins its parent's family, every other graph id is its own.
  _familyOf(req) {
    const p = req.payload || {}
    if (req.kind === 'compileForward') {
      const f = this.family.has(p.parentGraphId) ? this.family.get(p.parentGraphId) : p.parentGraphId
      this.family.set(p.graphId, f)
      return f
    }
    if (!this.family.has(p.graphId)) this.family.set(p.graphId, p.graphId)
    return this.family.get(p.graphId)
  }

  // Requests of one family run one after another in arrival order (the reference worker
  // handles its messages in order and chains its dispatches, src/runtime.ts:303-313);
  // families run independently. A failed request does not stop the ones behind it.
  _enqueue(req) {
    const fam = this._familyOf(req)
    const prev = this.queues.has(fam) ? this.queues.get(fam) : Promise.resolve()
    const turn = prev.catch(() => {}).then(() => {
      if (this.terminated) throw new Error('tensorgrad: worker terminated')
      return this._handle(req)
    })
    this.queues.set(fam, turn)
    return turn
  }

  /** Same contract as WorkerProxy.request: resolves with the handler's result, rejects
   *  with an Error whose `name` survives (AbortError for destroyed / replaced graphs).
   *  The native work runs off the JS thread. */
  request(req, transfer) {
    if (this.terminated) return Promise.reject(new Error('tensorgrad: worker has been terminated'))
    return this._enqueue(req)
  }

  send(req, transfer) {
    if (this.terminated) return
    this._enqueue(req).catch(() => { /* fire-and-forget, as WorkerProxy.send */ })
  }

  /** Stops the proxy: requests not yet started reject; each family's runtimes are
   *  destroyed once the request it is running (if any) has finished. Resolves when all
   *  are destroyed. */
  terminate() {
    if (this.terminated) return Promise.resolve()
    this.terminated = true
    const done = []
    const queued = new Set(this.queues.keys())
    for (const [fam, tail] of Array.from(this.queues.entries()))
      done.push(tail.catch(() => {}).then(() => this._destroyWhere(f => f === fam)))
    done.push(this._destroyWhere(f => !queued.has(f)))
    this.queues.clear()
    return Promise.all(done).then(() => undefined)
  }

  async _destroyWhere(pick) {
    for (const [id, slot] of Array.from(this.graphs.entries())) {
      if (!pick(this.family.has(id) ? this.family.get(id) : id)) continue
      this.graphs.delete(id)
      if (slot.parentGraphId === null) await native().destroy(slot.handle)
    }
  }
}

module.exports = { NativeWorkerProxy, toWire, native }

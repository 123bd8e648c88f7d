'use strict'
// Drives training through NativeWorkerProxy exactly as compile.ts drives WorkerProxy:
// createRuntime with a reference-shaped payload, `step` requests, downloadParams,
// a compileForward sibling with a `run`, and destroy. Input: one JSON file
// {payload, steps: [{name: {dtype, data}}], forward: {ir, inputs}}; output: one JSON
// line {losses, params, forward, abortedAfterDestroy}.
const fs = require('fs')
const { NativeWorkerProxy } = require('../../tensorgrad_amd/node/worker_shim.js')

function typed(rec) {
  const out = {}
  for (const k of Object.keys(rec)) {
    const v = rec[k]
    out[k] = v.dtype === 'f32' ? Float32Array.from(v.data) : Int32Array.from(v.data)
  }
  return out
}

async function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], 'utf8'))
  const proxy = new NativeWorkerProxy()
  const p = spec.payload
  const meta = await proxy.request({ kind: 'createRuntime', payload: {
    graphId: 0, ir: p.ir, initialParams: typed(p.initialParams), optimizer: p.optimizer } })
  const losses = []
  for (const s of spec.steps) {
    const r = await proxy.request({ kind: 'step', payload: { graphId: 0, inputs: typed(s) } })
    losses.push(r.loss)
  }
  const dl = await proxy.request({ kind: 'downloadParams', payload: { graphId: 0 } })
  const params = {}
  for (const k of Object.keys(dl.params)) params[k] = Array.from(dl.params[k])
  await proxy.request({ kind: 'compileForward', payload: { graphId: 1, parentGraphId: 0, ir: spec.forward.ir } })
  const run = await proxy.request({ kind: 'run', payload: { graphId: 1, inputs: typed(spec.forward.inputs) } })
  await proxy.request({ kind: 'destroy', payload: { graphId: 0 } })
  let aborted = null
  try {
    await proxy.request({ kind: 'run', payload: { graphId: 1, inputs: typed(spec.forward.inputs) } })
  } catch (e) {
    aborted = e.name
  }
  await proxy.terminate()
  process.stdout.write(JSON.stringify({ paramNames: meta.paramNames, kernelCount: meta.kernelCount, losses, params,
                                        forward: Array.from(run.output), abortedAfterDestroy: aborted }) + '\n')
}

main().catch(e => { process.stderr.write(String(e && e.stack || e) + '\n'); process.exit(1) })

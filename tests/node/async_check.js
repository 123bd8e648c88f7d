'use strict'
// The event loop keeps running while the backend works: a 1 ms setInterval counts ticks
// through createRuntime (IR lowering, kernel compilation, allocation, parameter upload)
// and through the training steps, which run off the JS thread. Input: one JSON file
// {payload, steps: [{name: {dtype, data}}]}; output: one JSON line {createMs,
// createTicks, stepMs, stepTicks, losses, concurrentTicks}.
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
  const steps = spec.steps.map(typed)
  const init = typed(spec.payload.initialParams)
  const proxy = new NativeWorkerProxy()
  let ticks = 0
  const iv = setInterval(() => { ticks++ }, 1)
  let t0 = Date.now(), k0 = ticks
  await proxy.request({ kind: 'createRuntime', payload: {
    graphId: 0, ir: spec.payload.ir, initialParams: init, optimizer: spec.payload.optimizer } })
  const createMs = Date.now() - t0, createTicks = ticks - k0
  const losses = []
  t0 = Date.now()
  k0 = ticks
  for (const s of steps) {
    const r = await proxy.request({ kind: 'step', payload: { graphId: 0, inputs: s } })
    losses.push(r.loss)
  }
  const stepMs = Date.now() - t0, stepTicks = ticks - k0
  // requests made without awaiting run in order, one after another, off the JS thread
  t0 = Date.now()
  k0 = ticks
  const pending = steps.slice(0, 4).map(s => proxy.request({ kind: 'step', payload: { graphId: 0, inputs: s } }))
  const more = (await Promise.all(pending)).map(r => r.loss)
  const concurrentTicks = ticks - k0
  clearInterval(iv)
  await proxy.terminate()
  process.stdout.write(JSON.stringify({ createMs, createTicks, stepMs, stepTicks, losses, more,
                                        concurrentMs: Date.now() - t0, concurrentTicks }) + '\n')
}

main().catch(e => { process.stderr.write(String(e && e.stack || e) + '\n'); process.exit(1) })

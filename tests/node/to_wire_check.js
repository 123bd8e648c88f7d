'use strict'
// Reads createRuntime-shaped payloads ({ir: {graph, plan, kernels}, optimizer}) and
// prints, one line each, the C ABI document toWire derives from them.
const fs = require('fs')
const { toWire } = require('../../tensorgrad_amd/node/worker_shim.js')
for (const f of process.argv.slice(2)) {
  const p = JSON.parse(fs.readFileSync(f, 'utf8'))
  process.stdout.write(JSON.stringify(toWire(p.ir, p.optimizer)) + '\n')
}

'use strict'
// Reads IR documents (one JSON file per argument) and prints, one line each, the launch
// schedule the N-API addon's host-only lowering returns for it.
const fs = require('fs')
const { native } = require('../../tensorgrad_amd/node/worker_shim.js')
for (const f of process.argv.slice(2)) process.stdout.write(native().plan(fs.readFileSync(f, 'utf8')) + '\n')

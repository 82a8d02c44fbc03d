'use strict';
// Runs the JavaScript host on the real Node-API binding (GPU) and prints the
// binding calls it made as JSON (run by tests/test_gpu_js.py).
// usage: node gpu_generate.js <model.gguf> <attention: reference|gemma3>
const path = require('path');
const JS = path.join(__dirname, '..', '..', 'webgpu-gemma_amd', 'js');
const { createGemmaEngine } = require(path.join(JS, 'engine'));

const real = require(path.join(__dirname, '..', '..', 'webgpu-gemma_amd', 'lib', 'gg_napi.node'));
const log = [];
// pass-through to the binding, recording prefill / select / step
const backend = Object.assign({}, real, {
  prefill: async (ctx, ids, pos) => { log.push({ op: 'prefill', ids: Array.from(ids), pos: pos }); return real.prefill(ctx, ids, pos); },
  select: async (ctx, t, p, r, u) => { const id = await real.select(ctx, t, p, r, u); log.push({ op: 'select', t: t, p: p, r: r, u: u, id: id }); return id; },
  step: async (ctx, tok, pos, t, p, r, u) => { const id = await real.step(ctx, tok, pos, t, p, r, u); log.push({ op: 'step', tok: tok, pos: pos, t: t, p: p, r: r, u: u, id: id }); return id; },
  penaltyReset: (ctx) => { log.push({ op: 'penaltyReset' }); return real.penaltyReset(ctx); },
  penaltyAdd: (ctx, ids) => { log.push({ op: 'penaltyAdd', ids: Array.from(ids) }); return real.penaltyAdd(ctx, ids); },
});

let seed = 12345;
function lcg() {   // deterministic uniform draws in [0, 1)
  seed = (Math.imul(seed, 1103515245) + 12345) >>> 0;
  return seed / 4294967296;
}

(async () => {
  const engine = await createGemmaEngine({ model: process.argv[2], attention: process.argv[3], contextLength: 256,
    backend: backend, random: lcg });
  const turns = [];
  engine.addUserMessage('Hello the a');
  let text = '';
  for await (const s of engine.generate({ temperature: 0, maxTokens: 12 })) text += s;
  turns.push(text);
  engine.addUserMessage('a the');
  text = '';
  for await (const s of engine.generate({ temperature: 0.7, topP: 0.9, repPenalty: 1.2, maxTokens: 16 })) text += s;
  turns.push(text);
  console.log(JSON.stringify({ log: log, turns: turns, kvPosition: engine.kvPosition }));
  engine.dispose();
})().catch((e) => {
  console.error(e && e.stack ? e.stack : e, e && e.code);
  process.exit(1);
});

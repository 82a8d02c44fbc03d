'use strict';
// Runs the JavaScript host on the real Node-API binding (GPU) and prints the
// binding calls it made as JSON (run by tests/test_gpu_js.py).
// usage: node gpu_generate.js <model.gguf> <attention: reference|gemma3>
const path = require('path');
const JS = path.join(__dirname, '..', '..', 'webgpu-gemma_amd', 'js');
const { createGemmaEngine } = require(path.join(JS, 'engine'));

const real = require(path.join(__dirname, '..', '..', 'webgpu-gemma_amd', 'lib', 'gg_napi.node'));
const log = [];
// pass-through to the binding, recording prefill / select / step; a queued
// step (stepSubmit / stepCollect) is logged as a step with its input id
// resolved (-1: the id of the step before it) once it is collected
const pending = [];
let lastId = -1;
const backend = Object.assign({}, real, {
  stepSubmit: (ctx, tok, pos, t, p, r, u) => {
    real.stepSubmit(ctx, tok, pos, t, p, r, u);
    pending.push({ op: 'step', tok: tok, pos: pos, t: t, p: p, r: r, u: u });
  },
  stepCollect: async (ctx) => {
    const id = await real.stepCollect(ctx);
    const c = pending.shift();
    if (c.tok < 0) c.tok = lastId;
    c.id = id;
    c.queued = true;
    lastId = id;
    log.push(c);
    return id;
  },
  prefill: async (ctx, ids, pos) => { log.push({ op: 'prefill', ids: Array.from(ids), pos: pos }); return real.prefill(ctx, ids, pos); },
  select: async (ctx, t, p, r, u) => { const id = await real.select(ctx, t, p, r, u); lastId = id; log.push({ op: 'select', t: t, p: p, r: r, u: u, id: id }); return id; },
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
  // a step at or past the turn's final kvPosition was queued ahead and dropped
  const markDropped = () => { for (const c of log) if (c.op === 'step' && c.pos >= engine.kvPosition) c.dropped = true; };
  engine.addUserMessage('Hello the a');
  let text = '';
  for await (const s of engine.generate({ temperature: 0, maxTokens: 12 })) text += s;
  turns.push(text);
  markDropped();
  engine.addUserMessage('a the');
  text = '';
  for await (const s of engine.generate({ temperature: 0.7, topP: 0.9, repPenalty: 1.2, maxTokens: 16 })) text += s;
  turns.push(text);
  markDropped();
  console.log(JSON.stringify({ log: log, turns: turns, kvPosition: engine.kvPosition }));
  engine.dispose();
})().catch((e) => {
  console.error(e && e.stack ? e.stack : e, e && e.code);
  process.exit(1);
});

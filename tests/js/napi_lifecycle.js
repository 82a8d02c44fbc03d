'use strict';
// Context lifetime of the Node-API binding (gg_napi.c) over a stub libgg
// whose prefill/select/step/stepCollect sleep: a second job on a busy context is refused
// with GG_ERR_INVALID, destroy() during a step is deferred until the step's
// completion, calls on a destroyed context are refused, and a context whose
// JavaScript handle is garbage-collected during a step is destroyed after it.
// The stub aborts on any use after destroy or overlapping call.
// usage: node --expose-gc napi_lifecycle.js <dir holding gg_napi.node>
const path = require('path');
const gg = require(path.join(process.argv[2], 'gg_napi.node'));

function expectCode(fn, code, what) {
  try {
    fn();
  } catch (e) {
    if (e.code !== code) throw new Error(what + ': expected ' + code + ', got ' + e.code + ' ' + e.message);
    return e;
  }
  throw new Error(what + ': expected an error');
}

const tick = () => new Promise((r) => setImmediate(r));
const sleep = (ms) => new Promise((r) => setTimeout(r, ms));

async function main() {
  const a = gg.create({ hidden_size: 8 });
  gg.finalize(a);

  // two jobs at once: the second is refused, the first completes
  const p1 = gg.step(a, 41, 0, 0, 1, 1, 0.5);
  expectCode(() => gg.step(a, 1, 1, 0, 1, 1, 0.5), 'GG_ERR_INVALID', 'second step');
  expectCode(() => gg.select(a, 0, 1, 1, 0.5), 'GG_ERR_INVALID', 'select while busy');
  expectCode(() => gg.read(a, 0, 0, new Float32Array(4)), 'GG_ERR_INVALID', 'read while busy');
  expectCode(() => gg.resetKV(a), 'GG_ERR_INVALID', 'resetKV while busy');
  if ((await p1) !== 42) throw new Error('step result');
  console.log('ok busy');

  // destroy() while a step runs: deferred to the step's completion
  const p2 = gg.step(a, 9, 1, 0, 1, 1, 0.5);
  await sleep(50);
  gg.destroy(a);
  expectCode(() => gg.step(a, 1, 2, 0, 1, 1, 0.5), 'GG_ERR_INVALID', 'step after destroy');
  if ((await p2) !== 10) throw new Error('step result after destroy');
  expectCode(() => gg.prefill(a, new Int32Array([1, 2]), 0), 'GG_ERR_INVALID', 'prefill after destroy');
  gg.destroy(a);  // a second destroy is a no-op
  console.log('ok destroy mid-step');

  // prefill then destroy right away, before the worker has started
  const b = gg.create({ hidden_size: 8 });
  const p3 = gg.prefill(b, new Int32Array([1, 2, 3]), 0);
  gg.destroy(b);
  await p3;
  console.log('ok destroy before start');

  // the handle is garbage-collected while its step runs
  let c = gg.create({ hidden_size: 8 });
  const p4 = gg.step(c, 99, 0, 0, 1, 1, 0.5);
  c = null;
  for (let i = 0; i < 5; ++i) {
    global.gc();
    await tick();
  }
  if ((await p4) !== 100) throw new Error('step result after gc');
  for (let i = 0; i < 5; ++i) {
    global.gc();
    await tick();
  }
  console.log('ok gc mid-step');

  // pipelined steps: stepSubmit is synchronous, stepCollect a job (the context
  // is busy until it completes), destroy() during a collect is deferred
  const d = gg.create({ hidden_size: 8 });
  gg.stepSubmit(d, 5, 0, 0, 1, 1, 0.5);
  const p5 = gg.stepCollect(d);
  expectCode(() => gg.stepSubmit(d, -1, 1, 0, 1, 1, 0.5), 'GG_ERR_INVALID', 'submit while a collect runs');
  if ((await p5) !== 6) throw new Error('collected id');
  gg.stepSubmit(d, -1, 1, 0, 1, 1, 0.5);
  const p6 = gg.stepCollect(d);
  await sleep(50);
  gg.destroy(d);
  if ((await p6) !== 7) throw new Error('collected id after destroy');
  expectCode(() => gg.stepSubmit(d, 1, 2, 0, 1, 1, 0.5), 'GG_ERR_INVALID', 'submit after destroy');
  console.log('ok pipelined steps');
  console.log('lifecycle passed');
}

main().catch((e) => {
  console.log('FAILED: ' + (e && e.stack ? e.stack : e));
  process.exit(1);
});

'use strict';
// CPU tests of the JavaScript host (run by tests/test_js_host.py):
// tokenizer, chat template, GGUF reader, and the generate() turn logic of
// engine.js against a recording fake of the Node-API binding.
// usage: node host_tests.js <tiny.gguf> <expect.json>
const assert = require('assert');
const fs = require('fs');
const path = require('path');

const JS = path.join(__dirname, '..', '..', 'webgpu-gemma_amd', 'js');
const { Tokenizer } = require(path.join(JS, 'tokenizer'));
const { buildChatPrompt, turnSuffix } = require(path.join(JS, 'conversation'));
const gguf = require(path.join(JS, 'gguf'));
const { createGemmaEngine } = require(path.join(JS, 'engine'));

const ggufPath = process.argv[2];
const expect = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
const results = [];
async function test(name, fn) {
  await fn();
  results.push(name);
  console.log('ok', name);
}

// ---- tokenizer (tokenizer.ts semantics) ----------------------------------
function vocab() {
  const v = [];
  for (let i = 0; i < 300; i++) v.push('<unused' + i + '>');
  v[0] = '<pad>'; v[1] = '<eos>'; v[2] = '<bos>'; v[105] = '<start_of_turn>'; v[106] = '<end_of_turn>';
  const words = ['▁', '▁the', '▁th', '▁t', 'h', 'e', '▁Hello', 'Hello', '▁world', 'user', 'model', '\n', '?',
    '▁a', 'a', '<end_function_call>', 'x', 'xx'];
  words.forEach((w, i) => { v[200 + i] = w; });
  return v;
}
const W = (w) => 200 + ['▁', '▁the', '▁th', '▁t', 'h', 'e', '▁Hello', 'Hello', '▁world', 'user', 'model', '\n', '?',
  '▁a', 'a', '<end_function_call>', 'x', 'xx'].indexOf(w);

async function tokenizerTests() {
  const tk = new Tokenizer(vocab());
  await test('tokenizer: BOS, leading space marker, longest match', () => {
    assert.deepStrictEqual(tk.encode('the'), [2, W('▁the')]);
    assert.deepStrictEqual(tk.encode('Hello world'), [2, W('▁Hello'), W('▁world')]);
    assert.deepStrictEqual(tk.encode('thee'), [2, W('▁the'), W('e')]);
  });
  await test('tokenizer: unknown characters are dropped', () => {
    assert.deepStrictEqual(tk.encode('the#'), [2, W('▁the')]);
    assert.deepStrictEqual(tk.encode('#'), [2, W('▁')]);
  });
  await test('tokenizer: special tokens split first, no space marker after one', () => {
    assert.deepStrictEqual(tk.encode('<start_of_turn>user\nHello<end_of_turn>'),
      [2, 105, W('user'), W('\n'), W('Hello'), 106]);
    assert.deepStrictEqual(tk.encode('a<eos>a'), [2, W('▁a'), 1, W('a')]);
  });
  await test('tokenizer: function tokens become specials when in the vocabulary', () => {
    assert.strictEqual(tk.funcTokens['<end_function_call>'], W('<end_function_call>'));
    // '▁x' is not in the vocabulary: '▁' then 'x'; no marker after the special
    assert.deepStrictEqual(tk.encode('x<end_function_call>x'), [2, W('▁'), W('x'), W('<end_function_call>'), W('x')]);
  });
  await test('tokenizer: decode maps the space marker back', () => {
    assert.strictEqual(tk.decodeTokens([W('▁Hello'), W('▁world'), W('?')]), ' Hello world?');
    assert.strictEqual(tk.decodeToken(99999), '<unk:99999>');
  });
}

// ---- chat template (conversation.ts) --------------------------------------
async function templateTests() {
  await test('chat template: turns and the model opening', () => {
    const p = buildChatPrompt([{ role: 'user', text: 'Hi' }, { role: 'model', text: 'Yo' },
      { role: 'user', text: 'Again' }], '[]');
    assert.strictEqual(p, '<start_of_turn>user\nHi<end_of_turn>\n<start_of_turn>model\nYo<end_of_turn>\n' +
      '<start_of_turn>user\nAgain<end_of_turn>\n<start_of_turn>model\n');
    assert.strictEqual(turnSuffix('Q'), '<end_of_turn>\n<start_of_turn>user\nQ<end_of_turn>\n<start_of_turn>model\n');
  });
  await test('chat template: tool declarations', () => {
    const tools = JSON.stringify([{ name: 'f', description: 'd', parameters: { type: 'OBJECT',
      properties: { a: { description: 'da', type: 'STRING', enum: ['x', 'y'] } }, required: ['a'] } }]);
    const p = buildChatPrompt([{ role: 'user', text: 'u' }], tools);
    assert.strictEqual(p, '<start_of_turn>developer\nYou are a model that can do function calling with the ' +
      'following functions\n<start_function_declaration>declaration:f{description:<escape>d<escape>,' +
      'parameters:{properties:{a:{description:<escape>da<escape>,type:<escape>STRING<escape>,enum:[<escape>x' +
      '<escape>,<escape>y<escape>]}},required:[<escape>a<escape>],type:<escape>OBJECT<escape>}}' +
      '<end_function_declaration>\n<end_of_turn>\n<start_of_turn>user\nu<end_of_turn>\n<start_of_turn>model\n');
    assert.strictEqual(buildChatPrompt([], 'not json'), '<start_of_turn>model\n');
  });
}

// ---- GGUF reader ------------------------------------------------------------
async function ggufTests() {
  await test('gguf: header, tensor table, data offset and bytes', () => {
    const fd = fs.openSync(ggufPath, 'r');
    const g = gguf.parseHeader(fd);
    assert.strictEqual(g.version, 3);
    assert.strictEqual(g.dataOffset, expect.data_offset);
    assert.strictEqual(g.tensors.length, expect.tensors.length);
    for (let i = 0; i < g.tensors.length; i++) {
      const t = g.tensors[i], e = expect.tensors[i];
      assert.strictEqual(t.name, e.name);
      assert.deepStrictEqual(t.dims, e.dims);
      assert.strictEqual(t.type, e.type);
      assert.strictEqual(t.offset, e.offset);
      assert.strictEqual(gguf.tensorByteSize(t), e.nbytes);
      const b = gguf.readTensor(fd, g, t);
      assert.strictEqual(require('crypto').createHash('sha256').update(b).digest('hex'), e.sha256);
    }
    const c = gguf.configFromGGUF(g, require(path.join(JS, 'engine')).defaultConfig(), 4096);
    assert.strictEqual(c.hidden_size, expect.hidden);
    assert.strictEqual(c.num_layers, expect.layers);
    assert.strictEqual(c.intermediate_size, expect.inter);
    assert.strictEqual(c.context_length, Math.min(expect.file_ctx, 4096));
    assert.strictEqual(c.vocab_size, expect.vocab);
    assert.strictEqual(c.file_rope_theta, expect.rope_base);
    assert.strictEqual(c.file_rope_theta_swa, expect.rope_base_swa);
    fs.closeSync(fd);
  });
}

// ---- engine turn logic against a fake binding -------------------------------
class FakeGG {
  constructor(script) {
    this.calls = [];
    this.script = script.slice();   // ids returned by select/step in order
    this.failOn = null;
  }
  rec(name, args) {
    this.calls.push([name].concat(args));
    if (this.failOn === name) {
      const e = new Error('device gone');
      e.code = 'GG_ERR_DEVICE_LOST';
      throw e;
    }
  }
  create(cfg) { this.rec('create', [cfg]); return { live: true }; }
  upload(ctx, name, type, dims, bytes) { this.rec('upload', [name, type, dims.slice(), bytes.length]); }
  finalize() { this.rec('finalize', []); }
  penaltyReset() { this.rec('penaltyReset', []); }
  penaltyAdd(ctx, ids) { this.rec('penaltyAdd', [Array.from(ids)]); }
  resetKV() { this.rec('resetKV', []); }
  destroy() { this.rec('destroy', []); }
  async prefill(ctx, ids, pos) { this.rec('prefill', [Array.from(ids), pos]); }
  async select(ctx, t, p, r, u) { this.rec('select', [t, p, r, u]); return this.script.shift(); }
  async step(ctx, tok, pos, t, p, r, u) { this.rec('step', [tok, pos, t, p, r, u]); return this.script.shift(); }
}

// Fakes whose step results depend only on the position (a table), so a
// sequential and a pipelined run of the same turn see the same ids.
class TableGG extends FakeGG {
  constructor(first, table) {
    super([]);
    this.first = first.slice();   // the id select() returns, per turn
    this.table = table;           // pos -> id of the step at pos
  }
  async select(ctx, t, p, r, u) { this.rec('select', [t, p, r, u]); return this.first.shift(); }
  async step(ctx, tok, pos, t, p, r, u) { this.rec('step', [tok, pos, t, p, r, u]); return this.table(pos); }
}
class PipeGG extends TableGG {
  constructor(first, table) {
    super(first, table);
    this.queue = [];
    this.last = -1;
  }
  select(ctx, t, p, r, u) {
    return super.select(ctx, t, p, r, u).then((id) => { this.last = id; return id; });
  }
  stepSubmit(ctx, tok, pos, t, p, r, u) {
    assert.ok(this.queue.length < 2, 'at most two steps outstanding');
    const input = tok < 0 ? this.last : tok;   // -1: the previous step's id, "on the device"
    this.rec('step', [input, pos, t, p, r, u]);
    this.last = this.table(pos);
    this.queue.push(this.last);
  }
  async stepCollect() { this.rec('collect', []); return this.queue.shift(); }
}

async function collect(gen) {
  const out = [];
  for await (const s of gen) out.push(s);
  return out;
}

async function engineTests() {
  const mk = async (script, extra) => {
    const gg = new FakeGG(script);
    const progress = [];
    let draws = 0;
    const e = await createGemmaEngine(Object.assign({ model: ggufPath, backend: gg, contextLength: 64,
      onProgress: (p) => progress.push(p), random: () => { draws++; return 0.25; } }, extra || {}));
    return { e: e, gg: gg, progress: progress, draws: () => draws };
  };
  await test('engine: init streams every tensor and reports progress', async () => {
    const { gg, progress } = await mk([]);
    const ups = gg.calls.filter((c) => c[0] === 'upload');
    assert.strictEqual(ups.length, expect.tensors.length);
    const total = expect.tensors.reduce((a, t) => a + t.nbytes, 0);
    assert.strictEqual(progress[progress.length - 1].loaded, total);
    assert.strictEqual(progress[progress.length - 1].total, total);
    const cfg = gg.calls[0][1];
    assert.strictEqual(cfg.vocab_size, expect.vocab);
    assert.strictEqual(cfg.context_length, 64);
    assert.strictEqual(gg.calls[gg.calls.length - 1][0], 'finalize');
  });
  await test('engine: model keys resolve to the reference\'s file names in modelDir', async () => {
    const os = require('os');
    const { MODEL_FILES } = require(path.join(JS, 'engine'));
    assert.deepStrictEqual(Object.keys(MODEL_FILES).sort(), ['1b', '270m', 'func']);
    const dir = fs.mkdtempSync(path.join(os.tmpdir(), 'gg-models-'));
    try {
      fs.symlinkSync(path.resolve(ggufPath), path.join(dir, 'gemma-3-270m-it-Q8_0.gguf'));
      const gg = new FakeGG([]);
      await createGemmaEngine({ model: '270m', modelDir: dir, backend: gg, contextLength: 64 });
      assert.strictEqual(gg.calls[0][0], 'create');
      await assert.rejects(createGemmaEngine({ model: '1b', modelDir: dir, backend: new FakeGG([]) }),
        /model file not found: .*gemma-3-1b-it-Q8_0\.gguf/);
      await assert.rejects(createGemmaEngine({ model: 'https://example.invalid/m.gguf', backend: new FakeGG([]) }),
        /model URLs are not fetched/);
      const saved = process.env.GEMMA_MODEL_DIR;
      process.env.GEMMA_MODEL_DIR = dir;
      try {
        const gg2 = new FakeGG([]);
        await createGemmaEngine({ model: '270m', backend: gg2, contextLength: 64 });
        assert.strictEqual(gg2.calls[gg2.calls.length - 1][0], 'finalize');
      } finally {
        if (saved === undefined) delete process.env.GEMMA_MODEL_DIR;
        else process.env.GEMMA_MODEL_DIR = saved;
      }
    } finally {
      fs.unlinkSync(path.join(dir, 'gemma-3-270m-it-Q8_0.gguf'));
      fs.rmdirSync(dir);
    }
  });
  await test('engine: batched MFMA prefill by default; a negative prefillBatch keeps the token-by-token order', async () => {
    assert.strictEqual((await mk([])).gg.calls[0][1].prefill_batch, 64);   // whole prompt, capped by the context
    assert.strictEqual((await mk([], { prefillBatch: 48 })).gg.calls[0][1].prefill_batch, 48);
    assert.strictEqual((await mk([], { prefillBatch: -1 })).gg.calls[0][1].prefill_batch, 0);
  });
  await test('engine: create() gets the file\'s rope bases (one base in reference mode)', async () => {
    const ref = (await mk([])).gg.calls[0][1];
    assert.strictEqual(ref.rope_theta_global, expect.rope_base);
    assert.strictEqual(ref.rope_theta_local, expect.rope_base);
    assert.strictEqual(ref.sliding_window, 0);
    const g3 = (await mk([], { attention: 'gemma3' })).gg.calls[0][1];
    assert.strictEqual(g3.rope_theta_global, expect.rope_base);
    assert.strictEqual(g3.rope_theta_local, expect.rope_base_swa);
    assert.strictEqual(g3.sliding_window, 512);
  });
  await test('engine: first turn prefill, first id from select, steps at kvPosition + writes, stop id', async () => {
    const { e, gg, draws } = await mk([210, 211, 212, 106]);
    e.addUserMessage('Hello');
    const out = await collect(e.generate({ temperature: 0.7, topP: 0.9, repPenalty: 1.2 }));
    const prompt = e.tokenizer.encode(buildChatPrompt([{ role: 'user', text: 'Hello' }], '[]'));
    const pf = gg.calls.find((c) => c[0] === 'prefill');
    assert.deepStrictEqual(pf.slice(1), [prompt, 0]);
    const steps = gg.calls.filter((c) => c[0] === 'step');
    assert.deepStrictEqual(steps.map((s) => [s[1], s[2]]),
      [[210, prompt.length], [211, prompt.length + 1], [212, prompt.length + 2]]);
    assert.deepStrictEqual(out, [210, 211, 212].map((id) => e.tokenizer.decodeToken(id)));
    assert.strictEqual(e.kvPosition, prompt.length + 3);    // the stop id is not written
    assert.strictEqual(draws(), 4);                         // one draw per selection when sampling
    const pa = gg.calls.filter((c) => c[0] === 'penaltyAdd');
    assert.deepStrictEqual(pa[0][1], prompt);               // the turn's prompt seeds the penalty set
  });
  await test('engine: second turn sends the suffix without BOS at kvPosition and rescopes the penalty set', async () => {
    const { e, gg } = await mk([210, 106, 220, 221, 1]);
    e.addUserMessage('Hello');
    await collect(e.generate({ temperature: 0 }));
    const kv1 = e.kvPosition;
    e.addUserMessage('the');
    await collect(e.generate({ temperature: 0 }));
    const pfs = gg.calls.filter((c) => c[0] === 'prefill');
    const suffix = e.tokenizer.encode(turnSuffix('the')).slice(1);
    assert.deepStrictEqual(pfs[1].slice(1), [suffix, kv1]);
    const resets = gg.calls.filter((c) => c[0] === 'penaltyReset');
    assert.strictEqual(resets.length, 2);
    assert.deepStrictEqual(gg.calls.filter((c) => c[0] === 'penaltyAdd')[1][1], suffix);
    assert.strictEqual(e.kvPosition, kv1 + suffix.length + 2);
    assert.strictEqual(e.conversationHistory.length, 4);
  });
  await test('engine: greedy takes no random draw', async () => {
    const { e, draws } = await mk([210, 211, 106]);
    e.addUserMessage('Hello');
    await collect(e.generate({ temperature: 0 }));
    assert.strictEqual(draws(), 0);
  });
  await test('engine: maxTokens, abort signal and end of context stop the loop', async () => {
    let r = await mk([210, 211, 212, 213, 214]);
    r.e.addUserMessage('Hello');
    assert.strictEqual((await collect(r.e.generate({ maxTokens: 2 }))).length, 2);
    r = await mk([210, 211, 212]);
    r.e.addUserMessage('Hello');
    assert.strictEqual((await collect(r.e.generate({ signal: { aborted: true } }))).length, 1);
    r = await mk(new Array(100).fill(210));
    r.e.addUserMessage('Hello');
    await collect(r.e.generate({}));
    const last = r.gg.calls.filter((c) => c[0] === 'step').pop();
    assert.strictEqual(last[2], 64 - 2);      // pos >= contextLength - 1 ends the turn
  });
  await test('engine: the pipelined loop (one step queued ahead) matches the sequential loop', async () => {
    const endCall = W('<end_function_call>');
    const scenarios = [
      { name: 'stop id', opts: { temperature: 0 }, table: (p) => (p === 20 ? 106 : 210 + (p % 5)) },
      { name: 'function call end', opts: { temperature: 0 }, table: (p) => (p === 18 ? endCall : 211) },
      { name: 'maxTokens', opts: { temperature: 0.7, maxTokens: 4 }, table: () => 212 },
      { name: 'end of context', opts: { temperature: 0 }, table: () => 213 },
      { name: 'abort after two ids', opts: { temperature: 0 }, table: () => 214, abortAfter: 2 },
    ];
    let dropped = 0;
    for (const sc of scenarios) {
      const runs = [];
      for (const Kind of [TableGG, PipeGG]) {
        const gg = new Kind([215, 216], sc.table);
        let draws = 0;
        const e = await createGemmaEngine({ model: ggufPath, backend: gg, contextLength: 64,
          random: () => { draws++; return 0.25; } });
        const outs = [];
        for (const text of ['Hello', 'the']) {
          e.addUserMessage(text);
          const signal = { aborted: false };
          const got = [];
          for await (const s of e.generate(Object.assign({ signal: signal }, sc.opts))) {
            got.push(s);
            if (sc.abortAfter && got.length === sc.abortAfter) signal.aborted = true;
          }
          outs.push({ got: got, kv: e.kvPosition });
        }
        const steps = gg.calls.filter((c) => c[0] === 'step').map((c) => [c[1], c[2]]);
        const collects = gg.calls.filter((c) => c[0] === 'collect').length;
        runs.push({ outs: outs, steps: steps, collects: collects, draws: draws, pipe: Kind === PipeGG });
      }
      const [seq, pipe] = runs;
      assert.deepStrictEqual(pipe.outs, seq.outs, sc.name);
      // every sequential step appears, in order, with its input id and position; the
      // pipelined run adds at most one queued step per turn, collected and dropped
      let i = 0;
      const extra = [];
      for (const st of pipe.steps) {
        if (i < seq.steps.length && st[0] === seq.steps[i][0] && st[1] === seq.steps[i][1]) i++;
        else extra.push(st);
      }
      assert.strictEqual(i, seq.steps.length, sc.name + ': sequential steps missing');
      assert.ok(extra.length <= 2, sc.name + ': at most one dropped step per turn');
      assert.strictEqual(pipe.collects, pipe.steps.length, sc.name + ': every queued step is collected');
      if (sc.opts.temperature > 0) assert.strictEqual(pipe.draws, seq.draws + extra.length, sc.name);
      assert.ok(pipe.steps.length > 0, sc.name);
      dropped += extra.length;
    }
    assert.ok(dropped > 0);   // the queued-ahead path ran and dropped its extra steps
  });
  await test('engine: a generator left unfinished has its queued step collected before the next call', async () => {
    const gg = new PipeGG([215, 216], () => 211);
    const e = await createGemmaEngine({ model: ggufPath, backend: gg, contextLength: 64 });
    e.addUserMessage('Hello');
    const it = e.generate({ temperature: 0 });
    await it.next();
    await it.next();                   // a step is queued; the generator is then abandoned
    assert.strictEqual(gg.queue.length, 1);
    e.resetConversation();             // the KV reset waits for the queued step
    assert.strictEqual(gg.calls.filter((c) => c[0] === 'resetKV').length, 0);
    e.addUserMessage('the');
    const out = await collect(e.generate({ temperature: 0, maxTokens: 3 }));
    assert.strictEqual(out.length, 3);
    assert.strictEqual(gg.queue.length, 0);
    assert.strictEqual(gg.calls.filter((c) => c[0] === 'resetKV').length, 1);
    const pfs = gg.calls.filter((c) => c[0] === 'prefill');
    assert.strictEqual(pfs[1][2], 0);  // a fresh conversation from position 0
  });
  await test('engine: on the graph path (decodePath 0) generate() steps one at a time, never queued', async () => {
    const seq = new TableGG([215, 216], (p) => (p === 20 ? 106 : 211));
    const gg = new PipeGG([215, 216], (p) => (p === 20 ? 106 : 211));
    gg.decodePath = () => 0;   // stepSubmit would run each step synchronously
    const outs = [];
    for (const b of [seq, gg]) {
      const e = await createGemmaEngine({ model: ggufPath, backend: b, contextLength: 64 });
      e.addUserMessage('Hello');
      outs.push(await collect(e.generate({ temperature: 0 })));
    }
    assert.deepStrictEqual(outs[1], outs[0]);
    assert.strictEqual(gg.calls.filter((c) => c[0] === 'collect').length, 0);
    assert.deepStrictEqual(gg.calls.filter((c) => c[0] === 'step'), seq.calls.filter((c) => c[0] === 'step'));
    gg.decodePath = () => 1;   // the persistent kernel: queued again
    const e = await createGemmaEngine({ model: ggufPath, backend: gg, contextLength: 64 });
    e.addUserMessage('Hello');
    await collect(e.generate({ temperature: 0 }));
    assert.ok(gg.calls.filter((c) => c[0] === 'collect').length > 0);
  });
  await test('engine: context overflow resets the KV cache and keeps only the last user message', async () => {
    const { e, gg } = await mk([210, 106, 210, 106]);
    e.addUserMessage('Hello');
    await collect(e.generate({}));
    e.addUserMessage(new Array(40).fill('the').join(' '));
    await collect(e.generate({}));
    assert.strictEqual(gg.calls.filter((c) => c[0] === 'resetKV').length, 1);
    const pfs = gg.calls.filter((c) => c[0] === 'prefill');
    assert.strictEqual(pfs[1][2], 0);
    assert.strictEqual(pfs[1][1][0], 2);       // a fresh prompt with BOS
  });
  await test('engine: device loss surfaces as deviceLost and blocks generate', async () => {
    const { e, gg } = await mk([210, 211]);
    gg.failOn = 'step';
    e.addUserMessage('Hello');
    await assert.rejects(() => collect(e.generate({})), /device gone/);
    assert.strictEqual(e.deviceLost, true);
    await assert.rejects(() => collect(e.generate({})), /device lost/);
  });
  await test('engine: resetConversation and dispose', async () => {
    const { e, gg } = await mk([210, 106]);
    e.addUserMessage('Hello');
    await collect(e.generate({}));
    e.resetConversation();
    assert.strictEqual(e.kvPosition, 0);
    assert.strictEqual(e.conversationHistory.length, 0);
    e.dispose();
    assert.strictEqual(gg.calls[gg.calls.length - 1][0], 'destroy');
  });
}

(async () => {
  await tokenizerTests();
  await templateTests();
  await ggufTests();
  await engineTests();
  console.log('passed', results.length);
})().catch((e) => {
  console.error(e && e.stack ? e.stack : e);
  process.exit(1);
});

'use strict';
// The JavaScript host: the reference's public engine API (index.ts:34-38,
// types.ts:86-97, engine.ts:31-1078) over the libgg.so C-ABI through the
// Node-API binding (gg_napi.node). The WebGPU device, pipelines, buffers and
// bind groups of engine.ts are replaced by one context of the binding; what
// stays here is what stays in JavaScript in the reference: GGUF parsing, the
// tokenizer, the chat template, conversation / KV-position bookkeeping, stop
// ids, the Math.random() draw and the per-turn penalty set.
const fs = require('fs');
const path = require('path');

const gguf = require('./gguf');
const { Tokenizer } = require('./tokenizer');
const { buildChatPrompt, turnSuffix } = require('./conversation');

const GG_ATTN_REFERENCE = 0;
const GG_ATTN_GEMMA3 = 1;

// Defaults of types.ts:19-36 (Gemma-3 270M), updated from the GGUF.
function defaultConfig() {
  return {
    hidden_size: 640, q_dim: 1024, kv_dim: 256, num_q_heads: 4, num_kv_heads: 1, head_dim: 256,
    intermediate_size: 2048, vocab_size: 262144, num_layers: 18, context_length: 2048,
    rms_norm_eps: 1e-6, rope_theta_global: 1000000.0, rope_theta_swa: 1000000.0, swa_period: 6,
    sliding_window: 0,
  };
}

// The reference's model keys (engine.ts:24-28, options.model in types.ts:51)
// name these Q8_0 files; with no network they are looked up in a local
// directory (options.modelDir, else $GEMMA_MODEL_DIR, else the working
// directory) instead of fetched. Any other model string is a file path.
const MODEL_FILES = {
  '1b': 'gemma-3-1b-it-Q8_0.gguf',
  '270m': 'gemma-3-270m-it-Q8_0.gguf',
  'func': 'functiongemma-270m-it-Q8_0.gguf',
};

function resolveModel(options) {
  const key = options.model || '1b';
  if (/^[a-z]+:\/\//i.test(key)) {
    throw new Error('model URLs are not fetched: download the .gguf and pass its path, or a model key ' +
                    'with modelDir: ' + key);
  }
  if (Object.prototype.hasOwnProperty.call(MODEL_FILES, key)) {
    const dir = options.modelDir || process.env.GEMMA_MODEL_DIR || process.cwd();
    return path.join(dir, MODEL_FILES[key]);
  }
  return key;
}

function loadBinding(dir) {
  const p = path.join(dir || path.join(__dirname, '..', 'lib'), 'gg_napi.node');
  return require(p);   // throws when the HIP library or the binding is missing
}

class GemmaEngineImpl {
  constructor(options) {
    this.config = defaultConfig();
    if (options.contextLength) this.config.context_length = options.contextLength;
    this.onProgress = options.onProgress;
    this.gg = options.backend || loadBinding(options.bindingDir);
    this.random = options.random || Math.random;
    // 'reference' (one theta, full attention: src/ as shipped) or 'gemma3'
    // (local layers: theta 1e4, 512-position window)
    this.attention = options.attention || 'reference';
    // rows per batched MFMA prefill slice: unset or 0 = the whole prompt
    // (at most 4096 rows per slice); a negative value keeps the reference's
    // token-by-token prefill (engine.ts:923-928)
    this.prefillBatch = options.prefillBatch || 0;
    this.ctx = null;
    this.conversationHistory = [];
    this.kvPosition = 0;
    this.deviceLost = false;
    this.inflight = 0;          // steps queued ahead and not yet collected
    this.resetPending = false;  // resetConversation() while a step was queued
  }

  reportProgress(loaded, total, status) {
    if (this.onProgress) this.onProgress({ loaded: loaded, total: total, status: status });
  }

  // init(): the model is a key of MODEL_FILES or the path of a local .gguf
  // file; tensors stream from the file to the device one at a time.
  async init(options) {
    const file = resolveModel(options);
    if (!fs.existsSync(file)) throw new Error('model file not found: ' + file);
    const fd = fs.openSync(file, 'r');
    try {
      this.reportProgress(0, 1, 'Reading header...');
      const g = gguf.parseHeader(fd);
      const cfg = gguf.configFromGGUF(g, this.config, options.contextLength);
      const emb = g.tensors.find((t) => t.name === 'token_embd.weight');
      if (!emb) throw new Error('GGUF has no token_embd.weight');
      cfg.vocab_size = emb.dims[1];
      // The file's rope base replaces the 1e6 default of types.ts:32-33 on
      // every layer (reference mode keeps one base, as types.ts does); in
      // gemma3 mode local layers take the file's sliding-window base, else 1e4.
      if (cfg.file_rope_theta) {
        cfg.rope_theta_global = cfg.file_rope_theta;
        cfg.rope_theta_swa = cfg.file_rope_theta;
      }
      if (this.attention === 'gemma3') {
        cfg.rope_theta_swa = cfg.file_rope_theta_swa || 10000.0;
        cfg.sliding_window = cfg.file_sliding_window || 512;
      }
      this.config = cfg;
      this.tokenizer = Tokenizer.fromGGUF(g);
      this.ctx = this.call(() => this.gg.create({
        hidden_size: cfg.hidden_size, num_layers: cfg.num_layers, num_q_heads: cfg.num_q_heads,
        num_kv_heads: cfg.num_kv_heads, head_dim: cfg.head_dim, intermediate_size: cfg.intermediate_size,
        vocab_size: cfg.vocab_size, context_length: cfg.context_length, rms_norm_eps: cfg.rms_norm_eps,
        rope_theta_global: cfg.rope_theta_global, rope_theta_local: cfg.rope_theta_swa,
        swa_period: cfg.swa_period, sliding_window: cfg.sliding_window,
        attention_mode: this.attention === 'gemma3' ? GG_ATTN_GEMMA3 : GG_ATTN_REFERENCE,
        prefill_batch: this.prefillBatch < 0 ? 0
          : this.prefillBatch > 0 ? this.prefillBatch : Math.min(4096, cfg.context_length),
      }));
      const total = g.tensors.reduce((a, t) => a + gguf.tensorByteSize(t), 0);
      let loaded = 0;
      for (const t of g.tensors) {
        const bytes = gguf.readTensor(fd, g, t);
        this.call(() => this.gg.upload(this.ctx, t.name, t.type, t.dims, bytes));
        loaded += bytes.length;
        this.reportProgress(loaded, total, 'Uploading weights...');
      }
      this.call(() => this.gg.finalize(this.ctx));
      this.reportProgress(total, total, 'Ready');
    } finally {
      fs.closeSync(fd);
    }
  }

  // Failures of the binding: GG_ERR_DEVICE_LOST sets deviceLost (engine.ts:134-137).
  call(fn) {
    try {
      return fn();
    } catch (e) {
      this.noteError(e);
      throw e;
    }
  }

  async callAsync(fn) {
    try {
      return await fn();
    } catch (e) {
      this.noteError(e);
      throw e;
    }
  }

  noteError(e) {
    if (e && e.code === 'GG_ERR_DEVICE_LOST') this.deviceLost = true;
  }

  addUserMessage(text) {
    this.conversationHistory.push({ role: 'user', text: text });
  }

  // generate(): engine.ts:957-1031 -- prompt (first turn) or turn suffix,
  // overflow reset at contextLength - 10, prefill, first token from the LM
  // head, then one forward + select per token until a stop id, the abort
  // signal, maxTokens or the end of the context.
  async *generate(options) {
    const o = options || {};
    if (this.deviceLost) throw new Error('GPU device lost - call dispose() and recreate the engine');
    const temperature = o.temperature === undefined ? 0.7 : o.temperature;
    const topP = o.topP === undefined ? 0.9 : o.topP;
    const repPenalty = o.repPenalty === undefined ? 1.2 : o.repPenalty;
    const maxTokens = o.maxTokens === undefined ? 32768 : o.maxTokens;
    const toolsJson = o.toolsJson === undefined ? '[]' : o.toolsJson;
    const signal = o.signal;
    // a previous generator left unfinished may still have a step queued
    await this.drain();
    if (this.resetPending) {
      this.resetPending = false;
      this.call(() => this.gg.resetKV(this.ctx));
    }
    // the uniform draw is taken only when sampling (engine.ts:878,894)
    const draw = () => (temperature === 0 ? 0 : this.random());

    let newTokens;
    if (this.kvPosition === 0) {
      newTokens = this.tokenizer.encode(buildChatPrompt(this.conversationHistory, toolsJson));
    } else {
      const lastUser = this.conversationHistory[this.conversationHistory.length - 1];
      newTokens = this.tokenizer.encode(turnSuffix(lastUser.text)).slice(1);   // no BOS
    }
    if (this.kvPosition + newTokens.length >= this.config.context_length - 10) {
      const lastUser = this.conversationHistory[this.conversationHistory.length - 1];
      this.conversationHistory = [{ role: 'user', text: lastUser.text }];
      newTokens = this.tokenizer.encode(buildChatPrompt(this.conversationHistory, toolsJson));
      this.call(() => this.gg.resetKV(this.ctx));
      this.kvPosition = 0;
    }

    // the turn's repetition-penalty set starts as its prompt tokens; the
    // device adds every selected id (allTokens, engine.ts:989,994,1021)
    const ids = Int32Array.from(newTokens);
    this.call(() => this.gg.penaltyReset(this.ctx));
    this.call(() => this.gg.penaltyAdd(this.ctx, ids));
    await this.callAsync(() => this.gg.prefill(this.ctx, ids, this.kvPosition));
    this.kvPosition += newTokens.length;

    let next = await this.callAsync(() => this.gg.select(this.ctx, temperature, topP, repPenalty, draw()));
    const endCall = this.tokenizer.funcTokens['<end_function_call>'];
    const generated = [next];
    let writes = 0;
    const isStop = (t) => t === 1 || t === 0 || t === 106;
    yield this.tokenizer.decodeToken(next);

    // the queued loop only where a submit returns before its step has run
    // (the persistent decode kernel: decodePath 1); on the graph path the
    // binding's stepSubmit would run each step synchronously on this thread
    const queued = typeof this.gg.stepSubmit === 'function' && typeof this.gg.stepCollect === 'function' &&
      (typeof this.gg.decodePath !== 'function' || this.gg.decodePath(this.ctx) === 1);
    if (queued) {
      // The same loop with one step queued ahead: step k + 1 is submitted
      // before step k's id reaches the host (it takes that id on the device),
      // so the GPU runs the steps back to back. The ids, the yields and the
      // stop rules are those of the loop below; a step queued past the end is
      // collected and dropped (its K/V row lies beyond kvPosition, its id in
      // the turn's penalty set, which the next turn resets). When sampling, that
      // dropped step has taken one draw.
      const canStep = (step, pos) =>
        step < maxTokens && pos < this.config.context_length - 1 && !(signal && signal.aborted);
      try {
        if (!isStop(next) && !(endCall !== undefined && next === endCall) && canStep(1, this.kvPosition)) {
          this.call(() => this.gg.stepSubmit(this.ctx, next, this.kvPosition, temperature, topP, repPenalty, draw()));
          this.inflight = 1;
          for (let step = 1; this.inflight > 0; step++) {
            const ahead = this.kvPosition + writes + 1;
            if (canStep(step + 1, ahead)) {
              this.call(() => this.gg.stepSubmit(this.ctx, -1, ahead, temperature, topP, repPenalty, draw()));
              this.inflight++;
            }
            next = await this.callAsync(() => this.gg.stepCollect(this.ctx));
            this.inflight--;
            writes++;
            if (isStop(next)) break;
            if (endCall !== undefined && next === endCall) {
              generated.push(next);
              break;
            }
            generated.push(next);
            yield this.tokenizer.decodeToken(next);
            if (signal && signal.aborted) break;
          }
        }
      } finally {
        await this.drain();
      }
    } else {
      for (let step = 1; step < maxTokens; step++) {
        if (isStop(next)) break;
        if (endCall !== undefined && next === endCall) break;
        if (signal && signal.aborted) break;
        const pos = this.kvPosition + writes;
        if (pos >= this.config.context_length - 1) break;
        const tok = next;
        next = await this.callAsync(() => this.gg.step(this.ctx, tok, pos, temperature, topP, repPenalty, draw()));
        writes++;
        if (isStop(next)) break;
        if (endCall !== undefined && next === endCall) {
          generated.push(next);
          break;
        }
        generated.push(next);
        yield this.tokenizer.decodeToken(next);
      }
    }
    this.conversationHistory.push({ role: 'model', text: this.tokenizer.decodeTokens(generated) });
    this.kvPosition += writes;
  }

  // Collects (and drops) any step still queued by a generator that was left
  // unfinished without being returned.
  async drain() {
    while (this.inflight > 0 && this.ctx) {
      this.inflight--;
      await this.callAsync(() => this.gg.stepCollect(this.ctx));
    }
    this.inflight = 0;
  }

  resetConversation() {
    this.conversationHistory = [];
    this.kvPosition = 0;
    if (!this.ctx) return;
    // with a step still queued the KV reset waits for the next generate()
    if (this.inflight > 0) this.resetPending = true;
    else this.call(() => this.gg.resetKV(this.ctx));
  }

  dispose() {
    if (this.ctx) this.gg.destroy(this.ctx);
    this.ctx = null;
  }
}

async function createGemmaEngine(options) {
  const o = options || {};
  const engine = new GemmaEngineImpl(o);
  await engine.init(o);
  return engine;
}

module.exports = { createGemmaEngine: createGemmaEngine, GemmaEngineImpl: GemmaEngineImpl,
  defaultConfig: defaultConfig, MODEL_FILES: MODEL_FILES, resolveModel: resolveModel };

'use strict';
// GGUF v3 reader for the JavaScript host (the reference's gguf.ts:3-91,
// 169-220): header, metadata, tensor table and data offset, read from a file
// descriptor so that tensor bytes stream straight to the device one tensor at
// a time (no whole-file buffer, no repack: the device takes GGUF Q8_0 bytes).
const fs = require('fs');

const GGUF_MAGIC = 0x46554747;   // "GGUF"
const TYPE_NAMES = ['uint8', 'int8', 'uint16', 'int16', 'uint32', 'int32', 'float32', 'bool', 'string',
  'array', 'uint64', 'int64', 'float64'];
const GGML_F32 = 0;
const GGML_F16 = 1;
const GGML_Q8_0 = 8;

// Sequential little-endian reader over a growable window of the file.
class FileCursor {
  constructor(fd, chunk) {
    this.fd = fd;
    this.chunk = chunk || (1 << 20);
    this.buf = Buffer.alloc(0);
    this.base = 0;      // file offset of buf[0]
    this.pos = 0;       // file offset of the next byte
  }
  need(n) {
    const have = this.base + this.buf.length - this.pos;
    if (have >= n) return;
    const start = this.pos;
    const len = Math.max(n, this.chunk);
    const b = Buffer.alloc(len);
    const got = fs.readSync(this.fd, b, 0, len, start);
    if (got < n) throw new Error('GGUF: unexpected end of file at byte ' + start);
    this.buf = b.slice(0, got);
    this.base = start;
  }
  take(n) {
    this.need(n);
    const off = this.pos - this.base;
    this.pos += n;
    return off;
  }
  u8() { const o = this.take(1); return this.buf.readUInt8(o); }
  i8() { const o = this.take(1); return this.buf.readInt8(o); }
  u16() { const o = this.take(2); return this.buf.readUInt16LE(o); }
  i16() { const o = this.take(2); return this.buf.readInt16LE(o); }
  u32() { const o = this.take(4); return this.buf.readUInt32LE(o); }
  i32() { const o = this.take(4); return this.buf.readInt32LE(o); }
  f32() { const o = this.take(4); return this.buf.readFloatLE(o); }
  f64() { const o = this.take(8); return this.buf.readDoubleLE(o); }
  u64() { const o = this.take(8); return this.buf.readBigUInt64LE(o); }
  i64() { const o = this.take(8); return this.buf.readBigInt64LE(o); }
  str() {
    const n = Number(this.u64());
    const o = this.take(n);
    return this.buf.toString('utf8', o, o + n);
  }
}

function readValue(cur, type) {
  switch (type) {
    case 0: return { type: 'uint8', value: cur.u8() };
    case 1: return { type: 'int8', value: cur.i8() };
    case 2: return { type: 'uint16', value: cur.u16() };
    case 3: return { type: 'int16', value: cur.i16() };
    case 4: return { type: 'uint32', value: cur.u32() };
    case 5: return { type: 'int32', value: cur.i32() };
    case 6: return { type: 'float32', value: cur.f32() };
    case 7: return { type: 'bool', value: cur.u8() !== 0 };
    case 8: return { type: 'string', value: cur.str() };
    case 9: {
      const elem = cur.u32();
      const count = Number(cur.u64());
      const out = new Array(count);
      for (let i = 0; i < count; i++) out[i] = readValue(cur, elem);
      return { type: 'array', value: out };
    }
    case 10: return { type: 'uint64', value: cur.u64() };
    case 11: return { type: 'int64', value: cur.i64() };
    case 12: return { type: 'float64', value: cur.f64() };
  }
  throw new Error('GGUF: unknown metadata value type ' + type);
}

// Parse the header of an open GGUF file: { version, kv: Map, tensors, dataOffset }.
function parseHeader(fd) {
  const cur = new FileCursor(fd);
  const magic = cur.u32();
  if (magic !== GGUF_MAGIC) throw new Error('Invalid GGUF magic: 0x' + magic.toString(16));
  const version = cur.u32();
  if (version < 2 || version > 3) throw new Error('Unsupported GGUF version ' + version);
  const tensorCount = Number(cur.u64());
  const kvCount = Number(cur.u64());
  const kv = new Map();
  for (let i = 0; i < kvCount; i++) {
    const key = cur.str();
    kv.set(key, readValue(cur, cur.u32()));
  }
  const tensors = [];
  for (let i = 0; i < tensorCount; i++) {
    const name = cur.str();
    const nd = cur.u32();
    const dims = [];
    for (let d = 0; d < nd; d++) dims.push(Number(cur.u64()));
    const type = cur.u32();
    const offset = Number(cur.u64());
    tensors.push({ name: name, dims: dims, type: type, offset: offset });
  }
  const align = kv.has('general.alignment') ? Number(kv.get('general.alignment').value) : 32;
  const dataOffset = Math.ceil(cur.pos / align) * align;
  return { version: version, kv: kv, tensors: tensors, dataOffset: dataOffset };
}

// Bytes of a tensor in the file (gguf.ts:169-176).
function tensorByteSize(t) {
  const n = t.dims.reduce((a, b) => a * b, 1);
  if (t.type === GGML_Q8_0) return n / 32 * 34;
  if (t.type === GGML_F32) return n * 4;
  if (t.type === GGML_F16) return n * 2;
  throw new Error('Unsupported tensor type ' + t.type + ' (' + t.name + ')');
}

// Read one tensor's bytes from the file.
function readTensor(fd, gguf, t) {
  const size = tensorByteSize(t);
  const b = Buffer.alloc(size);
  let got = 0;
  while (got < size) {
    const n = fs.readSync(fd, b, got, size - got, gguf.dataOffset + t.offset + got);
    if (n <= 0) throw new Error('GGUF: short read of ' + t.name);
    got += n;
  }
  return b;
}

function kvNumber(gguf, key) {
  const e = gguf.kv.get(key);
  return e === undefined ? null : Number(e.value);
}

// Model configuration from metadata (gguf.ts:180-220 keys, plus the sliding
// window and rope frequency bases that a Gemma-3 GGUF carries).
function configFromGGUF(gguf, base, maxContext) {
  const c = Object.assign({}, base);
  const arch = gguf.kv.has('general.architecture') ? gguf.kv.get('general.architecture').value : 'gemma3';
  const k = (s) => kvNumber(gguf, arch + '.' + s);
  const set = (field, v) => { if (v !== null) c[field] = v; };
  set('hidden_size', k('embedding_length'));
  set('num_layers', k('block_count'));
  set('intermediate_size', k('feed_forward_length'));
  set('num_q_heads', k('attention.head_count'));
  set('num_kv_heads', k('attention.head_count_kv'));
  set('head_dim', k('attention.key_length'));
  const ctx = k('context_length');
  const cap = maxContext === undefined || maxContext === null ? 2048 : maxContext;
  if (ctx !== null) c.context_length = Math.min(ctx, cap);
  const win = k('attention.sliding_window');
  if (win !== null) c.file_sliding_window = win;
  const theta = k('rope.freq_base');
  if (theta !== null) c.file_rope_theta = theta;
  const thetaSwa = k('rope.freq_base_swa');
  if (thetaSwa !== null) c.file_rope_theta_swa = thetaSwa;
  const tokens = gguf.kv.get('tokenizer.ggml.tokens');
  if (tokens && tokens.type === 'array') c.vocab_size = tokens.value.length;
  c.q_dim = c.num_q_heads * c.head_dim;
  c.kv_dim = c.num_kv_heads * c.head_dim;
  return c;
}

module.exports = {
  GGML_F32: GGML_F32, GGML_F16: GGML_F16, GGML_Q8_0: GGML_Q8_0, TYPE_NAMES: TYPE_NAMES,
  parseHeader: parseHeader, tensorByteSize: tensorByteSize, readTensor: readTensor,
  configFromGGUF: configFromGGUF,
};

'use strict';
// Tokenizer of the JavaScript host, same behaviour as the reference's
// tokenizer.ts:1-142: greedy longest match over the GGUF vocabulary with
// spaces as U+2581 (a leading U+2581 on each segment except right after a
// special token), special / function tokens split out first, unknown
// characters skipped, BOS (2) prepended; decoding maps U+2581 back to spaces.

const SPECIALS = { '<start_of_turn>': 105, '<end_of_turn>': 106, '<eos>': 1, '<bos>': 2 };
const FUNCTION_TOKENS = ['<start_function_declaration>', '<end_function_declaration>',
  '<start_function_call>', '<end_function_call>', '<start_function_response>',
  '<end_function_response>', '<escape>'];
const SPACE = '▁';

function escapeRegex(s) {
  return s.replace(/[.*+?^${}()|[\]\\<>]/g, (c) => '\\' + c);
}

class Tokenizer {
  constructor(vocab) {
    this.vocab = vocab;
    this.idOf = new Map();
    this.maxLen = 0;
    // the lengths of the entries that start with each first code unit,
    // longest first: only those can match there, so the longest match is
    // found with a lookup per such length instead of one per length up to
    // maxLen (same result)
    const lens = new Map();
    for (let i = 0; i < vocab.length; i++) {
      const t = vocab[i];
      if (!t) continue;
      if (!this.idOf.has(t)) this.idOf.set(t, i);
      if (t.length > this.maxLen) this.maxLen = t.length;
      const l = lens.get(t[0]);
      if (l) l.add(t.length);
      else lens.set(t[0], new Set([t.length]));
    }
    this.lensByFirst = new Map();
    for (const [c, l] of lens) this.lensByFirst.set(c, Array.from(l).sort((a, b) => b - a));
    this.special = Object.assign({}, SPECIALS);
    this.funcTokens = {};
    for (const name of FUNCTION_TOKENS) {
      const id = this.idOf.get(name);
      if (id !== undefined) {
        this.funcTokens[name] = id;
        this.special[name] = id;
      }
    }
    // longest names first so that no special token is split by a shorter one
    const names = Object.keys(this.special).sort((a, b) => b.length - a.length);
    this.specialSource = names.map(escapeRegex).join('|');
  }

  static fromGGUF(gguf) {
    const e = gguf.kv.get('tokenizer.ggml.tokens');
    if (!e || e.type !== 'array') throw new Error('No tokenizer found in GGUF metadata');
    return new Tokenizer(e.value.map((v) => v.value));
  }

  encodeSegment(text, prefix) {
    const str = (prefix ? SPACE : '') + text.replace(/ /g, SPACE);
    const out = [];
    let pos = 0;
    while (pos < str.length) {
      let hit = -1;
      let hitLen = 0;
      const lens = this.lensByFirst.get(str[pos]);
      if (lens) {
        const left = str.length - pos;
        for (const len of lens) {
          if (len > left) continue;
          const id = this.idOf.get(str.substring(pos, pos + len));
          if (id !== undefined) {
            hit = id;
            hitLen = len;
            break;
          }
        }
      }
      if (hitLen === 0) {
        pos += 1;   // no vocabulary entry starts here: drop one character
      } else {
        out.push(hit);
        pos += hitLen;
      }
    }
    return out;
  }

  encode(text) {
    const ids = [2];
    const re = new RegExp(this.specialSource, 'g');
    let last = 0;
    let afterSpecial = false;
    let m;
    while ((m = re.exec(text)) !== null) {
      const before = text.slice(last, m.index);
      if (before.length > 0) Array.prototype.push.apply(ids, this.encodeSegment(before, !afterSpecial));
      ids.push(this.special[m[0]]);
      last = m.index + m[0].length;
      afterSpecial = true;
    }
    const tail = text.slice(last);
    if (tail.length > 0) Array.prototype.push.apply(ids, this.encodeSegment(tail, !afterSpecial));
    return ids;
  }

  decodeToken(id) {
    if (id >= 0 && id < this.vocab.length && this.vocab[id]) return this.vocab[id].split(SPACE).join(' ');
    return '<unk:' + id + '>';
  }

  decodeTokens(ids) {
    let s = '';
    for (const id of ids) s += this.decodeToken(id);
    return s;
  }
}

module.exports = { Tokenizer: Tokenizer, SPECIALS: SPECIALS };

'use strict';
// Entry point of the JavaScript host (the reference's index.ts:34-47).
const { createGemmaEngine, defaultConfig } = require('./engine');
const { Tokenizer } = require('./tokenizer');
const { buildChatPrompt } = require('./conversation');
const gguf = require('./gguf');

module.exports = { createGemmaEngine: createGemmaEngine, defaultConfig: defaultConfig, Tokenizer: Tokenizer,
  buildChatPrompt: buildChatPrompt, gguf: gguf };

// Type declarations of the JavaScript host (index.js), matching the
// reference's public types (types.ts:1-97, index.ts:34-47) plus the options
// this host adds for a local, HIP-backed engine.

/** Model configuration: Gemma-3 270M defaults (types.ts:19-36), updated from the GGUF. */
export interface GemmaConfig {
  hidden_size: number;
  q_dim: number;
  kv_dim: number;
  num_q_heads: number;
  num_kv_heads: number;
  head_dim: number;
  intermediate_size: number;
  vocab_size: number;
  num_layers: number;
  context_length: number;
  rms_norm_eps: number;
  rope_theta_global: number;
  rope_theta_swa: number;
  swa_period: number;
  /** 0: full attention on every layer; otherwise the local layers' window. */
  sliding_window: number;
}

export interface ProgressInfo {
  /** Bytes uploaded so far. */
  loaded: number;
  /** Total bytes to upload. */
  total: number;
  /** Human-readable status message. */
  status: string;
}

export interface GemmaEngineOptions {
  /**
   * '270m', '1b', 'func' (the reference's model keys, resolved to their Q8_0
   * file names in modelDir) or the path of a local .gguf file. Default '1b'.
   * URLs are not fetched.
   */
  model?: string;
  /** Directory holding the keyed model files. Default: $GEMMA_MODEL_DIR, else the working directory. */
  modelDir?: string;
  /** Progress callback during weight loading. */
  onProgress?: (progress: ProgressInfo) => void;
  /** Maximum context length (tokens). Defaults to 2048. */
  contextLength?: number;
  /**
   * 'reference' (default): one rope base and full attention on every layer,
   * as the reference's shaders run. 'gemma3': local layers use base 1e4 (or
   * the file's sliding-window base) and a 512-position window.
   */
  attention?: 'reference' | 'gemma3';
  /**
   * Rows per batched MFMA prefill slice. Unset or 0: the whole prompt (at most
   * 4096 rows per slice). Negative: the reference's token-by-token prefill.
   */
  prefillBatch?: number;
  /** Directory holding gg_napi.node and libgg.so (default: ../lib beside this file). */
  bindingDir?: string;
  /** Uniform draw in [0, 1) for sampling. Default Math.random. */
  random?: () => number;
}

export interface GenerateOptions {
  /** Sampling temperature. 0 = greedy. Default: 0.7 */
  temperature?: number;
  /** Top-P nucleus sampling threshold. Default: 0.9 */
  topP?: number;
  /** Repetition penalty. 1.0 = no penalty. Default: 1.2 */
  repPenalty?: number;
  /** Maximum tokens to generate. Default: 32768 */
  maxTokens?: number;
  /** Tools JSON string for function calling. Default: '[]' */
  toolsJson?: string;
  /** Cancels generation between tokens. */
  signal?: { readonly aborted: boolean };
}

/** A single turn in conversation history. */
export interface ConversationTurn {
  role: 'user' | 'model';
  text: string;
}

export interface GemmaEngine {
  /** Add a user message to the conversation. */
  addUserMessage(text: string): void;
  /** Generate a response as an async iterator of token strings. */
  generate(options?: GenerateOptions): AsyncGenerator<string, void, undefined>;
  /** Reset conversation history and KV cache. */
  resetConversation(): void;
  /** Release the device context (deferred until a running call ends). */
  dispose(): void;
  /** Current config (read-only). */
  readonly config: Readonly<GemmaConfig>;
}

export function createGemmaEngine(options?: GemmaEngineOptions): Promise<GemmaEngine>;
export function defaultConfig(): GemmaConfig;

export class Tokenizer {
  constructor(vocab: string[]);
  encode(text: string): number[];
  decodeToken(id: number): string;
  decodeTokens(ids: number[]): string;
}

export function buildChatPrompt(history: ConversationTurn[], toolsJson?: string): string;

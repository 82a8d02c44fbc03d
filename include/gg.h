/*
 * gg.h -- C-ABI of the MI355X (gfx950) Gemma-3 Q8_0 token loop.
 *
 * Drop-in boundary: these entry points replace the private WebGPU layer of
 * GemmaEngineImpl in svenflow/webgpu-gemma (src/engine.ts). The JS host keeps
 * the public API (createGemmaEngine / addUserMessage / generate), the GGUF
 * parser, tokenizer and turn/KV-position bookkeeping, and calls these through
 * an N-API addon. Plain pointers and sizes only; every call returns 0 on
 * success or a negative GG_ERR_* code and never throws. Host pointers are
 * borrowed for the duration of the call. One context = one HIP stream; calls
 * on one context must be serialised by the caller (the reference relies on a
 * single-threaded caller too).
 */
#ifndef GG_H
#define GG_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GG_OK 0
#define GG_ERR_INVALID (-1)      /* bad argument, shape or state            */
#define GG_ERR_NO_DEVICE (-2)    /* no HIP device / not gfx950 ("No WebGPU adapter found", engine.ts:125-127) */
#define GG_ERR_HIP (-3)          /* HIP runtime error                       */
#define GG_ERR_DEVICE_LOST (-4)  /* sticky fault (a HIP error that poisons the context); recreate the
                                    context ("WebGPU device lost", engine.ts:134-137,812,958) */
#define GG_ERR_MISSING (-5)      /* gg_finalize: a required tensor was never uploaded */
#define GG_ERR_OOM (-6)          /* device allocation failed               */

/* ggml tensor types accepted by gg_upload_tensor (gguf.ts:160-171, 181-187) */
#define GG_TYPE_F32 0u
#define GG_TYPE_F16 1u
#define GG_TYPE_Q8_0 8u

/* attention modes: 0 = reference (src/ as shipped: one RoPE theta, full
 * attention on every layer, types.ts:32-33, shaders.ts:229-325);
 * 1 = gemma3 (local layers: rope_theta_local + sliding_window). */
#define GG_ATTN_REFERENCE 0
#define GG_ATTN_GEMMA3 1

/* gg_read targets: the reference's debug readback points
 * (debug.html:2636-2920, 3172-3243). */
#define GG_READ_HIDDEN 0        /* f32[H]  hidden after the last layer        */
#define GG_READ_NORMED 1        /* f32[H]  output-normed hidden (LM head input) */
#define GG_READ_LOGITS 2        /* f32[V]  logits of the last selection        */
#define GG_READ_TOPK256 3       /* 256 x {f32 val, u32 id} (topk256 layout, shaders.ts:382-383) */
#define GG_READ_LAYER_HIDDEN 4  /* f32[H]  hidden after layer `layer`          */
#define GG_READ_K_CACHE 5       /* f32[ctx][256] K cache of layer `layer`      */
#define GG_READ_V_CACHE 6       /* f32[ctx][256] V cache of layer `layer`      */
#define GG_READ_Q 7             /* f32[n_q*256] normed+roped q of layer `layer` (last token) */
#define GG_READ_ATTN_OUT 8      /* f32[n_q*256] attention output of the last layer */
#define GG_READ_EMBED 9         /* f32[H]  embedding row of token `layer` (embeddingLookup, shaders.ts:2-23),
                                   built by the device function both decode paths use */

/* GemmaConfig (types.ts:2-36) plus the build's attention-mode fields. */
typedef struct gg_config {
  int32_t hidden_size;
  int32_t num_layers;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t intermediate_size;
  int32_t vocab_size;
  int32_t context_length;
  float rms_norm_eps;
  float rope_theta_global;
  float rope_theta_local;   /* reference mode: equal to rope_theta_global (rope_theta_swa) */
  int32_t swa_period;       /* isSwaLayer(il) = il % swa_period < swa_period - 1 (types.ts:38-40) */
  int32_t sliding_window;   /* 0 = full attention */
  int32_t attention_mode;   /* GG_ATTN_* (documentation of intent; window/theta decide) */
  int32_t prefill_batch;    /* 0: gg_prefill runs the decode pass per token like the reference
                               (engine.ts:923-928); > 0: prompt rows per batched MFMA prefill
                               slice (no reference counterpart) */
} gg_config;

/* Sampling options of one selection (GenerateOptions, types.ts:65-78), kept
 * as doubles because the JS host computes with JS numbers. */
typedef struct gg_sample {
  double temperature;
  double top_p;
  double rep_penalty;
} gg_sample;

typedef struct gg_ctx gg_ctx;

/* Replaces initWebGPU + createUniformBuffers (engine.ts:124-138, 171-217).
 * Returns NULL on failure; gg_last_error(NULL) then says why. */
gg_ctx* gg_create(const gg_config* cfg);

/* Replaces uploadWeightsFromBuffer / uploadWeightsStreaming (engine.ts:219-400).
 * `name` is the GGUF tensor name (token_embd.weight, output_norm.weight,
 * blk.N.{attn_q,attn_k,attn_v,attn_output,ffn_gate,ffn_up,ffn_down,attn_norm,
 * ffn_norm,attn_q_norm,attn_k_norm,post_attention_norm,post_ffw_norm}.weight).
 * `bytes` are the tensor's GGUF bytes (34-byte Q8_0 blocks, F32 or F16);
 * no host repacking is needed. dims[0] is the input (ne0) dimension. */
int gg_upload_tensor(gg_ctx* ctx, const char* name, uint32_t ggml_type, const uint64_t* dims,
                     uint32_t ndims, const void* bytes, size_t nbytes);

/* Replaces createWorkBuffers + createBindGroups (engine.ts:402-732): checks
 * every tensor is present, allocates work buffers and the KV cache, and
 * captures the per-token HIP graphs. */
int gg_finalize(gg_ctx* ctx);

/* Replaces prefillBatched / forwardPassOnly (engine.ts:917-928): the tokens
 * at positions start_pos.. go through every layer (KV cache written), no LM
 * head; the last token's normed hidden is left for gg_select. Returns after
 * the device has finished (onSubmittedWorkDone). With prefill_batch > 0 and
 * n > 1 the prompt runs as M-row GEMMs on MFMA plus batched attention. */
int gg_prefill(gg_ctx* ctx, const int32_t* tokens, int32_t n, int32_t start_pos);

/* Replaces getFirstTokenAfterPrefill / sampleNextToken (engine.ts:805-902,
 * 941-949): LM head on the current normed hidden, then greedy argmax
 * (temperature 0 and rep_penalty <= 1) or topk256 + penalty + temperature +
 * top-p with the draw `u` in [0,1) (Math.random() in the reference). The
 * selected id is added to the penalty set. */
int gg_select(gg_ctx* ctx, const gg_sample* s, double u, int32_t* out_token);

/* Replaces forwardPassAndGetToken (engine.ts:904-915): forward + select. */
int gg_step(gg_ctx* ctx, int32_t token, int32_t pos, const gg_sample* s, double u,
            int32_t* out_token);

/* Pipelined decode steps. No counterpart in the reference, whose generate()
 * loop (engine.ts:1001-1030) awaits each step's id before encoding the
 * next; the host uses these in that loop to keep one step queued ahead.
 *
 * gg_step_submit queues a step (forward + select, as gg_step) at `pos` and
 * returns without waiting. Its input is `token`; with token < 0 it is the
 * id that the previously submitted step (or the last gg_step / gg_select)
 * selects, read on the device, so the step can be queued before that id
 * reaches the host. gg_step_collect waits for the oldest submitted step and
 * returns its id; on the persistent kernel's path it waits by polling the
 * mapped host word the launch stores the id into (the calling thread spins;
 * no event sits between the queued launches).
 *
 * At most two steps may be outstanding. Every other call except
 * gg_destroy fails with GG_ERR_INVALID while any is. A step that is
 * collected and not used leaves its K/V row at `pos` and its id in the
 * penalty set; the next prefill at `pos` overwrites the row, and
 * gg_penalty_reset clears the set. Without the persistent decode kernel's
 * single-launch step (gg_decode_path: GG_DECODE_GRAPH, or a vocabulary that
 * is not a multiple of 16384), gg_step_submit runs the step before it
 * returns. */
int gg_step_submit(gg_ctx* ctx, int32_t token, int32_t pos, const gg_sample* s, double u);
int gg_step_collect(gg_ctx* ctx, int32_t* out_token);

/* Repetition-penalty set (the reference's Set(allTokens), engine.ts:868-876,
 * 989, 994, 1021): cleared per turn, filled with the turn's prompt ids. */
int gg_penalty_reset(gg_ctx* ctx);
int gg_penalty_add(gg_ctx* ctx, const int32_t* ids, int32_t n);

/* Replaces resetKVCaches (engine.ts:930-939). */
int gg_reset_kv(gg_ctx* ctx);

/* Parity checkpoints (debug.html readBackBuffer, 2636-2648). Synchronous. */
int gg_read(gg_ctx* ctx, int32_t what, int32_t layer, void* dst, size_t nbytes);

/* Per-step device timing, off by default. With on != 0 every gg_step /
 * gg_select records three HIP events on the context's stream (about 9 us of
 * device time per step on MI355X), and gg_last_timing returns the last
 * call's forward and select time in milliseconds (GG_ERR_INVALID when timing
 * is off or no call has run since it was turned on). On the persistent
 * decode path a gg_step is one launch: its whole time is reported as the
 * forward time and the select time is 0. No counterpart in the reference
 * (WebGPU timestamp queries are not used in src/). */
int gg_set_timing(gg_ctx* ctx, int32_t on);
int gg_last_timing(gg_ctx* ctx, float* forward_ms, float* select_ms);

/* Probe: before gg_finalize, name one kernel launch of the captured graphs
 * to bracket with HIP event-record nodes; after each gg_step / gg_select,
 * gg_probe_elapsed returns that launch's device time in milliseconds. Used by
 * the benchmark to time the dominant kernel inside the timed loop. Where the
 * HIP runtime of the process does not take external event records into a
 * stream capture, the probed context launches the same kernels directly
 * (as with GG_NO_GRAPH=1) and brackets the launch with ordinary records.
 * No counterpart in the reference (WebGPU has no per-dispatch timestamps in
 * src/). */
#define GG_PROBE_NONE 0
#define GG_PROBE_QKV 1       /* fused QKV GEMV of layer `layer`           */
#define GG_PROBE_ATTN 2      /* decode attention of layer `layer`         */
#define GG_PROBE_O 3         /* O projection GEMV of layer `layer`        */
#define GG_PROBE_GATE_UP 4   /* gate/up GEMV + GeGLU of layer `layer`     */
#define GG_PROBE_DOWN 5      /* down projection GEMV of layer `layer`     */
#define GG_PROBE_LM_HEAD 6   /* tied LM head GEMV                         */
#define GG_PROBE_SELECT 7    /* vocab selector                            */
int gg_set_probe(gg_ctx* ctx, int32_t kind, int32_t layer);
int gg_probe_elapsed(gg_ctx* ctx, float* ms);
/* Device time between two event-record nodes placed back to back right
 * before the probed launch (same graph, same step): the cost of an event
 * bracket itself, to subtract from gg_probe_elapsed. */
int gg_probe_overhead(gg_ctx* ctx, float* ms);

/* Decode path of the per-token forward passes. GG_DECODE_FUSED (the default
 * where the model and device allow it: 4 query heads, hidden <= 1280, 256
 * compute units) runs a whole forward pass -- and, for a
 * vocabulary that is a multiple of 16384, the LM head and the selection --
 * as one launch of a persistent kernel whose 256 blocks hand their outputs
 * to each other in device memory; GG_DECODE_GRAPH replays one kernel per
 * phase (133 per 1B token). Both compute the same functions; summation
 * orders differ. The environment variable GG_DECODE=graph selects the
 * graph path when gg_set_decode_path was not called. No counterpart in the
 * reference (engine.ts:735-802 encodes one dispatch per kernel).
 *
 * The persistent kernel needs all 256 of its blocks resident at once. The
 * persistent launches of all contexts of a process on one device run one at
 * a time (each waits for the other contexts' latest one). Every hand-off wait
 * inside the kernel is bounded (20 ms): if a launch's blocks could not all
 * run together (CUs held by another process) or a hand-off stalled, the
 * launch ends, the context switches to GG_DECODE_GRAPH for good and the call
 * runs its work again there -- a token-by-token prefill, a step, or a
 * pipelined step and the one queued behind it -- so it still returns the
 * selection with GG_OK; gg_decode_path then reports GG_DECODE_GRAPH. With
 * GG_DEC_COOP=1 in the environment at gg_finalize, direct persistent
 * launches are cooperative launches instead (the runtime refuses a grid that
 * cannot be resident; 4% slower per step on MI355X). */
#define GG_DECODE_GRAPH 0
#define GG_DECODE_FUSED 1
int gg_set_decode_path(gg_ctx* ctx, int32_t path);   /* before gg_finalize */
int gg_decode_path(gg_ctx* ctx);                      /* after gg_finalize: the path in use */
/* Profiling: with GG_DEC_TIMELINE=1 in the environment at gg_finalize the
 * persistent kernel stamps the s_memrealtime clock (100 MHz) at 16 phase
 * events per (block, layer); this copies the last launch's stamps,
 * [256][layers][16] int64 (0 = not reached by that block). */
int gg_decode_timeline(gg_ctx* ctx, int64_t* dst, size_t n);

/* Message for the last failing call on ctx (or of gg_create when ctx is NULL). */
const char* gg_last_error(const gg_ctx* ctx);

/* Replaces dispose (engine.ts:1039-1077). */
void gg_destroy(gg_ctx* ctx);

/* ---- kernel-level entry points (device pointers, caller's HIP stream) ----
 * These expose single kernels of the path for isolated parity tests and the
 * GEMV benchmark; `stream` is a hipStream_t (NULL = default stream). */

/* Device bytes of the item-planar layout of a rows x k Q8_0 matrix
 * (>= the GGUF count rows*k/32*34; 0 for unsupported shapes: rows and k must
 * be multiples of 64, k <= 8192). */
size_t gg_q8_0_packed_size(int64_t rows, int64_t k);

/* Q8_0 GGUF bytes -> the device layout the GEMV reads (packQ8_0ForGPU's
 * role, gguf.ts:126-149, without changing the 34-byte blocks). */
int gg_q8_0_repack(const void* src_gguf, void* dst, int64_t rows, int64_t k, void* stream);

/* y[rows] = W[rows x k] x[k] on the device layout (linearQ8, shaders.ts:92-151). */
int gg_q8_0_gemv(const void* w, const float* x, float* y, int64_t rows, int64_t k, void* stream);

/* Bit-exact Q8_0 -> f32 (dequantizeQ8_0, gguf.ts:107-124), GGUF blocks in. */
int gg_q8_0_dequant(const void* src_gguf, float* out, int64_t n_elems, void* stream);

/* Token selection over a device logits vector (argmax / topk256 / sampler,
 * shaders.ts:327-384 + engine.ts:862-901). seen_bitmap: ceil(n/32) u32 words
 * (may be NULL when rep_penalty <= 1). topk_out: 256 x {f32, u32} or NULL.
 * Workspace: gg_select_workspace_size() bytes. out_token: host pointer. */
size_t gg_select_workspace_size(int32_t n);
int gg_select_logits(const float* logits, int32_t n, const uint32_t* seen_bitmap,
                     const gg_sample* s, double u, void* workspace, void* topk_out,
                     int32_t* out_token, void* stream);

/* gg_select_logits without a workspace argument and without any device
 * allocation: for callers that cannot allocate (tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. It is
 * not usable under HIP graph capture: it copies the sampling state from host
 * memory and synchronizes the stream, and returns only once the selection
 * has finished. The workspace is a static 67,840-byte device array, one
 * copy per GPU, held until the process ends; its address is looked up once
 * per device on the first call there. Every call on one GPU shares that
 * array: calls that overlap on one GPU (other streams or host threads) race.
 * Returns GG_ERR_INVALID, with a message on stderr, when n would need a
 * larger workspace than the static one (gg_select_workspace_size(n) bytes;
 * today that size does not depend on n). Same results as gg_select_logits. */
int gg_select_logits_noalloc(const float* logits, int32_t n, const uint32_t* seen_bitmap,
                             const gg_sample* s, double u, void* topk_out, int32_t* out_token,
                             void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GG_H */

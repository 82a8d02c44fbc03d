/*
 * gemma_oracle.h -- CPU restatement of the webgpu-gemma token loop.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle the HIP path is tested against:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. Nothing in the product (libgg.so, the JS host) links or calls it.
 *
 * Every function restates one piece of the reference in plain C, in the
 * reference's own arithmetic order (fp32 ops, no FMA contraction: the
 * library is compiled with -ffp-contract=off), citing the file:line it
 * follows in svenflow/webgpu-gemma:
 *   src/gguf.ts     GGUF container, f16 and Q8_0 decoding
 *   src/shaders.ts  the 15 WGSL kernels
 *   src/engine.ts   per-token op order and the host sampler
 *   src/types.ts    config defaults and the sliding-window layer predicate
 *
 * Two attention modes (config.window / config.theta_local):
 *   reference: theta_local == theta_global (1e6), window 0 = full causal
 *              attention on every layer (what src/ does, types.ts:32-33).
 *   gemma3:    theta_local 1e4 and window 512 on the layers isSwaLayer()
 *              selects; global layers use theta_global and full attention.
 */
#ifndef GEMMA_ORACLE_H
#define GEMMA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- formats (gguf.ts) ---------------------------------------------- */
float gor_f16_to_f32(uint16_t h);
void  gor_f16_to_f32_n(const uint16_t* h, size_t n, float* out);
void  gor_q8_0_dequant(const uint8_t* blocks, size_t n_elems, float* out);
void  gor_q8_0_pack36(const uint8_t* blocks, size_t n_elems, uint32_t* out);

/* ---- kernels (shaders.ts) ------------------------------------------- */
void  gor_embed(const uint8_t* emb, int token, int hidden, float* out);
void  gor_rms_norm(const float* x, const float* w, float* out, int n, float eps);
void  gor_fused_norm_add(const float* x, const float* w, const float* residual,
                         float* out, int n, float eps);
void  gor_linear_q8(const uint8_t* w, const float* x, float* y, int rows, int k);
void  gor_gelu_mul(const float* gate, const float* up, float* out, int n);
float gor_rope_freq(int i, int head_dim, float theta);
void  gor_per_head_norm_rope(float* data, const float* w, int n_heads, int head_dim,
                             float eps, int pos, float theta);
void  gor_attention(const float* q, const float* k_cache, const float* v_cache,
                    int n_q_heads, int n_kv_heads, int head_dim, int t_lo, int t_hi,
                    float scale, float* scores, float* out);
int   gor_argmax(const float* logits, int n);
void  gor_topk256(const float* logits, int n, float* vals, uint32_t* ids);

/* ---- host sampler (engine.ts:862-901) ------------------------------- */
int   gor_sample_candidates(const float* vals, const uint32_t* ids,
                            const uint32_t* seen_bitmap, double temperature,
                            double top_p, double rep_penalty, double u);

/* ---- whole model ---------------------------------------------------- */
typedef struct gor_config {
  int32_t hidden_size, num_layers, num_q_heads, num_kv_heads, head_dim;
  int32_t intermediate_size, vocab_size, context_length;
  float   rms_norm_eps, rope_theta_global, rope_theta_local;
  int32_t swa_period, sliding_window;
} gor_config;

typedef struct gor_model gor_model;

gor_model* gor_model_create(const gor_config* cfg);
/* Q8_0 tensors are borrowed (the caller keeps them alive); F32/F16 are copied. */
int   gor_model_set_tensor(gor_model* m, const char* name, uint32_t ggml_type,
                           const void* data, size_t nbytes);
void  gor_model_destroy(gor_model* m);
void  gor_model_reset_kv(gor_model* m);
int   gor_model_forward(gor_model* m, int token, int pos);
void  gor_model_lm_head(gor_model* m);
int   gor_model_select(gor_model* m, double temperature, double top_p,
                       double rep_penalty, double u, const int32_t* seen, int n_seen);
float* gor_model_buffer(gor_model* m, int what, int layer);
void  gor_set_threads(int n);
int   gor_get_threads(void);

enum { GOR_HIDDEN = 0, GOR_NORMED = 1, GOR_LOGITS = 2, GOR_LAYER_HIDDEN = 3,
       GOR_K_CACHE = 4, GOR_V_CACHE = 5, GOR_Q = 6, GOR_ATTN_OUT = 7 };

#ifdef __cplusplus
}
#endif
#endif

/*
 * gemma_oracle.c -- CPU restatement of the webgpu-gemma token loop.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle the HIP path is tested against; see
 * the header).
 * Built with -O2 -ffp-contract=off -fopenmp so that every fp32 expression
 * rounds exactly as written, in the order the WGSL source writes it.
 * OpenMP only splits independent output rows; each row's sum keeps the
 * reference order, so results do not depend on the thread count.
 */
#include "gemma_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ===================================================================== */
/* Formats                                                               */
/* ===================================================================== */

/* gguf.ts:95-105 -- f16ToF32. The JS computes a double and stores it into a
 * Float32Array; every f16 value is exact in f32, NaN stores as quiet NaN. */
float gor_f16_to_f32(uint16_t h) {
  int sign = (h >> 15) & 1, ex = (h >> 10) & 0x1f, mant = h & 0x3ff;
  double s = sign ? -1.0 : 1.0;
  if (ex == 0) {
    if (mant == 0) return sign ? -0.0f : 0.0f;
    return (float)(s * ldexp(1.0, -14) * ((double)mant / 1024.0));
  }
  if (ex == 31) return mant == 0 ? (sign ? -INFINITY : INFINITY) : NAN;
  return (float)(s * ldexp(1.0, ex - 15) * (1.0 + (double)mant / 1024.0));
}

void gor_f16_to_f32_n(const uint16_t* h, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = gor_f16_to_f32(h[i]);
}

static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* gguf.ts:107-124 -- dequantizeQ8_0: q * scale in double, stored as f32.
 * A Q8_0 block is 34 bytes: f16 LE scale, then 32 int8. */
void gor_q8_0_dequant(const uint8_t* blocks, size_t n_elems, float* out) {
  size_t idx = 0;
  const uint8_t* p = blocks;
  while (idx < n_elems) {
    double scale = (double)gor_f16_to_f32(rd_u16(p));
    p += 2;
    size_t in_block = n_elems - idx < 32 ? n_elems - idx : 32;
    for (size_t i = 0; i < in_block; ++i) out[idx++] = (float)((double)(int8_t)p[i] * scale);
    p += 32;
  }
}

/* gguf.ts:126-149 -- packQ8_0ForGPU: 36-byte device block = f32 scale,
 * then the 32 quant bytes as 8 little-endian u32 words. */
void gor_q8_0_pack36(const uint8_t* blocks, size_t n_elems, uint32_t* out) {
  size_t nb = n_elems / 32;
  const uint8_t* p = blocks;
  for (size_t b = 0; b < nb; ++b) {
    float scale = gor_f16_to_f32(rd_u16(p));
    memcpy(&out[b * 9], &scale, 4);
    p += 2;
    for (int j = 0; j < 8; ++j) {
      uint32_t packed = 0;
      for (int k = 0; k < 4; ++k) packed |= (uint32_t)p[j * 4 + k] << (k * 8);
      out[b * 9 + 1 + j] = packed;
    }
    p += 32;
  }
}

/* ===================================================================== */
/* Kernels                                                               */
/* ===================================================================== */

/* shaders.ts:2-23 -- embeddingLookup: (f32(q) * scale) * sqrt(f32(H)). */
void gor_embed(const uint8_t* emb, int token, int hidden, float* out) {
  size_t bpr = (size_t)hidden / 32;
  const uint8_t* row = emb + (size_t)token * bpr * 34;
  float sq = sqrtf((float)hidden);
  for (int i = 0; i < hidden; ++i) {
    const uint8_t* blk = row + (size_t)(i / 32) * 34;
    float scale = gor_f16_to_f32(rd_u16(blk));
    float q = (float)(int8_t)blk[2 + (i % 32)];
    float t = q * scale;
    out[i] = t * sq;
  }
}

/* The 256-lane "strided partials + halving tree" sum that rmsNorm, softmax
 * and fusedNormAdd use (shaders.ts:37-49, 280-293, 399-411). */
static float wg256_sum_sq(const float* x, int n) {
  float part[256];
  for (int t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (int i = t; i < n; i += 256) { float v = x[i]; float sq = v * v; s = s + sq; }
    part[t] = s;
  }
  for (int stride = 128; stride > 0; stride >>= 1)
    for (int t = 0; t < stride; ++t) part[t] = part[t] + part[t + stride];
  return part[0];
}

static float wg256_sum(const float* x, int n) {
  float part[256];
  for (int t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (int i = t; i < n; i += 256) s = s + x[i];
    part[t] = s;
  }
  for (int stride = 128; stride > 0; stride >>= 1)
    for (int t = 0; t < stride; ++t) part[t] = part[t] + part[t + stride];
  return part[0];
}

/* shaders.ts:25-56 -- rmsNorm: x * w / sqrt(sum/N + eps). */
void gor_rms_norm(const float* x, const float* w, float* out, int n, float eps) {
  float ss = wg256_sum_sq(x, n);
  float rms = sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) { float t = x[i] * w[i]; out[i] = t / rms; }
}

/* shaders.ts:386-418 -- fusedNormAdd: residual + x * w / rms. */
void gor_fused_norm_add(const float* x, const float* w, const float* residual,
                        float* out, int n, float eps) {
  float ss = wg256_sum_sq(x, n);
  float rms = sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) { float t = x[i] * w[i]; t = t / rms; out[i] = residual[i] + t; }
}

/* shaders.ts:92-151 -- linearQ8. Row m of W is K/32 Q8_0 blocks; the block
 * sum runs over j = 0..31 in order, then total += block_sum * scale with
 * blocks ascending (the 2048-wide x tile does not change that order). */
void gor_linear_q8(const uint8_t* w, const float* x, float* y, int rows, int k) {
  int nb = k / 32;
#pragma omp parallel for schedule(static)
  for (int m = 0; m < rows; ++m) {
    const uint8_t* row = w + (size_t)m * nb * 34;
    float total = 0.0f;
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = row + (size_t)b * 34;
      float scale = gor_f16_to_f32(rd_u16(blk));
      const float* xb = x + b * 32;
      float bs = 0.0f;
      for (int j = 0; j < 32; ++j) { float p = (float)(int8_t)blk[2 + j] * xb[j]; bs = bs + p; }
      float t = bs * scale;
      total = total + t;
    }
    y[m] = total;
  }
}

/* shaders.ts:153-170 -- geluMul (tanh GELU with the argument clamped to
 * +-15), times up. WGSL evaluates left to right. */
void gor_gelu_mul(const float* gate, const float* up, float* out, int n) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  for (int i = 0; i < n; ++i) {
    float x = gate[i];
    float a = k1 * x; a = a * x; a = 1.0f + a;
    float arg = k0 * x; arg = arg * a;
    if (arg < -15.0f) arg = -15.0f;
    if (arg > 15.0f) arg = 15.0f;
    float g = 0.5f * x; g = g * (1.0f + tanhf(arg));
    out[i] = g * up[i];
  }
}

/* shaders.ts:457 -- freq = 1.0 / pow(theta, f32(i*2) / f32(head_dim)). */
float gor_rope_freq(int i, int head_dim, float theta) {
  float e = (float)(i * 2) / (float)head_dim;
  return 1.0f / powf(theta, e);
}

/* shaders.ts:420-467 -- fusedPerHeadNormRope: per-head RMSNorm in place,
 * then NEOX rotation of the pairs (i, i + head_dim/2). */
void gor_per_head_norm_rope(float* data, const float* w, int n_heads, int head_dim,
                            float eps, int pos, float theta) {
  int half = head_dim / 2;
  for (int h = 0; h < n_heads; ++h) {
    float* d = data + (size_t)h * head_dim;
    float ss = wg256_sum_sq(d, head_dim);
    float rms = sqrtf(ss / (float)head_dim + eps);
    for (int i = 0; i < head_dim; ++i) { float t = d[i] * w[i]; d[i] = t / rms; }
    for (int i = 0; i < half; ++i) {
      float freq = gor_rope_freq(i, head_dim, theta);
      float angle = (float)pos * freq;
      float c = cosf(angle), s = sinf(angle);
      float x0 = d[i], x1 = d[i + half];
      float a = x0 * c, b = x1 * s;
      float e = x0 * s, f = x1 * c;
      d[i] = a - b;
      d[i + half] = e + f;
    }
  }
}

/* shaders.ts:229-325 -- attnScore, softmax, attnOutput for positions
 * t_lo..t_hi (the reference always uses t_lo = 0, t_hi = pos). Scores use
 * relative index t - t_lo. kv_head = head * n_kv / n_q (shaders.ts:243). */
void gor_attention(const float* q, const float* k_cache, const float* v_cache,
                   int n_q_heads, int n_kv_heads, int head_dim, int t_lo, int t_hi,
                   float scale, float* scores, float* out) {
  int seq = t_hi - t_lo + 1;
  int kv_stride = n_kv_heads * head_dim;
  for (int h = 0; h < n_q_heads; ++h) {
    int kvh = h * n_kv_heads / n_q_heads;
    const float* qh = q + (size_t)h * head_dim;
    float* s = scores + (size_t)h * seq;
    for (int i = 0; i < seq; ++i) {
      const float* kr = k_cache + (size_t)(t_lo + i) * kv_stride + (size_t)kvh * head_dim;
      float dot = 0.0f;
      for (int d = 0; d < head_dim; ++d) { float p = qh[d] * kr[d]; dot = dot + p; }
      s[i] = dot * scale;
    }
    /* softmax (shaders.ts:254-300): max init -1e30, strided partials, tree */
    float pm[256];
    for (int t = 0; t < 256; ++t) {
      float m = -1e30f;
      for (int i = t; i < seq; i += 256) m = fmaxf(m, s[i]);
      pm[t] = m;
    }
    for (int stride = 128; stride > 0; stride >>= 1)
      for (int t = 0; t < stride; ++t) pm[t] = fmaxf(pm[t], pm[t + stride]);
    float mx = pm[0];
    for (int i = 0; i < seq; ++i) s[i] = expf(s[i] - mx);
    float sum = wg256_sum(s, seq);
    for (int i = 0; i < seq; ++i) s[i] = s[i] / sum;
    /* attnOutput: serial over positions */
    for (int d = 0; d < head_dim; ++d) {
      float acc = 0.0f;
      for (int i = 0; i < seq; ++i) {
        float p = s[i] * v_cache[(size_t)(t_lo + i) * kv_stride + (size_t)kvh * head_dim + d];
        acc = acc + p;
      }
      out[(size_t)h * head_dim + d] = acc;
    }
  }
}

/* shaders.ts:327-361 -- argmax, simulated lane by lane: 256 strided local
 * maxima (strict >, init (-1e30, 0)), then the halving tree that takes the
 * right slot only when strictly greater. */
int gor_argmax(const float* logits, int n) {
  float mx[256];
  uint32_t ix[256];
  for (int t = 0; t < 256; ++t) {
    float m = -1e30f; uint32_t id = 0;
    for (int i = t; i < n; i += 256) if (logits[i] > m) { m = logits[i]; id = (uint32_t)i; }
    mx[t] = m; ix[t] = id;
  }
  for (int stride = 128; stride > 0; stride >>= 1)
    for (int t = 0; t < stride; ++t)
      if (mx[t + stride] > mx[t]) { mx[t] = mx[t + stride]; ix[t] = ix[t + stride]; }
  return (int)ix[0];
}

/* shaders.ts:363-384 -- topk256: lane t reports (max, first index) over the
 * indices congruent to t mod 256. */
void gor_topk256(const float* logits, int n, float* vals, uint32_t* ids) {
  for (int t = 0; t < 256; ++t) {
    float m = -1e30f; uint32_t id = 0;
    for (int i = t; i < n; i += 256) if (logits[i] > m) { m = logits[i]; id = (uint32_t)i; }
    vals[t] = m; ids[t] = id;
  }
}

/* ===================================================================== */
/* Host sampler -- engine.ts:862-901                                     */
/* ===================================================================== */

typedef struct { double val; uint32_t id; int ord; } cand_t;

/* candidates.sort((a, b) => b.val - a.val) is stable in V8 >= 7.0. */
static int cand_cmp(const void* a, const void* b) {
  const cand_t* x = (const cand_t*)a; const cand_t* y = (const cand_t*)b;
  if (x->val > y->val) return -1;
  if (x->val < y->val) return 1;
  return x->ord - y->ord;
}

int gor_sample_candidates(const float* vals, const uint32_t* ids,
                          const uint32_t* seen_bitmap, double temperature,
                          double top_p, double rep_penalty, double u) {
  cand_t c[256];
  int any_seen = 0;
  if (seen_bitmap)
    for (int i = 0; i < 8192 && !any_seen; ++i) any_seen = seen_bitmap[i] != 0;
  for (int i = 0; i < 256; ++i) { c[i].val = (double)vals[i]; c[i].id = ids[i]; c[i].ord = i; }
  if (rep_penalty > 1.0 && any_seen) {                       /* engine.ts:868-876 */
    for (int i = 0; i < 256; ++i) {
      uint32_t id = c[i].id;
      if (id < 262144u && ((seen_bitmap[id >> 5] >> (id & 31)) & 1u)) {
        if (c[i].val > 0) c[i].val /= rep_penalty; else c[i].val *= rep_penalty;
      }
    }
  }
  qsort(c, 256, sizeof(cand_t), cand_cmp);                   /* engine.ts:878 */
  if (temperature == 0.0) return (int)c[0].id;               /* engine.ts:879 */
  double max_logit = c[0].val, sum_exp = 0.0;
  float probs[256];
  for (int i = 0; i < 256; ++i) {                            /* engine.ts:881-887 */
    probs[i] = (float)exp((c[i].val - max_logit) / temperature);
    sum_exp += (double)probs[i];
  }
  double cum = 0.0; int cutoff = 256;
  for (int i = 0; i < 256; ++i) {                            /* engine.ts:889-893 */
    cum += (double)probs[i] / sum_exp;
    if (cum >= top_p) { cutoff = i + 1; break; }
  }
  double subset = 0.0;
  for (int i = 0; i < cutoff; ++i) subset += (double)probs[i];
  double r = u * subset;                                     /* engine.ts:896 */
  for (int i = 0; i < cutoff; ++i) {
    r -= (double)probs[i];
    if (r <= 0) return (int)c[i].id;
  }
  return (int)c[cutoff - 1].id;
}

/* ===================================================================== */
/* Whole model -- engine.ts:735-802 (forward), 805-902 (LM head + select) */
/* ===================================================================== */

enum { L_ATTN_Q, L_ATTN_K, L_ATTN_V, L_ATTN_O, L_FFN_GATE, L_FFN_UP, L_FFN_DOWN, L_NQ8 };
enum { N_ATTN, N_FFN, N_QN, N_KN, N_POST_ATTN, N_POST_FFW, N_NNORM };

static const char* q8_names[L_NQ8] = {"attn_q", "attn_k", "attn_v", "attn_output",
                                      "ffn_gate", "ffn_up", "ffn_down"};
static const char* norm_names[N_NNORM] = {"attn_norm", "ffn_norm", "attn_q_norm", "attn_k_norm",
                                          "post_attention_norm", "post_ffw_norm"};

typedef struct {
  const uint8_t* q8[L_NQ8];
  float* norm[N_NNORM];
  float* k_cache;
  float* v_cache;
} gor_layer;

struct gor_model {
  gor_config c;
  int q_dim, kv_dim;
  const uint8_t* embd;
  float* out_norm;
  gor_layer* layers;
  float *hidden, *residual, *normed, *q, *k, *v, *attn_out, *attn_proj;
  float *gate, *up, *mul, *down, *scores, *logits, *hist;
};

gor_model* gor_model_create(const gor_config* cfg) {
  gor_model* m = (gor_model*)calloc(1, sizeof(gor_model));
  if (!m) return NULL;
  m->c = *cfg;
  m->q_dim = cfg->num_q_heads * cfg->head_dim;
  m->kv_dim = cfg->num_kv_heads * cfg->head_dim;
  int H = cfg->hidden_size, I = cfg->intermediate_size;
  size_t kv = (size_t)cfg->context_length * m->kv_dim;
  m->layers = (gor_layer*)calloc((size_t)cfg->num_layers, sizeof(gor_layer));
  for (int l = 0; l < cfg->num_layers; ++l) {
    m->layers[l].k_cache = (float*)calloc(kv, sizeof(float));
    m->layers[l].v_cache = (float*)calloc(kv, sizeof(float));
  }
  m->hidden = (float*)calloc(H, 4); m->residual = (float*)calloc(H, 4);
  m->normed = (float*)calloc(H, 4); m->attn_proj = (float*)calloc(H, 4);
  m->down = (float*)calloc(H, 4);
  m->q = (float*)calloc(m->q_dim, 4); m->attn_out = (float*)calloc(m->q_dim, 4);
  m->k = (float*)calloc(m->kv_dim, 4); m->v = (float*)calloc(m->kv_dim, 4);
  m->gate = (float*)calloc(I, 4); m->up = (float*)calloc(I, 4); m->mul = (float*)calloc(I, 4);
  m->scores = (float*)calloc((size_t)cfg->num_q_heads * cfg->context_length, 4);
  m->logits = (float*)calloc((size_t)cfg->vocab_size, 4);
  m->hist = (float*)calloc((size_t)cfg->num_layers * H, 4);
  return m;
}

void gor_model_destroy(gor_model* m) {
  if (!m) return;
  for (int l = 0; l < m->c.num_layers; ++l) {
    free(m->layers[l].k_cache); free(m->layers[l].v_cache);
    for (int n = 0; n < N_NNORM; ++n) free(m->layers[l].norm[n]);
  }
  free(m->layers); free(m->out_norm);
  free(m->hidden); free(m->residual); free(m->normed); free(m->attn_proj); free(m->down);
  free(m->q); free(m->attn_out); free(m->k); free(m->v);
  free(m->gate); free(m->up); free(m->mul); free(m->scores); free(m->logits); free(m->hist);
  free(m);
}

static float* to_f32(uint32_t type, const void* data, size_t nbytes, size_t* n_out) {
  size_t n = type == 0 ? nbytes / 4 : nbytes / 2;
  float* f = (float*)malloc(n * 4);
  if (type == 0) memcpy(f, data, n * 4);
  else gor_f16_to_f32_n((const uint16_t*)data, n, f);
  *n_out = n;
  return f;
}

int gor_model_set_tensor(gor_model* m, const char* name, uint32_t type,
                         const void* data, size_t nbytes) {
  size_t n;
  if (strcmp(name, "token_embd.weight") == 0) {
    if (type != 8) return -1;
    m->embd = (const uint8_t*)data;
    return 0;
  }
  if (strcmp(name, "output_norm.weight") == 0) {
    if (type != 0 && type != 1) return -1;
    free(m->out_norm);
    m->out_norm = to_f32(type, data, nbytes, &n);
    return 0;
  }
  int layer = -1, off = 0;
  if (sscanf(name, "blk.%d.%n", &layer, &off) != 1 || layer < 0 || layer >= m->c.num_layers) return -2;
  const char* key = name + off;
  size_t klen = strlen(key);
  if (klen < 8 || strcmp(key + klen - 7, ".weight") != 0) return -2;
  char base[64];
  if (klen - 7 >= sizeof(base)) return -2;
  memcpy(base, key, klen - 7); base[klen - 7] = 0;
  for (int i = 0; i < L_NQ8; ++i)
    if (strcmp(base, q8_names[i]) == 0) {
      if (type != 8) return -1;
      m->layers[layer].q8[i] = (const uint8_t*)data;
      return 0;
    }
  for (int i = 0; i < N_NNORM; ++i)
    if (strcmp(base, norm_names[i]) == 0) {
      if (type != 0 && type != 1) return -1;
      free(m->layers[layer].norm[i]);
      m->layers[layer].norm[i] = to_f32(type, data, nbytes, &n);
      return 0;
    }
  return -2;
}

void gor_model_reset_kv(gor_model* m) {
  size_t kv = (size_t)m->c.context_length * m->kv_dim;
  for (int l = 0; l < m->c.num_layers; ++l) {
    memset(m->layers[l].k_cache, 0, kv * 4);
    memset(m->layers[l].v_cache, 0, kv * 4);
  }
}

/* types.ts:38-40 */
static int is_swa_layer(const gor_config* c, int il) {
  return (il % c->swa_period) < (c->swa_period - 1);
}

/* engine.ts:735-802 -- one token through every layer, ending with the final
 * rmsNorm into `normed`. */
int gor_model_forward(gor_model* m, int token, int pos) {
  const gor_config* c = &m->c;
  int H = c->hidden_size, I = c->intermediate_size, HD = c->head_dim;
  if (pos < 0 || pos >= c->context_length || token < 0 || token >= c->vocab_size) return -1;
  float scale = (float)(1.0 / sqrt((double)HD));           /* engine.ts:200 */
  gor_embed(m->embd, token, H, m->hidden);
  for (int l = 0; l < c->num_layers; ++l) {
    gor_layer* L = &m->layers[l];
    int swa = is_swa_layer(c, l);
    float theta = swa ? c->rope_theta_local : c->rope_theta_global;   /* types.ts:42-44 */
    int t_lo = 0;
    if (swa && c->sliding_window > 0 && pos - c->sliding_window + 1 > 0) t_lo = pos - c->sliding_window + 1;
    gor_rms_norm(m->hidden, L->norm[N_ATTN], m->normed, H, c->rms_norm_eps);
    gor_linear_q8(L->q8[L_ATTN_Q], m->normed, m->q, m->q_dim, H);
    gor_linear_q8(L->q8[L_ATTN_K], m->normed, m->k, m->kv_dim, H);
    gor_linear_q8(L->q8[L_ATTN_V], m->normed, m->v, m->kv_dim, H);
    gor_per_head_norm_rope(m->q, L->norm[N_QN], c->num_q_heads, HD, c->rms_norm_eps, pos, theta);
    gor_per_head_norm_rope(m->k, L->norm[N_KN], c->num_kv_heads, HD, c->rms_norm_eps, pos, theta);
    memcpy(L->k_cache + (size_t)pos * m->kv_dim, m->k, (size_t)m->kv_dim * 4);   /* kvCacheStore */
    memcpy(L->v_cache + (size_t)pos * m->kv_dim, m->v, (size_t)m->kv_dim * 4);
    gor_attention(m->q, L->k_cache, L->v_cache, c->num_q_heads, c->num_kv_heads, HD,
                  t_lo, pos, scale, m->scores, m->attn_out);
    gor_linear_q8(L->q8[L_ATTN_O], m->attn_out, m->attn_proj, H, m->q_dim);
    gor_fused_norm_add(m->attn_proj, L->norm[N_POST_ATTN], m->hidden, m->residual, H, c->rms_norm_eps);
    gor_rms_norm(m->residual, L->norm[N_FFN], m->normed, H, c->rms_norm_eps);
    gor_linear_q8(L->q8[L_FFN_GATE], m->normed, m->gate, I, H);
    gor_linear_q8(L->q8[L_FFN_UP], m->normed, m->up, I, H);
    gor_gelu_mul(m->gate, m->up, m->mul, I);
    gor_linear_q8(L->q8[L_FFN_DOWN], m->mul, m->down, H, I);
    gor_fused_norm_add(m->down, L->norm[N_POST_FFW], m->residual, m->hidden, H, c->rms_norm_eps);
    memcpy(m->hist + (size_t)l * H, m->hidden, (size_t)H * 4);
  }
  gor_rms_norm(m->hidden, m->out_norm, m->normed, H, c->rms_norm_eps);
  return 0;
}

/* engine.ts:817-821 -- LM head: linearQ8 with the tied embedding. */
void gor_model_lm_head(gor_model* m) {
  gor_linear_q8(m->embd, m->normed, m->logits, m->c.vocab_size, m->c.hidden_size);
}

/* engine.ts:805-902 -- LM head then greedy argmax or topk256 + sampler. */
int gor_model_select(gor_model* m, double temperature, double top_p, double rep_penalty,
                     double u, const int32_t* seen, int n_seen) {
  gor_model_lm_head(m);
  int V = m->c.vocab_size;
  if (temperature == 0.0 && rep_penalty <= 1.0) return gor_argmax(m->logits, V);
  float vals[256]; uint32_t ids[256];
  gor_topk256(m->logits, V, vals, ids);
  uint32_t* bm = (uint32_t*)calloc(8192, 4);
  for (int i = 0; i < n_seen; ++i)
    if (seen[i] >= 0 && seen[i] < 262144) bm[seen[i] >> 5] |= 1u << (seen[i] & 31);
  int r = gor_sample_candidates(vals, ids, bm, temperature, top_p, rep_penalty, u);
  free(bm);
  return r;
}

float* gor_model_buffer(gor_model* m, int what, int layer) {
  switch (what) {
    case GOR_HIDDEN: return m->hidden;
    case GOR_NORMED: return m->normed;
    case GOR_LOGITS: return m->logits;
    case GOR_LAYER_HIDDEN: return m->hist + (size_t)layer * m->c.hidden_size;
    case GOR_K_CACHE: return m->layers[layer].k_cache;
    case GOR_V_CACHE: return m->layers[layer].v_cache;
    case GOR_Q: return m->q;
    case GOR_ATTN_OUT: return m->attn_out;
  }
  return NULL;
}

void gor_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int gor_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

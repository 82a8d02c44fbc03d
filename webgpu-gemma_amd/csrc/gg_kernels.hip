// gg_kernels.hip -- gfx950 (CDNA4) kernels of the Gemma-3 Q8_0 token loop.
//
// One forward pass over a token is five kernels per layer:
//   k_gemv<EMBED_NORM|RESID_NORM, PARTIAL>  fused QKV projection; its prologue
//        finishes the previous layer (post-FFN norm + residual) and applies
//        attn_norm (engine.ts:768-774, 794)
//   k_attn      QK-norm + RoPE + KV store + split-K decode attention with the
//               last-arriving block combining the chunks (engine.ts:775-783)
//   k_gemv<NONE, PARTIAL>       attention output projection (engine.ts:784)
//   k_gemv<RESID_NORM, GEGLU>   post-attn norm + residual + ffn_norm, gate and
//               up rows side by side, GeGLU in the epilogue (engine.ts:785-792)
//   k_gemv<NONE, PARTIAL>       down projection (engine.ts:793)
// then k_final (post-FFN norm + residual + output_norm, engine.ts:794-801),
// and for a sampled step the LM head GEMV plus k_select (engine.ts:817-901).
//
// All arithmetic is fp32 except the int8 weight payload (dequantised exactly
// in registers) and the sampler's f64 steps, which mirror the JS host's.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gg_internal.h"

namespace gg {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sbyte(uint32_t w, int b) {
  // compiles to v_cvt_f32_i32_sdwa with a sign-extended byte select
  return (float)(int8_t)(w >> (8 * b));
}
__device__ __forceinline__ float f16_lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over a 256-thread block; every thread gets the same value.
__device__ __forceinline__ float block_sum256(float v, float* sh4) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh4[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((sh4[0] + sh4[1]) + sh4[2]) + sh4[3];
}
__device__ __forceinline__ float block_max256(float v, float* sh4) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh4[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(sh4[0], sh4[1]), fmaxf(sh4[2], sh4[3]));
}

// One 68-byte pair = blocks 2c and 2c+1 of a row: 17 dwords.
struct Pair {
  uint32_t w[17];
};

__device__ __forceinline__ void load_pair(const uint8_t* p, Pair& P) {
  const u32x4a4 a = *(const u32x4a4*)(p);
  const u32x4a4 b = *(const u32x4a4*)(p + 16);
  const u32x4a4 c = *(const u32x4a4*)(p + 32);
  const u32x4a4 d = *(const u32x4a4*)(p + 48);
  P.w[0] = a.x; P.w[1] = a.y; P.w[2] = a.z; P.w[3] = a.w;
  P.w[4] = b.x; P.w[5] = b.y; P.w[6] = b.z; P.w[7] = b.w;
  P.w[8] = c.x; P.w[9] = c.y; P.w[10] = c.z; P.w[11] = c.w;
  P.w[12] = d.x; P.w[13] = d.y; P.w[14] = d.z; P.w[15] = d.w;
  P.w[16] = *(const uint32_t*)(p + 64);
}

// acc += (sum_j q0[j] x[j]) * d0 + (sum_j q1[j] x[32+j]) * d1, each block sum
// running over j in order like linearQ8 (shaders.ts:123-142).
// Pair bytes: [0,2) d0 | [2,34) q0 | [34,36) d1 | [36,68) q1.
__device__ __forceinline__ float dot_pair(const Pair& P, const float* __restrict__ xc, float acc) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) s0 = fmaf(sbyte(P.w[(2 + j) >> 2], (2 + j) & 3), xc[j], s0);
#pragma unroll
  for (int j = 0; j < 32; ++j) s1 = fmaf(sbyte(P.w[9 + (j >> 2)], j & 3), xc[32 + j], s1);
  acc = fmaf(s0, f16_lo(P.w[0]), acc);
  acc = fmaf(s1, f16_hi(P.w[8]), acc);
  return acc;
}

// shaders.ts:153-170 (tanh GELU, argument clamped to +-15) times up.
__device__ __forceinline__ float gelu_mul(float x, float up) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  float a = 1.0f + (k1 * x) * x;
  float arg = (k0 * x) * a;
  arg = fminf(fmaxf(arg, -15.0f), 15.0f);
  float g = (0.5f * x) * (1.0f + tanhf(arg));
  return g * up;
}

// ---------------------------------------------------------------------------
// GEMV prologues: build the GEMV input x (K floats) in LDS.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float embed_elem(const GemvArgs& a, int token, int e) {
  // shaders.ts:2-23: (f32(q) * scale) * sqrt(f32(H)), row `token` of the
  // tied embedding, read from the pair-interleaved layout.
  const int g = token >> 6, ln = token & 63;
  const int b = e >> 5, c = b >> 1;
  const uint8_t* pr = a.embd + (((size_t)g * a.Kp_embd + c) * 64 + ln) * kPairBytes;
  const int off = (b & 1) ? 34 : 0;
  const uint16_t sb = (uint16_t)(pr[off] | (pr[off + 1] << 8));
  const float scale = (float)__builtin_bit_cast(_Float16, sb);
  const float q = (float)(int8_t)pr[off + 2 + (e & 31)];
  const float t = q * scale;
  return t * a.embed_scale;
}

template <int PRO>
__device__ __forceinline__ void gemv_prologue(const GemvArgs& a, float* xs, int K, float* sh4) {
  const int tid = threadIdx.x;
  if (PRO == PRO_NONE) {
    for (int e = tid; e < K; e += 256) xs[e] = a.x[e];
    return;
  }
  float ss = 0.f;
  if (PRO == PRO_EMBED_NORM) {
    const int token = a.tokens[a.st->cursor];
    for (int e = tid; e < K; e += 256) {
      const float h = embed_elem(a, token, e);
      xs[e] = h;
      ss = fmaf(h, h, ss);
      if (blockIdx.x == 0) a.res_out[e] = h;
    }
  } else {  // PRO_RESID_NORM: res = pre_res + norm(sum(parts)) * w_post
    float s1 = 0.f;
    for (int e = tid; e < K; e += 256) {
      float v = 0.f;
      for (int p = 0; p < a.pre_S; ++p) v += a.pre_part[(size_t)p * K + e];
      xs[e] = v;
      s1 = fmaf(v, v, s1);
    }
    const float ss1 = block_sum256(s1, sh4);
    const float rms1 = sqrtf(ss1 / (float)K + a.eps);
    for (int e = tid; e < K; e += 256) {
      const float t = (xs[e] * a.w_post[e]) / rms1;   // fusedNormAdd, shaders.ts:415
      const float r = a.pre_res[e] + t;
      xs[e] = r;
      ss = fmaf(r, r, ss);
      if (blockIdx.x == 0) {
        a.res_out[e] = r;
        if (a.hist_out) a.hist_out[e] = r;
      }
    }
  }
  const float ss2 = block_sum256(ss, sh4);
  const float rms = sqrtf(ss2 / (float)K + a.eps);       // rmsNorm, shaders.ts:50-53
  for (int e = tid; e < K; e += 256) xs[e] = (xs[e] * a.w_pre[e]) / rms;
}

// ---------------------------------------------------------------------------
// Q8_0 dequant-GEMV. Block = 256 threads = 4 wavefronts on one 64-row group;
// the block's pair-columns [c0, c1) are dealt round-robin to the waves, each
// lane owns one row. blockIdx.x = g * S + s.
// ---------------------------------------------------------------------------
template <int PRO, int EPI>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  extern __shared__ float xs[];
  __shared__ float red[4][64];
  __shared__ float sh4[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = blockIdx.x / a.S, s = blockIdx.x - g * a.S;
  const int c0 = s * a.CS;
  const int c1 = min(c0 + a.CS, a.Kp);
  const int K = a.Kp * 64;
  const uint8_t* base = a.W + ((size_t)g * a.Kp * 64 + lane) * kPairBytes;

  // Weights do not depend on x: start streaming before the prologue.
  int c = c0 + wv;
  Pair cur;
  if (c < c1) load_pair(base + (size_t)c * kColBytes, cur);

  gemv_prologue<PRO>(a, xs, K, sh4);
  __syncthreads();

  float acc = 0.f;
  for (; c < c1; c += 4) {
    const int cn = min(c + 4, c1 - 1);
    Pair nxt;
    load_pair(base + (size_t)cn * kColBytes, nxt);
    acc = dot_pair(cur, xs + c * 64, acc);
    cur = nxt;
  }
  red[wv][lane] = acc;
  __syncthreads();
  if (wv != 0) return;
  const float r = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
  const int row = g * 64 + lane;
  if (EPI == EPI_PARTIAL) {
    a.out[(size_t)s * a.N + row] = r;
  } else {
    // rows 32g'+i (gate) sit in lanes 0..31, the matching up rows in 32..63
    const float up = __shfl(r, lane + 32, 64);
    if (lane < 32) a.act_out[g * 32 + lane] = gelu_mul(r, up);
  }
}

__global__ __launch_bounds__(256) void k_sum_parts(const float* __restrict__ parts, int S, int N,
                                                   float* __restrict__ y) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  float v = 0.f;
  for (int p = 0; p < S; ++p) v += parts[(size_t)p * N + i];
  y[i] = v;
}

// ---------------------------------------------------------------------------
// Decode attention (one KV head, head_dim 256).
// Block b covers positions [t0, t1) of the attended span [t_lo, pos]; the
// chunk size grows with the span so at most kAttnMaxChunks blocks are live.
// Every block rebuilds q/k/v from the QKV partials and applies the per-head
// RMSNorm + NEOX RoPE itself (fusedPerHeadNormRope, shaders.ts:420-467); the
// block holding `pos` also stores k/v into the cache (kvCacheStore,
// shaders.ts:209-227). Scores/softmax/weighted-V follow shaders.ts:229-325
// per chunk; the last block to finish merges the chunks with the usual
// max-rescaled sums.
// ---------------------------------------------------------------------------
constexpr int kAttnMaxCh = 256;

__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
  __shared__ float qs[kMaxQHeads][kHeadDim];
  __shared__ float ks[kHeadDim];
  __shared__ float vs[kHeadDim];
  __shared__ float sc[kMaxQHeads][kAttnMaxCh];
  __shared__ float mh[kMaxQHeads], lh[kMaxQHeads];
  __shared__ float fac[kAttnMaxChunks];
  __shared__ float sh4[4];
  __shared__ int is_last;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nq = a.n_q;
  const int pos = a.st->pos;
  const int t_lo = a.window > 0 ? max(0, pos - a.window + 1) : 0;
  const int span = pos - t_lo + 1;
  const int ch = 32 * ((span + 32 * kAttnMaxChunks - 1) / (32 * kAttnMaxChunks));
  const int nch = (span + ch - 1) / ch;
  const int b = blockIdx.x;
  if (b >= nch) return;
  const int t0 = t_lo + b * ch;
  const int t1 = min(t0 + ch, pos + 1);

  // 1. q, k, v = sum of the QKV partials
  const int nqd = nq * kHeadDim;
  const int nel = nqd + 2 * kHeadDim;
  for (int e = tid; e < nel; e += 256) {
    float v = 0.f;
    for (int p = 0; p < a.S; ++p) v += a.qkv_part[(size_t)p * nel + e];
    if (e < nqd) qs[e >> 8][e & 255] = v;
    else if (e < nqd + kHeadDim) ks[e - nqd] = v;
    else vs[e - nqd - kHeadDim] = v;
  }
  __syncthreads();

  // 2. per-head RMSNorm (q heads, then the k head)
  for (int h = wv; h <= nq; h += 4) {
    float* hp = (h < nq) ? qs[h] : ks;
    const float* w = (h < nq) ? a.q_norm : a.k_norm;
    float x[4];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[i] = hp[lane + 64 * i]; ss = fmaf(x[i], x[i], ss); }
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)kHeadDim + a.eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) hp[lane + 64 * i] = (x[i] * w[lane + 64 * i]) / rms;
  }
  __syncthreads();

  // 3. NEOX RoPE on pairs (i, i+128): angle = f32(pos) * freq[i]
  for (int idx = tid; idx < (nq + 1) * (kHeadDim / 2); idx += 256) {
    const int h = idx >> 7, i = idx & 127;
    float* hp = (h < nq) ? qs[h] : ks;
    const float angle = (float)pos * a.freq[i];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    const float x0 = hp[i], x1 = hp[i + 128];
    hp[i] = x0 * cs - x1 * sn;
    hp[i + 128] = x0 * sn + x1 * cs;
  }
  __syncthreads();

  if (b == nch - 1) {
    a.k_cache[(size_t)pos * kHeadDim + tid] = ks[tid];
    a.v_cache[(size_t)pos * kHeadDim + tid] = vs[tid];
  }
  if (b == 0 && a.q_dbg)
    for (int e = tid; e < nqd; e += 256) a.q_dbg[e] = qs[e >> 8][e & 255];

  // 4. scores: wave w takes positions t0+w, t0+w+4, ...; lane holds 4 dims
  float4 q4[kMaxQHeads];
#pragma unroll
  for (int h = 0; h < kMaxQHeads; ++h)
    q4[h] = (h < nq) ? *(const float4*)&qs[h][4 * lane] : make_float4(0.f, 0.f, 0.f, 0.f);
  for (int t = t0 + wv; t < t1; t += 4) {
    float4 k4;
    if (t == pos) k4 = *(const float4*)&ks[4 * lane];
    else k4 = *(const float4*)(a.k_cache + (size_t)t * kHeadDim + 4 * lane);
#pragma unroll
    for (int h = 0; h < kMaxQHeads; ++h) {
      if (h < nq) {
        float d = q4[h].x * k4.x;
        d = fmaf(q4[h].y, k4.y, d);
        d = fmaf(q4[h].z, k4.z, d);
        d = fmaf(q4[h].w, k4.w, d);
        d = wave_sum(d);
        if (lane == 0) sc[h][t - t0] = d * a.scale;
      }
    }
  }
  __syncthreads();

  // 5. chunk softmax statistics
  const int n = t1 - t0;
  for (int h = wv; h < nq; h += 4) {
    float m = -INFINITY;
    for (int j = lane; j < n; j += 64) m = fmaxf(m, sc[h][j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < n; j += 64) {
      const float p = expf(sc[h][j] - m);
      sc[h][j] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) { mh[h] = m; lh[h] = l; }
  }
  __syncthreads();

  // 6. o[h][d] = sum_t p[h][t] * V[t][d]; thread = dimension
  float acc[kMaxQHeads];
#pragma unroll
  for (int h = 0; h < kMaxQHeads; ++h) acc[h] = 0.f;
  for (int t = t0; t < t1; ++t) {
    const float v = (t == pos) ? vs[tid] : a.v_cache[(size_t)t * kHeadDim + tid];
#pragma unroll
    for (int h = 0; h < kMaxQHeads; ++h)
      if (h < nq) acc[h] = fmaf(sc[h][t - t0], v, acc[h]);
  }
  const size_t pstride = (size_t)nq * (2 + kHeadDim);
  float* mypart = a.part + (size_t)b * pstride;
#pragma unroll
  for (int h = 0; h < kMaxQHeads; ++h)
    if (h < nq) mypart[h * (2 + kHeadDim) + 2 + tid] = acc[h];
  if (tid < nq) {
    mypart[tid * (2 + kHeadDim)] = mh[tid];
    mypart[tid * (2 + kHeadDim) + 1] = lh[tid];
  }

  // 7. the last block to arrive merges all chunks
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned int old =
        __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (old == (unsigned int)(nch - 1));
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int h = 0; h < nq; ++h) {
    float m = -INFINITY;
    for (int cc = tid; cc < nch; cc += 256) m = fmaxf(m, a.part[(size_t)cc * pstride + h * (2 + kHeadDim)]);
    const float M = block_max256(m, sh4);
    float l = 0.f;
    for (int cc = tid; cc < nch; cc += 256) {
      const float* pp = a.part + (size_t)cc * pstride + h * (2 + kHeadDim);
      const float f = expf(pp[0] - M);
      fac[cc] = f;
      l = fmaf(f, pp[1], l);
    }
    const float L = block_sum256(l, sh4);   // barrier also publishes fac[]
    float o = 0.f;
    for (int cc = 0; cc < nch; ++cc)
      o = fmaf(fac[cc], a.part[(size_t)cc * pstride + h * (2 + kHeadDim) + 2 + tid], o);
    a.attn_out[h * kHeadDim + tid] = o / L;
    __syncthreads();
  }
  if (tid == 0) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// End of a forward pass: hidden = residual + norm(down) * post_ffw_norm, then
// normed = rmsNorm(hidden, output_norm) (engine.ts:794-801); advance pos.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_final(FinalArgs a) {
  extern __shared__ float hs[];
  __shared__ float sh4[4];
  const int tid = threadIdx.x, H = a.H;
  float s1 = 0.f;
  for (int e = tid; e < H; e += 256) {
    float v = 0.f;
    for (int p = 0; p < a.pre_S; ++p) v += a.pre_part[(size_t)p * H + e];
    hs[e] = v;
    s1 = fmaf(v, v, s1);
  }
  const float rms1 = sqrtf(block_sum256(s1, sh4) / (float)H + a.eps);
  float s2 = 0.f;
  for (int e = tid; e < H; e += 256) {
    const float r = a.pre_res[e] + (hs[e] * a.w_post[e]) / rms1;
    hs[e] = r;
    a.hidden[e] = r;
    if (a.hist_out) a.hist_out[e] = r;
    s2 = fmaf(r, r, s2);
  }
  const float rms2 = sqrtf(block_sum256(s2, sh4) / (float)H + a.eps);
  for (int e = tid; e < H; e += 256) a.normed[e] = (hs[e] * a.w_out[e]) / rms2;
  if (tid == 0) {
    a.st->pos += 1;
    a.st->cursor += 1;
  }
}

// ---------------------------------------------------------------------------
// Token selection over the logits (engine.ts:823-901).
// Stage 1 (every block): per stride class c = i mod 256, the first index of
// the class maximum over the block's stripes (strict >, init (-1e30, 0)), as
// in argmax/topk256 (shaders.ts:337-347, 371-381).
// Stage 2 (last block): merge stripes in order -> topk256; then either the
// argmax halving tree (shaders.ts:351-357) or the host sampler
// (engine.ts:862-901): repetition penalty in f64, stable descending sort,
// f32-stored exp, f64 sums, top-p cutoff, walk with the injected draw u.
// ---------------------------------------------------------------------------
struct Cand {
  double val;
  int ord;
  uint32_t id;
};

__device__ __forceinline__ bool cand_before(const Cand& x, const Cand& y) {
  return x.val > y.val || (x.val == y.val && x.ord < y.ord);
}

__global__ __launch_bounds__(256) void k_select(SelectArgs a) {
  __shared__ float tv[256];
  __shared__ uint32_t ti[256];
  __shared__ Cand cs[256];
  __shared__ float probs[256];
  __shared__ int is_last;
  __shared__ int tok_sh;
  const int tid = threadIdx.x;
  const int nb = gridDim.x;
  const int stripes = (a.V + 255) / 256;
  const int per = (stripes + nb - 1) / nb;
  const int j0 = blockIdx.x * per, j1 = min(j0 + per, stripes);
  float m = -1e30f;
  uint32_t id = 0;
  for (int j = j0; j < j1; ++j) {
    const int i = j * 256 + tid;
    if (i < a.V) {
      const float v = a.logits[i];
      if (v > m) { m = v; id = (uint32_t)i; }
    }
  }
  a.cand_val[blockIdx.x * 256 + tid] = m;
  a.cand_id[blockIdx.x * 256 + tid] = id;
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned int old =
        __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (old == (unsigned int)(nb - 1));
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();

  // stage 2: class maxima in stripe order
  m = -1e30f;
  id = 0;
  for (int bb = 0; bb < nb; ++bb) {
    const float v = a.cand_val[bb * 256 + tid];
    if (v > m) { m = v; id = a.cand_id[bb * 256 + tid]; }
  }
  tv[tid] = m;
  ti[tid] = id;
  a.top[2 * tid] = __float_as_uint(m);
  a.top[2 * tid + 1] = id;
  __syncthreads();

  const DevState* st = a.st;
  const double T = st->temperature, rep = st->rep_penalty;
  int token;
  if (T == 0.0 && rep <= 1.0) {
    for (int stride = 128; stride > 0; stride >>= 1) {
      if (tid < stride && tv[tid + stride] > tv[tid]) {
        tv[tid] = tv[tid + stride];
        ti[tid] = ti[tid + stride];
      }
      __syncthreads();
    }
    token = (int)ti[0];
  } else {
    Cand cd;
    cd.val = (double)m;
    cd.ord = tid;
    cd.id = id;
    if (rep > 1.0 && st->seen_count > 0 && id < (uint32_t)a.V &&
        ((a.seen[id >> 5] >> (id & 31)) & 1u)) {
      if (cd.val > 0) cd.val /= rep;
      else cd.val *= rep;
    }
    cs[tid] = cd;
    __syncthreads();
    for (int k = 2; k <= 256; k <<= 1) {
      for (int jj = k >> 1; jj > 0; jj >>= 1) {
        const int ixj = tid ^ jj;
        if (ixj > tid) {
          const bool up = (tid & k) == 0;
          const Cand x = cs[tid], y = cs[ixj];
          const bool sw = up ? cand_before(y, x) : cand_before(x, y);
          if (sw) { cs[tid] = y; cs[ixj] = x; }
        }
        __syncthreads();
      }
    }
    if (T == 0.0) {
      token = (int)cs[0].id;
    } else {
      probs[tid] = (float)exp((cs[tid].val - cs[0].val) / T);
      __syncthreads();
      if (tid == 0) {
        double sum = 0.0;
        for (int i = 0; i < 256; ++i) sum += (double)probs[i];
        double cum = 0.0;
        int cutoff = 256;
        for (int i = 0; i < 256; ++i) {
          cum += (double)probs[i] / sum;
          if (cum >= st->top_p) { cutoff = i + 1; break; }
        }
        double subset = 0.0;
        for (int i = 0; i < cutoff; ++i) subset += (double)probs[i];
        double r = st->u * subset;
        int pick = -1;
        for (int i = 0; i < cutoff; ++i) {
          r -= (double)probs[i];
          if (r <= 0) { pick = i; break; }
        }
        if (pick < 0) pick = cutoff - 1;
        tok_sh = (int)cs[pick].id;
      }
      __syncthreads();
      token = tok_sh;
    }
  }
  if (tid == 0) {
    a.st->out_token = token;
    if (a.out_token) *a.out_token = token;
    if (a.auto_add && token >= 0 && token < a.V) {
      a.seen[token >> 5] |= 1u << (token & 31);
      a.st->seen_count += 1;
    }
    __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Upload helpers.
// k_repack: GGUF row-major Q8_0 (rows of Kp 68-byte pairs) -> pair-interleaved.
// interleave_half > 0 places source row r at fused row
// (r / half) * 64 + (r % half) + dst_row_offset, i.e. gate rows in lanes 0..31
// and (with dst_row_offset = 32) up rows in lanes 32..63 of each group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                long long rows, int Kp, long long off, int half) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = rows * Kp;
  if (idx >= total) return;
  const long long r = idx / Kp;
  const int c = (int)(idx - r * Kp);
  const long long R = half > 0 ? (r / half) * 64 + (r % half) + off : r + off;
  const long long g = R >> 6;
  const int ln = (int)(R & 63);
  const uint32_t* s = (const uint32_t*)(src + (size_t)idx * kPairBytes);
  uint32_t* d = (uint32_t*)(dst + (((size_t)g * Kp + c) * 64 + ln) * kPairBytes);
#pragma unroll
  for (int i = 0; i < 17; ++i) d[i] = s[i];
}

// Bit-exact Q8_0 dequantisation of GGUF blocks (gguf.ts:107-124).
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ src, float* __restrict__ out,
                                                 long long n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint8_t* blk = src + (size_t)(i >> 5) * 34;
  const uint16_t sb = (uint16_t)(blk[0] | (blk[1] << 8));
  const float scale = (float)__builtin_bit_cast(_Float16, sb);
  out[i] = (float)(int8_t)blk[2 + (i & 31)] * scale;
}

// Add ids to the repetition-penalty bitmap (the turn's prompt tokens).
__global__ __launch_bounds__(256) void k_seen_add(uint32_t* seen, DevState* st, const int32_t* ids, int n,
                                                  int V) {
  for (int i = threadIdx.x; i < n; i += 256) {
    const int id = ids[i];
    if (id >= 0 && id < V) atomicOr(&seen[id >> 5], 1u << (id & 31));
  }
  if (threadIdx.x == 0) st->seen_count += n;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int PRO, int EPI>
static int launch_gemv_t(const GemvArgs& a, hipStream_t s) {
  const size_t lds = (size_t)a.Kp * 64 * sizeof(float);
  hipLaunchKernelGGL((k_gemv<PRO, EPI>), dim3(a.G * a.S), dim3(256), lds, s, a);
  return (int)hipGetLastError();
}

int launch_gemv(int pro, int epi, const GemvArgs& a, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (a.Kp * 64 > kMaxK || a.Kp <= 0 || a.G <= 0 || a.S <= 0 || a.CS <= 0) return (int)hipErrorInvalidValue;
  if (epi == EPI_GEGLU && a.S != 1) return (int)hipErrorInvalidValue;
  if (pro == PRO_NONE && epi == EPI_PARTIAL) return launch_gemv_t<PRO_NONE, EPI_PARTIAL>(a, s);
  if (pro == PRO_EMBED_NORM && epi == EPI_PARTIAL) return launch_gemv_t<PRO_EMBED_NORM, EPI_PARTIAL>(a, s);
  if (pro == PRO_RESID_NORM && epi == EPI_PARTIAL) return launch_gemv_t<PRO_RESID_NORM, EPI_PARTIAL>(a, s);
  if (pro == PRO_RESID_NORM && epi == EPI_GEGLU) return launch_gemv_t<PRO_RESID_NORM, EPI_GEGLU>(a, s);
  return (int)hipErrorInvalidValue;
}

int launch_sum_parts(const float* parts, int S, int N, float* y, void* stream) {
  hipLaunchKernelGGL(k_sum_parts, dim3((N + 255) / 256), dim3(256), 0, (hipStream_t)stream, parts, S, N, y);
  return (int)hipGetLastError();
}

int launch_attention(const AttnArgs& a, int grid, void* stream) {
  if (a.n_q < 1 || a.n_q > kMaxQHeads || grid < 1 || grid > kAttnMaxChunks) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn, dim3(grid), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_final(const FinalArgs& a, void* stream) {
  hipLaunchKernelGGL(k_final, dim3(1), dim3(256), (size_t)a.H * sizeof(float), (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_select(const SelectArgs& a, void* stream) {
  const int stripes = (a.V + 255) / 256;
  const int nb = stripes < kSelBlocks ? stripes : kSelBlocks;
  hipLaunchKernelGGL(k_select, dim3(nb), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_repack(const uint8_t* src, uint8_t* dst, long long rows, int Kp, long long off, int half,
                  void* stream) {
  const long long total = rows * Kp;
  if (total <= 0) return 0;
  hipLaunchKernelGGL(k_repack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src,
                     dst, rows, Kp, off, half);
  return (int)hipGetLastError();
}

int launch_dequant(const uint8_t* src, float* out, long long n, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src, out,
                     n);
  return (int)hipGetLastError();
}

int launch_seen_add(uint32_t* seen, DevState* st, const int32_t* ids, int n, int V, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_seen_add, dim3(1), dim3(256), 0, (hipStream_t)stream, seen, st, ids, n, V);
  return (int)hipGetLastError();
}

}  // namespace gg

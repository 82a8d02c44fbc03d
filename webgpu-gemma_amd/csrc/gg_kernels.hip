// gg_kernels.hip -- gfx950 (CDNA4) kernels of the Gemma-3 Q8_0 token loop.
//
// One forward pass over a token is six kernels per layer:
//   k_gemv<EMBED_NORM|RESID_NORM, OUT>  fused QKV projection; its prologue
//        finishes the previous layer (post-FFN norm + residual) and applies
//        attn_norm (engine.ts:768-774, 794)
//   k_attn          QK-norm + RoPE + KV store + one chunk of decode attention
//                   per block (engine.ts:775-783)
//   k_attn_combine  merge of the chunk softmax statistics
//   k_gemv<NONE, OUT>          attention output projection (engine.ts:784)
//   k_gemv<RESID_NORM, GEGLU>  post-attn norm + residual + ffn_norm, gate and
//                   up rows side by side, GeGLU in the epilogue (engine.ts:785-792)
//   k_gemv<NONE, OUT>          down projection (engine.ts:793)
// then k_final (post-FFN norm + residual + output_norm, engine.ts:794-801),
// and for a sampled step the LM head GEMV plus k_select1/k_select2
// (engine.ts:817-901).
//
// No kernel communicates between its blocks: on this multi-XCD part a
// device-scope fence is an L2 write-back, so every cross-block dependency is
// a kernel boundary of the captured graph instead.
//
// All arithmetic is fp32 except the int8 weight payload (dequantised exactly
// in registers) and the sampler's f64 steps, which mirror the JS host's.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gg_internal.h"

namespace gg {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kXPad = 68;          // LDS floats per 64-wide x segment (4 pad: no bank conflicts)
constexpr int kAttnMaxCh = 256;    // largest attention chunk (positions per block)

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

__device__ __forceinline__ int xs_index(int e) { return (e >> 6) * kXPad + (e & 63); }

// ---------------------------------------------------------------------------
// GEMV prologues: build the GEMV input x (K floats) in LDS.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float embed_elem(const GemvArgs& a, int token, int e) {
  // shaders.ts:2-23: (f32(q) * scale) * sqrt(f32(H)), row `token` of the
  // tied embedding (layout with CI = 1, GR = 64).
  const int g = token >> 6, ln = token & 63;
  const int b = e >> 5, c = b >> 1;
  const uint8_t* pr = a.embd + (((size_t)g * a.embd_KpS + c) * 64 + ln) * kPairBytes;
  const int off = (b & 1) ? 34 : 0;
  const uint16_t sb = (uint16_t)(pr[off] | (pr[off + 1] << 8));
  const float scale = (float)__builtin_bit_cast(_Float16, sb);
  const float q = (float)(int8_t)pr[off + 2 + (e & 31)];
  const float t = q * scale;
  return t * a.embed_scale;
}

// Prologue inputs are read into registers before any reduction so that the
// prologue costs one memory latency, overlapped with the weight stream.
constexpr int kMaxEPT = kMaxK / 256;   // elements of x per thread

template <int PRO>
__device__ __forceinline__ void gemv_prologue(const GemvArgs& a, float* xs, int K, float* sh4) {
  const int tid = threadIdx.x;
  const int n = (K - tid + 255) / 256;   // elements this thread owns
  if (PRO == PRO_NONE) {
    float xv[kMaxEPT];
#pragma unroll
    for (int i = 0; i < kMaxEPT; ++i)
      if (i < n) xv[i] = a.x[tid + 256 * i];
#pragma unroll
    for (int i = 0; i < kMaxEPT; ++i)
      if (i < n) xs[xs_index(tid + 256 * i)] = xv[i];
    return;
  }
  float r[kMaxEPT / 4], wp[kMaxEPT / 4];  // K <= 2048 for the norm prologues
  float ss = 0.f;
  if (PRO == PRO_EMBED_NORM) {
    const int token = a.tokens[a.st->cursor];
#pragma unroll
    for (int i = 0; i < kMaxEPT / 4; ++i)
      if (i < n) {
        const int e = tid + 256 * i;
        r[i] = embed_elem(a, token, e);
        wp[i] = a.w_pre[e];
      }
#pragma unroll
    for (int i = 0; i < kMaxEPT / 4; ++i)
      if (i < n) {
        ss = fmaf(r[i], r[i], ss);
        if (blockIdx.x == 0) a.res_out[tid + 256 * i] = r[i];
      }
  } else {  // PRO_RESID_NORM: res = pre_res + norm(pre_vec) * w_post
    float v[kMaxEPT / 4], res[kMaxEPT / 4], wq[kMaxEPT / 4];
#pragma unroll
    for (int i = 0; i < kMaxEPT / 4; ++i)
      if (i < n) {
        const int e = tid + 256 * i;
        v[i] = a.pre_vec[e];
        res[i] = a.pre_res[e];
        wq[i] = a.w_post[e];
        wp[i] = a.w_pre[e];
      }
    float s1 = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxEPT / 4; ++i)
      if (i < n) s1 = fmaf(v[i], v[i], s1);
    const float rms1 = sqrtf(block_sum256(s1, sh4) / (float)K + a.eps);
#pragma unroll
    for (int i = 0; i < kMaxEPT / 4; ++i)
      if (i < n) {
        const float t = (v[i] * wq[i]) / rms1;   // fusedNormAdd, shaders.ts:415
        r[i] = res[i] + t;
        ss = fmaf(r[i], r[i], ss);
        if (blockIdx.x == 0) {
          a.res_out[tid + 256 * i] = r[i];
          if (a.hist_out) a.hist_out[tid + 256 * i] = r[i];
        }
      }
  }
  const float rms = sqrtf(block_sum256(ss, sh4) / (float)K + a.eps);   // rmsNorm, shaders.ts:50-53
#pragma unroll
  for (int i = 0; i < kMaxEPT / 4; ++i)
    if (i < n) xs[xs_index(tid + 256 * i)] = (r[i] * wp[i]) / rms;
}

// ---------------------------------------------------------------------------
// Q8_0 dequant-GEMV. Block = 256 threads = 4 wavefronts on one group of GR
// rows; lane l holds row l % GR and pair-column phase l / GR. Wave w takes
// column steps w, w+4, ...; each step is one 4352-byte contiguous load per
// wave. Up to kStepsInFlight steps per wave are issued at kernel entry,
// before the prologue (weights never depend on x), so a launch costs about
// one memory latency; longer rows continue with a two-step prefetch.
// ---------------------------------------------------------------------------
template <int PRO, int EPI, int CI, int kStepsInFlight>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  constexpr int GR = 64 / CI;
  extern __shared__ float xs[];
  __shared__ float red[4][GR];
  __shared__ float sh4[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = blockIdx.x;
  const int cp = lane / GR;
  const int Kp = a.Kp, KpS = a.KpS;
  const uint8_t* base = a.W + ((size_t)g * KpS * 64 + lane) * kPairBytes;

  Pair st[kStepsInFlight];
#pragma unroll
  for (int i = 0; i < kStepsInFlight; ++i) {
    const int s = wv + 4 * i;
    if (s < KpS && s * CI + cp < Kp) load_pair(base + (size_t)s * kColBytes, st[i]);
  }

  gemv_prologue<PRO>(a, xs, Kp * 64, sh4);
  __syncthreads();

  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < kStepsInFlight; ++i) {
    const int s = wv + 4 * i;
    const int c = s * CI + cp;
    if (s < KpS && c < Kp) acc = dot_pair(st[i], xs + c * kXPad, acc);
  }
  int s = wv + 4 * kStepsInFlight;
  if (s < KpS) {
    Pair cur, nxt;
    if (s * CI + cp < Kp) load_pair(base + (size_t)s * kColBytes, cur);
    if (s + 4 < KpS && (s + 4) * CI + cp < Kp) load_pair(base + (size_t)(s + 4) * kColBytes, nxt);
    for (; s < KpS; s += 4) {
      Pair nn;
      const int s3 = s + 8;
      if (s3 < KpS && s3 * CI + cp < Kp) load_pair(base + (size_t)s3 * kColBytes, nn);
      const int c = s * CI + cp;
      if (c < Kp) acc = dot_pair(cur, xs + c * kXPad, acc);
      cur = nxt;
      nxt = nn;
    }
  }
  // the CI column phases of a row sit in lanes r, r+GR, ...: butterfly sum
#pragma unroll
  for (int m = GR; m < 64; m <<= 1) acc += __shfl_xor(acc, m, 64);
  if (lane < GR) red[wv][lane] = acc;
  __syncthreads();
  if (wv != 0) return;
  const float r = lane < GR ? ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane] : 0.f;
  if (EPI == EPI_OUT) {
    if (lane < GR) a.out[g * GR + lane] = r;
  } else {
    // gate rows g*GR/2 + i sit in lanes 0..GR/2-1, the matching up rows in GR/2..GR-1
    const float up = __shfl(r, lane + GR / 2, 64);
    if (lane < GR / 2) a.act_out[g * (GR / 2) + lane] = gelu_mul(r, up);
  }
}

// ---------------------------------------------------------------------------
// Decode attention (one KV head, head_dim 256), one chunk of positions per
// block. Block b covers [t0, t1) of the attended span [t_lo, pos]; the chunk
// grows with the span so at most kAttnMaxChunks blocks are live. Every block
// rebuilds q/k from the QKV output with the per-head RMSNorm + NEOX RoPE
// (fusedPerHeadNormRope, shaders.ts:420-467); the block holding `pos` stores
// k/v into the cache (kvCacheStore, shaders.ts:209-227) and reads them from
// LDS. Scores/softmax/weighted-V follow shaders.ts:229-325 within the chunk
// and leave (max, sum, o) per head for k_attn_combine.
//
// Scores: wave w takes P = 64/NQP positions at a time with one float4 of the
// head per lane; the P*NQP = 64 partial dots per lane are finished by one
// reduce-scatter butterfly (63 shuffles) after which lane l owns dot l.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void attn_span(const AttnArgs& a, int pos, int* t_lo, int* ch, int* nch) {
  const int lo = a.window > 0 ? max(0, pos - a.window + 1) : 0;
  const int span = pos - lo + 1;
  const int c = kAttnChunk * ((span + kAttnChunk * kAttnMaxChunks - 1) / (kAttnChunk * kAttnMaxChunks));
  *t_lo = lo;
  *ch = c;
  *nch = (span + c - 1) / c;
}

template <int NQP>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
  constexpr int P = 64 / NQP;
  __shared__ float qs[NQP][kHeadDim];
  __shared__ float ks[kHeadDim];
  __shared__ float vs[kHeadDim];
  __shared__ float pw[4][64];
  __shared__ float wm[4][NQP], wl[4][NQP];
  __shared__ float wo[4][NQP][kHeadDim];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nq = a.n_q;
  const int pos = a.st->pos;
  int t_lo, ch, nch;
  attn_span(a, pos, &t_lo, &ch, &nch);
  const int b = blockIdx.x;
  if (b >= nch) return;
  const int t0 = t_lo + b * ch;
  const int t1 = min(t0 + ch, pos + 1);

  // 1. q, k, v from the QKV output (query heads beyond n_q are zero)
  const int nqd = nq * kHeadDim;
  for (int e = tid; e < NQP * kHeadDim; e += 256) qs[e >> 8][e & 255] = e < nqd ? a.qkv[e] : 0.f;
  ks[tid] = a.qkv[nqd + tid];
  vs[tid] = a.qkv[nqd + kHeadDim + tid];
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

  // 4. per-wave online softmax over passes of P positions; lane holds 4 dims
  float4 q4[NQP];
#pragma unroll
  for (int h = 0; h < NQP; ++h) q4[h] = *(const float4*)&qs[h][4 * lane];
  float m[NQP], l[NQP];
  float4 o4[NQP];
#pragma unroll
  for (int h = 0; h < NQP; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
    o4[h] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int my_h = lane % NQP;
  for (int tb = t0 + wv * P; tb < t1; tb += 4 * P) {
    float4 kr[P], vr[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int t = tb + i;
      if (t < pos) {
        kr[i] = *(const float4*)(a.k_cache + (size_t)t * kHeadDim + 4 * lane);
        vr[i] = *(const float4*)(a.v_cache + (size_t)t * kHeadDim + 4 * lane);
      } else if (t == pos) {
        kr[i] = *(const float4*)&ks[4 * lane];
        vr[i] = *(const float4*)&vs[4 * lane];
      } else {
        kr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        vr[i] = kr[i];
      }
    }
    float v[64];
#pragma unroll
    for (int i = 0; i < P; ++i)
#pragma unroll
      for (int h = 0; h < NQP; ++h) {
        float d = q4[h].x * kr[i].x;
        d = fmaf(q4[h].y, kr[i].y, d);
        d = fmaf(q4[h].z, kr[i].z, d);
        d = fmaf(q4[h].w, kr[i].w, d);
        v[i * NQP + h] = d;
      }
    // reduce-scatter: afterwards lane l owns the full dot of index l
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) {
      const bool hi = (lane & msk) != 0;
#pragma unroll
      for (int i = 0; i < msk; ++i) {
        const float send = hi ? v[i] : v[i + msk];
        const float keep = hi ? v[i + msk] : v[i];
        v[i] = keep + __shfl_xor(send, msk, 64);
      }
    }
    const bool valid = tb + lane / NQP < t1 && my_h < nq;
    const float sco = valid ? v[0] * a.scale : -INFINITY;
    // pass maximum of head my_h over the lanes holding that head
    float mx = sco;
#pragma unroll
    for (int msk = NQP; msk < 64; msk <<= 1) mx = fmaxf(mx, __shfl_xor(mx, msk, 64));
    float alpha[NQP], m_own = -INFINITY;
#pragma unroll
    for (int h = 0; h < NQP; ++h) {
      const float mn = fmaxf(m[h], __shfl(mx, h, 64));
      alpha[h] = (m[h] == -INFINITY) ? 0.f : expf(m[h] - mn);
      m[h] = mn;
      if (h == my_h) m_own = mn;
    }
    const float p = valid ? expf(sco - m_own) : 0.f;
    float ps = p;
#pragma unroll
    for (int msk = NQP; msk < 64; msk <<= 1) ps += __shfl_xor(ps, msk, 64);
    pw[wv][lane] = p;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < NQP; ++h) {
      l[h] = fmaf(l[h], alpha[h], __shfl(ps, h, 64));
      o4[h].x *= alpha[h];
      o4[h].y *= alpha[h];
      o4[h].z *= alpha[h];
      o4[h].w *= alpha[h];
    }
#pragma unroll
    for (int i = 0; i < P; ++i)
#pragma unroll
      for (int h = 0; h < NQP; ++h) {
        const float pp = pw[wv][i * NQP + h];
        o4[h].x = fmaf(pp, vr[i].x, o4[h].x);
        o4[h].y = fmaf(pp, vr[i].y, o4[h].y);
        o4[h].z = fmaf(pp, vr[i].z, o4[h].z);
        o4[h].w = fmaf(pp, vr[i].w, o4[h].w);
      }
    __builtin_amdgcn_wave_barrier();
  }

  // 5. merge the four waves (fixed order) into this chunk's (max, sum, o)
  if (lane < NQP) {
    float mm = m[0], ll = l[0];
#pragma unroll
    for (int h = 1; h < NQP; ++h)
      if (lane == h) { mm = m[h]; ll = l[h]; }
    wm[wv][lane] = mm;
    wl[wv][lane] = ll;
  }
#pragma unroll
  for (int h = 0; h < NQP; ++h) *(float4*)&wo[wv][h][4 * lane] = o4[h];
  __syncthreads();
  const size_t pstride = (size_t)nq * (2 + kHeadDim);
  float* mypart = a.part + (size_t)b * pstride;
  for (int h = 0; h < nq; ++h) {
    const float M = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = wm[w][h] == -INFINITY ? 0.f : expf(wm[w][h] - M);
      L = fmaf(f, wl[w][h], L);
      O = fmaf(f, wo[w][h][tid], O);
    }
    mypart[h * (2 + kHeadDim) + 2 + tid] = O;
    if (tid == 0) {
      mypart[h * (2 + kHeadDim)] = M;
      mypart[h * (2 + kHeadDim) + 1] = L;
    }
  }
}

// Merge the chunk statistics: block = (head, quarter of the head dims).
// Loads of all chunk statistics and outputs are issued before any arithmetic.
__global__ __launch_bounds__(64) void k_attn_combine(AttnArgs a) {
  __shared__ float fac[kAttnMaxChunks];
  const int lane = threadIdx.x;
  const int h = blockIdx.x >> 2, d = (blockIdx.x & 3) * 64 + lane;
  const int pos = a.st->pos;
  int t_lo, ch, nch;
  attn_span(a, pos, &t_lo, &ch, &nch);
  const size_t pstride = (size_t)a.n_q * (2 + kHeadDim);
  const float* ph = a.part + h * (2 + kHeadDim);
  float mc[kAttnMaxChunks / 64], lc[kAttnMaxChunks / 64];
#pragma unroll
  for (int i = 0; i < kAttnMaxChunks / 64; ++i) {
    const int c = lane + 64 * i;
    mc[i] = c < nch ? ph[c * pstride] : -INFINITY;
    lc[i] = c < nch ? ph[c * pstride + 1] : 0.f;
  }
  float o = 0.f, L = 0.f;
  for (int c0 = 0; c0 < nch; c0 += 32) {
    float ov[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) ov[k] = c0 + k < nch ? ph[(c0 + k) * pstride + 2 + d] : 0.f;
    if (c0 == 0) {
      float m = -INFINITY;
#pragma unroll
      for (int i = 0; i < kAttnMaxChunks / 64; ++i) m = fmaxf(m, mc[i]);
      const float M = wave_max(m);
      float l = 0.f;
#pragma unroll
      for (int i = 0; i < kAttnMaxChunks / 64; ++i) {
        const int c = lane + 64 * i;
        if (c < nch) {
          const float f = expf(mc[i] - M);
          fac[c] = f;
          l = fmaf(f, lc[i], l);
        }
      }
      L = wave_sum(l);
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (c0 + k < nch) o = fmaf(fac[c0 + k], ov[k], o);
  }
  a.attn_out[h * kHeadDim + d] = o / L;
}

// ---------------------------------------------------------------------------
// End of a forward pass: hidden = residual + norm(down) * post_ffw_norm, then
// normed = rmsNorm(hidden, output_norm) (engine.ts:794-801); advance pos.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_final(FinalArgs a) {
  __shared__ float sh4[4];
  const int tid = threadIdx.x, H = a.H;
  const int n = (H - tid + 255) / 256;
  float v[8], res[8], wq[8], wo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) {
      const int e = tid + 256 * i;
      v[i] = a.pre_vec[e];
      res[i] = a.pre_res[e];
      wq[i] = a.w_post[e];
      wo[i] = a.w_out[e];
    }
  float s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) s1 = fmaf(v[i], v[i], s1);
  const float rms1 = sqrtf(block_sum256(s1, sh4) / (float)H + a.eps);
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) {
      const float r = res[i] + (v[i] * wq[i]) / rms1;
      v[i] = r;
      a.hidden[tid + 256 * i] = r;
      if (a.hist_out) a.hist_out[tid + 256 * i] = r;
      s2 = fmaf(r, r, s2);
    }
  const float rms2 = sqrtf(block_sum256(s2, sh4) / (float)H + a.eps);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) a.normed[tid + 256 * i] = (v[i] * wo[i]) / rms2;
  if (tid == 0) {
    a.st->pos += 1;
    a.st->cursor += 1;
  }
}

// ---------------------------------------------------------------------------
// Token selection over the logits (engine.ts:823-901).
// k_select1: per stride class c = i mod 256, the first index of the class
// maximum over the block's stripes (strict >, init (-1e30, 0)), as in
// argmax/topk256 (shaders.ts:337-347, 371-381).
// k_select2: merge stripes in order -> topk256; then either the argmax
// halving tree (shaders.ts:351-357) or the host sampler (engine.ts:862-901):
// repetition penalty in f64, stable descending sort, f32-stored exp, f64
// sums, top-p cutoff, walk with the injected draw u.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_select1(SelectArgs a) {
  const int tid = threadIdx.x;
  const int nb = gridDim.x;
  const int stripes = (a.V + 255) / 256;
  const int per = (stripes + nb - 1) / nb;
  const int j0 = blockIdx.x * per, j1 = min(j0 + per, stripes);
  float m = -1e30f;
  uint32_t id = 0;
  for (int j = j0; j < j1; j += 32) {
    float v[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const int i = (j + k) * 256 + tid;
      v[k] = (j + k < j1 && i < a.V) ? a.logits[i] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (v[k] > m) { m = v[k]; id = (uint32_t)((j + k) * 256 + tid); }
  }
  a.cand_val[blockIdx.x * 256 + tid] = m;
  a.cand_id[blockIdx.x * 256 + tid] = id;
}

struct Cand {
  double val;
  int ord;
  uint32_t id;
};

__device__ __forceinline__ bool cand_before(const Cand& x, const Cand& y) {
  return x.val > y.val || (x.val == y.val && x.ord < y.ord);
}

__global__ __launch_bounds__(256) void k_select2(SelectArgs a, int nb) {
  __shared__ float tv[256];
  __shared__ uint32_t ti[256];
  __shared__ Cand cs[256];
  __shared__ float probs[256];
  __shared__ int tok_sh;
  const int tid = threadIdx.x;
  float m = -1e30f;
  uint32_t id = 0;
  for (int b0 = 0; b0 < nb; b0 += 32) {
    float v[32];
    uint32_t ix[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      v[k] = b0 + k < nb ? a.cand_val[(b0 + k) * 256 + tid] : -INFINITY;
      ix[k] = b0 + k < nb ? a.cand_id[(b0 + k) * 256 + tid] : 0u;
    }
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (v[k] > m) { m = v[k]; id = ix[k]; }
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
    if (rep > 1.0 && st->seen_count > 0 && id < (uint32_t)a.V && ((a.seen[id >> 5] >> (id & 31)) & 1u)) {
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
    if (a.auto_add && token >= 0 && token < a.V) {
      a.seen[token >> 5] |= 1u << (token & 31);
      a.st->seen_count += 1;
    }
  }
}

// ---------------------------------------------------------------------------
// Upload helpers.
// k_repack: GGUF row-major Q8_0 (rows of Kp 68-byte pairs) -> the
// pair-interleaved layout L. interleave_half > 0 places source row r at fused
// row (r / half) * GR + (r % half) + dst_row_offset with half = GR / 2, i.e.
// gate rows in the first half of each row group and (dst_row_offset = half)
// the matching up rows in the second half.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                long long rows, Q8Layout L, long long off, int half) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = rows * L.Kp;
  if (idx >= total) return;
  const long long r = idx / L.Kp;
  const int c = (int)(idx - r * L.Kp);
  const long long R = half > 0 ? (r / half) * L.GR + (r % half) + off : r + off;
  const long long g = R / L.GR;
  const int ln = (int)(R - g * L.GR);
  const uint32_t* s = (const uint32_t*)(src + (size_t)idx * kPairBytes);
  uint32_t* d = (uint32_t*)(dst + (((size_t)g * L.KpS + c / L.CI) * 64 + (c % L.CI) * L.GR + ln) * kPairBytes);
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
template <int PRO, int EPI, int CI, int NIF>
static int launch_gemv_t(const GemvArgs& a, hipStream_t s) {
  const size_t lds = (size_t)a.Kp * kXPad * sizeof(float);
  hipLaunchKernelGGL((k_gemv<PRO, EPI, CI, NIF>), dim3(a.N / (64 / CI)), dim3(256), lds, s, a);
  return (int)hipGetLastError();
}

// Steps a wave issues before the prologue: all of them when a row group has
// at most 4, 8 or 20 column steps; longer rows continue with a prefetch loop.
template <int PRO, int EPI, int CI>
static int launch_gemv_nif(const GemvArgs& a, hipStream_t s) {
  if (a.KpS <= 4) return launch_gemv_t<PRO, EPI, CI, 1>(a, s);
  if (a.KpS <= 8) return launch_gemv_t<PRO, EPI, CI, 2>(a, s);
  return launch_gemv_t<PRO, EPI, CI, 5>(a, s);
}

template <int PRO, int EPI>
static int launch_gemv_ci(int ci, const GemvArgs& a, hipStream_t s) {
  switch (ci) {
    case 1: return launch_gemv_nif<PRO, EPI, 1>(a, s);
    case 8: return launch_gemv_nif<PRO, EPI, 8>(a, s);
  }
  return (int)hipErrorInvalidValue;
}

int launch_gemv(int pro, int epi, int ci, const GemvArgs& a, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (a.Kp * 64 > kMaxK || a.Kp <= 0 || a.N <= 0 || (ci != 1 && ci != 8) || a.N % (64 / ci) ||
      a.KpS != (a.Kp + ci - 1) / ci)
    return (int)hipErrorInvalidValue;
  if (pro != PRO_NONE && a.Kp * 64 > kMaxEPT / 4 * 256) return (int)hipErrorInvalidValue;
  if (epi == EPI_GEGLU) {
    if (pro != PRO_RESID_NORM) return (int)hipErrorInvalidValue;
    return launch_gemv_ci<PRO_RESID_NORM, EPI_GEGLU>(ci, a, s);
  }
  if (pro == PRO_NONE) return launch_gemv_ci<PRO_NONE, EPI_OUT>(ci, a, s);
  if (pro == PRO_EMBED_NORM) return launch_gemv_ci<PRO_EMBED_NORM, EPI_OUT>(ci, a, s);
  if (pro == PRO_RESID_NORM) return launch_gemv_ci<PRO_RESID_NORM, EPI_OUT>(ci, a, s);
  return (int)hipErrorInvalidValue;
}

int launch_attention(const AttnArgs& a, int grid, void* stream) {
  if (a.n_q < 1 || a.n_q > kMaxQHeads || grid < 1 || grid > kAttnMaxChunks) return (int)hipErrorInvalidValue;
  hipStream_t s = (hipStream_t)stream;
  if (a.n_q <= 4) hipLaunchKernelGGL(k_attn<4>, dim3(grid), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(k_attn<8>, dim3(grid), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(k_attn_combine, dim3(a.n_q * 4), dim3(64), 0, s, a);
  return (int)hipGetLastError();
}

int launch_final(const FinalArgs& a, void* stream) {
  if (a.H > 2048) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_final, dim3(1), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_select(const SelectArgs& a, void* stream) {
  const int stripes = (a.V + 255) / 256;
  const int nb = stripes < kSelBlocks ? stripes : kSelBlocks;
  hipLaunchKernelGGL(k_select1, dim3(nb), dim3(256), 0, (hipStream_t)stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(k_select2, dim3(1), dim3(256), 0, (hipStream_t)stream, a, nb);
  return (int)hipGetLastError();
}

int launch_repack(const uint8_t* src, uint8_t* dst, const Q8Layout& L, long long rows, long long off, int half,
                  void* stream) {
  const long long total = rows * L.Kp;
  if (total <= 0) return 0;
  hipLaunchKernelGGL(k_repack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src,
                     dst, rows, L, off, half);
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

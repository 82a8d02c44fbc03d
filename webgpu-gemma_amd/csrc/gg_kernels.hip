// gg_kernels.hip -- gfx950 (CDNA4) kernels of the Gemma-3 Q8_0 token loop.
//
// One forward pass over a token is five kernels per layer:
//   k_gemv_mg<EMBED_NORM|RESID_NORM, OUT>  fused QKV projection; its prologue
//        finishes the previous layer (post-FFN norm + residual) and applies
//        attn_norm (engine.ts:768-774, 794)
//   k_attn_dec      QK-norm + RoPE + KV store + one chunk of decode attention
//                   per block, chunk partials to memory (engine.ts:775-783)
//   k_gemv_mg<ATTN_MERGE, OUT>  merges the attention chunks in its prologue,
//                   then the attention output projection (engine.ts:784);
//                   spans above 4096 positions: k_attn_merge, then
//                   k_gemv_mg<NONE, OUT>
//   k_gemv_mg<RESID_NORM, GEGLU>  post-attn norm + residual + ffn_norm, gate
//                   and up rows side by side, GeGLU in the epilogue (engine.ts:785-792)
//   k_gemv_mg<NONE, OUT>       down projection (engine.ts:793)
// then k_final (post-FFN norm + residual + output_norm, engine.ts:794-801),
// and for a sampled step the LM head GEMV plus k_select1/k_select2
// (engine.ts:817-901).
//
// A batched prefill runs per layer the bf16-MFMA GEMMs (k_gemm: int8 weights
// exact in bf16, activations split into bf16 hi + lo), the row kernels
// (norms, residuals, QK-norm + RoPE + KV store) and the MFMA attention
// k_attn_pf (+ k_attn_pf_merge for long spans); the GEMM tiles are 128 x 128,
// or 128 x 144 for 1152-wide outputs with a K split.
//
// On this multi-XCD part a device-scope fence is a whole-L2 write-back, so
// kernels never fence and never exchange data across blocks of one launch:
// every cross-block step is a kernel boundary.
//
// Decode arithmetic is fp32 except the int8 weight payload (dequantised
// exactly in registers) and the sampler's f64 steps, which mirror the JS
// host's. The batched prefill's bf16 products use hi + lo splits of their
// fp32 operands and accumulate in fp32.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gg_device.h"
#include "gg_internal.h"

namespace gg {


// ---------------------------------------------------------------------------
// GEMV prologues: build the GEMV input x (K floats) in LDS.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float embed_elem(const GemvArgs& a, int token, int e) {
  return embed_value(a.embd, a.embd_KpS, a.embed_scale, token, e);
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
    const int cur = a.st->cursor;
    const int token = cur < 0 ? a.st->token : a.tokens[cur];
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
    const float ri1 = rsq(block_sum256(s1, sh4) / (float)K + a.eps);
#pragma unroll
    for (int i = 0; i < kMaxEPT / 4; ++i)
      if (i < n) {
        const float t = (v[i] * wq[i]) * ri1;   // fusedNormAdd, shaders.ts:415
        r[i] = res[i] + t;
        ss = fmaf(r[i], r[i], ss);
        if (blockIdx.x == 0) {
          a.res_out[tid + 256 * i] = r[i];
          if (a.hist_out) a.hist_out[tid + 256 * i] = r[i];
        }
      }
  }
  const float ri = rsq(block_sum256(ss, sh4) / (float)K + a.eps);   // rmsNorm, shaders.ts:50-53
#pragma unroll
  for (int i = 0; i < kMaxEPT / 4; ++i)
    if (i < n) {
      const float x = (r[i] * wp[i]) * ri;
      xs[xs_index(tid + 256 * i)] = x;
      if (PRO == PRO_RESID_NORM && blockIdx.x == 0 && a.x_out) a.x_out[tid + 256 * i] = x;
    }
  // the LM head carrying k_final's work also carries its step of the state
  if (PRO == PRO_RESID_NORM && blockIdx.x == 0 && tid == 0 && a.st_advance) {
    a.st_advance->pos += 1;
    a.st_advance->cursor += 1;
  }
}

// ---------------------------------------------------------------------------
// Q8_0 dequant-GEMV, one row group per block (used with CI = 1: the tied LM
// head, 64 rows per block). Block = 256 threads = 4 wavefronts on one group
// of GR rows; lane l holds slot l of each item (row l % GR, pair-column phase
// l / GR). Wave w takes items w, w+4, ... of the group. Up to kStepsInFlight
// items per wave are issued at kernel entry, before the prologue (weights
// never depend on x); longer rows continue with a two-item prefetch.
// ---------------------------------------------------------------------------
template <int PRO, int EPI, int CI, int kStepsInFlight>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  constexpr int GR = 64 / CI;
  extern __shared__ float4 xs4[];
  float* xs = (float*)xs4;
  __shared__ float red[4][GR];
  __shared__ float sh4[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = blockIdx.x;
  const int cp = lane / GR;
  const int Kp = a.Kp, KpS = a.KpS;
  const uint8_t* base = a.W + (size_t)g * KpS * kColBytes;

  Pair st[kStepsInFlight];
#pragma unroll
  for (int i = 0; i < kStepsInFlight; ++i) {
    const int s = wv + 4 * i;
    if (s < KpS && s * CI + cp < Kp) load_planes(base + (size_t)s * kColBytes, lane, st[i]);
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
    if (s * CI + cp < Kp) load_planes(base + (size_t)s * kColBytes, lane, cur);
    if (s + 4 < KpS && (s + 4) * CI + cp < Kp) load_planes(base + (size_t)(s + 4) * kColBytes, lane, nxt);
    for (; s < KpS; s += 4) {
      Pair nn;
      const int s3 = s + 8;
      if (s3 < KpS && s3 * CI + cp < Kp) load_planes(base + (size_t)s3 * kColBytes, lane, nn);
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
// Q8_0 dequant-GEMV over balanced ranges of row groups (used with CI = 8 or 2:
// QKV, O, gate/up, down). Block b owns groups [b G / nb, (b+1) G / nb); their
// items (memory-contiguous, KpS per group) are split evenly over the W
// waves. Every load is issued unconditionally (indices clamped into range)
// so the wait counters stay exact: the prologue's vector loads go first, then
// all NIF weight items of the wave, and the prologue only waits for its own
// loads. Dot products accumulate per lane while a wave stays in one group;
// one butterfly over the CI column phases per group lands the row sums in
// the wave's LDS slots, and a fixed-order sum over the waves gives the rows
// (deterministic). Prologue reductions run on the DPP network.
// ---------------------------------------------------------------------------
constexpr size_t kDecStatOff = (size_t)kDecMaxChunks * kAttnMaxQ * kHeadDim;   // (m, l) after the o block

constexpr int kMgRows = 256;   // rows one block may own
template <int PRO, int EPI, int CI, int W, int NIF, int EPT>
__global__ __launch_bounds__(64 * W) void k_gemv_mg(GemvArgs a) {
  // the prologue (x from the previous kernel's output: a latency chain of
  // loads and block reductions) runs at raised wave priority over the other
  // block's dot products on the CU (0.7797 -> 0.7780 ms per 1B token)
  __builtin_amdgcn_s_setprio(1);
  constexpr int GR = 64 / CI;
  constexpr int NT = 64 * W;
  extern __shared__ float4 xs4[];
  float* xs = (float*)xs4;
  __shared__ float red[W][kMgRows];
  __shared__ float shw[2][W];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int cp = lane / GR;
  const int Kp = a.Kp, KpS = a.KpS, K = Kp * 64;
  const int G = a.N / GR;
  const int b = blockIdx.x, nb = gridDim.x;
  const int g0 = (int)(((long long)b * G) / nb), g1 = (int)(((long long)(b + 1) * G) / nb);
  const int i0 = g0 * KpS, ni = (g1 - g0) * KpS;
  const int wi0 = i0 + (wv * ni) / W, wi1 = i0 + ((wv + 1) * ni) / W;
  const int K4 = K / 4;   // thread t owns the float4 chunks t + NT i (i < EPT) of x

  // Lanes of a padding column phase (c >= Kp, the tail item of a row group
  // when Kp % CI != 0) load the phase-0 lane of their row instead: the same
  // cache lines, so the padding bytes are not fetched (their products are
  // masked below).
  auto issue_weights = [&](Pair* w) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NIF; ++k) {
      const int it = max(min(wi0 + k, wi1 - 1), i0);
      const int sp = it % KpS;
      const int ll = sp * CI + cp < Kp ? lane : (lane & (GR - 1));
      load_planes(a.W + (size_t)it * kColBytes, ll, w[k]);
    }
  };
  Pair st[NIF];
  // 1. prologue loads (16 bytes per lane, clamped indices: always issued)
  float4 v[EPT], res[EPT], wq[EPT], wp[EPT];
  // PRO_ATTN_MERGE: thread t merges x[4t .. 4t+3] (head t / 64) from the
  // first 16 chunk partials (more are merged in batches of 16 below)
  constexpr int kMB = 16;
  float am_m[kMB], am_l[kMB];
  float4 am_o[kMB];
  int nch = 0, ahd = 0;
  if (PRO == PRO_ATTN_MERGE) {
    issue_weights(st);
    nch = a.attn_chunks;   // every chunk of the launch, empty ones included: no wait for the position
    // head of this wave (uniform): its (max, sum) pairs come through scalar loads
    ahd = __builtin_amdgcn_readfirstlane(min(wv, K / kHeadDim - 1));
#pragma unroll
    for (int k = 0; k < kMB; ++k) {
      const int c = min(k, nch - 1);
      const float2 ml = *(const float2*)(a.attn_part + kDecStatOff + ((size_t)c * kAttnMaxQ + ahd) * 2);
      am_m[k] = ml.x;
      am_l[k] = ml.y;
      am_o[k] = *(const float4*)(a.attn_part + ((size_t)c * kAttnMaxQ + ahd) * kHeadDim + 4 * (tid & 63));
    }
  } else if (PRO == PRO_EMBED_NORM) {
    const int cur = a.st->cursor;
    const int token = cur < 0 ? a.st->token : a.tokens[cur];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = min(tid + NT * i, K4 - 1);
      v[i] = make_float4(embed_elem(a, token, 4 * c), embed_elem(a, token, 4 * c + 1),
                         embed_elem(a, token, 4 * c + 2), embed_elem(a, token, 4 * c + 3));
      wp[i] = ((const float4*)a.w_pre)[c];
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = min(tid + NT * i, K4 - 1);
      if (PRO == PRO_NONE) {
        v[i] = ((const float4*)a.x)[c];
      } else {
        v[i] = ((const float4*)a.pre_vec)[c];
        res[i] = ((const float4*)a.pre_res)[c];
        wq[i] = ((const float4*)a.w_post)[c];
        wp[i] = ((const float4*)a.w_pre)[c];
      }
    }
  }
  // 2. this wave's weight items (clamped into the block's range); with
  // ATTN_MERGE they went out first, ahead of the position-dependent chunk loads
  if (PRO != PRO_ATTN_MERGE) issue_weights(st);
  for (int i = tid; i < W * kMgRows; i += NT) (&red[0][0])[i] = 0.f;

  // 3. prologue -> x in LDS
  auto has = [&](int i) { return tid + NT * i < K4; };
  auto sq4 = [](float4 q, float acc) {
    acc = fmaf(q.x, q.x, acc);
    acc = fmaf(q.y, q.y, acc);
    acc = fmaf(q.z, q.z, acc);
    return fmaf(q.w, q.w, acc);
  };
  if (PRO == PRO_NONE) {
#pragma unroll
    for (int i = 0; i < EPT; ++i)
      if (has(i)) *(float4*)&xs[xs_index(4 * (tid + NT * i))] = v[i];
  } else if (PRO == PRO_ATTN_MERGE) {
    // chunk weights 2^(m_c - M) (maxima in log2 units) with M the running
    // max, in chunk order
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMB; ++k)
      if (k < nch) M = fmaxf(M, am_m[k]);
    float L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](int k, float Mx) {
      const float f = __builtin_amdgcn_exp2f(am_m[k] - Mx);
      L = fmaf(f, am_l[k], L);
      acc.x = fmaf(f, am_o[k].x, acc.x);
      acc.y = fmaf(f, am_o[k].y, acc.y);
      acc.z = fmaf(f, am_o[k].z, acc.z);
      acc.w = fmaf(f, am_o[k].w, acc.w);
    };
#pragma unroll
    for (int k = 0; k < kMB; ++k)
      if (k < nch) add(k, M);
    for (int c0 = kMB; c0 < nch; c0 += kMB) {   // spans above 4096 positions
#pragma unroll
      for (int k = 0; k < kMB; ++k) {
        const int c = min(c0 + k, nch - 1);
        const float2 ml = *(const float2*)(a.attn_part + kDecStatOff + ((size_t)c * kAttnMaxQ + ahd) * 2);
        am_m[k] = ml.x;
        am_l[k] = ml.y;
        am_o[k] = *(const float4*)(a.attn_part + ((size_t)c * kAttnMaxQ + ahd) * kHeadDim + 4 * (tid & 63));
      }
      float Mb = M;
#pragma unroll
      for (int k = 0; k < kMB; ++k)
        if (c0 + k < nch) Mb = fmaxf(Mb, am_m[k]);
      const float sc = __builtin_amdgcn_exp2f(M - Mb);
      L *= sc;
      acc.x *= sc;
      acc.y *= sc;
      acc.z *= sc;
      acc.w *= sc;
      M = Mb;
#pragma unroll
      for (int k = 0; k < kMB; ++k)
        if (c0 + k < nch) add(k, M);
    }
    if (4 * tid < K) {
      const float iL = 1.f / L;
      const float4 xo = make_float4(acc.x * iL, acc.y * iL, acc.z * iL, acc.w * iL);
      *(float4*)&xs[xs_index(4 * tid)] = xo;
      if (b == 0) *(float4*)(a.x_out + 4 * tid) = xo;
    }
  } else {
    float4 r[EPT];
    if (PRO == PRO_EMBED_NORM) {
#pragma unroll
      for (int i = 0; i < EPT; ++i) r[i] = v[i];
    } else {   // res = pre_res + norm(pre_vec) * w_post (fusedNormAdd, shaders.ts:415)
      float s1 = 0.f;
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        if (has(i)) s1 = sq4(v[i], s1);
      s1 = wave_sum_dpp(s1);
      if (lane == 0) shw[0][wv] = s1;
      __syncthreads();
      float t1 = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) t1 += shw[0][w];
      const float ri1 = rsq(t1 / (float)K + a.eps);
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        r[i] = make_float4(res[i].x + (v[i].x * wq[i].x) * ri1, res[i].y + (v[i].y * wq[i].y) * ri1,
                           res[i].z + (v[i].z * wq[i].z) * ri1, res[i].w + (v[i].w * wq[i].w) * ri1);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < EPT; ++i)
      if (has(i)) ss = sq4(r[i], ss);
    if (b == 0) {
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        if (has(i)) {
          ((float4*)a.res_out)[tid + NT * i] = r[i];
          if (PRO == PRO_RESID_NORM && a.hist_out) ((float4*)a.hist_out)[tid + NT * i] = r[i];
        }
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) shw[1][wv] = ss;
    __syncthreads();
    float t2 = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) t2 += shw[1][w];
    const float ri = rsq(t2 / (float)K + a.eps);   // rmsNorm, shaders.ts:50-53
#pragma unroll
    for (int i = 0; i < EPT; ++i)
      if (has(i))
        *(float4*)&xs[xs_index(4 * (tid + NT * i))] =
            make_float4((r[i].x * wp[i].x) * ri, (r[i].y * wp[i].y) * ri, (r[i].z * wp[i].z) * ri,
                        (r[i].w * wp[i].w) * ri);
  }
  __syncthreads();

  // 4. dot products in item order
  __builtin_amdgcn_s_setprio(0);
  float acc = 0.f;
  int gcur = wi0 / KpS - g0;
  auto flush = [&](int gl) {
    float t = acc;
#pragma unroll
    for (int m = GR; m < 64; m <<= 1) t += __shfl_xor(t, m, 64);
    if (lane < GR) red[wv][gl * GR + lane] = t;
  };
#pragma unroll
  for (int k = 0; k < NIF; ++k) {
    const int it = wi0 + k;
    const int g = it / KpS, s = it - g * KpS;
    const int c = s * CI + cp;
    float d = dot_pair(st[k], xs + min(c, Kp - 1) * kXPad, 0.f);
    d = (c < Kp && it < wi1) ? d : 0.f;
    if (it < wi1 && g - g0 != gcur) {
      flush(gcur);
      gcur = g - g0;
      acc = 0.f;
    }
    acc += d;
  }
  if (wi1 > wi0) flush(gcur);
  __syncthreads();

  // 5. fixed-order sum over the waves; epilogue
  const int nrows = (g1 - g0) * GR;
  for (int t = tid; t < nrows; t += NT) {
    float r = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) r += red[w][t];
    if (EPI == EPI_OUT) {
      a.out[g0 * GR + t] = r;
    } else {
      // gate rows of a group in its first GR/2 slots, the matching up rows next
      const int rr = t % GR;
      if (rr < GR / 2) {
        float up = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) up += red[w][t + GR / 2];
        a.act_out[(g0 * GR + t - rr) / 2 + rr] = gelu_mul(r, up);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Decode attention (one KV head, head_dim 256, up to 4 query heads). Block
// (x, y) = (chunk of positions, query head); the chunk partials (max, sum, o)
// go to memory and the attention output projection merges them in its
// prologue (no cross-block step here). Chunks: 32 * ceil(span / (32 * mc))
// positions, mc = 16 while the span is <= 4096 (else kDecMaxChunks), so the
// merge reads at most 16 partials per head at Gemma-3 1B lengths. Blocks past
// the span write empty partials (m = -inf), so the merge always reads the
// launch's chunk count and does not wait for the position. One head
// per block keeps each wave's serial chain short (the pass is bound by
// instruction latency, not by the K/V bytes).
//
// Per block: QK-norm + NEOX RoPE of query head y and, in the chunk holding
// `pos`, of the key; that chunk's head-0 block also stores k/v to the cache
// (fusedPerHeadNormRope + kvCacheStore, shaders.ts:209-227, 420-467). Wave w
// then runs passes of 8 positions t0 + 32 p + 8 w + i: lane (i, o) =
// (lane / 8, lane % 8) holds key dims 4 (o + 8 j) .. +3 (j < 8), so each key
// load instruction reads 8 whole 128-byte segments, and the dot product
// finishes with a butterfly over the 8 lanes of a position; lane l holds
// value dims 4 l .. 4 l + 3 for the weighted sum (shaders.ts:229-325).
// Softmax statistics are kept online per pass; all reductions run on DPP,
// probabilities reach every lane through readlane.
// ---------------------------------------------------------------------------
template <int HPB>
__global__ __launch_bounds__(256) void k_attn_dec(AttnArgs a) {
  __shared__ float4 qs4[HPB][64];
  __shared__ float4 ks4[64], vs4[64];
  __shared__ float4 wo[4][HPB][64];
  __shared__ float wm[4][HPB], wl[4][HPB];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nq = a.n_q;
  const int nqd = nq * kHeadDim;
  const int h0 = HPB == 1 ? (int)blockIdx.y : 0;   // first query head of the block
  // loads that do not depend on the position: q of the head this wave
  // normalises (HPB = 1: wave 0, head h0; else wave w, head w), this token's
  // k and v, the norm weights
  const int qh = HPB == 1 ? h0 : min(wv, nq - 1);
  float hx[4], kx[4], nwt[4], kwt[4], cs[2], sn[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hx[i] = a.qkv[qh * kHeadDim + lane + 64 * i];
    nwt[i] = a.q_norm[lane + 64 * i];
    kx[i] = a.qkv[nqd + lane + 64 * i];
    kwt[i] = a.k_norm[lane + 64 * i];
  }
  const float4 vme = *(const float4*)(a.qkv + nqd + kHeadDim + 4 * lane);
  const int pos = a.st->pos;
  int t_lo, ch, nch;
  dec_span(pos, a.window, gridDim.x, &t_lo, &ch, &nch);
  const int b = blockIdx.x;
  if (b >= nch) {   // past the span: empty partials, so that the merge needs no position
#pragma unroll
    for (int hh = 0; hh < HPB; ++hh) {
      const int h = h0 + hh;
      if (h >= nq) break;
      if (tid < 64) *(float4*)(a.part + ((size_t)b * kAttnMaxQ + h) * kHeadDim + 4 * tid) = make_float4(0.f, 0.f, 0.f, 0.f);
      if (tid == 0) {
        a.part[kDecStatOff + ((size_t)b * kAttnMaxQ + h) * 2] = -INFINITY;
        a.part[kDecStatOff + ((size_t)b * kAttnMaxQ + h) * 2 + 1] = 0.f;
      }
    }
    return;
  }
  const int t0 = t_lo + b * ch;
  const int t1 = min(t0 + ch, pos + 1);
  const int npass = (t1 - t0 + 31) >> 5;
  const int kv_last = max(pos - 1, 0);     // cache rows [0, pos) hold earlier tokens
  const int pl = lane >> 3, oc = lane & 7;
  const bool holder = (b == nch - 1);      // this block's chunk contains pos

  // loads of pass p: key rows in the score layout, value rows in the PV
  // layout; rows are clamped into the cache (positions >= t1 are masked,
  // pos itself is substituted from LDS). Nontemporal: with HPB = 1 each row
  // is read by the four head blocks of its chunk (same XCD) within one launch.
  float4 kr[8], vr[8];
  auto load_k = [&](int p) {
    const int t = min(t0 + 32 * p + 8 * wv + pl, kv_last);
    const f32x4* kp = (const f32x4*)(a.k_cache + (size_t)t * kHeadDim);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 v = __builtin_nontemporal_load(kp + oc + 8 * j);
      kr[j] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
  auto load_v = [&](int p) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = min(t0 + 32 * p + 8 * wv + i, kv_last);
      const f32x4 v = __builtin_nontemporal_load((const f32x4*)(a.v_cache + (size_t)t * kHeadDim) + lane);
      vr[i] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
  // this position's RoPE row, then the first pass of K / V rows (the norm
  // below waits only for the loads issued before these)
  const float* rt = a.rope + (size_t)pos * kHeadDim;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cs[j] = rt[lane + 64 * j];
    sn[j] = rt[kHeadDim / 2 + lane + 64 * j];
  }
  load_k(0);
  load_v(0);

  // RMSNorm + NEOX RoPE of one head: lane owns dims lane + 64 i; pairs (i, i + 128)
  auto norm_rope = [&](float* x, const float* w, float* dst) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
    ss = wave_sum_dpp(ss);
    const float ri = rsq(ss / (float)kHeadDim + a.eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (x[i] * w[i]) * ri;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float x0 = x[j], x1 = x[j + 2];
      dst[lane + 64 * j] = x0 * cs[j] - x1 * sn[j];
      dst[lane + 64 * j + 128] = x0 * sn[j] + x1 * cs[j];
    }
  };
  if (HPB == 1) {
    if (wv == 0) norm_rope(hx, nwt, (float*)qs4[0]);
  } else if (wv < HPB) {
    if (wv < nq) norm_rope(hx, nwt, (float*)qs4[wv]);
    else qs4[wv][lane] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (holder && wv == 1) norm_rope(kx, kwt, (float*)ks4);
  if (holder && wv == 2) vs4[lane] = vme;
  __syncthreads();
  if (holder && h0 == 0) {
    a.k_cache[(size_t)pos * kHeadDim + tid] = ((const float*)ks4)[tid];
    a.v_cache[(size_t)pos * kHeadDim + tid] = ((const float*)vs4)[tid];
  }
  if (b == 0 && a.q_dbg && tid < 64)
#pragma unroll
    for (int hh = 0; hh < HPB; ++hh)
      if (h0 + hh < nq) *(float4*)(a.q_dbg + (h0 + hh) * kHeadDim + 4 * tid) = qs4[hh][tid];

  float4 qr[HPB][8];
#pragma unroll
  for (int hh = 0; hh < HPB; ++hh)
#pragma unroll
    for (int j = 0; j < 8; ++j) qr[hh][j] = qs4[hh][oc + 8 * j];

  // scores in log2 units: the online softmax and every merge of its
  // partials (chunk maxima in the same units) run in base 2 on v_exp_f32
  const float sl2 = a.scale * 1.4426950408889634f;
  float m[HPB], l[HPB];
  float4 o4[HPB];
#pragma unroll
  for (int hh = 0; hh < HPB; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.f;
    o4[hh] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int p = 0; p < npass; ++p) {
    const int tb = t0 + 32 * p + 8 * wv;       // first position of this wave's pass
    const int t = tb + pl;
    if (t == pos) {
#pragma unroll
      for (int j = 0; j < 8; ++j) kr[j] = ks4[oc + 8 * j];
    }
    float sc[HPB];
#pragma unroll
    for (int hh = 0; hh < HPB; ++hh) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        d = fmaf(qr[hh][j].x, kr[j].x, d);
        d = fmaf(qr[hh][j].y, kr[j].y, d);
        d = fmaf(qr[hh][j].z, kr[j].z, d);
        d = fmaf(qr[hh][j].w, kr[j].w, d);
      }
      d = group8_sum(d);
      sc[hh] = (t < t1 && h0 + hh < nq) ? d * sl2 : -INFINITY;
    }
    if (p + 1 < npass) load_k(p + 1);          // next pass (wave-uniform)
    float pr[HPB], alpha[HPB];
#pragma unroll
    for (int hh = 0; hh < HPB; ++hh) {
      const float mx = across8_max(sc[hh]);
      const float mn = fmaxf(m[hh], mx);
      alpha[hh] = (m[hh] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[hh] - mn);
      pr[hh] = (sc[hh] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sc[hh] - mn);
      l[hh] = fmaf(l[hh], alpha[hh], across8_sum(pr[hh]));
      m[hh] = mn;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (tb + i == pos) vr[i] = vs4[lane];
#pragma unroll
    for (int hh = 0; hh < HPB; ++hh) {
      o4[hh].x *= alpha[hh];
      o4[hh].y *= alpha[hh];
      o4[hh].z *= alpha[hh];
      o4[hh].w *= alpha[hh];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr[hh]), 8 * i));
        o4[hh].x = fmaf(pv, vr[i].x, o4[hh].x);
        o4[hh].y = fmaf(pv, vr[i].y, o4[hh].y);
        o4[hh].z = fmaf(pv, vr[i].z, o4[hh].z);
        o4[hh].w = fmaf(pv, vr[i].w, o4[hh].w);
      }
    }
    if (p + 1 < npass) load_v(p + 1);
  }

  // merge the four waves (fixed order) into the chunk's (max, sum, o) per
  // head: one barrier, then every lane of wave 0 forms the weights itself
#pragma unroll
  for (int hh = 0; hh < HPB; ++hh) {
    wo[wv][hh][lane] = o4[hh];
    if (lane == 0) {
      wm[wv][hh] = m[hh];
      wl[wv][hh] = l[hh];
    }
  }
  __syncthreads();
  if (tid < 64) {
#pragma unroll
    for (int hh = 0; hh < HPB; ++hh) {
      const int h = h0 + hh;
      if (h >= nq) break;
      const float M = fmaxf(fmaxf(wm[0][hh], wm[1][hh]), fmaxf(wm[2][hh], wm[3][hh]));
      float L = 0.f;
      float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = wm[w][hh] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm[w][hh] - M);
        L = fmaf(f, wl[w][hh], L);
        const float4 v = wo[w][hh][tid];
        O.x = fmaf(f, v.x, O.x);
        O.y = fmaf(f, v.y, O.y);
        O.z = fmaf(f, v.z, O.z);
        O.w = fmaf(f, v.w, O.w);
      }
      *(float4*)(a.part + ((size_t)b * kAttnMaxQ + h) * kHeadDim + 4 * tid) = O;
      if (tid == 0) {
        a.part[kDecStatOff + ((size_t)b * kAttnMaxQ + h) * 2] = M;
        a.part[kDecStatOff + ((size_t)b * kAttnMaxQ + h) * 2 + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Long-span decode attention merge: per query head, the softmax-weighted sum
// of the launch's nch chunk partials, o = sum_c f_c o_c / sum_c f_c l_c with
// f_c = 2^(m_c - max_c m_c) (maxima in log2 units; empty chunks have m_c =
// -inf, f_c = 0), written
// to attn_out, the O GEMV's input. Block (32-dim slice, head); thread (chunk
// group tid / 32 of 8, dim tid % 32) sums chunks g, g + 8, ..., then the
// groups add in a fixed order (deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a, int nch) {
  constexpr int kPer = kDecMaxChunks / 8;   // chunks per thread
  __shared__ float gmax[8], gl[8], go[8][32];
  const int tid = threadIdx.x, cg = tid >> 5, d = tid & 31;
  const int h = blockIdx.y, dim = 32 * blockIdx.x + d;
  const float* ml = a.part + kDecStatOff;
  // every partial of this thread is loaded before any is used (the loads
  // are independent; one at a time each would wait a full memory latency)
  float2 st[kPer];
  float ov[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int c = min(cg + 8 * k, nch - 1);
    st[k] = *(const float2*)(ml + ((size_t)c * kAttnMaxQ + h) * 2);
    ov[k] = a.part[((size_t)c * kAttnMaxQ + h) * kHeadDim + dim];
  }
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (cg + 8 * k < nch) mx = fmaxf(mx, st[k].x);
  if (d == 0) gmax[cg] = mx;
  __syncthreads();
  float M = gmax[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) M = fmaxf(M, gmax[i]);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (cg + 8 * k < nch) {
      const float f = __builtin_amdgcn_exp2f(st[k].x - M);
      L = fmaf(f, st[k].y, L);
      O = fmaf(f, ov[k], O);
    }
  go[cg][d] = O;
  if (d == 0) gl[cg] = L;
  __syncthreads();
  if (cg == 0) {
    float So = 0.f, Sl = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      So += go[i][d];
      Sl += gl[i];
    }
    a.attn_out[h * kHeadDim + dim] = So / Sl;
  }
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
      for (int p = 1; p < a.pre_planes; ++p) v[i] += a.pre_vec[p * a.pre_stride + e];
      res[i] = a.pre_res[e];
      wq[i] = a.w_post[e];
      wo[i] = a.w_out[e];
    }
  float s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) s1 = fmaf(v[i], v[i], s1);
  const float ri1 = rsq(block_sum256(s1, sh4) / (float)H + a.eps);
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) {
      const float r = res[i] + (v[i] * wq[i]) * ri1;
      v[i] = r;
      a.hidden[tid + 256 * i] = r;
      if (a.hist_out) a.hist_out[tid + 256 * i] = r;
      s2 = fmaf(r, r, s2);
    }
  const float ri2 = rsq(block_sum256(s2, sh4) / (float)H + a.eps);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) a.normed[tid + 256 * i] = (v[i] * wo[i]) * ri2;
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

__global__ __launch_bounds__(256) void k_select2(SelectArgs a, int nb) {
  __shared__ SelShared sh;
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
  a.top[2 * tid] = __float_as_uint(m);
  a.top[2 * tid + 1] = id;
  const int token = select_token(sh, m, id, true, sample_of(a.st), a.seen, a.V);
  if (tid == 0) {
    a.st->out_token = token;
    if (a.host_out) a.host_out[0] = token;
    if (a.auto_add && token >= 0 && token < a.V) {
      a.seen[token >> 5] |= 1u << (token & 31);
      a.st->seen_count += 1;
    }
  }
}

// ---------------------------------------------------------------------------
// Batched prefill attention (no reference counterpart: the reference attends
// one prompt token per decode pass, engine.ts:923-928, with the
// scores / softmax / weighted V of shaders.ts:229-325).
//
// Block (x = key chunk, y = query tile) covers 32 prompt rows with 8 waves;
// wave w computes query head w % 4 of rows 16 (w / 4) .. + 15 over the
// chunk's keys, which are staged 32 rows at a time in LDS and shared by the
// heads (one KV head) and both row halves, so each key's hi / lo split
// serves 128 (row, head) pairs.
//   S^T = K Q^T  on v_mfma_f32_16x16x32_bf16 with q and k split into bf16
//                hi + lo (k and v when they are staged, q once per block):
//                per 32 dims the products hi.hi, lo.hi and hi.lo, fp32
//                accumulate (the dropped lo.lo term is below 2^-16 |k| |q|). Operand row
//                c of key tile j (j < 2) is key 8 (c / 4) + 4 j + c % 4, so
//                lane l holds S^T[key 8 g + 4 j + r][row l % 16] for r < 4,
//                g = lane / 16.
//   O += P V     on v_mfma_f32_16x16x32_bf16, the same three products of
//                bf16 hi + lo splits: A = P from lane l's own S^T registers
//                (keys 8 g .. 8 g + 7 in order), B = V^T rows staged per
//                dim; lane l holds O[row 4 g + r][16 i + l % 16] for i < 16.
// Softmax statistics of row l % 16 stay online per lane: the max is reduced
// over the four lane groups each tile, the sum once at the end. LDS rows are
// unpadded and XOR-swizzled so that the ds_read_b128 operand reads (16 rows
// per lane group) hit distinct banks: 16-byte unit u of K row k sits at
// u ^ ((k % 4) + 4 (k / 8)), unit u (keys 8u .. 8u + 7) of V^T dim row d at
// u ^ ((d / 2) % 4). A query tile whose span fits one chunk writes
// O / l; otherwise every chunk leaves (m, l, O) in `part` for
// k_attn_pf_merge.
// ---------------------------------------------------------------------------

// x = hi + lo + e with hi = bf16(x), lo = bf16(x - hi), |e| <= 2^-17 |x|
// (the input format of the prefill GEMMs).
__device__ __forceinline__ void split_bf16(float x, uint16_t* hi, uint16_t* lo) {
  const __bf16 h = (__bf16)x;
  *hi = __builtin_bit_cast(uint16_t, h);
  *lo = __builtin_bit_cast(uint16_t, (__bf16)(x - (float)h));
}

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
// The same split for two values at once, as packed bf16 pairs (element 0 in
// the low half): one packed conversion for hi, hi widened back by a shift and
// a mask, one packed conversion for lo.
__device__ __forceinline__ void split2_bf16(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){x0, x1}, bf16x2));
  const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){x0 - h0, x1 - h1}, bf16x2));
}
// bf16 hi / lo of four values as packed pairs
__device__ __forceinline__ void split4_bf16(float x0, float x1, float x2, float x3, bf16x4& hi, bf16x4& lo) {
  uint32_t h[2], l[2];
  split2_bf16(x0, x1, h[0], l[0]);
  split2_bf16(x2, x3, h[1], l[1]);
  hi = __builtin_bit_cast(bf16x4, h);
  lo = __builtin_bit_cast(bf16x4, l);
}

// max / sum with lane ^ 16 and lane ^ 32 on the gfx950 half-row and
// half-wave swaps (VALU) instead of ds_bpermute shuffles (an LDS round trip)
__device__ __forceinline__ float pf_xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pf_xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

constexpr int kPfRows = 32;   // query rows per block: two 16-row MFMA tiles
__device__ __forceinline__ bf16x8 lds_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *(const u32x4*)p);
}

constexpr int kPfKeys = 32;   // keys per LDS tile

__device__ __forceinline__ int pf_key_lo(const AttnArgs& a, int pos) {
  return a.window > 0 ? max(0, pos - a.window + 1) : 0;
}

// Keys of query tile qt (kPfRows rows): [lo(first row), last row], chunks of
// pf_chunk keys.
__device__ __forceinline__ void pf_tile_span(const AttnArgs& a, int qt, int* klo, int* khi, int* nkc) {
  const int p_first = a.pf_start + qt * kPfRows;
  const int p_last = a.pf_start + min(qt * kPfRows + kPfRows - 1, a.pf_rows - 1);
  *klo = pf_key_lo(a, p_first);
  *khi = p_last;
  *nkc = (p_last - *klo + a.pf_chunk) / a.pf_chunk;
}

__global__ __launch_bounds__(512, 1) void k_attn_pf(AttnArgs a) {
  __shared__ __align__(16) uint16_t Kh[kPfKeys * kHeadDim];
  __shared__ __align__(16) uint16_t Kl[kPfKeys * kHeadDim];
  __shared__ __align__(16) uint16_t Vh[kHeadDim * kPfKeys];   // V^T: [dim][key]
  __shared__ __align__(16) uint16_t Vl[kHeadDim * kPfKeys];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, h = wv & 3, rt = wv >> 2;
  const int g = lane >> 4, c16 = lane & 15;
  const int M = a.pf_rows, nq = a.n_q, qt = blockIdx.y, kc = blockIdx.x;
  int klo, khi, nkc;
  pf_tile_span(a, qt, &klo, &khi, &nkc);
  if (kc >= nkc) return;
  const int k0 = klo + kc * a.pf_chunk, k1 = min(k0 + a.pf_chunk, khi + 1);
  const bool active = h < nq;

  // K staging: wave w moves key rows 8 i + w of a tile, lane = float4 slot.
  // V of a tile is fetched while its scores run, K of the next tile while
  // the weighted sum runs, so the two staging sets are never live together.
  float4 st[4];
  auto fetch = [&](const float* cache, int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kt + 8 * i + wv;
      st[i] = *(const float4*)(cache + (size_t)(key < k1 ? key : k0) * kHeadDim + 4 * lane);
      if (key >= k1) st[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  // K rows as bf16 hi / lo planes (hi = bf16(k), lo = bf16(k - hi)); the
  // 16-byte unit u of row kr sits at u ^ kswz(kr), kswz = key bits 0, 1, 3, 4,
  // so that the 16 rows of one MFMA operand read cover all 16 bank groups
  auto kswz = [](int kr) { return (kr & 3) | ((kr >> 3) << 2); };
  auto stage_k = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kr = 8 * i + wv;
      const float4 x = st[i];
      bf16x4 hi, lo;
      split4_bf16(x.x, x.y, x.z, x.w, hi, lo);
      const int o = kr * kHeadDim + 8 * ((lane >> 1) ^ kswz(kr)) + 4 * (lane & 1);
      *(bf16x4*)&Kh[o] = hi;
      *(bf16x4*)&Kl[o] = lo;
    }
  };
  // V^T as bf16 hi / lo planes, 32 keys (64 bytes) per dim row; the 16-byte
  // unit u (keys 8u .. 8u + 7) of dim row d sits at u ^ ((d / 2) % 4). Wave w
  // fetches keys 4 w .. 4 w + 3, lane l dims 4 l .. 4 l + 3 (one 16-byte load
  // per key), and writes half w % 2 of unit w / 2 of its four dim rows.
  float vv[4][4];
  auto fetch_v = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kt + 4 * wv + i;
      const float4 x = *(const float4*)(a.v_cache + (size_t)(key < k1 ? key : k0) * kHeadDim + 4 * lane);
      vv[i][0] = key < k1 ? x.x : 0.f;
      vv[i][1] = key < k1 ? x.y : 0.f;
      vv[i][2] = key < k1 ? x.z : 0.f;
      vv[i][3] = key < k1 ? x.w : 0.f;
    }
  };
  auto stage_v = [&]() {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bf16x4 hi, lo;
      split4_bf16(vv[0][e], vv[1][e], vv[2][e], vv[3][e], hi, lo);
      const int d = 4 * lane + e;
      const int o = d * kPfKeys + 8 * ((wv >> 1) ^ ((d >> 1) & 3)) + 4 * (wv & 1);
      *(bf16x4*)&Vh[o] = hi;
      *(bf16x4*)&Vl[o] = lo;
    }
  };
  fetch(a.k_cache, k0);

  // q (normed + roped) of row l % 16, dims 32 t + 8 g .. +7, as bf16 hi / lo
  const int row = qt * kPfRows + rt * 16 + c16;
  const bool row_ok = row < M;
  const int prow = a.pf_start + row, plo = pf_key_lo(a, prow);
  const float sl2 = a.scale * 1.4426950408889634f;   // scores in log2 units (softmax in base 2)
  // keys [kt, kt + 31] are valid for every row of the tile: all rows exist,
  // the last key is <= the first row's position and < k1, and the first key
  // is >= the last row's window start
  const int r_first = a.pf_start + qt * kPfRows + rt * 16, r_last = r_first + 15;
  const bool rows_full = qt * kPfRows + rt * 16 + 16 <= M;
  const int lo_last = pf_key_lo(a, r_last);
  auto tile_full = [&](int kt) { return rows_full && kt + kPfKeys - 1 <= r_first && kt + kPfKeys <= k1 && kt >= lo_last; };
  const float* qp = a.qkv + (size_t)min(row, M - 1) * (nq * kHeadDim + 2 * kHeadDim) + min(h, nq - 1) * kHeadDim + 8 * g;
  bf16x8 qh[8], ql[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float4 x0 = *(const float4*)(qp + 32 * t), x1 = *(const float4*)(qp + 32 * t + 4);
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    uint32_t h4[4], l4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split2_bf16(xs[2 * e], xs[2 * e + 1], h4[e], l4[e]);
    qh[t] = __builtin_bit_cast(bf16x8, h4);
    ql[t] = __builtin_bit_cast(bf16x8, l4);
  }
  stage_k();

  f32x4 o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  for (int kt = k0; kt < k1; kt += kPfKeys) {
    fetch_v(kt);
    __syncthreads();   // K of this tile staged; the previous tile's V reads done
    float p[2][4];
    float alpha = 1.f;
    if (active) {
      f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      // S^T = K Q^T on bf16 MFMA: per 32 dims the products hi hi, lo hi and
      // hi lo (the dropped lo lo term is below 2^-16 of |k| |q|). Operand row
      // c16 of key tile j is key 8 (c16 / 4) + 4 j + c16 % 4, so register r of
      // lane group g holds key 8 g + 4 j + r.
#pragma unroll
      for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int kr = 8 * (c16 >> 2) + 4 * j + (c16 & 3);
          const int o = kr * kHeadDim + 8 * ((4 * t + g) ^ c16);
          const bf16x8 kh = lds_bf16x8(&Kh[o]), kl = lds_bf16x8(&Kl[o]);
          s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[t], s[j], 0, 0, 0);
          s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[t], s[j], 0, 0, 0);
          s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[t], s[j], 0, 0, 0);
        }
      }
      // scale (to log2 units) + causal / window mask; online softmax of row
      // l % 16 in base 2. A tile inside every row's key range needs no mask.
      float mx = -INFINITY;
      if (tile_full(kt)) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[j][r] = s[j][r] * sl2;
            mx = fmaxf(mx, p[j][r]);
          }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kt + 8 * g + 4 * j + r;
            const bool ok = row_ok && key < k1 && key >= plo && key <= prow;
            p[j][r] = ok ? s[j][r] * sl2 : -INFINITY;
            mx = fmaxf(mx, p[j][r]);
          }
      }
      mx = pf_xor32_max(pf_xor16_max(mx));
      const float mn = fmaxf(m, mx);
      const float mb = mn == -INFINITY ? 0.f : mn;   // a row with no key yet keeps p = 0
      alpha = __builtin_amdgcn_exp2f(m - mb);
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[j][r] = __builtin_amdgcn_exp2f(p[j][r] - mb);
          ps += p[j][r];
        }
      l = fmaf(l, alpha, ps);
      m = mn;
    }
    __syncthreads();   // every K read of this tile done
    stage_v();
    if (kt + kPfKeys < k1) fetch(a.k_cache, kt + kPfKeys);
    __syncthreads();   // V of this tile staged
    if (active) {
      // O rows 4 g + r take the factors of the lanes that hold those rows
      // (skipped when no row's running max moved: every factor is then 1)
      if (__ballot(alpha != 1.f)) {
        float ar[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[i][r] *= ar[r];
      }
      // O += P V on bf16 MFMA: A = P (row l % 16, keys 8 g .. 8 g + 7 =
      // p[j][r] for key 8 g + 4 j + r), B = V^T rows; hi.hi, lo.hi, hi.lo
      uint32_t ph4[4], pl4[4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        split2_bf16(p[j][0], p[j][1], ph4[2 * j], pl4[2 * j]);
        split2_bf16(p[j][2], p[j][3], ph4[2 * j + 1], pl4[2 * j + 1]);
      }
      const bf16x8 ph = __builtin_bit_cast(bf16x8, ph4), pl = __builtin_bit_cast(bf16x8, pl4);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 16 * i + c16;
        const int ov = d * kPfKeys + 8 * (g ^ ((d >> 1) & 3));
        const bf16x8 vh = lds_bf16x8(&Vh[ov]), vl = lds_bf16x8(&Vl[ov]);
        o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, vh, o[i], 0, 0, 0);
        o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, vh, o[i], 0, 0, 0);
        o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, vl, o[i], 0, 0, 0);
      }
    }
    if (kt + kPfKeys < k1) stage_k();   // no K reads until the next barrier
  }
  if (!active) return;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  float lr[4], mr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lr[r] = __shfl(l, 4 * g + r, 64);
    mr[r] = __shfl(m, 4 * g + r, 64);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int orow = qt * kPfRows + rt * 16 + 4 * g + r;
    if (orow >= M) continue;
    if (nkc == 1) {
      uint16_t* out = a.pf_out + (size_t)orow * nq * kHeadDim + h * kHeadDim + c16;
      const size_t plane = (size_t)M * nq * kHeadDim;
      const float il = 1.f / lr[r];
#pragma unroll
      for (int i = 0; i < 16; ++i) split_bf16(o[i][r] * il, &out[16 * i], &out[plane + 16 * i]);
    } else {
      float* pp = a.part + (((size_t)orow * kPrefillChunks + kc) * nq + h) * (2 + kHeadDim);
#pragma unroll
      for (int i = 0; i < 16; ++i) pp[2 + 16 * i + c16] = o[i][r];
      if (c16 == 0) {
        pp[0] = mr[r];
        pp[1] = lr[r];
      }
    }
  }
}

// Rows of query tiles with more than one chunk: softmax-weighted sum of the
// chunks' (m, l, O) (maxima in log2 units, as k_attn_pf keeps them), one
// block per (row, query head), thread = head dim.
__global__ __launch_bounds__(256) void k_attn_pf_merge(AttnArgs a) {
  // one block per prompt row: wave h merges head h, lane l dims 4 l .. 4 l + 3
  // (16-byte loads of each chunk's o); the same per-element sums, in chunk
  // order, as one thread per dim
  const int row = blockIdx.x, tid = threadIdx.x, nq = a.n_q, h = tid >> 6, d4 = tid & 63;
  int klo, khi, nkc;
  pf_tile_span(a, row / kPfRows, &klo, &khi, &nkc);
  if (nkc == 1 || h >= nq) return;
  const float* pr = a.part + (size_t)row * kPrefillChunks * nq * (2 + kHeadDim);
  // chunks in groups of four, each group's loads issued together (clamped
  // indices; a group's chunks past nkc are skipped in the sums)
  constexpr int G = 4;
  float M = -INFINITY;
  for (int c0 = 0; c0 < nkc; c0 += G) {
    float m[G];
#pragma unroll
    for (int j = 0; j < G; ++j) m[j] = pr[(min(c0 + j, nkc - 1) * nq + h) * (2 + kHeadDim)];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (c0 + j < nkc) M = fmaxf(M, m[j]);
  }
  float L = 0.f;
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int c0 = 0; c0 < nkc; c0 += G) {
    float m[G], l[G];
    float4 o[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float* pc = pr + (min(c0 + j, nkc - 1) * nq + h) * (2 + kHeadDim);
      m[j] = pc[0];
      l[j] = pc[1];
      // a partial's o starts 2 floats into its 258-float record: 8-byte aligned
      const float2 lo2 = *(const float2*)(pc + 2 + 4 * d4), hi2 = *(const float2*)(pc + 4 + 4 * d4);
      o[j] = make_float4(lo2.x, lo2.y, hi2.x, hi2.y);
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (c0 + j < nkc) {
        const float f = m[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[j] - M);
        L = fmaf(f, l[j], L);
        O.x = fmaf(f, o[j].x, O.x);
        O.y = fmaf(f, o[j].y, O.y);
        O.z = fmaf(f, o[j].z, O.z);
        O.w = fmaf(f, o[j].w, O.w);
      }
    }
  }
  const size_t e = (size_t)row * nq * kHeadDim + h * kHeadDim + 4 * d4;
  const size_t lo = (size_t)a.pf_rows * nq * kHeadDim;
  split_bf16(O.x / L, &a.pf_out[e], &a.pf_out[lo + e]);
  split_bf16(O.y / L, &a.pf_out[e + 1], &a.pf_out[lo + e + 1]);
  split_bf16(O.z / L, &a.pf_out[e + 2], &a.pf_out[lo + e + 2]);
  split_bf16(O.w / L, &a.pf_out[e + 3], &a.pf_out[lo + e + 3]);
}

// ---------------------------------------------------------------------------
// Batched prefill GEMMs (no reference counterpart: the reference runs the
// decode pass once per prompt token, engine.ts:923-928).
//
// k_gemm: C[M x N] = A[M x K] * W[N x K]^T on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16, K = 32 = one Q8_0 block). W holds the int8
// weights as bf16 (exact); A is split by its producer into hi = bf16(x) and
// lo = bf16(x - hi), so x - hi - lo is within 2^-17 |x| and every product
// q * hi, q * lo is exact in the fp32 accumulator. Per 32-block the two
// MFMAs give sum_j q_j x_j, which is scaled by the block's fp32 scale d and
// added to the output in fp32 -- the linearQ8 structure (shaders.ts:123-142)
// with the block sum on the matrix cores.
//
// Block tile 128 (rows) x BN (features) x 64 (k step), four waves of
// 16 NI x 16 NJ (NI x NJ MFMA tiles): 2 x 2 waves of 64 x 64 (BN = 128),
// 4 x 1 waves of 32 x 144 (BN = 144; 1152-wide outputs then split into 8
// tiles, so that a K split of 4 fills the 512 block slots of the chip
// exactly) or 2 x 2 waves of 64 x 48 (BN = 96; the 1536 QKV outputs in 16
// tiles, so that a K split of 2 gives 512 blocks at 2048 rows). LDS rows are padded to 72 bf16 so that the 16 lanes of a lane
// group (16 rows, one 16-byte chunk) cover all banks; the next step's global
// loads are issued before the current step's MFMAs.
// ---------------------------------------------------------------------------
constexpr int kGBM = 128, kGBP = 72;

template <int EPI, int NI, int NJ>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs a) {
  constexpr int WM = 128 / (16 * NI), WN = 4 / WM;   // waves along rows / features
  constexpr int BN = WN * 16 * NJ;
  constexpr int WI = (BN * 8 + 255) / 256;   // 16-byte W chunks per thread and step
  constexpr int DI = (BN * 2 + 255) / 256;   // block scales per thread and step
  static_assert(WM * WN == 4 && WM * 16 * NI == kGBM, "four waves cover the 128-row tile");
  static_assert(EPI == EPI_OUT || NJ % 2 == 0, "GeGLU pairs adjacent column tiles");
  __shared__ __align__(16) uint16_t Ah[kGBM * kGBP];
  __shared__ __align__(16) uint16_t Al[kGBM * kGBP];
  __shared__ __align__(16) uint16_t Ws[BN * kGBP];
  __shared__ float Ds[BN * 2];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int M = a.M, K = a.K;
  // Tile order: workgroups go to the XCDs round-robin (from an XCD that
  // depends on earlier dispatches), so the blocks with one value of b % 8
  // (launch order) share an XCD; they take the contiguous range
  // [(b % 8) G / 8, (b % 8 + 1) G / 8) of an order with the K slice
  // slowest, then groups of 4 tile rows with the rows fastest, so that the
  // blocks sharing an XCD's L2 share A rows and W tiles (fewer L2 misses).
  const int NT = gridDim.x, MT = gridDim.y, G = NT * MT * gridDim.z;
  const int bid = blockIdx.x + NT * (blockIdx.y + MT * blockIdx.z);
  const int L = (G % 8 == 0) ? (bid % 8) * (G / 8) + bid / 8 : bid;
  const int kz = L / (NT * MT), Lp = L % (NT * MT);
  const int fm = (Lp / (4 * NT)) * 4, gm = min(MT - fm, 4);
  const int m0 = (fm + (Lp % (4 * NT)) % gm) * kGBM, n0 = ((Lp % (4 * NT)) / gm) * BN;
  const int kn = K / a.ks;   // this block's K slice [kz kn, (kz + 1) kn)
  const int wm = (wv / WN) * 16 * NI, wn = (wv % WN) * 16 * NJ;
  const size_t MK = (size_t)M * K;
  // staging: rows tid / 8 + 32 i, 16-byte chunk tid % 8 of the 64-wide step;
  // scale (row tid / 2 + 128 i, block tid % 2)
  const int sr = tid >> 3, sc = (tid & 7) * 8;
  const uint16_t* a0 = a.A + sc;
  const uint16_t* w0 = a.W + (size_t)(n0 + sr) * K + sc;
  const float* dp = a.D + (size_t)(n0 + (tid >> 1)) * (K / 32) + (tid & 1);
  u32x4 rh[4], rl[4], rw[WI];
  float rd[DI];
  auto fetch = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t* ar = a0 + (size_t)min(m0 + sr + 32 * i, M - 1) * K + k0;
      rh[i] = *(const u32x4*)ar;
      rl[i] = *(const u32x4*)(ar + MK);
    }
#pragma unroll
    for (int i = 0; i < WI; ++i)
      if (BN >= 32 * (i + 1) || sr + 32 * i < BN) rw[i] = *(const u32x4*)(w0 + (size_t)(32 * i) * K + k0);
#pragma unroll
    for (int i = 0; i < DI; ++i)
      if (BN >= 128 * (i + 1) || tid + 256 * i < 2 * BN) rd[i] = dp[(size_t)(128 * i) * (K / 32) + k0 / 32];
  };
  auto stage = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (sr + 32 * i) * kGBP + sc;
      *(u32x4*)&Ah[r] = rh[i];
      *(u32x4*)&Al[r] = rl[i];
    }
#pragma unroll
    for (int i = 0; i < WI; ++i)
      if (BN >= 32 * (i + 1) || sr + 32 * i < BN) *(u32x4*)&Ws[(sr + 32 * i) * kGBP + sc] = rw[i];
#pragma unroll
    for (int i = 0; i < DI; ++i)
      if (BN >= 128 * (i + 1) || tid + 256 * i < 2 * BN) Ds[tid + 256 * i] = rd[i];
  };

  f32x4 acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int kb = kz * kn, ke = kb + kn;
  fetch(kb);
  for (int k0 = kb; k0 < ke; k0 += 64) {
    __syncthreads();   // the previous step's LDS reads are done
    stage();
    __syncthreads();
    if (k0 + 64 < ke) fetch(k0 + 64);
    // the MFMA phase runs at raised wave priority: with two blocks on a CU
    // the one computing issues ahead of the one staging (down 97 -> 85 us,
    // O 24.3 -> 22.2 us at the 1B prefill shapes; no effect alone on a CU)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      bf16x8 xh[NI], xl[NI], w[NJ];
      float d[NJ];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int o = (wm + 16 * i + c16) * kGBP + 32 * b + 8 * g;
        xh[i] = lds_bf16x8(&Ah[o]);
        xl[i] = lds_bf16x8(&Al[o]);
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        w[j] = lds_bf16x8(&Ws[(wn + 16 * j + c16) * kGBP + 32 * b + 8 * g]);
        d[j] = Ds[(wn + 16 * j + c16) * 2 + b];
      }
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh[i], w[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl[i], w[j], p, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(d[j], p[r], acc[i][j][r]);
        }
    }
    __builtin_amdgcn_s_setprio(0);
  }
  // D[i][j] of a 16x16 tile: lane l, register r -> row 4 (l / 16) + r, col l % 16
  const size_t half_plane = (size_t)M * (a.N / 2);
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm + 16 * i + 4 * g + r;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int n = n0 + wn + 16 * j + c16;
        if (EPI == EPI_OUT) {
          a.C[(size_t)kz * M * a.N + (size_t)m * a.N + n] = acc[i][j][r];
        } else if ((j & 1) == 0) {
          // 16 gate rows (tile j), then their 16 up rows (tile j + 1)
          const size_t o = (size_t)m * (a.N / 2) + (n >> 5) * 16 + (n & 15);
          split_bf16(gelu_mul(acc[i][j][r], acc[i][j | 1][r]), &a.act[o], &a.act[half_plane + o]);
        }
      }
    }
}

// Row kernels (one block per prompt row, H <= 2048).
__device__ __forceinline__ void row_norm_out(const float* r, const float* w, int H, float eps, uint16_t* out,
                                             size_t plane, float* sh4, int n) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) ss = fmaf(r[i], r[i], ss);
  const float ri = rsq(block_sum256(ss, sh4) / (float)H + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) {
      const int e = threadIdx.x + 256 * i;
      split_bf16((r[i] * w[e]) * ri, &out[e], &out[plane + e]);
    }
}

__global__ __launch_bounds__(256) void k_rows_embed(RowArgs a) {
  __shared__ float sh4[4];
  const int row = blockIdx.x, tid = threadIdx.x, H = a.H;
  const int n = (H - tid + 255) / 256;
  const int token = a.tokens[row];
  float h[8];
  GemvArgs g{};
  g.embd = a.embd;
  g.embd_KpS = a.embd_KpS;
  g.embed_scale = a.embed_scale;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) {
      h[i] = embed_elem(g, token, tid + 256 * i);
      a.res_out[(size_t)row * H + tid + 256 * i] = h[i];
    }
  row_norm_out(h, a.w_pre, H, a.eps, a.x_out + (size_t)row * H, (size_t)a.M * H, sh4, n);
}

__global__ __launch_bounds__(256) void k_rows_resid(RowArgs a) {
  // one wave per prompt row, four rows per block: lane l holds float4s
  // l + 64 k of the row, so both sums of squares are wave reductions (no
  // LDS, no barrier); every load of the row is issued before the sums
  constexpr int KF = 2048 / 4 / 64;   // float4s per lane at the largest hidden size
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), H = a.H;
  if (row >= a.M) return;
  const int F4 = H / 4;
  const size_t o4 = (size_t)row * F4;
  const float4* pre = (const float4*)a.pre;
  const float4* res = (const float4*)a.res;
  const float4* wpost = (const float4*)a.w_post;
  const float4* wpre = (const float4*)a.w_pre;
  const size_t ps4 = a.pre_stride / 4;
  float4 v[KF], rs[KF], wq[KF];
#pragma unroll
  for (int k = 0; k < KF; ++k) {
    const int f = lane + 64 * k;
    if (f < F4) {
      v[k] = pre[o4 + f];
      float4 pv[kGemmMaxSlices - 1];
#pragma unroll
      for (int p = 1; p < kGemmMaxSlices; ++p)
        if (p < a.pre_planes) pv[p - 1] = pre[p * ps4 + o4 + f];
      rs[k] = res[o4 + f];
      wq[k] = wpost[f];
      // K slices of the previous GEMM, added in slice order
#pragma unroll
      for (int p = 1; p < kGemmMaxSlices; ++p)
        if (p < a.pre_planes) {
          v[k].x += pv[p - 1].x;
          v[k].y += pv[p - 1].y;
          v[k].z += pv[p - 1].z;
          v[k].w += pv[p - 1].w;
        }
    }
  }
  float s1 = 0.f;
#pragma unroll
  for (int k = 0; k < KF; ++k)
    if (lane + 64 * k < F4) {
      s1 = fmaf(v[k].x, v[k].x, s1);
      s1 = fmaf(v[k].y, v[k].y, s1);
      s1 = fmaf(v[k].z, v[k].z, s1);
      s1 = fmaf(v[k].w, v[k].w, s1);
    }
  const float ri1 = rsq(wave_sum_dpp(s1) / (float)H + a.eps);
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < KF; ++k) {
    const int f = lane + 64 * k;
    if (f < F4) {
      float4 r;
      r.x = rs[k].x + (v[k].x * wq[k].x) * ri1;
      r.y = rs[k].y + (v[k].y * wq[k].y) * ri1;
      r.z = rs[k].z + (v[k].z * wq[k].z) * ri1;
      r.w = rs[k].w + (v[k].w * wq[k].w) * ri1;
      ((float4*)a.res_out)[o4 + f] = r;
      if (a.last_hidden && row == a.M - 1) ((float4*)a.last_hidden)[f] = r;
      v[k] = r;
      ss = fmaf(r.x, r.x, ss);
      ss = fmaf(r.y, r.y, ss);
      ss = fmaf(r.z, r.z, ss);
      ss = fmaf(r.w, r.w, ss);
    }
  }
  const float ri = rsq(wave_sum_dpp(ss) / (float)H + a.eps);
  const size_t plane = (size_t)a.M * H;
#pragma unroll
  for (int k = 0; k < KF; ++k) {
    const int f = lane + 64 * k;
    if (f < F4) {
      const float4 w = wpre[f];
      const float y[4] = {(v[k].x * w.x) * ri, (v[k].y * w.y) * ri, (v[k].z * w.z) * ri, (v[k].w * w.w) * ri};
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) split_bf16(y[j], &hi[j], &lo[j]);
      const size_t e = (size_t)row * H + 4 * f;
      *(uint2*)(a.x_out + e) = make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
      *(uint2*)(a.x_out + plane + e) = make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
    }
  }
}

// One block per prompt row: RMSNorm + NEOX RoPE of the key head (into the
// cache, with v) and of every query head, the latter in place in the QKV
// rows for the attention kernel (fusedPerHeadNormRope, shaders.ts:420-467).
__global__ __launch_bounds__(320) void k_rows_kv(RowArgs a) {
  // wave w < n_q: query head w of the row, in place; wave n_q: the key head
  // (into the cache) and the value row. Lane l holds dims l + 64 j, so the
  // NEOX pairs (i, i + 128) are its own j and j + 2, and the head's sum of
  // squares is one wave reduction: no LDS, no barrier
  const int row = blockIdx.x, wv = threadIdx.x >> 6, lane = threadIdx.x & 63, nq = a.n_q;
  if (wv > nq) return;
  const int pos = a.pf_start + row;
  float* qrow = const_cast<float*>(a.qkv) + (size_t)row * (nq * kHeadDim + 2 * kHeadDim);
  float* src = qrow + wv * kHeadDim;   // wave nq: the key head
  const float* w = wv < nq ? a.q_norm : a.k_norm;
  const float* rt = a.rope + (size_t)pos * kHeadDim;
  // the QKV GEMM's K slices (pre_planes of them, pre_stride floats apart)
  // are added in slice order; the sum stays in slice 0
  const int ns = a.pre_planes > 1 ? a.pre_planes : 1;
  float x[4], nw[4], cs[2], sn[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[j] = src[lane + 64 * j];
    nw[j] = w[lane + 64 * j];
  }
  for (int p = 1; p < ns; ++p)
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] += src[p * a.pre_stride + lane + 64 * j];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cs[j] = rt[lane + 64 * j];
    sn[j] = rt[kHeadDim / 2 + lane + 64 * j];
  }
  float v[4];
  if (wv == nq) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = src[kHeadDim + lane + 64 * j];
    for (int p = 1; p < ns; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += src[p * a.pre_stride + kHeadDim + lane + 64 * j];
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) ss = fmaf(x[j], x[j], ss);
  const float ri = rsq(wave_sum_dpp(ss) / (float)kHeadDim + a.eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = (x[j] * nw[j]) * ri;
  float* dst = wv < nq ? src : a.k_cache + (size_t)pos * kHeadDim;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float x0 = x[j], x1 = x[j + 2];
    dst[lane + 64 * j] = x0 * cs[j] - x1 * sn[j];
    dst[lane + 64 * j + 128] = x0 * sn[j] + x1 * cs[j];
  }
  if (wv == nq) {
#pragma unroll
    for (int j = 0; j < 4; ++j) a.v_cache[(size_t)pos * kHeadDim + lane + 64 * j] = v[j];
  }
}

// ---------------------------------------------------------------------------
// Upload helpers.
// k_repack: GGUF row-major Q8_0 (rows of Kp 68-byte pairs) -> the
// item-planar layout L. interleave_half > 0 places source row r at fused
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
  uint8_t* item = dst + ((size_t)g * L.KpS + c / L.CI) * kColBytes;
  const int slot = (c % L.CI) * L.GR + ln;
#pragma unroll
  for (int i = 0; i < 17; ++i) *(uint32_t*)(item + plane_offset(i, slot)) = s[i];
}

// Class-major copy of a CI = 1 item-planar matrix (the tied LM head): row
// c + 256 k (vocabulary stride class c, shaders.ts:337-347) goes to row
// c * (rows / 256) + k, so each 64-row group of the copy holds one class.
__global__ __launch_bounds__(256) void k_class_major(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                     long long rows, int Kp) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * Kp) return;
  const long long r = idx / Kp;
  const int c = (int)(idx - r * Kp);
  const long long p = (r & 255) * (rows >> 8) + (r >> 8);
  const uint8_t* si = src + ((size_t)(r >> 6) * Kp + c) * kColBytes;
  uint8_t* di = dst + ((size_t)(p >> 6) * Kp + c) * kColBytes;
  const int ss = (int)(r & 63), ds = (int)(p & 63);
#pragma unroll
  for (int i = 0; i < 17; ++i) *(uint32_t*)(di + plane_offset(i, ds)) = *(const uint32_t*)(si + plane_offset(i, ss));
}

// Column-block layout of a Q8_0 matrix (the down projection of the
// persistent decode kernel): for each 32-wide input block m, the f16 scales
// of all rows [rows], then their 32 int8 values [rows][32]: 34 * rows bytes
// per block, so one block's column slice is contiguous.
__global__ __launch_bounds__(256) void k_repack_colblock(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         long long rows, int nblk) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * nblk) return;
  const long long r = idx / nblk;
  const int m = (int)(idx - r * nblk);
  const uint8_t* blk = src + (size_t)idx * 34;
  uint8_t* col = dst + (size_t)m * 34 * rows;
  col[2 * r] = blk[0];
  col[2 * r + 1] = blk[1];
  uint8_t* q = col + 2 * rows + 32 * r;
#pragma unroll
  for (int i = 0; i < 32; ++i) q[i] = blk[2 + i];
}

// Gate/up copy of the persistent decode kernel laid out as the B operands of
// v_mfma_i32_16x16x64_i8. Group g holds gate rows 32g .. 32g + 31 and up rows
// 32g .. 32g + 31 as four 16-row tiles t (0, 1: gate; 2, 3: up). For pair
// column c (k in [64c, 64c + 64)) tile t is 1 KB at c * 4096 + t * 1024, where
// lane l's 16 bytes are row 16 (t & 1) + l % 16 of its half at k = 64c +
// 16 (l / 16) .. +15. After the Kp * 4096 int8 bytes come the block scales,
// [t][m][lane < 32] dwords: the f16 scales of pair columns 2m (low half) and
// 2m + 1 (high half) for row 16 (t & 1) + lane % 16, Q8_0 block 2c + lane / 16.
// One thread per 16-byte chunk, then one per scale dword, of the gate (up = 0)
// or up (up = 1) half.
__global__ __launch_bounds__(256) void k_repack_gum(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                    long long rows, int K, int up) {
  const int Kp = K / 64, Kh = (Kp + 1) / 2;
  const size_t gbytes = gum_group_bytes(K), rowb = (size_t)K / 32 * 34;
  const long long groups = rows / 32;
  const long long nch = groups * Kp * 2 * 64, nsc = groups * 2 * Kh * 32;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < nch) {
    const int lane = (int)(i % 64);
    long long q = i / 64;
    const int th = (int)(q % 2);
    q /= 2;
    const int c = (int)(q % Kp);
    const long long g = q / Kp;
    const long long row = 32 * g + 16 * th + lane % 16;
    const int k0 = 64 * c + 16 * (lane / 16);
    const uint8_t* sp = src + row * rowb + (size_t)(k0 / 32) * 34 + 2 + k0 % 32;
    uint8_t* dp = dst + g * gbytes + (size_t)c * 4096 + (size_t)(th + 2 * up) * 1024 + (size_t)lane * 16;
#pragma unroll
    for (int j = 0; j < 16; ++j) dp[j] = sp[j];
  } else if (i < nch + nsc) {
    long long q = i - nch;
    const int lane = (int)(q % 32);
    q /= 32;
    const int m = (int)(q % Kh);
    q /= Kh;
    const int th = (int)(q % 2);
    const long long g = q / 2;
    const long long row = 32 * g + 16 * th + lane % 16;
    uint32_t v = 0;
    for (int h = 0; h < 2; ++h) {
      const int c = 2 * m + h;
      if (c < Kp) {
        const uint8_t* bp = src + row * rowb + (size_t)(2 * c + lane / 16) * 34;
        v |= (uint32_t)(bp[0] | (bp[1] << 8)) << (16 * h);
      }
    }
    *(uint32_t*)(dst + g * gbytes + (size_t)Kp * 4096 + ((size_t)((th + 2 * up) * Kh + m) * 32 + lane) * 4) = v;
  }
}

// Embedding row of one token through embed_value (parity reads).
__global__ __launch_bounds__(256) void k_embed_row(const uint8_t* embd, int kps, float scale, int token, int H,
                                                   float* out) {
  for (int e = threadIdx.x; e < H; e += 256) out[e] = embed_value(embd, kps, scale, token, e);
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

// GGUF Q8_0 rows -> the prefill GEMM's weights: int8 values as bf16 (exact)
// and fp32 block scales, one thread per 32-block. Source row r goes to row
// r + off, or with half = 16 to (r / 16) * 32 + r % 16 + off (gate / up
// groups of 16 + 16 rows).
__global__ __launch_bounds__(256) void k_q8_bf16(const uint8_t* __restrict__ src, uint16_t* __restrict__ wb,
                                                 float* __restrict__ wd, long long rows, int K, long long off,
                                                 int half) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const int nb = K / 32;
  if (idx >= rows * nb) return;
  const long long r = idx / nb;
  const int b = (int)(idx - r * nb);
  const long long R = half > 0 ? (r / half) * 2 * half + r % half + off : r + off;
  const uint8_t* blk = src + (size_t)idx * 34;
  wd[R * nb + b] = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[0] | (blk[1] << 8)));
  uint32_t* o = (uint32_t*)(wb + R * K + 32 * b);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float f0 = (float)(int8_t)blk[2 + 2 * j], f1 = (float)(int8_t)blk[3 + 2 * j];
    o[j] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
  }
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
    case 2: return launch_gemv_nif<PRO, EPI, 2>(a, s);
    case 8: return launch_gemv_nif<PRO, EPI, 8>(a, s);
  }
  return (int)hipErrorInvalidValue;
}

// Launch plan of k_gemv_mg: W = 4 waves for K <= 2048, 16 above; about two
// blocks per CU (512 or 256 blocks, at most one per row group), more blocks
// when a wave would otherwise hold more than three items in registers.
// Returns false when no plan keeps every wave at <= 3 items.
struct MgPlan { int W, nb, nif, ept; };
static bool mg_plan(const GemvArgs& a, int pro, int ci, MgPlan& p) {
  const int K = a.Kp * 64, GR = 64 / ci, G = a.N / GR;
  p.W = K > 2048 ? 16 : 4;
  if ((pro != PRO_NONE || ci != 8) && p.W != 4) return false;
  p.ept = (K / 4 + 64 * p.W - 1) / (64 * p.W);   // float4 chunks of x per thread: 1 or 2
  if (p.ept > 2) return false;
  int nb = min(G, p.W == 4 ? 512 : 256);
  for (;;) {
    const int gpb = (G + nb - 1) / nb;
    const int nif = (gpb * a.KpS + p.W - 1) / p.W;
    if (nif <= 3 && gpb * GR <= kMgRows) {
      p.nb = nb;
      p.nif = nif;
      return true;
    }
    if (nb == G) return false;
    nb = min(G, nb * 2);
  }
}

template <int PRO, int EPI, int CI, int W, int NIF>
static int launch_mg_ept(const GemvArgs& a, const MgPlan& p, hipStream_t s) {
  const size_t lds = (size_t)a.Kp * kXPad * sizeof(float);
  switch (p.ept) {
#define GG_MG_EPT(E) \
    case E: hipLaunchKernelGGL((k_gemv_mg<PRO, EPI, CI, W, NIF, E>), dim3(p.nb), dim3(64 * W), lds, s, a); break;
    GG_MG_EPT(1) GG_MG_EPT(2)
#undef GG_MG_EPT
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}
template <int PRO, int EPI, int CI, int W>
static int launch_mg_nif(const GemvArgs& a, const MgPlan& p, hipStream_t s) {
  switch (p.nif) {
    case 1: return launch_mg_ept<PRO, EPI, CI, W, 1>(a, p, s);
    case 2: return launch_mg_ept<PRO, EPI, CI, W, 2>(a, p, s);
    case 3: return launch_mg_ept<PRO, EPI, CI, W, 3>(a, p, s);
  }
  return (int)hipErrorInvalidValue;
}
template <int CI>
static int launch_mg_ci(int pro, int epi, const GemvArgs& a, const MgPlan& p, hipStream_t s) {
  if (pro == PRO_ATTN_MERGE) return launch_mg_nif<PRO_ATTN_MERGE, EPI_OUT, CI, 4>(a, p, s);
  if (pro == PRO_NONE) {
    if (CI == 8 && p.W == 16) return launch_mg_nif<PRO_NONE, EPI_OUT, 8, 16>(a, p, s);
    return launch_mg_nif<PRO_NONE, EPI_OUT, CI, 4>(a, p, s);
  }
  if (epi == EPI_GEGLU) return launch_mg_nif<PRO_RESID_NORM, EPI_GEGLU, CI, 4>(a, p, s);
  if (pro == PRO_EMBED_NORM) return launch_mg_nif<PRO_EMBED_NORM, EPI_OUT, CI, 4>(a, p, s);
  return launch_mg_nif<PRO_RESID_NORM, EPI_OUT, CI, 4>(a, p, s);
}
static int launch_mg(int pro, int epi, int ci, const GemvArgs& a, const MgPlan& p, hipStream_t s) {
  return ci == 2 ? launch_mg_ci<2>(pro, epi, a, p, s) : launch_mg_ci<8>(pro, epi, a, p, s);
}

int launch_gemv(int pro, int epi, int ci, const GemvArgs& a, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (a.Kp * 64 > kMaxK || a.Kp <= 0 || a.N <= 0 || (ci != 1 && ci != 2 && ci != 8) || a.N % (64 / ci) ||
      a.KpS != (a.Kp + ci - 1) / ci)
    return (int)hipErrorInvalidValue;
  if (pro != PRO_NONE && a.Kp * 64 > kMaxEPT / 4 * 256) return (int)hipErrorInvalidValue;
  if (epi == EPI_GEGLU && pro != PRO_RESID_NORM) return (int)hipErrorInvalidValue;
  MgPlan plan;
  if (pro == PRO_ATTN_MERGE) {   // only the multi-group kernel merges: K = n_q * 256 <= 1024 on 256 threads
    if (ci == 1 || a.Kp * 64 > kAttnMaxQ * kHeadDim || a.Kp % 4 || a.attn_chunks < 1 ||
        a.attn_chunks > kDecMaxChunks || !mg_plan(a, pro, ci, plan))
      return (int)hipErrorInvalidValue;
    return launch_mg(pro, epi, ci, a, plan, s);
  }
  if (ci != 1 && mg_plan(a, pro, ci, plan)) return launch_mg(pro, epi, ci, a, plan, s);
  if (epi == EPI_GEGLU) return launch_gemv_ci<PRO_RESID_NORM, EPI_GEGLU>(ci, a, s);
  if (pro == PRO_NONE) return launch_gemv_ci<PRO_NONE, EPI_OUT>(ci, a, s);
  if (pro == PRO_EMBED_NORM) return launch_gemv_ci<PRO_EMBED_NORM, EPI_OUT>(ci, a, s);
  if (pro == PRO_RESID_NORM) return launch_gemv_ci<PRO_RESID_NORM, EPI_OUT>(ci, a, s);
  return (int)hipErrorInvalidValue;
}

int launch_attention(const AttnArgs& a, int grid, void* stream) {
  if (a.n_q < 1 || a.n_q > kAttnMaxQ || grid < 1 || grid > kDecMaxChunks) return (int)hipErrorInvalidValue;
  if (grid <= kDecMergeInO) hipLaunchKernelGGL(k_attn_dec<1>, dim3(grid, a.n_q), dim3(256), 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(k_attn_dec<kAttnMaxQ>, dim3(grid), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_attention_merge(const AttnArgs& a, int chunks, void* stream) {
  if (a.n_q < 1 || a.n_q > kAttnMaxQ || chunks < 1 || chunks > kDecMaxChunks || !a.part || !a.attn_out)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_merge, dim3(kHeadDim / 32, a.n_q), dim3(256), 0, (hipStream_t)stream, a, chunks);
  return (int)hipGetLastError();
}

int launch_prefill_attention(const AttnArgs& a, int M, void* stream) {
  if (a.n_q < 1 || a.n_q > kAttnMaxQ || M < 1 || a.pf_rows != M || a.pf_start < 0 || a.window < 0 ||
      a.pf_chunk < kPfKeys || a.pf_chunk % kPfKeys)
    return (int)hipErrorInvalidValue;
  const int span = prefill_max_span(a.window, a.pf_start, M);
  const int nkc = (span + a.pf_chunk - 1) / a.pf_chunk;
  if (nkc > kPrefillChunks) return (int)hipErrorInvalidValue;   // `part` holds kPrefillChunks per row
  hipLaunchKernelGGL(k_attn_pf, dim3(nkc, (M + kPfRows - 1) / kPfRows), dim3(512), 0, (hipStream_t)stream, a);
  if (nkc > 1) hipLaunchKernelGGL(k_attn_pf_merge, dim3(M), dim3(256), 0, (hipStream_t)stream, a);
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

int launch_embed_row(const uint8_t* embd, int kps, float scale, int token, int H, float* out, void* stream) {
  hipLaunchKernelGGL(k_embed_row, dim3(1), dim3(256), 0, (hipStream_t)stream, embd, kps, scale, token, H, out);
  return (int)hipGetLastError();
}

int launch_repack_gum(const uint8_t* src, uint8_t* dst, long long rows, int K, int up, void* stream) {
  if (rows <= 0 || rows % 32 || K <= 0 || K % 64) return (int)hipErrorInvalidValue;
  const int Kp = K / 64, Kh = (Kp + 1) / 2;
  const long long total = rows / 32 * (Kp * 2 * 64 + 2 * Kh * 32);
  hipLaunchKernelGGL(k_repack_gum, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src,
                     dst, rows, K, up);
  return (int)hipGetLastError();
}

int launch_repack_colblock(const uint8_t* src, uint8_t* dst, long long rows, int K, void* stream) {
  if (rows <= 0 || K <= 0 || K % 32) return (int)hipErrorInvalidValue;
  const long long total = rows * (K / 32);
  hipLaunchKernelGGL(k_repack_colblock, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     src, dst, rows, K / 32);
  return (int)hipGetLastError();
}

int launch_class_major(const uint8_t* src, uint8_t* dst, long long rows, int Kp, void* stream) {
  if (rows <= 0 || rows % 16384 || Kp <= 0) return (int)hipErrorInvalidValue;
  const long long total = rows * Kp;
  hipLaunchKernelGGL(k_class_major, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src,
                     dst, rows, Kp);
  return (int)hipGetLastError();
}

int launch_q8_bf16(const uint8_t* src, uint16_t* wb, float* wd, long long rows, int K, long long off, int half,
                   void* stream) {
  if (K % 32 || off < 0 || (half != 0 && half != 16)) return (int)hipErrorInvalidValue;
  const long long total = rows * (K / 32);
  if (total <= 0) return 0;
  hipLaunchKernelGGL(k_q8_bf16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src, wb,
                     wd, rows, K, off, half);
  return (int)hipGetLastError();
}

int launch_dequant(const uint8_t* src, float* out, long long n, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, src, out,
                     n);
  return (int)hipGetLastError();
}

int launch_gemm(int epi, const GemmArgs& a, void* stream) {
  const int bn = a.bn;
  if (a.M < 1 || (bn != 128 && bn != 144 && bn != 96) || (bn != 128 && epi != EPI_OUT) || a.N < bn || a.N % bn ||
      a.K < 64 || a.ks < 1 || a.ks > kGemmMaxSlices || a.K % (64 * a.ks) || !a.A || !a.W || !a.D ||
      (epi == EPI_OUT ? !a.C : (!a.act || a.ks != 1)))
    return (int)hipErrorInvalidValue;
  dim3 grid(a.N / bn, (a.M + kGBM - 1) / kGBM, a.ks);
  if (epi == EPI_GEGLU) hipLaunchKernelGGL((k_gemm<EPI_GEGLU, 4, 4>), grid, dim3(256), 0, (hipStream_t)stream, a);
  else if (bn == 128) hipLaunchKernelGGL((k_gemm<EPI_OUT, 4, 4>), grid, dim3(256), 0, (hipStream_t)stream, a);
  else if (bn == 96) hipLaunchKernelGGL((k_gemm<EPI_OUT, 4, 3>), grid, dim3(256), 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL((k_gemm<EPI_OUT, 2, 9>), grid, dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_rows_embed(const RowArgs& a, void* stream) {
  if (a.H > 2048 || a.M < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rows_embed, dim3(a.M), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_rows_resid(const RowArgs& a, void* stream) {
  if (a.H > 2048 || a.M < 1) return (int)hipErrorInvalidValue;
  if (a.H % 4 || a.pre_stride % 4) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rows_resid, dim3((a.M + 3) / 4), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_rows_kv(const RowArgs& a, void* stream) {
  if (a.M < 1) return (int)hipErrorInvalidValue;
  if (a.n_q < 1 || a.n_q > kAttnMaxQ || a.pre_planes > kQkvMaxSlices ||
      (a.pre_planes > 1 && a.pre_stride < (size_t)a.M * (a.n_q + 2) * kHeadDim))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rows_kv, dim3(a.M), dim3(64 * (a.n_q + 1)), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_seen_add(uint32_t* seen, DevState* st, const int32_t* ids, int n, int V, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_seen_add, dim3(1), dim3(256), 0, (hipStream_t)stream, seen, st, ids, n, V);
  return (int)hipGetLastError();
}

}  // namespace gg

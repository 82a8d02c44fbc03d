// gg_device.h -- gfx950 device helpers shared by the per-kernel token loop
// (gg_kernels.hip) and the persistent decode kernel (gg_decode.hip):
// Q8_0 item loads and dot products, DPP wave reductions, GeGLU.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gg_internal.h"

namespace gg {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kXPad = 68;          // LDS floats per 64-wide x segment (4 pad: no bank conflicts)

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sbyte(uint32_t w, int b) {
  // compiles to v_cvt_f32_i32_sdwa with a sign-extended byte select
  return (float)(int8_t)(w >> (8 * b));
}
// 1 / sqrt(x) on v_rsq_f32 (about 1 ulp): every RMSNorm multiplies by it,
// where the reference divides by sqrt(mean + eps) (shaders.ts:50-53, 415)
__device__ __forceinline__ float rsq(float x) { return __builtin_amdgcn_rsqf(x); }
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

// Full-wave sum on the DPP network (no LDS round trips), the total
// broadcast through lane 63: pairs, quads, half rows, rows, then the
// row_bcast15 / row_bcast31 steps that fold rows 0-2 into row 3.
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float x) {
  x += dpp_mov<0xB1>(x);         // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);         // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);        // row_half_mirror
  x += dpp_mov<0x140>(x);        // row_mirror
  x += dpp_mov<0x142, 0xa>(x);   // row_bcast15 into rows 1 and 3
  x += dpp_mov<0x143, 0xc>(x);   // row_bcast31 into rows 2 and 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// DPP move whose rows outside ROWMASK read -inf (for max reductions).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_mov_ninf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY),
                                                               __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xf, false));
}
// Sum over each aligned group of 8 lanes, result in all 8 (quad_perm xor 1,
// xor 2, then row_half_mirror pairs the two quads).
__device__ __forceinline__ float group8_sum(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x141>(x);
  return x;
}
// Sum / max over the whole wave of values that are uniform within each group
// of 8 lanes: row_mirror pairs the two groups of a row, the row_bcast15 /
// row_bcast31 steps fold rows 0-2 into row 3, lane 63 is broadcast.
__device__ __forceinline__ float across8_sum(float x) {
  x += dpp_mov<0x140>(x);
  x += dpp_mov<0x142, 0xa>(x);
  x += dpp_mov<0x143, 0xc>(x);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
__device__ __forceinline__ float across8_max(float x) {
  x = fmaxf(x, dpp_mov<0x140>(x));
  x = fmaxf(x, dpp_mov_ninf<0x142, 0xa>(x));
  x = fmaxf(x, dpp_mov_ninf<0x143, 0xc>(x));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// One 68-byte pair = blocks 2c and 2c+1 of a row: 17 dwords.
struct Pair {
  uint32_t w[17];
};

// Lane `lane` of a wave loads slot `lane` of a 4352-byte item (item-planar
// layout): four dwordx4 loads over 1024 contiguous bytes each, one dword load.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Weight items are read once per token: nontemporal loads (the `nt` bit)
// keep them from displacing the activations, chunk partials and K/V rows
// that the next kernels read from L2 (0.826 -> 0.789 ms per 1B token).
__device__ __forceinline__ void load_planes(const uint8_t* item, int lane, Pair& P) {
  const u32x4* p4 = (const u32x4*)item;
  const u32x4 a = __builtin_nontemporal_load(p4 + lane), b = __builtin_nontemporal_load(p4 + 64 + lane),
              c = __builtin_nontemporal_load(p4 + 128 + lane), d = __builtin_nontemporal_load(p4 + 192 + lane);
  P.w[0] = a.x; P.w[1] = a.y; P.w[2] = a.z; P.w[3] = a.w;
  P.w[4] = b.x; P.w[5] = b.y; P.w[6] = b.z; P.w[7] = b.w;
  P.w[8] = c.x; P.w[9] = c.y; P.w[10] = c.z; P.w[11] = c.w;
  P.w[12] = d.x; P.w[13] = d.y; P.w[14] = d.z; P.w[15] = d.w;
  P.w[16] = __builtin_nontemporal_load((const uint32_t*)(item + 4096) + lane);
}

// The same load through a global-address-space pointer. Pointers read from
// device memory (a layer table) are generic to the compiler, which then emits
// flat loads, and flat loads also count against lgkmcnt: every LDS access or
// scalar load after them would wait for the whole weight stream.
#define GG_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ void load_planes_g(const GG_GLOBAL uint8_t* item, int lane, Pair& P) {
  const GG_GLOBAL u32x4* p4 = (const GG_GLOBAL u32x4*)item;
  const u32x4 a = __builtin_nontemporal_load(p4 + lane), b = __builtin_nontemporal_load(p4 + 64 + lane),
              c = __builtin_nontemporal_load(p4 + 128 + lane), d = __builtin_nontemporal_load(p4 + 192 + lane);
  P.w[0] = a.x; P.w[1] = a.y; P.w[2] = a.z; P.w[3] = a.w;
  P.w[4] = b.x; P.w[5] = b.y; P.w[6] = b.z; P.w[7] = b.w;
  P.w[8] = c.x; P.w[9] = c.y; P.w[10] = c.z; P.w[11] = c.w;
  P.w[12] = d.x; P.w[13] = d.y; P.w[14] = d.z; P.w[15] = d.w;
  P.w[16] = __builtin_nontemporal_load((const GG_GLOBAL uint32_t*)(item + 4096) + lane);
}
template <class T>
__device__ __forceinline__ const GG_GLOBAL T* gmem(const T* p) { return (const GG_GLOBAL T*)p; }
template <class T>
__device__ __forceinline__ GG_GLOBAL T* gmem(T* p) { return (GG_GLOBAL T*)p; }

// acc += (sum_j q0[j] x[j]) * d0 + (sum_j q1[j] x[32+j]) * d1, each block sum
// running over j in order like linearQ8 (shaders.ts:123-142). xc is 16-byte
// aligned (LDS). Pair bytes: [0,2) d0 | [2,34) q0 | [34,36) d1 | [36,68) q1.
__device__ __forceinline__ float dot_pair(const Pair& P, const float* __restrict__ xc, float acc) {
  const float4* x4 = (const float4*)xc;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j4 = 0; j4 < 8; ++j4) {
    const float4 xv = x4[j4];
    const int j = 4 * j4;
    s0 = fmaf(sbyte(P.w[(2 + j) >> 2], (2 + j) & 3), xv.x, s0);
    s0 = fmaf(sbyte(P.w[(3 + j) >> 2], (3 + j) & 3), xv.y, s0);
    s0 = fmaf(sbyte(P.w[(4 + j) >> 2], (4 + j) & 3), xv.z, s0);
    s0 = fmaf(sbyte(P.w[(5 + j) >> 2], (5 + j) & 3), xv.w, s0);
  }
#pragma unroll
  for (int j4 = 0; j4 < 8; ++j4) {
    const float4 xv = x4[8 + j4];
    s1 = fmaf(sbyte(P.w[9 + j4], 0), xv.x, s1);
    s1 = fmaf(sbyte(P.w[9 + j4], 1), xv.y, s1);
    s1 = fmaf(sbyte(P.w[9 + j4], 2), xv.z, s1);
    s1 = fmaf(sbyte(P.w[9 + j4], 3), xv.w, s1);
  }
  acc = fmaf(s0, f16_lo(P.w[0]), acc);
  acc = fmaf(s1, f16_hi(P.w[8]), acc);
  return acc;
}

// shaders.ts:153-170 (tanh GELU, argument clamped to +-15) times up.
// 0.5 x (1 + tanh(arg)) = x / (1 + e^(-2 arg)), evaluated as
// x * rcp(1 + 2^(-2 log2(e) arg)) on v_exp_f32 / v_rcp_f32 (a few ulp; the
// tanh form loses the relative precision of 1 + tanh for negative arg).
__device__ __forceinline__ float gelu_mul(float x, float up) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  float a = 1.0f + (k1 * x) * x;
  float arg = (k0 * x) * a;
  arg = fminf(fmaxf(arg, -15.0f), 15.0f);
  const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(arg * -2.8853900817779268f));
  return (x * sg) * up;
}

__device__ __forceinline__ int xs_index(int e) { return (e >> 6) * kXPad + (e & 63); }

// Element e of row `token` of the tied embedding in the item-planar layout
// with CI = 1 (GR = 64): (f32(q) * scale) * sqrt(f32(H)) (shaders.ts:2-23).
__device__ __forceinline__ float embed_value(const uint8_t* embd, int embd_KpS, float embed_scale, int token, int e) {
  const int g = token >> 6, ln = token & 63;
  const int b = e >> 5, c = b >> 1;
  const uint8_t* item = embd + ((size_t)g * embd_KpS + c) * kColBytes;
  // byte o of the pair: dword o / 4 of slot ln, byte o % 4
  auto pb = [&](int o) { return item[plane_offset(o >> 2, ln) + (o & 3)]; };
  const int off = (b & 1) ? 34 : 0;
  const uint16_t sb = (uint16_t)(pb(off) | (pb(off + 1) << 8));
  const float scale = (float)__builtin_bit_cast(_Float16, sb);
  const float q = (float)(int8_t)pb(off + 2 + (e & 31));
  const float t = q * scale;
  return t * embed_scale;
}

// Decode attention chunking: the span split into at most mc (the launch's
// chunk count) chunks of a multiple of 32 positions.
__device__ __forceinline__ void dec_span(int pos, int window, int mc, int* t_lo, int* ch, int* nch) {
  const int lo = window > 0 ? max(0, pos - window + 1) : 0;
  const int span = pos - lo + 1;
  const int c = kAttnChunk * ((span + kAttnChunk * mc - 1) / (kAttnChunk * mc));
  *t_lo = lo;
  *ch = c;
  *nch = (span + c - 1) / c;
}

// Candidate of the sampler's stable descending sort: value after the
// repetition penalty, then the candidate's slot (its class) as the tie order.
struct Cand {
  double val;
  int ord;
  uint32_t id;
};

// Non-short-circuit (| and &): both fields are read before any test, so a
// loop of comparisons against LDS entries has no branches and its loads
// issue together.
__device__ __forceinline__ bool cand_before(const Cand& x, const Cand& y) {
  return (x.val > y.val) | ((x.val == y.val) & (x.ord < y.ord));
}

struct SelShared {
  union {
    struct {
      float tv[256];
      uint32_t ti[256];
    };
    double q[256];      // sampling: probs[i] / sum, once the candidates are sorted
  };
  Cand cs[256];
  union {
    Cand ws[256];       // sampling: each wave's 64 candidates in sorted order
    struct {
      double pd[256];   // sampling: (double) of the f32 probability of rank k
      double pre_g[17]; // sampling: pre_g[g] = pd[0] + ... + pd[16 g - 1], summed in order
    };
  };
  int tok;
};

// Token selection from the 256 per-class candidates (topk256 in slot order,
// shaders.ts:363-384): thread t < 256 (`active`) holds class t's (m, id).
// Greedy (temperature 0, rep_penalty <= 1): the argmax halving tree
// (shaders.ts:351-357); otherwise the host sampler (engine.ts:862-901):
// repetition penalty in f64 for ids in the bitmap, stable descending sort
// (by value then slot: each candidate's rank within its wave's 64 by
// comparison, plus a binary search of each other wave's sorted 64),
// f32-stored exp of the scaled differences, f64 sums, top-p cutoff and the
// walk with the draw u. The sums keep the host's sequential order: one pass
// of running sums gives the total and every prefix (the top-p subset is the
// prefix up to the cutoff), the quotients probs[i] / sum are formed in
// parallel and only their cumulative sum and the walk run on one thread.
// Every thread of the block calls it (it holds block barriers); the token is
// returned to all threads.
static __device__ SampleIn sample_of(const DevState* st) {
  SampleIn p;
  p.temperature = st->temperature;
  p.top_p = st->top_p;
  p.rep_penalty = st->rep_penalty;
  p.u = st->u;
  p.seen_count = st->seen_count;
  return p;
}

// The sampling branch of select_token, out of line (one copy per kernel).
static __device__ __attribute__((noinline)) int select_sampled(SelShared& sh, float m, uint32_t id, bool active,
                                                               const SampleIn& p, const uint32_t* seen, int V);

// Greedy selection alone (temperature 0, rep_penalty <= 1).
static __device__ int select_greedy(SelShared& sh, float m, uint32_t id, bool active) {
  const int tid = threadIdx.x;
  if (active) {
    sh.tv[tid] = m;
    sh.ti[tid] = id;
  }
  __syncthreads();
  // the tree of strides 128, 64, ..., 1 where slot t takes slot t + s when
  // that value is strictly greater: the two widest levels from LDS, the
  // rest in wave 0 (one barrier instead of eight, same comparisons)
  if (tid < 64) {
    float v0 = sh.tv[tid], v1 = sh.tv[tid + 64];
    uint32_t i0 = sh.ti[tid], i1 = sh.ti[tid + 64];
    const float v2 = sh.tv[tid + 128], v3 = sh.tv[tid + 192];
    if (v2 > v0) { v0 = v2; i0 = sh.ti[tid + 128]; }
    if (v3 > v1) { v1 = v3; i1 = sh.ti[tid + 192]; }
    if (v1 > v0) { v0 = v1; i0 = i1; }
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
      const float o = __shfl_down(v0, s, 64);
      const uint32_t oi = (uint32_t)__shfl_down((int)i0, s, 64);
      if (tid < s && o > v0) { v0 = o; i0 = oi; }
    }
    if (tid == 0) sh.tok = (int)i0;
  }
  __syncthreads();
  return sh.tok;
}

static __device__ int select_token(SelShared& sh, float m, uint32_t id, bool active, const SampleIn& p,
                                   const uint32_t* seen, int V) {
  if (p.temperature == 0.0 && p.rep_penalty <= 1.0) return select_greedy(sh, m, id, active);
  return select_sampled(sh, m, id, active, p, seen, V);
}

static __device__ __attribute__((noinline)) int select_sampled(SelShared& sh, float m, uint32_t id, bool active,
                                                               const SampleIn& p, const uint32_t* seen, int V) {
  const int tid = threadIdx.x;
  const double T = p.temperature, rep = p.rep_penalty;
  Cand cd;
  cd.val = (double)m;
  cd.ord = tid;
  cd.id = id;
  if (active) {
    if (rep > 1.0 && p.seen_count > 0 && id < (uint32_t)V && ((seen[id >> 5] >> (id & 31)) & 1u)) {
      if (cd.val > 0) cd.val /= rep;
      else cd.val *= rep;
    }
    sh.cs[tid] = cd;
  }
  __syncthreads();
  // the order is total (slots are distinct), so the ranks are a permutation:
  // the rank within the wave's 64 sorts each wave's list into ws, then each
  // other list contributes the count of its entries ordered before cd, found
  // by a branch-free binary search (monotone predicate over a sorted list)
  const int w0 = tid & ~63;
  int rank = 0;
  if (active) {
#pragma unroll 8
    for (int j = 0; j < 64; ++j) rank += cand_before(sh.cs[w0 + j], cd) ? 1 : 0;
    sh.ws[w0 + rank] = cd;
  }
  __syncthreads();
  if (active) {
    int cnt[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const Cand* L = sh.ws + 64 * w;
      int pos = 0;
#pragma unroll
      for (int step = 32; step >= 1; step >>= 1) pos += cand_before(L[pos + step - 1], cd) ? step : 0;
      pos += (pos == 63 && cand_before(L[63], cd)) ? 1 : 0;
      cnt[w] = 64 * w == w0 ? 0 : pos;
    }
    rank += (cnt[0] + cnt[1]) + (cnt[2] + cnt[3]);
    sh.cs[rank] = cd;
  }
  __syncthreads();
  if (T == 0.0) return (int)sh.cs[0].id;
  if (active) sh.pd[tid] = (double)(float)exp((sh.cs[tid].val - sh.cs[0].val) / T);
  __syncthreads();
  // thread 0's sequential passes carry one dependent f64 add per element and
  // nothing else: every sum is non-decreasing (terms >= 0), so a group of 16
  // is searched for its first qualifying element only when the group's last
  // sum qualifies (or is NaN); the prefix sums are kept per group and the one
  // the walk needs is finished from its group's start in the same order
  constexpr int G = 16;
  // (each group's reads are issued before the previous group's adds, so the
  // LDS latency stays off the chains)
  if (tid == 0) {
    double s = 0.0, nx[G];
#pragma unroll
    for (int k = 0; k < G; ++k) nx[k] = sh.pd[k];
#pragma unroll
    for (int g = 0; g < 256 / G; ++g) {
      double cur[G];
#pragma unroll
      for (int k = 0; k < G; ++k) cur[k] = nx[k];
      if (g + 1 < 256 / G) {
#pragma unroll
        for (int k = 0; k < G; ++k) nx[k] = sh.pd[G * (g + 1) + k];
      }
      sh.pre_g[g] = s;
#pragma unroll
      for (int k = 0; k < G; ++k) s += cur[k];
    }
    sh.pre_g[256 / G] = s;
  }
  __syncthreads();
  if (active) sh.q[tid] = sh.pd[tid] / sh.pre_g[256 / G];
  __syncthreads();
  if (tid == 0) {
    double cum = 0.0, nx[G];
    int cutoff = 256;
#pragma unroll
    for (int k = 0; k < G; ++k) nx[k] = sh.q[k];
    for (int c = 0; c < 256 && cutoff == 256; c += G) {
      double cs[G];
#pragma unroll
      for (int k = 0; k < G; ++k) cs[k] = nx[k];
      const int cn = min(c + G, 256 - G);
#pragma unroll
      for (int k = 0; k < G; ++k) nx[k] = sh.q[cn + k];
#pragma unroll
      for (int k = 0; k < G; ++k) {
        cum += cs[k];
        cs[k] = cum;
      }
      if (!(cum < p.top_p)) {
        int first = G;
#pragma unroll
        for (int k = G - 1; k >= 0; --k) first = cs[k] >= p.top_p ? k : first;
        if (first < G) cutoff = c + first + 1;
      }
    }
    // prefix sum of the cutoff's candidates: pd[0] + ... + pd[cutoff - 1]
    double pc = sh.pre_g[cutoff / G];
    for (int k = cutoff & ~(G - 1); k < cutoff; ++k) pc += sh.pd[k];
    // the walk: r after element k is r - pd[0] - ... - pd[k] in this order;
    // the first k < cutoff where it reaches 0 is the pick
    double r = p.u * pc;
    int pick = -1;
#pragma unroll
    for (int k = 0; k < G; ++k) nx[k] = sh.pd[k];
    for (int c = 0; c < cutoff && pick < 0; c += G) {
      double rs[G];
#pragma unroll
      for (int k = 0; k < G; ++k) rs[k] = nx[k];
      const int cn = min(c + G, 256 - G);
#pragma unroll
      for (int k = 0; k < G; ++k) nx[k] = sh.pd[cn + k];
#pragma unroll
      for (int k = 0; k < G; ++k) {
        r -= rs[k];
        rs[k] = r;
      }
      if (!(r > 0)) {
#pragma unroll
        for (int k = G - 1; k >= 0; --k) pick = (c + k < cutoff && rs[k] <= 0) ? c + k : pick;
      }
    }
    if (pick < 0) pick = cutoff - 1;
    sh.tok = (int)sh.cs[pick].id;
  }
  __syncthreads();
  return sh.tok;
}

}  // namespace gg

// gg_decode.hip -- the persistent decode kernel: one launch per token.
//
// The per-kernel token loop (gg_kernels.hip) pays a dependent kernel launch
// for each of its 133 phases per token (2.4-3.7 us each on MI355X, measured
// in a graph-replay chain), and each kernel starts its weight stream only
// after its launch. Here 256 co-resident blocks (one per CU, four waves each)
// run every phase of every layer in one launch and hand outputs over through
// LL words: a 64-bit {f32 value, 32-bit tag} pair written and polled with
// device-scope relaxed atomics (global_store/load ... sc1). A word is valid
// when its tag equals the (launch, layer) tag, so a consumer needs no flag,
// no counter and no fence; an agent-scope release/acquire fence (a whole-L2
// write-back or invalidate on this multi-XCD part) cost 32 us per phase in a
// 256-block exchange. A block issues the weight loads of its next phase
// before it polls that phase's input, so the weight stream overlaps the
// hand-off.
//
// Phases per layer (engine.ts:766-795 order):
//   Q   blocks [0, 192): 8-row groups of the fused QKV GEMV. Every block
//       first rebuilds the residual stream from the previous layer's down
//       output (post-FFN norm + residual, engine.ts:794) into its own LDS:
//       the residual is never exchanged, each block keeps an identical copy.
//   A   blocks [192, 256): decode attention, block = (chunk of the span,
//       query head), 16 chunks per head in sliding-window layers, 32 in
//       full-attention layers with blocks [0, 64) taking chunks 16..31 after
//       their QKV rows (fusedPerHeadNormRope, kvCacheStore,
//       attnScore/softmax/attnOutput, shaders.ts:209-325); the blocks of
//       chunks 0..3 of each head merge the head's chunk partials, 64 dims
//       each. Full-attention
//       layers at spans above 4096 positions (k_decode<MODE, true>, for
//       contexts above 4096): every block takes one of 256 chunks for all
//       four heads (each K/V row read once), blocks [192, 256) merge.
//   O   blocks [0, H / 8): attention output projection.
//   F   all blocks: post-attention norm + residual; blocks [0, I / 32):
//       ffn_norm, the gate/up rows of 32 GeGLU outputs and their product
//       with W_down's matching 32-wide input block, a split-K partial of the
//       down output (engine.ts:785-793), both on int8 MFMA.
//   R   blocks [0, H / 8): sums of the I / 32 down partials, fixed order.
// Then DEC_FWD: block 0 finishes the pass (output norm, engine.ts:794-801);
// DEC_STEP: every block takes one vocabulary class c (rows c + 256 k, the
// stride classes of argmax / topk256, shaders.ts:327-384) of the tied LM
// head, from a class-major copy of the embedding, and hands over its
// class candidate; block 0 selects the token (engine.ts:805-902): the
// halving tree in the SAMPLE = false copy that greedy steps launch, the
// sampler in the SAMPLE = true copy. A step whose token argument is negative
// embeds the id the previous launch selected (DevState::out_token), so the
// host can queue the next step before that id reaches it.
//
// Every wait is bounded (a.spin_limit ticks of s_memrealtime): a block that
// times out raises the host-visible flag and leaves, so the launch always
// ends (the hand-off needs all 256 blocks resident: one per CU).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gg_device.h"
#include "gg_internal.h"

namespace gg {
namespace {

constexpr int NT = kDecThreads;
constexpr int NW = kDecThreads / 64;
constexpr int kEPT = (kDecMaxH + NT - 1) / NT;   // residual elements per thread (H <= kDecMaxH)
constexpr int kMaxKq = kDecMaxH / 64;                  // pair columns of a gate/up row (64 k each)
constexpr int kMaxKh = (kMaxKq + 1) / 2;                // gate/up scale dwords per lane
constexpr int kDT = (kDecMaxH / 32 + NW - 1) / NW;      // W_down 32-row tiles per wave
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Thread / block index as values the compiler cannot hoist out of the layer
// loop: loop-invariant addresses and offsets derived from them would stay
// live in registers across every phase of the loop.
__device__ __forceinline__ int tidx() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int bidx() {
  int b = blockIdx.x;
  asm volatile("" : "+s"(b));
  return b;
}

__device__ __forceinline__ uint64_t ll_ld(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_st(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ll_val(uint64_t w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ bool ll_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

// Thread t polls words t + NT k (k < PER) until each of its words below n
// carries `tag` (buffers hold NT * PER words, so every load of a round is
// issued unconditionally before any is checked). Returns false on timeout.
template <int PER>
__device__ __forceinline__ bool ll_wait(const uint64_t* src, int n, uint32_t tag, float* v, long long limit) {
  const int tid = tidx();
  const char* sb = (const char*)src;
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
    uint64_t w[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) w[k] = ll_ld((const uint64_t*)(sb + (uint32_t)(8 * (tid + NT * k))));
    bool ok = true;   // no short circuit: one compare per word, no branches
#pragma unroll
    for (int k = 0; k < PER; ++k) ok &= (tid + NT * k >= n) | ll_ok(w[k], tag);
    if (ok) {
#pragma unroll
      for (int k = 0; k < PER; ++k) v[k] = ll_val(w[k]);
      return true;
    }
    if (now_ - t0 > limit) return false;
  }
}

// Four 16-byte device-scope loads (two LL words each: value, tag, value,
// tag), waited for inside the same asm statement so that no result register
// is read before its load has returned. Each 8-byte word is read whole, as
// by ll_ld; the tag test per word keeps the hand-off valid word by word.
__device__ __forceinline__ void ll_ld4x2(const uint64_t* p0, const uint64_t* p1, const uint64_t* p2,
                                         const uint64_t* p3, u32x4 (&w)[4]) {
  asm volatile(
      "global_load_dwordx4 %0, %4, off sc1\n\t"
      "global_load_dwordx4 %1, %5, off sc1\n\t"
      "global_load_dwordx4 %2, %6, off sc1\n\t"
      "global_load_dwordx4 %3, %7, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
      : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
      : "memory");
}

// v + v of lane ^ 8 / ^ 16 / ^ 32 in every lane, on DPP (row_ror:8) and the
// gfx950 half-row / half-wave swaps (v_permlane16/32_swap) rather than
// ds_bpermute: the same IEEE sums as a shuffle, at VALU latency.
__device__ __forceinline__ float xor8_add(float v) { return v + dpp_mov<0x128>(v); }
__device__ __forceinline__ float xor16_add(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over the block (NW waves, fixed order); `sh` holds NW floats and must
// not be reused before the next barrier.
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum_dpp(v);
  const int id = tidx();
  if ((id & 63) == 0) sh[id >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += sh[w];
  return t;
}

// ---- block-level Q8_0 GEMV over item-planar row groups ----------------------
// Items [i0, i0 + ni) (row groups g0.. of KpS items each) split evenly over
// the 8 waves; every load is issued with clamped indices (exact wait counts).
template <int CI, int NIF>
__device__ __forceinline__ void mg_issue(const uint8_t* W, int Kp, int KpS, int i0, int ni, Pair* w) {
  constexpr int GR = 64 / CI;
  const int t = tidx(), lane = t & 63, wv = t >> 6, cp = lane / GR;
  const int wi0 = i0 + (wv * ni) / NW, wi1 = i0 + ((wv + 1) * ni) / NW;
#pragma unroll
  for (int k = 0; k < NIF; ++k) {
    const int it = max(min(wi0 + k, wi1 - 1), i0);
    const int sp = it % KpS;
    // lanes of a padding column phase load the phase-0 lane of their row
    const int ll = sp * CI + cp < Kp ? lane : (lane & (GR - 1));
    load_planes_g(gmem(W) + (size_t)it * kColBytes, ll, w[k]);
  }
}

// Dot products of the wave's items against x (LDS, kXPad layout); row sums of
// each touched group land in red[wave][row - g0 * GR] (red zeroed before).
template <int CI, int NIF>
__device__ __forceinline__ void mg_dots(const Pair* w, const float* xs, int Kp, int KpS, int g0, int i0, int ni,
                                        float (*red)[kDecMaxRows]) {
  constexpr int GR = 64 / CI;
  const int t = tidx(), lane = t & 63, wv = t >> 6, cp = lane / GR;
  const int wi0 = i0 + (wv * ni) / NW, wi1 = i0 + ((wv + 1) * ni) / NW;
  float acc = 0.f;
  int gcur = wi0 / KpS - g0;
  auto flush = [&](int gl) {
    float v = acc;
    static_assert(GR >= 8, "flush folds lane bits 3 and up");
    if (GR <= 8) v = xor8_add(v);
    if (GR <= 16) v = xor16_add(v);
    if (GR <= 32) v = xor32_add(v);
    if (lane < GR) red[wv][gl * GR + lane] = v;
  };
#pragma unroll
  for (int k = 0; k < NIF; ++k) {
    const int it = wi0 + k;
    const int g = it / KpS, s = it - g * KpS;
    const int c = s * CI + cp;
    float d = dot_pair(w[k], xs + min(c, Kp - 1) * kXPad, 0.f);
    d = (c < Kp && it < wi1) ? d : 0.f;
    if (it < wi1 && g - g0 != gcur) {
      flush(gcur);
      gcur = g - g0;
      acc = 0.f;
    }
    acc += d;
  }
  if (wi1 > wi0) flush(gcur);
}

__device__ __forceinline__ void zero_red(float (*red)[kDecMaxRows]) {
  for (int i = tidx(); i < NW * kDecMaxRows; i += NT) (&red[0][0])[i] = 0.f;
}

__device__ __forceinline__ float red_row(const float (*red)[kDecMaxRows], int t) {
  float r = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) r += red[w][t];
  return r;
}

// The kernel arguments read through a pointer the compiler cannot follow
// across loop iterations: fields used in a layer are loaded (s_load from the
// kernarg segment) where the layer needs them instead of being kept live in
// scalar registers across the whole layer loop, where most of them spilled.
typedef __attribute__((address_space(4))) const DecodeArgs KArgs;
__device__ __forceinline__ KArgs& kargs() {
  uint64_t p = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *(KArgs*)p;
}

struct Smem {
  union {
    float4 xs4[kMaxK / 64 * kXPad / 4]; // GEMV input x (K <= 8192)
    SelShared sel;                      // block 0's token selection, after its LM head has read x
  };
  i32x4 xq4[kMaxKq * 12];               // FFN input as int8 planes: [pair column][plane][64]
  float4 xsc4[2][kMaxKq / 4];           // ... block scales: [block parity][pair column]
  i32x4 xa4[6];                         // GeGLU output as int8 planes: [plane][32]
  i32x4 zq;                             // zero A operand of the lanes outside the planes
  float sact;                           // ... the GeGLU planes' scale
  float red[NW][kDecMaxRows];
  float shw[2][NW];
  float sh4[4][NW];                     // resid_norm's four block sums
  int fail;
  float4 qs4[64], ks4[64], vs4[64];     // attention: normed + roped q, k; v
  float4 wo[NW][64];
  float wm[NW], wl[NW];
  float act[32];                        // the FFN block's GeGLU outputs
  float cand_v[NW];
  uint32_t cand_i[NW];
};

// Timeline stamp (profiling builds of a step only): thread 0 of each block
// records s_memrealtime at event ev of layer l.
template <class DA>
__device__ __forceinline__ void stamp(const DA& a, int b, int l, int ev) {
  if (a.timeline && tidx() == 0)
    a.timeline[((size_t)b * a.L + l) * kDecEvents + ev] = __builtin_amdgcn_s_memrealtime();
}

// A block whose hand-off wait ran out: raises the launch's flags in mapped
// host memory (the context then continues on the graph path).
template <class DA>
__device__ __forceinline__ void report_timeout(const DA& a) {
  if (tidx() == 0) {
    __hip_atomic_store(a.host_out + 8 + a.out_slot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(a.host_out + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Block-uniform failure check after a poll (one barrier).
__device__ __forceinline__ bool failed(Smem& S, bool ok) {
  if (!ok) S.fail = 1;
  __syncthreads();
  return S.fail != 0;
}

// Failure check without a barrier, for polls whose consumer reaches a
// barrier anyway: a block whose poll timed out carries on with whatever it
// read (no index or branch depends on polled values; later polls of the
// layer time out in turn, each bounded by the spin limit) and leaves,
// reporting, at the end-of-layer check.
__device__ __forceinline__ void soft_fail(Smem& S, bool ok) {
  if (!ok) S.fail = 1;
}

// Four block sums at once (fixed order over the waves; one barrier).
__device__ __forceinline__ void block_sum4(float (&v)[4], float (*sh)[NW]) {
  const int id = tidx();
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = wave_sum_dpp(v[k]);
  if ((id & 63) == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) sh[k][id >> 6] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += sh[k][w];
    v[k] = t;
  }
}

// The residual stream r (this thread's elements e = tid + NT i < H, kept in
// registers) += rmsNorm(v) * wpost (fusedNormAdd, shaders.ts:386-418) and,
// with NORM, x = rmsNorm(r) * wpre into the GEMV input (rmsNorm,
// shaders.ts:25-56), from one block reduction: with u = v * wpost and
// a = 1 / rms(v), the new residual's sum of squares is
// sum r^2 + 2 a sum r u + a^2 sum u^2, reduced together with sum v^2.
template <bool NORM>
__device__ __forceinline__ void resid_norm(Smem& S, const float* v, const float* wpost, const float* wpre, int H,
                                           float eps, float* r) {
  const int tid = tidx();
  float sm[4] = {0.f, 0.f, 0.f, 0.f};
  float u[kEPT];
#pragma unroll
  for (int i = 0; i < kEPT; ++i) {
    u[i] = v[i] * wpost[i];
    if (tid + NT * i < H) {
      sm[0] = fmaf(v[i], v[i], sm[0]);
      sm[1] = fmaf(r[i], r[i], sm[1]);
      sm[2] = fmaf(r[i], u[i], sm[2]);
      sm[3] = fmaf(u[i], u[i], sm[3]);
    }
  }
  block_sum4(sm, S.sh4);
  const float ra = rsq(sm[0] / (float)H + eps);
#pragma unroll
  for (int i = 0; i < kEPT; ++i)
    if (tid + NT * i < H) r[i] = r[i] + u[i] * ra;
  if (NORM) {
    const float ri = rsq((sm[1] + ra * (2.f * sm[2] + ra * sm[3])) / (float)H + eps);
    float* xs = (float*)S.xs4;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) {
      const int e = tid + NT * i;
      if (e < H) xs[xs_index(e)] = (r[i] * wpre[i]) * ri;
    }
  }
}

// This thread's elements e = tid + NT i < H of a norm weight vector, loaded
// before the poll they follow so that their latency overlaps the hand-off.
__device__ __forceinline__ void load_norm(const float* w, int H, float* dst) {
  const int tid = tidx();
#pragma unroll
  for (int i = 0; i < kEPT; ++i) dst[i] = gmem(w)[min(tid + NT * i, H - 1)];
}

// x = rmsNorm(r) * w into the GEMV input (rmsNorm, shaders.ts:25-56).
__device__ __forceinline__ void norm_to_xs(Smem& S, const float* r, const float* w, int H, float eps, int shi) {
  const int tid = tidx();
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kEPT; ++i)
    if (tid + NT * i < H) ss = fmaf(r[i], r[i], ss);
  const float ri = rsq(block_sum(ss, S.shw[shi]) / (float)H + eps);
  float* xs = (float*)S.xs4;
#pragma unroll
  for (int i = 0; i < kEPT; ++i) {
    const int e = tid + NT * i;
    if (e < H) xs[xs_index(e)] = (r[i] * w[i]) * ri;
  }
}

// ---- int8-MFMA FFN ----------------------------------------------------------
// A 32-element block of an activation vector with max |v| = m is carried as
// three int8 planes, v = S (p0 + p1 / 254 + p2 / 254^2) with S = m / 127
// (p0 = rint(v / S), each next plane the rounded remainder times 254; a base
// of 256 would let a plane reach 128): within 2e-7 m of v, a few f32 ulps of
// the block maximum. The MFMA's int32 sums of weight x plane are exact; the
// scales S and the Q8_0 block scale apply in f32 afterwards.
__device__ __forceinline__ void split3(float y, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
  const float a = rintf(y);
  const float r = (y - a) * 254.f;
  const float bq = rintf(r);
  const float cq = rintf((r - bq) * 254.f);
  p0 = (uint32_t)(int)a & 255u;
  p1 = (uint32_t)(int)bq & 255u;
  p2 = (uint32_t)(int)cq & 255u;
}
__device__ __forceinline__ float planes_value(int c0, int c1, int c2) {
  return fmaf((float)c2, 1.f / 64516.f, fmaf((float)c1, 1.f / 254.f, (float)c0));
}
// Max over the 32 lanes of a half wave.
__device__ __forceinline__ float half_wave_max(float m) {
  m = fmaxf(m, dpp_mov<0xB1>(m));
  m = fmaxf(m, dpp_mov<0x4E>(m));
  m = fmaxf(m, dpp_mov<0x141>(m));
  m = fmaxf(m, dpp_mov<0x140>(m));
  return xor16_max(m);
}

// The gate/up GEMV input x (f32 in xs) as int8 planes: four threads per
// 32-element block, eight elements each, one pass over H / 32 blocks.
__device__ __forceinline__ void planes_from_xs(Smem& S, int H) {
  const int tid = tidx();
  if (tid < H / 8) {
    const int blk = tid >> 2, sub = tid & 3;
    const float* xs = (const float*)S.xs4 + xs_index(32 * blk) + 8 * sub;
    const float4 v0 = *(const float4*)xs, v1 = *(const float4*)(xs + 4);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
    m = fmaxf(m, dpp_mov<0xB1>(m));   // quad_perm [1,0,3,2]
    m = fmaxf(m, dpp_mov<0x4E>(m));   // quad_perm [2,3,0,1]
    const float inv = m > 0.f ? 127.f * __builtin_amdgcn_rcpf(m) : 0.f;
    uint32_t q[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t p0, p1, p2;
      split3(v[j] * inv, p0, p1, p2);
      q[0][j >> 2] |= p0 << (8 * (j & 3));
      q[1][j >> 2] |= p1 << (8 * (j & 3));
      q[2][j >> 2] |= p2 << (8 * (j & 3));
    }
    uint8_t* dst = (uint8_t*)S.xq4 + (blk >> 1) * 192 + (blk & 1) * 32 + 8 * sub;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) *(uint2*)(dst + 64 * pl) = make_uint2(q[pl][0], q[pl][1]);
    if (sub == 0) ((float*)S.xsc4[blk & 1])[blk >> 1] = m * (1.f / 127.f);
  }
}

// Gate/up rows of tile wv (16 rows: gate rows 16 wv .. for wv < 2, up rows
// 16 (wv - 2) .. otherwise) over the pair columns on v_mfma_i32_16x16x64_i8.
// A: the input planes, rows 0-2 for block 2c and rows 4-6 for block 2c + 1,
// each at the k-groups of its block (lane l: row l % 16, k-group l / 16);
// the other lanes read a zero operand, and so does every lane past Kq (the
// plane rows of pair columns >= Kq are never written), so the loop has no
// branch. B: the tile's weights (lane l: weight row l % 16, the same
// k-group). Result lanes 0-15 / 16-31 hold the three plane sums of block
// 2c / 2c + 1 for weight row l % 16; returns that lane's f32 sum over all c.
__device__ __forceinline__ float gate_up_mfma(const Smem& S, const i32x4* wb, const uint32_t* wsc) {
  const int lane = tidx() & 63, i = lane & 15, g = lane >> 4;
  const bool valid = (i < 3 && g < 2) || (i >= 4 && i < 7 && g >= 2);
  const int p = i < 3 ? i : i - 4;
  const int hb = (lane >> 4) & 1;
  const uint8_t* ab = valid ? (const uint8_t*)S.xq4 + p * 64 + 16 * g : (const uint8_t*)&S.zq;
  const int as = valid ? 192 : 0;
  const float* sc = (const float*)S.xsc4[hb];
  const i32x4 zero = {0, 0, 0, 0};
  // all products first, each into its own accumulator, so that the MFMAs
  // issue back to back instead of each waiting for the previous result to be
  // read out; then the f32 sums in increasing c
  i32x4 C[kMaxKq];
#pragma unroll
  for (int c = 0; c < kMaxKq; ++c) {
    const i32x4 A = *(const i32x4*)(ab + c * as);
    C[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, wb[c], zero, 0, 0, 0);
  }
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxKq; ++c) {
    const uint32_t w2 = wsc[c >> 1];
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? w2 >> 16 : w2 & 0xffffu));
    acc = fmaf(planes_value(C[c][0], C[c][1], C[c][2]), sc[c] * d, acc);
  }
  return acc;
}

// Poll n <= NT * PER LL words into the GEMV input x.
template <int PER>
__device__ __forceinline__ bool poll_to_xs(Smem& S, const uint64_t* src, int n, uint32_t tag, long long lim) {
  float v[PER];
  const bool ok = ll_wait<PER>(src, n, tag, v, lim);
  float* xs = (float*)S.xs4;
  if (ok) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = tidx() + NT * k;
      if (e < n) xs[xs_index(e)] = v[k];
    }
  }
  return ok;
}

// ---- attention block: chunk c of head h (16 chunks per head) ---------------
// Wave w runs passes of 8 positions t0 + 64 p + 8 w + i; lane (i, o) =
// (lane / 8, lane % 8) holds key dims 4 (o + 8 j) .. +3, lane l value dims
// 4 l .. 4 l + 3; online softmax in base 2 (scores scaled by log2(e) / 16).
// Layer l's tensors, formed from the slab bases and strides.
struct LayerView {
  const uint8_t *qkv, *o, *guf, *dcb;
  const float* norms;      // norm j at norms + j * norm_stride
  float *kc, *vc;
  const float* rope;
  int window;
};
template <class DA>
__device__ __forceinline__ LayerView layer_view(const DA& a, int l) {
  LayerView v;
  v.qkv = a.w_qkv + (size_t)l * a.st_qkv;
  v.o = a.w_o + (size_t)l * a.st_o;
  v.guf = a.w_guf + (size_t)l * a.st_guf;
  v.dcb = a.w_dcb + (size_t)l * a.st_dcb;
  v.norms = a.norms + (size_t)l * 6 * a.norm_stride;
  v.kc = a.kc + (size_t)l * a.kv_stride;
  v.vc = a.vc + (size_t)l * a.kv_stride;
  const bool swa = (l % a.swa_period) < a.swa_period - 1;
  v.rope = swa ? a.rope_local : a.rope_global;
  v.window = swa ? a.window : 0;
  return v;
}
template <class DA>
__device__ __forceinline__ const float* norm_of(const DA& a, const LayerView& v, int j) {
  return v.norms + (size_t)j * a.norm_stride;
}

template <class DA>
__device__ __forceinline__ bool attention_block(const DA& a, Smem& S, const LayerView& Ly, int l, int c,
                                                int h, int pos, uint32_t tag, int nchunks) {
  const int tid = tidx(), lane = tid & 63, wv = tid >> 6;
  const long long lim = a.spin_limit;
  int t_lo, ch, nch;
  dec_span(pos, Ly.window, nchunks, &t_lo, &ch, &nch);
  uint64_t* part = a.x_part + (size_t)(h * kDecChunksG + c) * kDecPart;
  if (c >= nch) {   // past the span: an empty partial (m = -inf)
    for (int d = tid; d < kDecPart; d += NT) ll_st(part + d, d == kHeadDim ? -INFINITY : 0.f, tag);
    return true;
  }
  const int t0 = t_lo + c * ch;
  const int t1 = min(t0 + ch, pos + 1);
  const int npass = (t1 - t0 + 8 * NW - 1) / (8 * NW);
  const int kv_last = max(pos - 1, 0);   // cache rows [0, pos) hold earlier tokens
  const int pl = lane >> 3, oc = lane & 7;
  const bool holder = (c == nch - 1);
  float4 kr[8], kn[8], vr[8], vn[8];
  auto load_k = [&](int p, float4* dst) {
    const int t = min(t0 + 8 * NW * p + 8 * wv + pl, kv_last);
    const GG_GLOBAL f32x4* kp = (const GG_GLOBAL f32x4*)(gmem(Ly.kc) + (size_t)t * kHeadDim);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 v = __builtin_nontemporal_load(kp + oc + 8 * j);
      dst[j] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
  auto load_v = [&](int p, float4* dst) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = min(t0 + 8 * NW * p + 8 * wv + i, kv_last);
      const f32x4 v = __builtin_nontemporal_load((const GG_GLOBAL f32x4*)(gmem(Ly.vc) + (size_t)t * kHeadDim) + lane);
      dst[i] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
  // K/V rows of the first pass and the RoPE row go out before the q/k/v poll
  load_k(0, kr);
  load_v(0, vr);
  const GG_GLOBAL float* rt = gmem(Ly.rope) + (size_t)pos * kHeadDim;
  float cs[2], sn[2], nw[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cs[j] = rt[lane + 64 * j];
    sn[j] = rt[kHeadDim / 2 + lane + 64 * j];
  }
  const GG_GLOBAL float* wnorm = gmem(norm_of(a, Ly, wv == 1 ? 3 : 2));
#pragma unroll
  for (int i = 0; i < 4; ++i) nw[i] = wnorm[lane + 64 * i];
  // wave 0: q of head h; holder wave 1: this token's k, wave 2: its v
  bool ok = true;
  float hx[4];
  if (wv == 0 || (holder && wv <= 2)) {
    const uint64_t* src = a.x_qkv + (wv == 0 ? h * kHeadDim : a.QD + (wv - 1) * kHeadDim);
    const long long st0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
      uint64_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = ll_ld(src + (wv == 2 ? 4 * lane + i : lane + 64 * i));
      bool good = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) good &= ll_ok(w[i], tag);
      if (good) {
#pragma unroll
        for (int i = 0; i < 4; ++i) hx[i] = ll_val(w[i]);
        break;
      }
      if (now_ - st0 > lim) { ok = false; break; }
    }
  }
  // QK-norm + NEOX RoPE (fusedPerHeadNormRope): lane owns dims lane + 64 i
  auto norm_rope = [&](float* x, float4* dst4) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
    ss = wave_sum_dpp(ss);
    const float ri = rsq(ss / (float)kHeadDim + a.eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (x[i] * nw[i]) * ri;
    float* dst = (float*)dst4;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float x0 = x[j], x1 = x[j + 2];
      dst[lane + 64 * j] = x0 * cs[j] - x1 * sn[j];
      dst[lane + 64 * j + 128] = x0 * sn[j] + x1 * cs[j];
    }
  };
  if (ok) {
    if (wv == 0) norm_rope(hx, S.qs4);
    if (holder && wv == 1) norm_rope(hx, S.ks4);
    if (holder && wv == 2) S.vs4[lane] = make_float4(hx[0], hx[1], hx[2], hx[3]);
  }
  if (failed(S, ok)) return false;
  stamp(a, blockIdx.x, l, 12);

  float4 qr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) qr[j] = S.qs4[oc + 8 * j];
  const float sl2 = a.attn_scale * 1.4426950408889634f;
  float m = -INFINITY, lsum = 0.f;
  float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int p = 0; p < npass; ++p) {
    const int tb = t0 + 8 * NW * p + 8 * wv;
    const int t = tb + pl;
    // the next pass's K/V rows go out before this pass's products (a second
    // register set), so a pass after the first waits for less of their
    // latency
    if (p + 1 < npass) {
      load_k(p + 1, kn);
      load_v(p + 1, vn);
    }
    if (t == pos) {
#pragma unroll
      for (int j = 0; j < 8; ++j) kr[j] = S.ks4[oc + 8 * j];
    }
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      d = fmaf(qr[j].x, kr[j].x, d);
      d = fmaf(qr[j].y, kr[j].y, d);
      d = fmaf(qr[j].z, kr[j].z, d);
      d = fmaf(qr[j].w, kr[j].w, d);
    }
    d = group8_sum(d);
    const float sc = t < t1 ? d * sl2 : -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) kr[j] = kn[j];
    const float mx = across8_max(sc);
    const float mn = fmaxf(m, mx);
    const float alpha = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mn);
    const float pr = (sc == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sc - mn);
    lsum = fmaf(lsum, alpha, across8_sum(pr));
    m = mn;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (tb + i == pos) vr[i] = S.vs4[lane];
    o4.x *= alpha;
    o4.y *= alpha;
    o4.z *= alpha;
    o4.w *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr), 8 * i));
      o4.x = fmaf(pv, vr[i].x, o4.x);
      o4.y = fmaf(pv, vr[i].y, o4.y);
      o4.z = fmaf(pv, vr[i].z, o4.z);
      o4.w = fmaf(pv, vr[i].w, o4.w);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = vn[i];
  }
  // merge the eight waves (fixed order) into the chunk's (max, sum, o)
  S.wo[wv][lane] = o4;
  if (lane == 0) {
    S.wm[wv] = m;
    S.wl[wv] = lsum;
  }
  __syncthreads();
  if (tid < 64) {
    float M = S.wm[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, S.wm[w]);
    float L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = S.wm[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(S.wm[w] - M);
      L = fmaf(f, S.wl[w], L);
      const float4 v = S.wo[w][tid];
      O.x = fmaf(f, v.x, O.x);
      O.y = fmaf(f, v.y, O.y);
      O.z = fmaf(f, v.z, O.z);
      O.w = fmaf(f, v.w, O.w);
    }
    ll_st(part + 4 * tid, O.x, tag);
    ll_st(part + 4 * tid + 1, O.y, tag);
    ll_st(part + 4 * tid + 2, O.z, tag);
    ll_st(part + 4 * tid + 3, O.w, tag);
    if (tid == 0) {
      ll_st(part + kHeadDim, M, tag);
      ll_st(part + kHeadDim + 1, L, tag);
    }
  }
  // this token's K/V row and the debug copy of q go out last: a store issued
  // before the dot products would hold their wait for the K/V loads (the
  // vector memory counter also counts stores) until it is acknowledged; the
  // chunks read row pos from LDS, later launches from the cache
  if (holder && h == 0 && tid < kHeadDim) {
    gmem(Ly.kc)[(size_t)pos * kHeadDim + tid] = ((const float*)S.ks4)[tid];
    gmem(Ly.vc)[(size_t)pos * kHeadDim + tid] = ((const float*)S.vs4)[tid];
  }
  if (c == 0 && tid < 64) *(float4*)(a.q_dbg + (size_t)l * a.QD + h * kHeadDim + 4 * tid) = S.qs4[tid];
  return true;
}

// Chunk block p < 4 of head h: dims 64 p .. 64 p + 63 of the head's merge,
// o = sum_c f_c o_c / sum_c f_c l_c with f_c = 2^(m_c - max m) (maxima in
// log2 units; empty chunks have m_c = -inf), into the O GEMV's input (the
// four quarters run in four blocks, each polling a quarter of the partial
// words). Wave g polls dim 64 p + lane of chunks g, g + 4, ...;
// threads 0..2 NC - 1 also poll the (m, l) words. Every thread forms the
// head's max and l-sum in chunk order; wave g sums its chunks in order and
// the four waves' sums are added in wave order.
template <int NC, class DA>
__device__ __forceinline__ bool merge_head_part(const DA& a, Smem& S, int l, int h, int p, uint32_t tag) {
  constexpr int KC = NC / 4;
  const int tid = tidx(), lane = tid & 63, wv = tid >> 6;
  const uint64_t* base = a.x_part + (size_t)h * kDecChunksG * kDecPart;
  const int d = 64 * p + lane;
  bool ok = true;
  float oc[KC];
  {
    const long long t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
      uint64_t wo[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) wo[k] = ll_ld(base + (wv + 4 * k) * kDecPart + d);
      const int si = min(tid, 2 * NC - 1);   // (m, l) word of threads < 2 NC
      const uint64_t ws = ll_ld(base + (si >> 1) * kDecPart + kHeadDim + (si & 1));
      bool good = (tid >= 2 * NC) | ll_ok(ws, tag);
#pragma unroll
      for (int k = 0; k < KC; ++k) good &= ll_ok(wo[k], tag);
      if (good) {
#pragma unroll
        for (int k = 0; k < KC; ++k) oc[k] = ll_val(wo[k]);
        if (tid < 2 * NC) S.red[0][tid] = ll_val(ws);
        break;
      }
      if (now_ - t0 > a.spin_limit) { ok = false; break; }
    }
  }
  if (failed(S, ok)) return false;
  stamp(a, blockIdx.x, l, 13);
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c) M = fmaxf(M, S.red[0][2 * c]);
  float L = 0.f, acc = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) L = fmaf(__builtin_amdgcn_exp2f(S.red[0][2 * c] - M), S.red[0][2 * c + 1], L);
#pragma unroll
  for (int k = 0; k < KC; ++k) acc = fmaf(__builtin_amdgcn_exp2f(S.red[0][2 * (wv + 4 * k)] - M), oc[k], acc);
  if (wv > 0) S.red[wv][lane] = acc;
  __syncthreads();
  if (wv == 0) {
    const float x = (((acc + S.red[1][lane]) + S.red[2][lane]) + S.red[3][lane]) * (1.f / L);
    ll_st(a.x_attn + h * kHeadDim + d, x, tag);
    if (l == a.L - 1) a.attn_out[h * kHeadDim + d] = x;
  }
  return true;
}

// ---- long spans: full-attention layers past kDecMaxCtx positions ----------
// Block b takes chunk b of kDecChunksL for all four query heads, so each K/V
// row is read once per launch (one head per block would stream it four
// times); blocks [192, 256) then merge the partials, block 192 + 16 h + s
// dims 16 s .. 16 s + 15 of head h. Its LDS overlays the GEMV input x, which
// is free between the QKV dots and the O poll (barriers on both sides).
struct LongAttn {
  float4 qs[kAttnMaxQ][64];       // normed + roped q of the four heads
  float4 wo[NW][kAttnMaxQ][64];   // per-wave (o, max, sum) of each head
  float wm[NW][kAttnMaxQ], wl[NW][kAttnMaxQ];
  float mx[NW], ls[NW];           // merge: per-wave max of the chunk maxima, sum of f_c l_c
  float f[kDecChunksL];           // merge: chunk weights f_c
  float pm[NW][16];               // merge: per-wave sums of the 16-dim slice
};
static_assert(sizeof(LongAttn) <= sizeof(Smem::xs4), "long-span attention LDS exceeds the x buffer it overlays");

__device__ __forceinline__ float wave_max_dpp(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));
  x = fmaxf(x, dpp_mov<0x4E>(x));
  x = fmaxf(x, dpp_mov<0x141>(x));
  return across8_max(x);
}

// RMSNorm (weights w) + NEOX RoPE of one head held as dims lane + 64 i
// (fusedPerHeadNormRope, shaders.ts:209-227) into dst[256].
__device__ __forceinline__ void head_norm_rope(float* x, const float* w, const float* cs, const float* sn,
                                               float eps, int lane, float* dst) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
  ss = wave_sum_dpp(ss);
  const float ri = rsq(ss / (float)kHeadDim + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = (x[i] * w[i]) * ri;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float x0 = x[j], x1 = x[j + 2];
    dst[lane + 64 * j] = x0 * cs[j] - x1 * sn[j];
    dst[lane + 64 * j + 128] = x0 * sn[j] + x1 * cs[j];
  }
}

// Chunk c of a long span for the four query heads (the passes of
// attention_block with every K/V row scored against all four heads):
// wave w polls and normalises q of head w; in the block whose chunk holds
// pos, wave 1 also takes this token's k and wave 2 its v, and the block
// stores both into the cache. Partial of head h at (h * kDecChunksL + c).
template <class DA>
__device__ __forceinline__ bool attention_long(const DA& a, Smem& S, const LayerView& Ly, int l, int c,
                                               int pos, uint32_t tag) {
  LongAttn& LA = *reinterpret_cast<LongAttn*>(S.xs4);
  const int tid = tidx(), lane = tid & 63, wv = tid >> 6;
  const long long lim = a.spin_limit;
  int t_lo, ch, nch;
  dec_span(pos, 0, kDecChunksL, &t_lo, &ch, &nch);
  if (c >= nch) {   // past the span: empty partials (m = -inf)
    for (int i = tid; i < kAttnMaxQ * kDecPart; i += NT) {
      const int hh = i / kDecPart, d = i - hh * kDecPart;
      ll_st(a.x_part + ((size_t)hh * kDecChunksL + c) * kDecPart + d, d == kHeadDim ? -INFINITY : 0.f, tag);
    }
    return true;
  }
  const int t0 = t_lo + c * ch;
  const int t1 = min(t0 + ch, pos + 1);
  const int npass = (t1 - t0 + 8 * NW - 1) / (8 * NW);
  const int kv_last = max(pos - 1, 0);   // cache rows [0, pos) hold earlier tokens
  const int pl = lane >> 3, oc = lane & 7;
  const bool holder = (c == nch - 1);
  float4 kr[8], vr[8];
  auto load_k = [&](int p) {
    const int t = min(t0 + 8 * NW * p + 8 * wv + pl, kv_last);
    const GG_GLOBAL f32x4* kp = (const GG_GLOBAL f32x4*)(gmem(Ly.kc) + (size_t)t * kHeadDim);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 v = __builtin_nontemporal_load(kp + oc + 8 * j);
      kr[j] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
  auto load_v = [&](int p) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = min(t0 + 8 * NW * p + 8 * wv + i, kv_last);
      const f32x4 v = __builtin_nontemporal_load((const GG_GLOBAL f32x4*)(gmem(Ly.vc) + (size_t)t * kHeadDim) + lane);
      vr[i] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
  load_k(0);
  load_v(0);
  const GG_GLOBAL float* rt = gmem(Ly.rope) + (size_t)pos * kHeadDim;
  float cs[2], sn[2], nq[4], nk[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cs[j] = rt[lane + 64 * j];
    sn[j] = rt[kHeadDim / 2 + lane + 64 * j];
  }
  const GG_GLOBAL float* wq = gmem(norm_of(a, Ly, 2));
  const GG_GLOBAL float* wk = gmem(norm_of(a, Ly, 3));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    nq[i] = wq[lane + 64 * i];
    nk[i] = wk[lane + 64 * i];
  }
  // q of head wv (dims lane + 64 i); holder: wave 1 this token's k (same
  // layout), wave 2 its v (dims 4 lane .. 4 lane + 3)
  const bool extra = holder && (wv == 1 || wv == 2);
  const uint64_t* qsrc = a.x_qkv + wv * kHeadDim;
  const uint64_t* esrc = a.x_qkv + a.QD + (wv == 2 ? kHeadDim : 0);
  bool ok = true;
  float hx[4], ex[4];
  {
    const long long st0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
      uint64_t w[4], e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = ll_ld(qsrc + lane + 64 * i);
      if (extra) {
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = ll_ld(esrc + (wv == 2 ? 4 * lane + i : lane + 64 * i));
      }
      bool good = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) good &= ll_ok(w[i], tag);
      if (extra) {
#pragma unroll
        for (int i = 0; i < 4; ++i) good &= ll_ok(e[i], tag);
      }
      if (good) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hx[i] = ll_val(w[i]);
          ex[i] = extra ? ll_val(e[i]) : 0.f;
        }
        break;
      }
      if (now_ - st0 > lim) { ok = false; break; }
    }
  }
  if (ok) {
    head_norm_rope(hx, nq, cs, sn, a.eps, lane, (float*)LA.qs[wv]);
    if (holder && wv == 1) head_norm_rope(ex, nk, cs, sn, a.eps, lane, (float*)S.ks4);
    if (holder && wv == 2) S.vs4[lane] = make_float4(ex[0], ex[1], ex[2], ex[3]);
  }
  if (failed(S, ok)) return false;
  stamp(a, blockIdx.x, l, 12);

  float4 qr[kAttnMaxQ][8];
#pragma unroll
  for (int hh = 0; hh < kAttnMaxQ; ++hh)
#pragma unroll
    for (int j = 0; j < 8; ++j) qr[hh][j] = LA.qs[hh][oc + 8 * j];
  const float sl2 = a.attn_scale * 1.4426950408889634f;
  float m[kAttnMaxQ], ls[kAttnMaxQ];
  float4 o4[kAttnMaxQ];
#pragma unroll
  for (int hh = 0; hh < kAttnMaxQ; ++hh) {
    m[hh] = -INFINITY;
    ls[hh] = 0.f;
    o4[hh] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int p = 0; p < npass; ++p) {
    const int tb = t0 + 8 * NW * p + 8 * wv;
    const int t = tb + pl;
    if (t == pos) {
#pragma unroll
      for (int j = 0; j < 8; ++j) kr[j] = S.ks4[oc + 8 * j];
    }
    float sc[kAttnMaxQ];
#pragma unroll
    for (int hh = 0; hh < kAttnMaxQ; ++hh) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        d = fmaf(qr[hh][j].x, kr[j].x, d);
        d = fmaf(qr[hh][j].y, kr[j].y, d);
        d = fmaf(qr[hh][j].z, kr[j].z, d);
        d = fmaf(qr[hh][j].w, kr[j].w, d);
      }
      d = group8_sum(d);
      sc[hh] = t < t1 ? d * sl2 : -INFINITY;
    }
    if (p + 1 < npass) load_k(p + 1);
    float pr[kAttnMaxQ], alpha[kAttnMaxQ];
#pragma unroll
    for (int hh = 0; hh < kAttnMaxQ; ++hh) {
      const float mx = across8_max(sc[hh]);
      const float mn = fmaxf(m[hh], mx);
      alpha[hh] = (m[hh] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[hh] - mn);
      pr[hh] = (sc[hh] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sc[hh] - mn);
      ls[hh] = fmaf(ls[hh], alpha[hh], across8_sum(pr[hh]));
      m[hh] = mn;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (tb + i == pos) vr[i] = S.vs4[lane];
#pragma unroll
    for (int hh = 0; hh < kAttnMaxQ; ++hh) {
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
  // the four waves' (max, sum, o) per head, merged in a fixed order; wave
  // hh writes head hh's partial
#pragma unroll
  for (int hh = 0; hh < kAttnMaxQ; ++hh) {
    LA.wo[wv][hh][lane] = o4[hh];
    if (lane == 0) {
      LA.wm[wv][hh] = m[hh];
      LA.wl[wv][hh] = ls[hh];
    }
  }
  __syncthreads();
  {
    const int hh = wv;
    const float M = fmaxf(fmaxf(LA.wm[0][hh], LA.wm[1][hh]), fmaxf(LA.wm[2][hh], LA.wm[3][hh]));
    float L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = LA.wm[w][hh] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(LA.wm[w][hh] - M);
      L = fmaf(f, LA.wl[w][hh], L);
      const float4 v = LA.wo[w][hh][lane];
      O.x = fmaf(f, v.x, O.x);
      O.y = fmaf(f, v.y, O.y);
      O.z = fmaf(f, v.z, O.z);
      O.w = fmaf(f, v.w, O.w);
    }
    uint64_t* part = a.x_part + ((size_t)hh * kDecChunksL + c) * kDecPart;
    ll_st(part + 4 * lane, O.x, tag);
    ll_st(part + 4 * lane + 1, O.y, tag);
    ll_st(part + 4 * lane + 2, O.z, tag);
    ll_st(part + 4 * lane + 3, O.w, tag);
    if (lane == 0) {
      ll_st(part + kHeadDim, M, tag);
      ll_st(part + kHeadDim + 1, L, tag);
    }
  }
  // this token's K/V row and the debug copy of q go out last (as in
  // attention_block)
  if (holder) {
    gmem(Ly.kc)[(size_t)pos * kHeadDim + tid] = ((const float*)S.ks4)[tid];
    gmem(Ly.vc)[(size_t)pos * kHeadDim + tid] = ((const float*)S.vs4)[tid];
  }
  if (c == 0) *(float4*)(a.q_dbg + (size_t)l * a.QD + 4 * tid) = LA.qs[wv][lane];
  return true;
}

// Merge of a long span: block hs = 16 h + s forms dims 16 s .. 16 s + 15 of
// head h, o = sum_c f_c o_c / sum_c f_c l_c over the kDecChunksL partials
// (f_c = 2^(m_c - max m), maxima in log2 units, empty chunks f_c = 0).
// Thread t polls chunk t's (m, l) and dim t % 16 of chunks t / 16 + 16 k;
// sums run in a fixed order (per thread in k, then xor trees over the
// wave's chunk groups and the four waves in order).
template <class DA>
__device__ __forceinline__ bool merge_long(const DA& a, Smem& S, int l, int hs, uint32_t tag) {
  LongAttn& LA = *reinterpret_cast<LongAttn*>(S.xs4);
  const int tid = tidx(), lane = tid & 63, wv = tid >> 6;
  const int h = hs >> 4, s = hs & 15, g = tid >> 4, d = tid & 15;
  const uint64_t* base = a.x_part + (size_t)h * kDecChunksL * kDecPart;
  constexpr int KC = kDecChunksL / 16;
  float ov[KC], mt = -INFINITY, lt = 0.f;
  bool ok = true;
  {
    const long long t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
      uint64_t w[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) w[k] = ll_ld(base + (size_t)(g + 16 * k) * kDecPart + 16 * s + d);
      const uint64_t wm = ll_ld(base + (size_t)tid * kDecPart + kHeadDim);
      const uint64_t wl = ll_ld(base + (size_t)tid * kDecPart + kHeadDim + 1);
      bool good = ll_ok(wm, tag) & ll_ok(wl, tag);
#pragma unroll
      for (int k = 0; k < KC; ++k) good &= ll_ok(w[k], tag);
      if (good) {
#pragma unroll
        for (int k = 0; k < KC; ++k) ov[k] = ll_val(w[k]);
        mt = ll_val(wm);
        lt = ll_val(wl);
        break;
      }
      if (now_ - t0 > a.spin_limit) { ok = false; break; }
    }
  }
  if (failed(S, ok)) return false;
  stamp(a, blockIdx.x, l, 13);
  const float wmx = wave_max_dpp(mt);
  if (lane == 0) LA.mx[wv] = wmx;
  __syncthreads();
  const float M = fmaxf(fmaxf(LA.mx[0], LA.mx[1]), fmaxf(LA.mx[2], LA.mx[3]));
  const float f = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mt - M);
  LA.f[tid] = f;
  const float wls = wave_sum_dpp(f * lt);
  if (lane == 0) LA.ls[wv] = wls;
  __syncthreads();
  const float L = ((LA.ls[0] + LA.ls[1]) + LA.ls[2]) + LA.ls[3];
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < KC; ++k) acc = fmaf(LA.f[g + 16 * k], ov[k], acc);
  acc = xor32_add(xor16_add(acc));
  if (lane < 16) LA.pm[wv][lane] = acc;
  __syncthreads();
  if (tid < 16) {
    const float x = (((LA.pm[0][tid] + LA.pm[1][tid]) + LA.pm[2][tid]) + LA.pm[3][tid]) * (1.f / L);
    ll_st(a.x_attn + h * kHeadDim + 16 * s + tid, x, tag);
    if (l == a.L - 1) a.attn_out[h * kHeadDim + 16 * s + tid] = x;
  }
  return true;
}

}  // namespace

template <int MODE, bool LONG, bool SAMPLE>
__global__ __launch_bounds__(kDecThreads, 1) void k_decode(DecodeArgs a) {
  __shared__ Smem S;
  const int tid = threadIdx.x, b = blockIdx.x;
  const int H = a.H;
  const long long lim = a.spin_limit;
  if (tid == 0) S.fail = 0;
  // plane rows of pair columns >= Kq and their scales stay zero all launch
  for (int i = tid; i < kMaxKq * 12; i += NT) S.xq4[i] = i32x4{0, 0, 0, 0};
  if (tid < 2 * kMaxKq / 4) (&S.xsc4[0][0])[tid] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tid == 0) S.zq = i32x4{0, 0, 0, 0};
  const DevState* st = a.st;
  const uint32_t epoch = st->epoch;
  const bool args_in = MODE == DEC_STEP && a.in_use != 0;
  const int pos = args_in ? a.in_pos : st->pos;
  const int cur = args_in ? -1 : st->cursor;
  const int token = args_in ? (a.in_token >= 0 ? a.in_token : st->out_token) : cur < 0 ? st->token : a.tokens[cur];
  const uint32_t base = epoch * (uint32_t)(a.L + 2);
  __syncthreads();

  const int Kq = H / 64;
  float r[kEPT];
  // layer 0's residual stream: the embedding row (shaders.ts:2-23)
#pragma unroll
  for (int i = 0; i < kEPT; ++i) {
    const int e = tid + NT * i;
    if (e < H) {
      r[i] = embed_value(a.embd, a.kps_embd, a.embed_scale, token, e);
    } else {
      r[i] = 0.f;
    }
  }

  for (int l = 0; l < a.L; ++l) {
    KArgs& a = kargs();
    const int tid = tidx(), b = bidx();
    const LayerView Ly = layer_view(a, l);
    const uint32_t tag = base + (uint32_t)l + 1;
    stamp(a, b, l, 0);
    // ---- Q: residual stream update in every block; QKV rows in [0, 192) ----
    const bool qb = b < kDecQBlocks;
    const bool ffb = b < a.g_f;                     // this block runs the FFN block b
    Pair wq[1];
    i32x4 wgb[kMaxKq];                              // gate/up tile wv: B operands per pair column
    uint32_t wgs[kMaxKh];                           // and its block scales (lanes 0-31)
    i32x4 wdb[kDT];                                 // W_down input block b, 32-row tiles wv + NW k
    uint16_t wds[kDT];                              // and the f16 scale of row 32 T + lane (lanes 0-31)
    float wn[kEPT];
    // the FFN weights are issued as soon as the block's Q or A work is done:
    // they stream in while attention runs and the O hand-off waits
    auto issue_ffn = [&]() {
      if (!ffb) return;
      const int lane = tid & 63, wv = tid >> 6;
      const int Kh = (Kq + 1) / 2, nT = H / 32;
      const GG_GLOBAL uint8_t* gb =
          gmem(Ly.guf) + (size_t)b * ((size_t)Kq * 4096 + (size_t)Kh * 512);
#pragma unroll
      for (int c = 0; c < kMaxKq; ++c)
        wgb[c] = __builtin_nontemporal_load(
            (const GG_GLOBAL i32x4*)(gb + (size_t)min(c, Kq - 1) * 4096 + wv * 1024 + lane * 16));
#pragma unroll
      for (int m = 0; m < kMaxKh; ++m)
        wgs[m] = __builtin_nontemporal_load(
            (const GG_GLOBAL uint32_t*)(gb + (size_t)Kq * 4096 + ((size_t)(wv * Kh + min(m, Kh - 1)) * 32 + (lane & 31)) * 4));
      const GG_GLOBAL uint8_t* col = gmem(Ly.dcb) + (size_t)b * 34 * H;
      // tile T as the B operand of v_mfma_i32_16x16x64_i8: lane l holds row
      // 32 T + 16 (l / 32) + l % 16, input bytes 16 ((l / 16) & 1) .. +15
#pragma unroll
      for (int k = 0; k < kDT; ++k) {
        const int t0 = 32 * min(wv + NW * k, nT - 1);
        const int rb = t0 + 16 * (lane >> 5) + (lane & 15);
        wdb[k] = __builtin_nontemporal_load(
            (const GG_GLOBAL i32x4*)(col + 2 * H + 32 * rb + 16 * ((lane >> 4) & 1)));
        wds[k] = ((const GG_GLOBAL uint16_t*)col)[t0 + (lane & 31)];
      }
    };
    if (qb) mg_issue<8, 1>(Ly.qkv, Kq, a.kps_qkv, b * a.kps_qkv, a.kps_qkv, wq);
    if (qb) load_norm(norm_of(a, Ly, 0), H, wn);
    // the previous layer's down output into the residual stream; attention
    // blocks of the chunk layout without an FFN block defer it until after
    // their chunk (they need the residual only for the LM head), so they
    // start their K/V loads and q poll at once and poll x_down when it is
    // long there
    const bool defer = !qb && !ffb && !(LONG && Ly.window == 0 && pos >= kDecMaxCtx);
    auto update_resid = [&]() __attribute__((always_inline)) {
      float dv[kEPT], wpost[kEPT];
      load_norm(norm_of(a, layer_view(a, l - 1), 5), H, wpost);
      const bool ok = ll_wait<kEPT>(a.x_down + ((l - 1) & 1) * kDecXW, H, tag - 1, dv, lim);
      soft_fail(S, ok);
      stamp(a, b, l, 1);
      if (qb) {
        zero_red(S.red);
        resid_norm<true>(S, dv, wpost, wn, H, a.eps, r);
      } else {
        resid_norm<false>(S, dv, wpost, wn, H, a.eps, r);
      }
    };
    if (l > 0 && !defer) {
      update_resid();
      if (b == 0) {
#pragma unroll
        for (int i = 0; i < kEPT; ++i)
          if (tid + NT * i < H) a.hist[(size_t)(l - 1) * H + tid + NT * i] = r[i];
      }
    } else if (qb) {
      zero_red(S.red);
      norm_to_xs(S, r, wn, H, a.eps, 1);
    }
    if (qb) {
      __syncthreads();
      stamp(a, b, l, 8);
      mg_dots<8, 1>(wq, (const float*)S.xs4, Kq, a.kps_qkv, b, b * a.kps_qkv, a.kps_qkv, S.red);
      __syncthreads();
      if (tid < 8) ll_st(a.x_qkv + 8 * b + tid, red_row(S.red, tid), tag);
      stamp(a, b, l, 2);
      if (LONG && Ly.window == 0 && pos >= kDecMaxCtx) {
        // long span: every block takes a chunk of the four heads
        if (!attention_long(a, S, Ly, l, b, pos, tag)) { report_timeout(a); return; }
        stamp(a, b, l, 14);
      } else if (Ly.window == 0 && b < 64) {
        // full-attention layers: blocks [0, 64) also take chunks 16..31
        const int c = 16 + (b & 7) + 8 * (b >> 5), h = (b >> 3) & 3;
        if (!attention_block(a, S, Ly, l, c, h, pos, tag, kDecChunksG)) { report_timeout(a); return; }
      }
      issue_ffn();
    } else if (LONG && Ly.window == 0 && pos >= kDecMaxCtx) {
      // ---- A, long span: chunk b of the four heads, then the merge ----
      if (!attention_long(a, S, Ly, l, b, pos, tag)) { report_timeout(a); return; }
      stamp(a, b, l, 2);
      if (!merge_long(a, S, l, b - kDecQBlocks, tag)) { report_timeout(a); return; }
      stamp(a, b, l, 3);
      issue_ffn();
    } else {
      // ---- A: attention (blocks [192, 256): chunks 0..15 of each head) ----
      const int ab = b - kDecQBlocks;
      const int c = (ab & 7) + 8 * (ab >> 5), h = (ab >> 3) & 3;
      const bool glob = Ly.window == 0;
      if (!attention_block(a, S, Ly, l, c, h, pos, tag, glob ? kDecChunksG : kDecChunks)) {
        report_timeout(a);
        return;
      }
      stamp(a, b, l, 2);
      if (c < 4) {
        const bool mok =
            glob ? merge_head_part<kDecChunksG>(a, S, l, h, c, tag) : merge_head_part<kDecChunks>(a, S, l, h, c, tag);
        if (!mok) { report_timeout(a); return; }
        stamp(a, b, l, 3);
      }
      if (l > 0 && defer) update_resid();
      issue_ffn();
    }
    __syncthreads();

    // ---- O: attention output projection (blocks [0, H / 8)) ----
    if (b < a.g_o) {
      Pair wo[1];
      mg_issue<8, 1>(Ly.o, a.QD / 64, a.kps_o, b * a.kps_o, a.kps_o, wo);
      zero_red(S.red);
      const bool ok = poll_to_xs<kAttnMaxQ * kHeadDim / NT>(S, a.x_attn, a.QD, tag, lim);
      if (failed(S, ok)) { report_timeout(a); return; }
      stamp(a, b, l, 3);
      mg_dots<8, 1>(wo, (const float*)S.xs4, a.QD / 64, a.kps_o, b, b * a.kps_o, a.kps_o, S.red);
      __syncthreads();
      if (tid < 8) ll_st(a.x_o + 8 * b + tid, red_row(S.red, tid), tag);
      stamp(a, b, l, 4);
      __syncthreads();
    }

    // ---- F: post-attention norm + residual + ffn_norm, then in block b < I / 32
    // the gate/up rows of act[32 b .. 32 b + 31] (GeGLU) and that act slice
    // times W_down's 32-wide input block b: a partial down output. Both
    // products run on the int8 MFMA with the activations as int8 planes ----
    {
      float ov[kEPT], wpa[kEPT], wffn[kEPT];
      load_norm(norm_of(a, Ly, 4), H, wpa);
      load_norm(norm_of(a, Ly, 1), H, wffn);
      const bool ok = ll_wait<kEPT>(a.x_o, H, tag, ov, lim);
      soft_fail(S, ok);
      stamp(a, b, l, 5);
      if (ffb) resid_norm<true>(S, ov, wpa, wffn, H, a.eps, r);
      else resid_norm<false>(S, ov, wpa, wffn, H, a.eps, r);
      if (ffb) {
        const int lane = tid & 63, wv = tid >> 6;
        __syncthreads();
        planes_from_xs(S, H);
        __syncthreads();
        stamp(a, b, l, 9);
        float g = gate_up_mfma(S, wgb, wgs);
        g = xor16_add(g);
        if (lane < 16) S.red[0][16 * wv + lane] = g;
        __syncthreads();
        stamp(a, b, l, 10);
        // gate rows 0..31 of the group, the matching up rows 32..63
        if (tid < 32) {
          const float v = gelu_mul(S.red[0][tid], S.red[0][32 + tid]);
          const float m = half_wave_max(fabsf(v));
          const float inv = m > 0.f ? 127.f * __builtin_amdgcn_rcpf(m) : 0.f;
          uint32_t p0, p1, p2;
          split3(v * inv, p0, p1, p2);
          uint8_t* xa = (uint8_t*)S.xa4;
          xa[tid] = (uint8_t)p0;
          xa[32 + tid] = (uint8_t)p1;
          xa[64 + tid] = (uint8_t)p2;
          if (tid == 0) S.sact = m * (1.f / 127.f);
        }
        __syncthreads();
        // partial down output of this input block on v_mfma_i32_16x16x64_i8,
        // two 16-row halves of a 32-row tile per product: A rows 0-2 are the
        // act planes at k-groups 0-1 (the first half's rows in B), rows 4-6
        // the same planes at k-groups 2-3 (the second half's rows); result
        // lanes 0-31 hold the three plane sums of row 32 T + lane
        const int pi = lane & 15, pg = lane >> 4;
        const bool av = (pi < 3 && pg < 2) || (pi >= 4 && pi < 7 && pg >= 2);
        const i32x4 A = *(const i32x4*)(av ? (const uint8_t*)S.xa4 + 32 * (pi & 3) + 16 * (pg & 1)
                                           : (const uint8_t*)&S.zq);
        const float sact = S.sact;
        const i32x4 zero = {0, 0, 0, 0};
        float y[kDT];
#pragma unroll
        for (int k = 0; k < kDT; ++k) {
          const i32x4 C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, wdb[k], zero, 0, 0, 0);
          y[k] = (planes_value(C[0], C[1], C[2]) * sact) * (float)__builtin_bit_cast(_Float16, wds[k]);
        }
#pragma unroll
        for (int k = 0; k < kDT; ++k) {
          const int T = wv + NW * k;
          if (lane < 32 && T < H / 32) ll_st(a.x_dpart + (size_t)b * H + 32 * T + lane, y[k], tag);
        }
        stamp(a, b, l, 6);
      }
    }

    // ---- R: down output rows 8 b .. 8 b + 7 = sum over the I / 32 partials ----
    if (b < a.g_down) {
      // thread t: rows 2 jp, 2 jp + 1 (jp = t % 4) of partials m = t / 4 +
      // 64 k, one 16-byte load (two LL words) each, so four consecutive
      // lanes read the eight rows of one partial (one 64-byte line); each
      // thread sums its partials in increasing m, then a fixed tree over the
      // wave's m slots and the four waves in order
      constexpr int PR = (kDecMaxFBlocks + 63) / 64;
      static_assert(PR == 4, "the partial poll issues four 16-byte loads");
      const int jp = tid & 3, mt = tid >> 2;
      const uint64_t* src = a.x_dpart + 8 * b + 2 * jp;
      const long long t0 = __builtin_amdgcn_s_memrealtime();
      float acc0 = 0.f, acc1 = 0.f;
      bool ok = true;
      for (;;) {
        const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
        u32x4 w[PR];
        ll_ld4x2(src + (size_t)min(mt, a.g_f - 1) * H, src + (size_t)min(mt + 64, a.g_f - 1) * H,
                 src + (size_t)min(mt + 128, a.g_f - 1) * H, src + (size_t)min(mt + 192, a.g_f - 1) * H, w);
        bool good = true;
#pragma unroll
        for (int k = 0; k < PR; ++k) good &= (mt + 64 * k >= a.g_f) | ((w[k][1] == tag) & (w[k][3] == tag));
        if (good) {
#pragma unroll
          for (int k = 0; k < PR; ++k)
            if (mt + 64 * k < a.g_f) {
              acc0 += __uint_as_float(w[k][0]);
              acc1 += __uint_as_float(w[k][2]);
            }
          break;
        }
        if (now_ - t0 > lim) { ok = false; break; }
      }
      soft_fail(S, ok);
      stamp(a, b, l, 7);
      // lanes i, i + 4, i + 8, i + 12 of each 16-lane row (rotations by 8, then 4), then the half-rows and halves
      acc0 += dpp_mov<0x128>(acc0);
      acc1 += dpp_mov<0x128>(acc1);
      acc0 += dpp_mov<0x124>(acc0);
      acc1 += dpp_mov<0x124>(acc1);
      acc0 = xor32_add(xor16_add(acc0));
      acc1 = xor32_add(xor16_add(acc1));
      if ((tid & 63) < 4) {
        S.red[tid >> 6][2 * jp] = acc0;
        S.red[tid >> 6][2 * jp + 1] = acc1;
      }
      __syncthreads();
      if (tid < 8) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += S.red[w][tid];
        ll_st(a.x_down + (l & 1) * kDecXW + 8 * b + tid, sum, tag);
      }
      stamp(a, b, l, 11);
    }
    __syncthreads();
    if (S.fail) { report_timeout(a); return; }
  }

  // ---- end of the pass: post-FFN norm + residual, output norm ----
  const uint32_t tagL = base + (uint32_t)a.L;   // the last layer's down output
  if (MODE == DEC_FWD && b != 0) return;
  // ---- LM head (DEC_STEP), vocabulary class b: rows b + 256 k, class-major
  // copy. Wave w takes the class's 64-row groups j = w + 4 q; lane = row, so
  // each lane runs a whole row's dot product over its Kp items, streamed
  // with kLmDepth items in flight per wave. The first kLmDepth items are
  // issued here, before the last hand-off: the weights do not depend on it.
  const int lane = tid & 63, wv = tid >> 6;
  const int R = a.V / 256, R64 = R / 64;   // rows and 64-row groups per class
  const int Kp = H / 64;
  const int ngw = (R64 - wv + NW - 1) / NW;
  const int nit = ngw * Kp;
  auto item_ptr = [&](int i) {   // clamped into the class (a wave without groups loads its last one)
    const int q = i / Kp, cc = i - q * Kp;
    const int P = b * R64 + min(wv + NW * q, R64 - 1);
    return a.lm + ((size_t)P * Kp + cc) * kColBytes;
  };
  constexpr int kLmDepth = 6;
  Pair p[kLmDepth];
  if (MODE == DEC_STEP) {
#pragma unroll
    for (int d = 0; d < kLmDepth; ++d) load_planes(item_ptr(max(min(d, nit - 1), 0)), lane, p[d]);
  }
  {
    float dv[kEPT], wpost[kEPT], wout[kEPT];
    load_norm(norm_of(a, layer_view(a, a.L - 1), 5), H, wpost);
    load_norm(a.out_norm, H, wout);
    const bool ok = ll_wait<kEPT>(a.x_down + ((a.L - 1) & 1) * kDecXW, H, tagL, dv, lim);
    soft_fail(S, ok);
    resid_norm<true>(S, dv, wpost, wout, H, a.eps, r);
    __syncthreads();
    if (S.fail) { report_timeout(a); return; }
    if (b == 0) {
      const float* xs = (const float*)S.xs4;
#pragma unroll
      for (int i = 0; i < kEPT; ++i) {
        const int e = tid + NT * i;
        if (e < H) {
          a.hidden[e] = r[i];
          a.hist[(size_t)(a.L - 1) * H + e] = r[i];
          a.normed[e] = xs[xs_index(e)];
        }
      }
    }
  }
  if (MODE == DEC_FWD) {
    if (tid == 0) {
      a.st->pos = pos + 1;
      a.st->cursor = cur + 1;
      a.st->epoch = epoch + 1;
    }
    return;
  }

  stamp(a, b, a.L - 1, 14);
  const float* xs = (const float*)S.xs4;
  // the class candidate: the first index of the maximum above -1e30, else
  // (-1e30, 0) (strict >, shaders.ts:337-347); this lane's rows come in
  // increasing index order (group q = 0, 1, ...)
  float bv = -1e30f;
  uint32_t bi = 0;
  if (nit > 0) {
    float acc = 0.f;
    int q = 0, cc = 0;
    for (int i = 0; i < nit; i += kLmDepth) {
#pragma unroll
      for (int d = 0; d < kLmDepth; ++d) {
        const int it = i + d;
        if (it < nit) {
          acc = dot_pair(p[d], xs + cc * kXPad, acc);
          if (++cc == Kp) {   // row group finished: logit (class-major) and candidate
            const int j = wv + NW * q;
            a.logits[(size_t)(b * R64 + j) * 64 + lane] = acc;
            if (acc > bv) { bv = acc; bi = (uint32_t)(b + 256 * (64 * j + lane)); }
            acc = 0.f;
            cc = 0;
            ++q;
          }
        }
        if (it + kLmDepth < nit) load_planes(item_ptr(it + kLmDepth), lane, p[d]);
      }
    }
  }
  // wave max with the lowest index on ties: an associative, commutative
  // choice (bv is never NaN), so any pairing order gives the same result;
  // pairs over lane bits 0-5 on DPP and the half-row / half-wave swaps
  auto take = [&](float ov, uint32_t oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  };
  take(dpp_mov<0xB1>(bv), (uint32_t)__builtin_amdgcn_update_dpp(0, (int)bi, 0xB1, 0xf, 0xf, false));
  take(dpp_mov<0x4E>(bv), (uint32_t)__builtin_amdgcn_update_dpp(0, (int)bi, 0x4E, 0xf, 0xf, false));
  take(dpp_mov<0x141>(bv), (uint32_t)__builtin_amdgcn_update_dpp(0, (int)bi, 0x141, 0xf, 0xf, false));
  take(dpp_mov<0x128>(bv), (uint32_t)__builtin_amdgcn_update_dpp(0, (int)bi, 0x128, 0xf, 0xf, false));
  {
    const auto rv = __builtin_amdgcn_permlane16_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap(bi, bi, false, false);
    const bool lo = ((lane >> 4) & 1) == 0;   // this lane's own value is r[0] in even rows, r[1] in odd
    take(__uint_as_float(lo ? rv[1] : rv[0]), lo ? ri[1] : ri[0]);
  }
  {
    const auto rv = __builtin_amdgcn_permlane32_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap(bi, bi, false, false);
    const bool lo = lane < 32;
    take(__uint_as_float(lo ? rv[1] : rv[0]), lo ? ri[1] : ri[0]);
  }
  if (lane == 0) {
    S.cand_v[wv] = bv;
    S.cand_i[wv] = bi;
  }
  __syncthreads();
  const uint32_t tagC = base + (uint32_t)a.L + 1;
  stamp(a, b, a.L - 1, 15);
  if (tid == 0) {
    float v = S.cand_v[0];
    uint32_t id = S.cand_i[0];
    for (int w = 1; w < NW; ++w)
      if (S.cand_v[w] > v || (S.cand_v[w] == v && S.cand_i[w] < id)) { v = S.cand_v[w]; id = S.cand_i[w]; }
    ll_st(a.x_cand + 2 * b, v, tagC);
    ll_st(a.x_cand + 2 * b + 1, __uint_as_float(id), tagC);
  }
  if (b != 0) return;

  // ---- block 0: topk256 and the selection ----
  // the sampling inputs are read before the candidate poll, so their
  // latency overlaps it
  SampleIn sp = sample_of(st);
  if (args_in) {
    sp.temperature = a.in_temperature;
    sp.top_p = a.in_top_p;
    sp.rep_penalty = a.in_rep_penalty;
    sp.u = a.in_u;
  }
  float m = -1e30f;
  uint32_t id = 0;
  bool ok = true;
  if (tid < 256) {
    const long long t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      const long long now_ = __builtin_amdgcn_s_memrealtime();   // in flight with the loads
      const uint64_t wv0 = ll_ld(a.x_cand + 2 * tid), wi0 = ll_ld(a.x_cand + 2 * tid + 1);
      if (ll_ok(wv0, tagC) & ll_ok(wi0, tagC)) {
        m = ll_val(wv0);
        id = __float_as_uint(ll_val(wi0));
        break;
      }
      if (now_ - t0 > lim) { ok = false; break; }
    }
  }
  if (failed(S, ok)) { report_timeout(a); return; }
  if (tid < 256) {
    a.top[2 * tid] = __float_as_uint(m);
    a.top[2 * tid + 1] = id;
  }
  // greedy steps run the SAMPLE = false copy, which holds no sampler code
  const int tok = SAMPLE ? select_token(S.sel, m, id, tid < 256, sp, a.seen, a.V)
                         : select_greedy(S.sel, m, id, tid < 256);
  if (tid == 0) {
    a.st->out_token = tok;
    // system scope: the host polls this mapped word for the id of a queued step
    __hip_atomic_store(a.host_out + a.out_slot, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (tok >= 0 && tok < a.V) {
      // no-return atomic OR: no load round trip at the end of the launch
      __hip_atomic_fetch_or(a.seen + (tok >> 5), 1u << (tok & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      a.st->seen_count = sp.seen_count + 1;
    }
    a.st->pos = pos + 1;
    a.st->cursor = cur + 1;
    a.st->epoch = epoch + 1;
  }
}

int decode_occupancy() {
  int occ = 1 << 30;
  const void* ks[] = {(const void*)k_decode<DEC_STEP, false, false>, (const void*)k_decode<DEC_STEP, false, true>,
                      (const void*)k_decode<DEC_STEP, true, false>, (const void*)k_decode<DEC_STEP, true, true>};
  for (const void* k : ks) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kDecThreads, 0) != hipSuccess) return 0;
    occ = min(occ, n);
  }
  return occ;
}

int launch_decode(int mode, const DecodeArgs& a, void* stream, bool coop) {
  hipStream_t s = (hipStream_t)stream;
  if (mode == DEC_STEP && !a.lm) return (int)hipErrorInvalidValue;
  if (a.H > kDecMaxH || a.g_f > kDecMaxFBlocks) return (int)hipErrorInvalidValue;
  const dim3 grid(kDecBlocks), block(kDecThreads);
  // a step whose sampling options are arguments and greedy takes the copy
  // without the sampler
  const bool sample = !(a.in_use && a.in_temperature == 0.0 && a.in_rep_penalty <= 1.0);
  const void* k;
  if (mode == DEC_FWD) {
    k = a.long_ctx ? (const void*)k_decode<DEC_FWD, true, false> : (const void*)k_decode<DEC_FWD, false, false>;
  } else if (a.long_ctx) {
    k = sample ? (const void*)k_decode<DEC_STEP, true, true> : (const void*)k_decode<DEC_STEP, true, false>;
  } else {
    k = sample ? (const void*)k_decode<DEC_STEP, false, true> : (const void*)k_decode<DEC_STEP, false, false>;
  }
  DecodeArgs arg = a;
  void* args[] = {&arg};
  if (coop) return (int)hipLaunchCooperativeKernel(k, grid, block, args, 0, s);
  const hipError_t e = hipLaunchKernel(k, grid, block, args, 0, s);
  return e != hipSuccess ? (int)e : (int)hipGetLastError();
}

}  // namespace gg

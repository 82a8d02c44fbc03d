// gg_internal.h -- argument blocks shared by the gfx950 kernels
// (gg_kernels.hip) and the runtime that launches them (gg_runtime.hip).
//
// Device weight layout ("item-planar Q8_0"). A Q8_0 weight matrix with N
// output rows and K inputs keeps the bytes of the GGUF 34-byte blocks (f16 LE
// scale + 32 int8) but orders them so that one wavefront reads 4352
// contiguous bytes with fully coalesced 16-byte loads:
//   * two consecutive blocks of a row form a 68-byte "pair" (64 weights,
//     17 dwords); Kp = K / 64 pairs per row;
//   * rows are grouped GR at a time and pair-columns CI at a time, GR * CI =
//     64 pairs per "item"; slot s = (c % CI) * GR + r % GR of item
//     g * KpS + c / CI holds pair (row r, pair-column c), g = r / GR,
//     KpS = ceil(Kp / CI) items per row group; items are 4352 bytes apart;
//   * inside an item the 64 pairs are stored as planes: dwords 4j..4j+3 of
//     slot s at byte 1024 j + 16 s (j < 4) and dword 16 at 4096 + 4 s, so
//     lane s of a wave loads its pair with four dwordx4 loads that each
//     cover 1024 contiguous bytes, plus one dword load.
// When CI does not divide Kp the last item of each group has unused slots;
// they are allocated but hold no weights. Bytes read per token are the GGUF
// count plus those slots (none for the Gemma-3 1B shapes but K = 1152 with
// CI = 8, where a third of the last item of each group is padding).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace gg {

constexpr int kHeadDim = 256;        // Gemma-3 270M/1B head_dim
constexpr int kAttnMaxQ = 4;         // query heads per KV head the attention kernel takes
constexpr int kPairBytes = 68;
constexpr int kColBytes = 64 * kPairBytes;   // one wavefront step: 4352 bytes
constexpr int kMaxK = 8192;          // largest GEMV input (x staged in LDS)
constexpr int kSelBlocks = 32;       // stage-1 blocks of the vocab selector
constexpr int kAttnChunk = 32;       // base positions per decode attention block (4 waves x 8)
constexpr int kDecMaxChunks = 256;   // decode attention chunks of a long-span launch (else 16)
constexpr int kDecMergeInO = 16;     // launches of at most this many chunks are merged by the O GEMV
constexpr int kMaxContext = 65536;   // largest context_length

// Byte offset of dword j (0..16) of slot s (0..63) inside a 4352-byte item.
inline constexpr int plane_offset(int j, int s) {
  return j < 16 ? 1024 * (j >> 2) + 16 * s + 4 * (j & 3) : 4096 + 4 * s;
}

// Q8_0 matrix in the item-planar layout.
struct Q8Layout {
  int rows, K, Kp, CI, GR, KpS;
  size_t bytes() const { return (size_t)(rows / GR) * KpS * kColBytes; }
};

// The layout of a matrix: whole 64-row groups (CI = 1) for tall matrices,
// 8-row groups with 8 pair-columns per step (CI = 8) below 8192 rows, so that
// even N = 1152 gets 144 blocks without splitting K. force_ci = 2 (32-row
// groups) leaves no padding when Kp is even but not a multiple of 8.
// CI without padding for a row of Kp pair-columns: 8 when it divides Kp, else 2.
inline int padfree_ci(int Kp) { return (Kp % 8 == 0 || Kp % 2) ? 8 : 2; }

inline Q8Layout q8_layout(int rows, int K, int force_ci = 0) {
  Q8Layout L;
  L.rows = rows;
  L.K = K;
  L.Kp = K / 64;
  const int ci = force_ci ? force_ci : (rows >= 8192 ? 1 : 8);
  const int gr = 64 / ci;
  L.GR = gr;
  L.CI = 64 / gr;
  L.KpS = (L.Kp + L.CI - 1) / L.CI;
  return L;
}

// Per-step scalars the captured graphs read from device memory.
// The host rewrites the fields before `seen_count` ahead of every launch;
// `seen_count` and `out_token` are maintained by the kernels.
// Sampling inputs of one token selection (engine.ts:862-901 reads them from
// the generate() options and Math.random()).
struct SampleIn {
  double temperature;
  double top_p;
  double rep_penalty;
  double u;
  int32_t seen_count;
};

struct DevState {
  int32_t pos;          // position of the token being processed
  int32_t cursor;       // index into the device token array; < 0: embed `token`
  double temperature;
  double top_p;
  double rep_penalty;
  double u;             // uniform draw in [0,1) injected by the host
  int32_t token;        // gg_step: the token to embed (cursor < 0)
  int32_t seen_count;   // number of ids added to the penalty bitmap
  int32_t out_token;    // last selected token
  uint32_t epoch;       // launches of the persistent decode kernel so far (its hand-off tags)
};

struct GemvArgs {
  const uint8_t* W;     // item-planar weights
  int Kp;               // pairs per row (K / 64)
  int KpS;              // column steps per row group
  int N;                // output rows
  float* out;           // [N] result (EPI_OUT)
  const float* x;       // input vector (prologue NONE)
  // prologue inputs (RESID_NORM / EMBED_NORM); the prologue builds x in LDS
  const float* pre_vec;    // [K] output of the previous GEMV to post-norm
  const float* pre_res;    // residual stream vector entering the add
  const float* w_post;     // post-norm weight applied to pre_vec
  const float* w_pre;      // pre-norm weight producing x
  float* res_out;          // block 0 writes the new residual stream vector here
  float* hist_out;         // optional second copy (per-layer hidden history)
  const uint8_t* embd;     // item-planar token embedding (EMBED_NORM)
  int embd_KpS;            // its column steps per group (CI = 1)
  const DevState* st;
  const int32_t* tokens;
  float eps;
  float embed_scale;       // sqrtf((float)hidden)
  float* act_out;          // GEGLU epilogue output [N/2]
  // PRO_ATTN_MERGE (attention output projection): x is the merge of the
  // decode attention chunk partials of this token
  const float* attn_part;  // o [kDecMaxChunks][kAttnMaxQ][256], then (m, l) [kDecMaxChunks][kAttnMaxQ][2]
  int attn_chunks;         // chunks the attention launch wrote (blocks past the span leave empty ones)
  float* x_out;            // block 0 stores the merged x here (the attention output; for the
                           // LM head with PRO_RESID_NORM: the normed hidden state)
  DevState* st_advance;    // LM head with the final norm fused: block 0 advances pos / cursor
};

struct AttnArgs {
  const float* qkv;        // [n_q*256 + 512] QKV projection output (prefill: row stride)
  int n_q;                 // query heads (one KV head)
  const float* q_norm;     // [256]
  const float* k_norm;     // [256]
  const float* rope;       // [ctx][2][128] cos / sin of f32(pos) * freq[i], this layer's theta
  float* k_cache;          // [ctx][256]
  float* v_cache;          // [ctx][256]
  int window;              // 0: full causal attention
  float eps;
  float scale;             // 1/sqrt(head_dim)
  const DevState* st;
  float* part;             // decode: o [kDecMaxChunks][kAttnMaxQ][256] then (m, l) [kDecMaxChunks][kAttnMaxQ][2];
                           // batched prefill: (m, l, o[256]) [row][kPrefillChunks][n_q]
  float* attn_out;         // decode [n_q * 256]
  uint16_t* pf_out;        // batched prefill: hi plane [row][n_q * 256], then lo plane
  float* q_dbg;            // decode, optional: normed+roped q of this token
  // batched prefill: prompt row r sits at position pf_start + r; q of every
  // row is already normed + roped in `qkv`, K/V of every position are in the
  // cache; keys of a 16-row query tile are split in chunks of pf_chunk
  int pf_start;
  int pf_rows;
  int pf_chunk;
};

// Prefill GEMM on bf16 MFMA: C[M x N] = A[M x K] * W[N x K]^T. A comes as two
// bf16 planes (hi = bf16(x), lo = bf16(x - hi)); W as its int8 values in
// bf16 (exact) with the fp32 scale of every 32-wide block, applied to each
// block's MFMA partial in fp32.
struct GemmArgs {
  const uint16_t* A;       // hi plane [M][K], then lo plane [M][K]
  const uint16_t* W;       // [N][K]
  const float* D;          // [N][K / 32]
  int M, N, K;
  int ks;                  // K slices (1..kGemmMaxSlices, EPI_OUT only): slice z covers K/ks and writes C + z M N
  int bn;                  // block tile width: 128, or 144 / 96 (EPI_OUT: 4 waves of 32 x 144 / 64 x 48)
  float* C;                // EPI_OUT: [M][N] per slice
  uint16_t* act;           // EPI_GEGLU: hi plane [M][N/2], then lo plane; gate / up rows
                           // alternate in groups of 16 (16 gate rows, then their up rows)
};

// Row-wise prefill helpers: one block per prompt row.
struct RowArgs {
  int M, H;
  float eps;
  int pf_start;
  const int32_t* tokens;   // EMBED: prompt ids
  const uint8_t* embd;
  int embd_KpS;
  float embed_scale;
  const float* pre;        // RESID: output of the previous GEMM [M][H]
  int pre_planes;          // K slices of `pre` to add (0 or 1: one)
  size_t pre_stride;       // floats between the slices
  const float* res;        // RESID: residual stream entering the add [M][H]
  const float* w_post;
  const float* w_pre;
  float* res_out;          // [M][H] new residual stream
  uint16_t* x_out;         // normed GEMM input: hi plane [M][H], then lo plane
  float* last_hidden;      // optional: row M-1 of res_out (per-layer history)
  // KV: k/v of each row into the cache, q heads normed + roped in place
  const float* qkv;
  int n_q;
  const float* q_norm;
  const float* k_norm;
  const float* rope;
  float* k_cache;
  float* v_cache;
};

struct FinalArgs {
  const float* pre_vec;
  int pre_planes;          // K slices of pre_vec to add (0 or 1: one)
  size_t pre_stride;       // floats between the slices
  const float* pre_res;
  const float* w_post;
  const float* w_out;
  float* hidden;
  float* hist_out;
  float* normed;
  int H;
  float eps;
  DevState* st;            // pos += 1, cursor += 1 after each forward
};

struct SelectArgs {
  const float* logits;
  int V;
  float* cand_val;         // [kSelBlocks][256]
  uint32_t* cand_id;
  uint32_t* top;           // [256] x {f32 bits, id}: the topk256 layout
  uint32_t* seen;          // [ceil(V/32)] penalty bitmap
  DevState* st;
  int auto_add;            // add the chosen id to the bitmap
  int32_t* host_out;       // optional: mapped pinned host word that also receives the token
};

// ---- persistent decode kernel (gg_decode.hip) -------------------------------
// One launch runs a whole token: every layer's QKV, attention, O, gate/up and
// down phases on 256 co-resident blocks (one per CU) that hand their outputs
// over through "LL" words in device memory: 64-bit {f32 value, 32-bit tag}
// written and polled with device-scope relaxed atomics, so a word carries its
// own validity and no fence is needed. Tags are unique per (launch, layer).
constexpr int kDecBlocks = 256;      // blocks of the persistent decode kernel
constexpr int kDecThreads = 256;     // threads per block (4 waves, one per SIMD: 512 registers each)
constexpr int kDecQBlocks = 192;     // QKV phase: blocks [0, 192), one 8-row group each (1536 rows)
constexpr int kDecChunks = 16;       // attention chunks per head, sliding-window layers: blocks [192, 256)
constexpr int kDecChunksG = 32;      // ... full-attention layers: blocks [192, 256) and [0, 64)
constexpr int kDecPart = kHeadDim + 2;   // LL words of one chunk partial: o[256], m, l
constexpr int kDecMaxRows = 128;     // rows of one phase a block may own
constexpr int kDecMaxH = 1280;       // hidden sizes of the persistent kernel (its W_down rows per thread)
constexpr int kDecMaxFBlocks = 256;  // FFN blocks: intermediate / 32 <= 256
constexpr int kDecXW = 2048;        // LL words of one all-gathered hidden-size row (H <= kDecMaxH)
constexpr int kDecMaxCtx = 4096;     // spans up to 4096: 16 / 32 chunks per head, one head per block
constexpr int kDecChunksL = 256;     // longer spans of full-attention layers: chunk b of all four heads in block b
enum DecMode { DEC_FWD = 0, DEC_STEP = 1 };

// Every per-layer tensor kind is one layer-strided slab: layer l's copy is
// at base + l * stride, formed from these arguments (scalar registers), so
// the kernel never loads a pointer from memory in the middle of a phase.
struct DecodeArgs {
  const uint8_t* w_qkv;    // item-planar weights of every layer (CI = 8)
  const uint8_t* w_o;
  const uint8_t* w_guf;    // gate/up, CI = 1: 64-row group g = gate rows 32 g.. then up rows 32 g..
  const uint8_t* w_dcb;    // down, column blocks: per 32-wide input block f16 scales [H], int8 [H][32]
  size_t st_qkv, st_o, st_guf, st_dcb;   // bytes per layer
  const float* norms;      // [L][6][norm_stride]: attn, ffn, q, k, post_attention, post_ffw
  int norm_stride;
  float* kc;               // [L][ctx][256]
  float* vc;
  size_t kv_stride;        // floats per layer (ctx * 256)
  const float* rope_local; // [ctx][cos|sin][128]
  const float* rope_global;
  int swa_period;          // layer l is local when l % swa_period < swa_period - 1
  int window;              // local layers' sliding window (0: full attention)
  int L, H, I, QD, NQKV, V;
  int kps_qkv, kps_o, kps_embd;
  int g_f;                 // FFN blocks (intermediate / 32): block b < g_f takes act[32 b .. 32 b + 31]
  int g_o, g_down;         // 8-row groups of O / of the down output: blocks [0, g) take one each
  float eps, embed_scale, attn_scale;
  const uint8_t* embd;     // tied embedding (CI = 1 layout, original row order)
  const uint8_t* lm;       // DEC_STEP: the same rows class-major (row c + 256 k at c * V/256 + k)
  const float* out_norm;
  DevState* st;
  const int32_t* tokens;
  // hand-off buffers (LL words)
  uint64_t* x_qkv;         // [NQKV]
  uint64_t* x_part;        // chunk partials: head h, chunk c at (h * kDecChunksG + c) * kDecPart
                           // (spans <= kDecMaxCtx) or (h * kDecChunksL + c) * kDecPart (longer)
  uint64_t* x_attn;        // [QD]
  uint64_t* x_o;           // [H]
  uint64_t* x_dpart;       // [g_f][H] partial down outputs
  uint64_t* x_down;        // [2][kDecXW]: layer l's down output in row l & 1, so a block that
                           // polls layer l - 1's row late never finds it overwritten by layer l's
  uint64_t* x_cand;        // [256][2]: per vocab class (value, id)
  // parity outputs
  float* hidden;
  float* normed;
  float* hist;             // [L][H]
  float* q_dbg;            // [L][QD]
  float* attn_out;         // [QD] (last layer)
  float* logits;           // DEC_STEP: [V] class-major
  uint32_t* top;           // [256] x {f32 bits, id}
  uint32_t* seen;          // penalty bitmap
  int32_t* host_out;       // mapped host words: [0] token, [1] hand-off timeout flag, [4..5] pipelined tokens,
                           // [8 + out_slot] timeout flag of the launch that writes host_out[out_slot]
  long long spin_limit;    // s_memrealtime ticks (100 MHz) one hand-off may wait
  long long* timeline;     // optional [256][L][kDecEvents] s_memrealtime stamps (null: off)
  // in_use != 0: this launch's position, token and sampling parameters are
  // these arguments rather than DevState's host-written head, so a decode step
  // needs no state upload before its launch (DEC_STEP only); in_token < 0:
  // the id the previous launch selected (DevState::out_token); the id is
  // written to host_out[out_slot]
  int32_t in_use, in_pos, in_token, out_slot;
  double in_temperature, in_top_p, in_rep_penalty, in_u;
  // context_length > kDecMaxCtx: launches run k_decode<MODE, true>, whose
  // full-attention layers take the 256-chunk path at spans above kDecMaxCtx
  int32_t long_ctx;
};
constexpr int kDecEvents = 16;  // timeline events per (block, layer)
// coop: a cooperative launch (hipLaunchCooperativeKernel), for launches
// outside stream capture.
int launch_decode(int mode, const DecodeArgs& a, void* stream, bool coop);
// Blocks of the persistent kernel one CU can hold (it needs 1).
int decode_occupancy();

// ---- launchers (gg_kernels.hip) -------------------------------------------
enum Prologue { PRO_NONE = 0, PRO_EMBED_NORM = 1, PRO_RESID_NORM = 2, PRO_ATTN_MERGE = 3 };
enum Epilogue { EPI_OUT = 0, EPI_GEGLU = 1 };

int launch_gemv(int pro, int epi, int ci, const GemvArgs& a, void* stream);
int launch_attention(const AttnArgs& a, int grid, void* stream);
int launch_attention_merge(const AttnArgs& a, int chunks, void* stream);
// Decode attention chunks of a layer: 16 while its span cannot exceed 4096
// positions (a window <= 4096, or a context <= 4096), else kDecMaxChunks.
inline int decode_attention_chunks(int ctx, int window) {
  return (ctx <= 4096 || (window > 0 && window <= 4096)) ? kDecMergeInO : kDecMaxChunks;
}
int launch_final(const FinalArgs& a, void* stream);
int launch_select(const SelectArgs& a, void* stream);
int launch_repack(const uint8_t* src, uint8_t* dst, const Q8Layout& L, long long src_rows,
                  long long dst_row_offset, int interleave_half, void* stream);
int launch_dequant(const uint8_t* src, float* out, long long n, void* stream);
// One embedding row (embed_value) into out[H].
int launch_embed_row(const uint8_t* embd, int kps, float scale, int token, int H, float* out, void* stream);
// GGUF Q8_0 rows -> column-block layout (per 32-wide block: f16 scales [rows], int8 [rows][32]).
int launch_repack_colblock(const uint8_t* src, uint8_t* dst, long long rows, int K, void* stream);
// Gate/up copy of the persistent decode kernel in the int8-MFMA tile layout
// (bytes per 32-row pair of gate and up rows: gum_group_bytes(K)); up = 0
// writes the gate tiles, up = 1 the up tiles.
__host__ __device__ inline size_t gum_group_bytes(int K) { return (size_t)(K / 64) * 4096 + (size_t)((K / 64 + 1) / 2) * 512; }
int launch_repack_gum(const uint8_t* src, uint8_t* dst, long long rows, int K, int up, void* stream);
// Class-major copy of the CI = 1 LM head (rows a multiple of 16384).
int launch_class_major(const uint8_t* src, uint8_t* dst, long long rows, int Kp, void* stream);
// GGUF Q8_0 rows -> prefill GEMM weights: source row r to row r + off, or
// with half = 16 to (r / 16) * 32 + r % 16 + off (gate: off 0, up: off 16).
int launch_q8_bf16(const uint8_t* src, uint16_t* wb, float* wd, long long rows, int K, long long off, int half,
                   void* stream);
int launch_seen_add(uint32_t* seen, DevState* st, const int32_t* ids, int n, int V, void* stream);
int launch_prefill_attention(const AttnArgs& a, int M, void* stream);
int launch_gemm(int epi, const GemmArgs& a, void* stream);
int launch_rows_embed(const RowArgs& a, void* stream);
int launch_rows_resid(const RowArgs& a, void* stream);
int launch_rows_kv(const RowArgs& a, void* stream);
constexpr int kGemmMaxSlices = 4;   // K slices of a prefill GEMM (summed by the consumer)
constexpr int kQkvMaxSlices = 2;    // ... of the QKV GEMM (summed by k_rows_kv)
constexpr int kPrefillChunks = 16;   // key chunks per query tile in the batched prefill attention
constexpr int kPrefillMinChunk = 160;
// Longest key span of a 32-row query tile of a prefill of M rows at `start`.
inline int prefill_max_span(int window, int start, int M) {
  const int full = start + M;
  return window > 0 && window + 31 < full ? window + 31 : full;
}
// Keys per chunk: a multiple of 32, >= kPrefillMinChunk, at most kPrefillChunks chunks.
inline int prefill_chunk(int window, int start, int M) {
  const int span = prefill_max_span(window, start, M);
  const int c = 32 * ((span + 32 * kPrefillChunks - 1) / (32 * kPrefillChunks));
  return c > kPrefillMinChunk ? c : kPrefillMinChunk;
}

}  // namespace gg

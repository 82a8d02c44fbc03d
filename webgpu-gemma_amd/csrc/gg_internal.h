// gg_internal.h -- argument blocks shared by the gfx950 kernels
// (gg_kernels.hip) and the runtime that launches them (gg_runtime.hip).
//
// Device weight layout ("pair-interleaved Q8_0"). A Q8_0 weight matrix with
// N output rows and K inputs keeps the GGUF 34-byte blocks verbatim (f16 LE
// scale + 32 int8) but orders them so one wavefront streams contiguous bytes:
//   * two consecutive blocks of a row form a 68-byte "pair" (64 weights);
//   * rows are grouped 64 at a time (one row per lane of a wavefront);
//   * pair (row r, pair-column c) lives at byte
//       ((g * Kp + c) * 64 + (r % 64)) * 68,  g = r / 64,  Kp = K / 64.
// A wavefront that reads pair-column c of group g therefore loads 64 x 68 =
// 4352 contiguous bytes, every lane's 68 bytes starting on a 4-byte boundary.
// Byte count is exactly the GGUF count (34 bytes per 32 weights).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace gg {

constexpr int kHeadDim = 256;        // Gemma-3 270M/1B head_dim
constexpr int kMaxQHeads = 8;
constexpr int kPairBytes = 68;
constexpr int kGroupRows = 64;
constexpr int kColBytes = kGroupRows * kPairBytes;   // 4352
constexpr int kMaxK = 8192;          // largest GEMV input (x staged in LDS)
constexpr int kSelBlocks = 128;      // stage-1 blocks of the vocab selector
constexpr int kAttnMaxChunks = 256;  // attention split-K chunks per token

// Per-step scalars the captured graphs read from device memory.
// The host rewrites the fields before `seen_count` ahead of every launch;
// `seen_count` and `out_token` are maintained by the kernels.
struct DevState {
  int32_t pos;          // position of the token being processed
  int32_t cursor;       // index into the device token array
  double temperature;
  double top_p;
  double rep_penalty;
  double u;             // uniform draw in [0,1) injected by the host
  int32_t seen_count;   // number of ids added to the penalty bitmap
  int32_t out_token;    // last selected token
};

struct GemvArgs {
  const uint8_t* W;     // pair-interleaved weights
  int Kp;               // pairs per row (K / 64)
  int G;                // row groups (N / 64)
  int S;                // column splits across blocks
  int CS;               // pair-columns per split
  int N;                // output rows
  float* out;           // [S][N] partial sums (S == 1: the result)
  const float* x;       // input vector (prologue NONE)
  // prologue inputs (RESID_NORM / EMBED_NORM); the prologue builds x in LDS
  const float* pre_part;   // [pre_S][K] partial sums of the vector to post-norm
  int pre_S;
  const float* pre_res;    // residual stream vector entering the add
  const float* w_post;     // post-norm weight applied to the summed partials
  const float* w_pre;      // pre-norm weight producing x
  float* res_out;          // block 0 writes the new residual stream vector here
  float* hist_out;         // optional second copy (per-layer hidden history)
  const uint8_t* embd;     // pair-interleaved token embedding (EMBED_NORM)
  int Kp_embd;
  const DevState* st;
  const int32_t* tokens;
  float eps;
  float embed_scale;       // sqrtf((float)hidden)
  float* act_out;          // GEGLU epilogue output [N/2]
};

struct AttnArgs {
  const float* qkv_part;   // [S][n_q*256 + 512] QKV partial sums
  int S;
  int n_q;                 // query heads (one KV head)
  const float* q_norm;     // [256]
  const float* k_norm;     // [256]
  const float* freq;       // [128] RoPE inverse frequencies for this layer
  float* k_cache;          // [ctx][256]
  float* v_cache;          // [ctx][256]
  int window;              // 0: full causal attention
  float eps;
  float scale;             // 1/sqrt(head_dim)
  const DevState* st;
  float* part;             // [kAttnMaxChunks][n_q][2 + 256]
  unsigned int* counter;   // arrival counter for the last-block combine
  float* attn_out;         // [n_q * 256]
  float* q_dbg;            // optional: normed+roped q of this token
};

struct FinalArgs {
  const float* pre_part; int pre_S;
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
  int32_t* out_token;      // optional extra copy
  unsigned int* counter;
  int auto_add;            // add the chosen id to the bitmap
};

// ---- launchers (gg_kernels.hip) -------------------------------------------
enum Prologue { PRO_NONE = 0, PRO_EMBED_NORM = 1, PRO_RESID_NORM = 2 };
enum Epilogue { EPI_PARTIAL = 0, EPI_GEGLU = 1 };

int launch_gemv(int pro, int epi, const GemvArgs& a, void* stream);
int launch_sum_parts(const float* parts, int S, int N, float* y, void* stream);
int launch_attention(const AttnArgs& a, int grid, void* stream);
int launch_final(const FinalArgs& a, void* stream);
int launch_select(const SelectArgs& a, void* stream);
int launch_repack(const uint8_t* src, uint8_t* dst, long long rows, int Kp,
                  long long dst_row_offset, int interleave_half, void* stream);
int launch_dequant(const uint8_t* src, float* out, long long n, void* stream);
int launch_seen_add(uint32_t* seen, DevState* st, const int32_t* ids, int n, int V, void* stream);

}  // namespace gg

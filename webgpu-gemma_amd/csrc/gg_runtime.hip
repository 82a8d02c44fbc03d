// gg_runtime.hip -- context, weight upload, captured token graphs and the
// C-ABI of include/gg.h.
//
// Replaces the WebGPU resource layer of GemmaEngineImpl (src/engine.ts:54-110,
// 124-732, 1039-1077) and drives the gfx950 kernels in gg_kernels.hip.
// All device memory of a context is allocated in gg_create/gg_finalize; the
// per-token calls allocate nothing. Per-token work is two captured HIP graphs
// (forward pass, LM head + selection) that read the token, position and
// sampling options from a small device struct the host refreshes with one
// async copy before each launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "gg.h"
#include "gg_internal.h"

using namespace gg;

namespace {

thread_local std::string g_create_error;

enum NormIdx { N_ATTN, N_FFN, N_QN, N_KN, N_POST_ATTN, N_POST_FFW, N_NNORM };
const char* kNormNames[N_NNORM] = {"attn_norm", "ffn_norm", "attn_q_norm", "attn_k_norm",
                                   "post_attention_norm", "post_ffw_norm"};
enum Q8Idx { Q_ATTN_Q, Q_ATTN_K, Q_ATTN_V, Q_ATTN_O, Q_GATE, Q_UP, Q_DOWN, Q_NQ8 };
const char* kQ8Names[Q_NQ8] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};

struct Layer {
  uint8_t* qkv = nullptr;   // fused [q | k | v] rows, item-planar
  uint8_t* o = nullptr;
  uint8_t* gu = nullptr;    // gate/up rows interleaved GR/2 + GR/2 per row group
  uint8_t* down = nullptr;
  // batched prefill GEMM weights (prefill_batch > 0): int8 values as bf16
  // [N][K] and fp32 block scales [N][K / 32]; gate / up in groups of 16 + 16
  uint16_t *qkv_b = nullptr, *o_b = nullptr, *gu_b = nullptr, *down_b = nullptr;
  float *qkv_d = nullptr, *o_d = nullptr, *gu_d = nullptr, *down_d = nullptr;
  float* norm[N_NNORM] = {};
  float* kc = nullptr;
  float* vc = nullptr;
  uint32_t have = 0;        // bit i: kQ8Names[i]; bit 8 + j: kNormNames[j]
};

constexpr uint32_t kAllLayerBits = ((1u << Q_NQ8) - 1) | (((1u << N_NNORM) - 1) << 8);

// ceil-division helpers
inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// f16 -> f32 (exact; gguf.ts:95-105 semantics, NaN quietened)
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  int ex = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x3ff;
  uint32_t bits;
  if (ex == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      int e = -1;
      do { mant <<= 1; ++e; } while (!(mant & 0x400));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ff) << 13);
    }
  } else if (ex == 31) {
    bits = mant ? 0x7fc00000u : (sign | 0x7f800000u);
  } else {
    bits = sign | ((uint32_t)(ex - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

struct gg_ctx {
  gg_config c{};
  int H = 0, L = 0, NQ = 0, I = 0, V = 0, CTX = 0, QD = 0, NQKV = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<Layer> layers;
  uint8_t* embd = nullptr;
  float* out_norm = nullptr;
  bool have_embd = false, have_out_norm = false;
  Q8Layout lay_embd{}, lay_qkv{}, lay_o{}, lay_gu{}, lay_down{};
  // per-layer tensors of one kind live in one layer-strided slab, so a
  // kernel forms layer l's address as base + l * stride from its arguments
  uint8_t *s_qkv = nullptr, *s_o = nullptr, *s_gu = nullptr, *s_down = nullptr;
  float* s_norm = nullptr;            // [L][6][norm_stride]
  int norm_stride = 0;
  float *s_kc = nullptr, *s_vc = nullptr;   // [L][ctx][256]
  // the persistent kernel's FFN copies: gate/up in 64-row groups (32 gate +
  // the 32 matching up rows, CI = 1) and down in 32-wide column blocks
  uint8_t *s_guf = nullptr, *s_dcb = nullptr;
  size_t st_guf = 0, st_dcb = 0;

  // work buffers
  float *qkv_out = nullptr, *attn_part = nullptr, *attn_out = nullptr, *o_out = nullptr;
  float *act = nullptr, *down_out = nullptr, *hidden = nullptr, *residual = nullptr, *normed = nullptr;
  float *logits = nullptr, *hist = nullptr, *q_dbg = nullptr;
  float* normed_tmp = nullptr;        // parity reads (GG_READ_EMBED)
  float *rope_local = nullptr, *rope_global = nullptr;   // [ctx][cos|sin][128]
  float* cand_val = nullptr;
  uint32_t *cand_id = nullptr, *top = nullptr, *seen = nullptr;
  DevState* st = nullptr;
  int32_t* tokens = nullptr;
  int32_t* d_ids = nullptr;           // staging for gg_penalty_add
  uint8_t* staging = nullptr;         // Q8_0 upload staging
  size_t staging_bytes = 0;

  // batched prefill (prefill_batch > 0)
  int pf_M = 0;
  float *pf_hidden = nullptr, *pf_residual = nullptr, *pf_qkv = nullptr, *pf_o = nullptr, *pf_part = nullptr;
  // GEMM inputs as bf16 hi / lo planes (the slice's M rows each)
  uint16_t *pf_xn = nullptr, *pf_attn = nullptr, *pf_act = nullptr;

  // pinned host mirrors
  DevState* h_st = nullptr;
  int32_t* h_tokens = nullptr;
  int32_t* h_out = nullptr;           // mapped: the selector writes the token here
  int32_t* d_out = nullptr;           // h_out's device address

  hipGraphExec_t g_fwd = nullptr, g_sel = nullptr;
  hipGraphExec_t g_step = nullptr;   // state upload + forward + select: one launch per gg_step
  // persistent decode kernel (gg_decode.hip): one launch per forward pass
  int decode_req = -1;                // gg_set_decode_path; -1: GG_DECODE environment / default
  bool fused = false;                 // forward passes run on the persistent kernel
  bool fused_step = false;            // ... and so do the LM head and the selection of gg_step
  std::string fused_why;              // why the persistent kernel is not used
  uint64_t* xll = nullptr;            // its hand-off words
  uint8_t* lm_cm = nullptr;           // class-major copy of the tied LM head
  DecodeArgs dargs{};
  hipGraphExec_t g_ffwd = nullptr, g_fstep = nullptr;
  uint64_t dec_launches = 0;          // since the hand-off words were last cleared
  size_t xll_words = 0;
  // pipelined steps (gg_step_submit / gg_step_collect): a FIFO of at most two
  int pipe_n = 0, pipe_head = 0;      // outstanding steps, slot of the oldest
  bool pipe_launched[2] = {false, false};   // slot's step is a launch in flight (else its id is known)
  int32_t pipe_tok[2] = {0, 0};       // ids of steps that ran synchronously
  struct PipeArgs { int32_t token, pos; gg_sample s; double u; };
  PipeArgs pipe_args[2] = {};         // each outstanding step's arguments (re-run after a fallback)
  bool have_prev = false;             // a selection has run: a step may take its id on the device
  int32_t last_tok = 0;               // ... that id, when the host knows it
  int32_t sel_id = 0;                 // id of the last selection whose result the host has
  hipEvent_t fence_ev = nullptr;      // follows this context's latest persistent launch (shared device)
  bool fence_reg = false;             // registered as a persistent-kernel context of its device
  bool coop = false;                  // GG_DEC_COOP=1: direct persistent launches are cooperative
  bool logits_cm = false;             // the last logits are in class-major order
  long long* timeline = nullptr;      // GG_DEC_TIMELINE=1: phase stamps of the last launch
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  int probe_kind = GG_PROBE_NONE, probe_layer = 0;
  hipError_t probe_err = hipSuccess;  // first failed probe event record of a capture
  bool capturing = false;             // a graph capture of c->stream is in progress
  hipEvent_t probe_ev[4] = {nullptr, nullptr, nullptr, nullptr};   // kernel bracket [0, 1], empty bracket [2, 3]
  bool probe_done = false;
  bool finalized = false, lost = false, timed = false, probed = false;
  bool step_timing = false;   // gg_set_timing: event records around each step
  bool use_graphs = true;   // GG_NO_GRAPH=1: launch the same kernels directly (profilers)
  std::vector<void*> allocs;
  std::string err;
};

namespace {

int set_err(gg_ctx* c, int code, const std::string& msg) {
  if (c) c->err = msg;
  else g_create_error = msg;
  return code;
}

// Map a HIP status to a gg code; faults that poison the context are sticky.
int hip_fail(gg_ctx* c, hipError_t e, const char* what) {
  std::string m = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  if (c && (e == hipErrorIllegalAddress || e == hipErrorLaunchFailure || e == hipErrorECCNotCorrectable ||
            e == hipErrorLaunchTimeOut || e == hipErrorAssert)) {
    c->lost = true;
    return set_err(c, GG_ERR_DEVICE_LOST, "device lost: " + m);
  }
  if (e == hipErrorOutOfMemory) return set_err(c, GG_ERR_OOM, m);
  return set_err(c, GG_ERR_HIP, m);
}

#define GG_HIP(ctx, call)                                   \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return hip_fail((ctx), e_, #call); \
  } while (0)

template <class T>
int dalloc(gg_ctx* c, T** p, size_t bytes) {
  void* v = nullptr;
  hipError_t e = hipMalloc(&v, bytes ? bytes : 4);
  if (e != hipSuccess) return hip_fail(c, e, "hipMalloc");
  c->allocs.push_back(v);
  *p = (T*)v;
  return GG_OK;
}

#define GG_TRY(x)          \
  do {                     \
    int r_ = (x);          \
    if (r_ != GG_OK) return r_; \
  } while (0)

int launch_rc(gg_ctx* c, int rc, const char* what) {
  if (rc != 0) return hip_fail(c, (hipError_t)rc, what);
  return GG_OK;
}

bool is_swa(const gg_config& c, int il) { return (il % c.swa_period) < (c.swa_period - 1); }


int check_ready(gg_ctx* c) {
  if (!c) return GG_ERR_INVALID;
  if (c->lost) return set_err(c, GG_ERR_DEVICE_LOST, "device lost: recreate the context");
  if (!c->finalized) return set_err(c, GG_ERR_INVALID, "context not finalized");
  return GG_OK;
}

// Ready, and no pipelined step outstanding (calls that use the device
// state or buffers must not interleave with them).
int check_idle(gg_ctx* c) {
  GG_TRY(check_ready(c));
  if (c->pipe_n > 0) return set_err(c, GG_ERR_INVALID, "pipelined steps outstanding: gg_step_collect them first");
  return GG_OK;
}

// Bracket a launch with external event-record nodes when it is the probe.
// A failed record is kept in probe_err (capture reports it) and cleared from
// the runtime's last-error state, so the bracketed launch's status stays its
// own.
struct ProbeScope {
  gg_ctx* c;
  bool on;
  ProbeScope(gg_ctx* c_, int kind, int layer) : c(c_), on(c_->probe_kind == kind && (layer < 0 || c_->probe_layer == layer)) {
    if (on) {
      record(c->probe_ev[2]);
      record(c->probe_ev[3]);
      record(c->probe_ev[0]);
    }
  }
  void record(hipEvent_t e) {
    // inside a capture an external record becomes a record node of the
    // graph; on direct launches it is an ordinary record
    const hipError_t r =
        c->capturing ? hipEventRecordWithFlags(e, c->stream, hipEventRecordExternal) : hipEventRecord(e, c->stream);
    if (r != hipSuccess) {
      if (c->probe_err == hipSuccess) c->probe_err = r;
      (void)hipGetLastError();
    }
  }
  ~ProbeScope() {
    if (on) record(c->probe_ev[1]);
  }
};

// Why the persistent decode kernel cannot run this model here ("" = it can).
std::string fused_unsupported(gg_ctx* c) {
  if (c->NQ != kAttnMaxQ) return "needs 4 query heads";
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, c->device) != hipSuccess || p.multiProcessorCount < kDecBlocks)
    return "needs 256 compute units";
  if (!c->s_guf) return "needs hidden <= 1280 and intermediate a multiple of 32 below 8193";
  if (c->lay_qkv.KpS > 4 || c->lay_o.KpS > 4) return "items per block";
  if (c->lay_qkv.rows / 8 != kDecQBlocks || c->lay_o.rows / 8 > kDecBlocks) return "row groups";
  if (decode_occupancy() < 1) return "kernel does not fit one CU";
  return "";
}

// Persistent launches of every context of the process on one device run one
// at a time: a launch needs all 256 of its blocks resident, and two launches
// side by side would each hold part of the CUs until their hand-off waits ran
// out. While a device has more than one persistent-kernel context, every
// persistent launch records its context's fence event, and a launch from
// another context first waits for the latest one.
int sync(gg_ctx* c, const char* what);
constexpr int kMaxFenceDevices = 64;
struct DevFence {
  std::vector<gg_ctx*> ctxs;   // persistent-kernel contexts of the device
  gg_ctx* last = nullptr;      // whose fence event follows the device's latest persistent launch
};
std::mutex g_fence_mu;
DevFence g_fence[kMaxFenceDevices];

int fence_register(gg_ctx* c) {
  if (c->device < 0 || c->device >= kMaxFenceDevices) return set_err(c, GG_ERR_INVALID, "device index");
  std::lock_guard<std::mutex> lk(g_fence_mu);
  DevFence& f = g_fence[c->device];
  if (f.ctxs.size() == 1) {
    // the device's only context has not fenced its launches so far
    gg_ctx* o = f.ctxs[0];
    GG_HIP(c, hipEventRecord(o->fence_ev, o->stream));
    f.last = o;
  }
  f.ctxs.push_back(c);
  c->fence_reg = true;
  return GG_OK;
}

void fence_unregister(gg_ctx* c) {
  if (!c->fence_reg) return;
  std::lock_guard<std::mutex> lk(g_fence_mu);
  DevFence& f = g_fence[c->device];
  for (size_t i = 0; i < f.ctxs.size(); ++i)
    if (f.ctxs[i] == c) {
      f.ctxs.erase(f.ctxs.begin() + (long)i);
      break;
    }
  if (f.last == c) f.last = nullptr;
  c->fence_reg = false;
}

// Start a persistent-kernel launch (lk holds the device's launch order until
// persistent_end): wait for another context's latest launch, and clear the
// hand-off words (and the launch counter that feeds their tags) before the
// 32-bit tags could wrap.
int persistent_begin(gg_ctx* c, std::unique_lock<std::mutex>& lk) {
  lk = std::unique_lock<std::mutex>(g_fence_mu);
  DevFence& f = g_fence[c->device];
  if (f.last && f.last != c) GG_HIP(c, hipStreamWaitEvent(c->stream, f.last->fence_ev, 0));
  const uint64_t limit = 0xffffffffull / (uint64_t)(c->L + 2) - 2;
  if (c->dec_launches >= limit) {
    GG_HIP(c, hipMemsetAsync(c->xll, 0, c->xll_words * 8, c->stream));
    GG_HIP(c, hipMemsetAsync((char*)c->st + offsetof(DevState, epoch), 0, 4, c->stream));
    c->dec_launches = 0;
  }
  c->dec_launches += 1;
  return GG_OK;
}

int persistent_end(gg_ctx* c) {
  DevFence& f = g_fence[c->device];
  if (f.ctxs.size() > 1) {
    GG_HIP(c, hipEventRecord(c->fence_ev, c->stream));
    f.last = c;
  }
  return GG_OK;
}

// Every hand-off wait of the persistent kernel is bounded, so a launch whose
// blocks were not all resident (CUs held by another process's work) or that
// stalled ends with its flags raised in mapped host memory. The context then
// drains its stream, clears the hand-off words and continues on the graph
// path (one kernel per phase, nothing to keep resident); the caller re-runs
// the work. Returns kRetry after that switch, GG_OK when no flag is raised.
constexpr int kRetry = 1;
constexpr int32_t kNoId = (int32_t)0x80000000;   // a queued step's id word before the launch stores it
int fall_back_to_graphs(gg_ctx* c) {
  GG_TRY(sync(c, "persistent decode kernel"));
  for (int i : {1, 8, 12, 13}) c->h_out[i] = 0;
  GG_HIP(c, hipMemsetAsync(c->xll, 0, c->xll_words * 8, c->stream));
  GG_HIP(c, hipMemsetAsync((char*)c->st + offsetof(DevState, epoch), 0, 4, c->stream));
  GG_TRY(sync(c, "hand-off reset"));
  c->dec_launches = 0;
  c->fused = c->fused_step = false;
  fence_unregister(c);
  c->fused_why = "a hand-off of the persistent decode kernel timed out (its 256 blocks were not all resident at "
                 "once, e.g. on a GPU shared with other work); switched to the graph path";
  return kRetry;
}

int check_fused(gg_ctx* c) {
  if (!c->fused || c->h_out[1] == 0) return GG_OK;
  return fall_back_to_graphs(c);
}

GemvArgs gemv_base(const uint8_t* W, const Q8Layout& L, float* out) {
  GemvArgs a{};
  a.W = W;
  a.Kp = L.Kp;
  a.KpS = L.KpS;
  a.N = L.rows;
  a.out = out;
  return a;
}

// Record the forward pass of one token (engine.ts:735-802).
// `final_norm` false: stop after the last down GEMV; the LM head then
// carries k_final's work (record_select_impl with fused_final).
int record_forward_impl(gg_ctx* c, bool final_norm) {
  const float eps = c->c.rms_norm_eps;
  for (int l = 0; l < c->L; ++l) {
    Layer& Ly = c->layers[l];
    // QKV with the previous layer's post-FFN norm + residual and attn_norm
    GemvArgs q = gemv_base(Ly.qkv, c->lay_qkv, c->qkv_out);
    q.w_pre = Ly.norm[N_ATTN];
    q.res_out = c->hidden;
    q.eps = eps;
    q.st = c->st;
    q.tokens = c->tokens;
    {
    ProbeScope ps(c, GG_PROBE_QKV, l);
    if (l == 0) {
      q.embd = c->embd;
      q.embd_KpS = c->lay_embd.KpS;
      q.embed_scale = sqrtf((float)c->H);
      GG_TRY(launch_rc(c, launch_gemv(PRO_EMBED_NORM, EPI_OUT, c->lay_qkv.CI, q, c->stream), "qkv gemv"));
    } else {
      q.pre_vec = c->down_out;
      q.pre_res = c->residual;
      q.w_post = c->layers[l - 1].norm[N_POST_FFW];
      q.hist_out = c->hist + (size_t)(l - 1) * c->H;
      GG_TRY(launch_rc(c, launch_gemv(PRO_RESID_NORM, EPI_OUT, c->lay_qkv.CI, q, c->stream), "qkv gemv"));
    }
    }
    // attention
    AttnArgs at{};
    at.qkv = c->qkv_out;
    at.n_q = c->NQ;
    at.q_norm = Ly.norm[N_QN];
    at.k_norm = Ly.norm[N_KN];
    const bool swa = is_swa(c->c, l);
    at.rope = swa ? c->rope_local : c->rope_global;
    at.k_cache = Ly.kc;
    at.v_cache = Ly.vc;
    at.window = swa ? c->c.sliding_window : 0;
    at.eps = eps;
    at.scale = (float)(1.0 / std::sqrt((double)kHeadDim));
    at.st = c->st;
    at.part = c->attn_part;
    at.attn_out = c->attn_out;
    at.q_dbg = c->q_dbg + (size_t)l * c->QD;
    // up to 16 chunks (spans <= 4096): one block per (chunk, head), merged by
    // the O GEMV's prologue; longer spans: 256 chunks of all four heads, merged
    // by k_attn_merge into attn_out
    const int nch = decode_attention_chunks(c->CTX, at.window);
    const bool merge_in_o = nch <= kDecMergeInO;
    {
      ProbeScope ps(c, GG_PROBE_ATTN, l);
      GG_TRY(launch_rc(c, launch_attention(at, nch, c->stream), "attention"));
      if (!merge_in_o) GG_TRY(launch_rc(c, launch_attention_merge(at, nch, c->stream), "attention merge"));
    }
    GemvArgs o = gemv_base(Ly.o, c->lay_o, c->o_out);
    if (merge_in_o) {
      o.attn_part = c->attn_part;
      o.attn_chunks = nch;
      o.x_out = c->attn_out;
      o.st = c->st;
    } else {
      o.x = c->attn_out;
    }
    {
      ProbeScope ps(c, GG_PROBE_O, l);
      GG_TRY(launch_rc(c, launch_gemv(merge_in_o ? PRO_ATTN_MERGE : PRO_NONE, EPI_OUT, c->lay_o.CI, o, c->stream),
                       "o gemv"));
    }
    // gate/up with post-attn norm + residual + ffn_norm, GeGLU epilogue
    GemvArgs gu = gemv_base(Ly.gu, c->lay_gu, nullptr);
    gu.pre_vec = c->o_out;
    gu.pre_res = c->hidden;
    gu.w_post = Ly.norm[N_POST_ATTN];
    gu.w_pre = Ly.norm[N_FFN];
    gu.res_out = c->residual;
    gu.eps = eps;
    gu.act_out = c->act;
    {
      ProbeScope ps(c, GG_PROBE_GATE_UP, l);
      GG_TRY(launch_rc(c, launch_gemv(PRO_RESID_NORM, EPI_GEGLU, c->lay_gu.CI, gu, c->stream), "gate/up gemv"));
    }
    // down projection
    GemvArgs d = gemv_base(Ly.down, c->lay_down, c->down_out);
    d.x = c->act;
    {
      ProbeScope ps(c, GG_PROBE_DOWN, l);
      GG_TRY(launch_rc(c, launch_gemv(PRO_NONE, EPI_OUT, c->lay_down.CI, d, c->stream), "down gemv"));
    }
  }
  if (!final_norm) return GG_OK;
  FinalArgs f{};
  f.pre_vec = c->down_out;
  f.pre_res = c->residual;
  f.w_post = c->layers[c->L - 1].norm[N_POST_FFW];
  f.w_out = c->out_norm;
  f.hidden = c->hidden;
  f.hist_out = c->hist + (size_t)(c->L - 1) * c->H;
  f.normed = c->normed;
  f.H = c->H;
  f.eps = eps;
  f.st = c->st;
  return launch_rc(c, launch_final(f, c->stream), "final norm");
}

int record_forward(gg_ctx* c) { return record_forward_impl(c, true); }

int record_fused_fwd(gg_ctx* c) {
  return launch_rc(c, launch_decode(DEC_FWD, c->dargs, c->stream, false), "persistent decode kernel");
}

// Record LM head + selection (engine.ts:805-902). With `fused_final` the LM
// head's prologue does k_final's work (post-FFN norm + residual, output norm,
// hidden / normed / history stores and the position step, engine.ts:794-801)
// from the last down GEMV's output: one launch fewer per decode step.
int record_select_impl(gg_ctx* c, bool fused_final) {
  GemvArgs lm = gemv_base(c->embd, c->lay_embd, c->logits);
  lm.x = c->normed;
  if (fused_final) {
    lm.pre_vec = c->down_out;
    lm.pre_res = c->residual;
    lm.w_post = c->layers[c->L - 1].norm[N_POST_FFW];
    lm.w_pre = c->out_norm;
    lm.res_out = c->hidden;
    lm.hist_out = c->hist + (size_t)(c->L - 1) * c->H;
    lm.x_out = c->normed;
    lm.st_advance = c->st;
    lm.eps = c->c.rms_norm_eps;
  }
  {
    ProbeScope ps(c, GG_PROBE_LM_HEAD, -1);
    GG_TRY(launch_rc(c, launch_gemv(fused_final ? PRO_RESID_NORM : PRO_NONE, EPI_OUT, c->lay_embd.CI, lm, c->stream),
                     "lm head"));
  }
  SelectArgs s{};
  s.logits = c->logits;
  s.V = c->V;
  s.cand_val = c->cand_val;
  s.cand_id = c->cand_id;
  s.top = c->top;
  s.seen = c->seen;
  s.st = c->st;
  s.auto_add = 1;
  s.host_out = c->d_out;
  ProbeScope ps(c, GG_PROBE_SELECT, -1);
  return launch_rc(c, launch_select(s, c->stream), "select");
}

int record_select(gg_ctx* c) { return record_select_impl(c, false); }

int capture(gg_ctx* c, int (*rec)(gg_ctx*), hipGraphExec_t* out) {
  GG_HIP(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed));
  c->capturing = true;
  c->probe_err = hipSuccess;   // direct launches' records are not this capture's
  int rc = rec(c);
  c->capturing = false;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  // a failed probe record belongs to this capture alone, whatever its outcome
  const hipError_t pe = c->probe_err;
  c->probe_err = hipSuccess;
  if (rc != GG_OK || e != hipSuccess || pe != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    if (rc != GG_OK) return rc;
    return e != hipSuccess ? hip_fail(c, e, "hipStreamEndCapture") : hip_fail(c, pe, "probe event record");
  }
  e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(c, e, "hipGraphInstantiate");
  return GG_OK;
}

int push_state(gg_ctx* c, size_t from, size_t to);

// Whether this runtime takes an external event record into a stream capture
// (a throw-away capture of one record of the probe's first event).
bool external_records_capture(gg_ctx* c) {
  if (hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const hipError_t r = hipEventRecordWithFlags(c->probe_ev[0], c->stream, hipEventRecordExternal);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (g) (void)hipGraphDestroy(g);
  (void)hipGetLastError();
  return r == hipSuccess && e == hipSuccess;
}

// One decode step as a single graph: the DevState upload (a memcpy node
// that reads the pinned host copy when the graph runs), the forward pass and
// the selection.
int record_step(gg_ctx* c) {
  GG_TRY(push_state(c, 0, offsetof(DevState, seen_count)));
  GG_TRY(record_forward_impl(c, false));
  return record_select_impl(c, true);
}

// The step on the persistent kernel when its LM head and selection cannot
// run in the same launch (a vocabulary that is not a multiple of 16384):
// forward launch, then the selection kernels. Otherwise the whole step is
// one launch_fused_step.
int record_fused_step(gg_ctx* c) {
  GG_TRY(push_state(c, 0, offsetof(DevState, seen_count)));
  GG_TRY(record_fused_fwd(c));
  return record_select(c);
}

// A decode step on the persistent kernel (DEC_STEP) whose position, token and
// sampling parameters are kernel arguments: one launch, no state upload.
int launch_fused_step(gg_ctx* c) {
  DecodeArgs a = c->dargs;
  a.in_use = 1;
  a.in_pos = c->h_st->pos;
  a.in_token = c->h_st->token;
  a.in_temperature = c->h_st->temperature;
  a.in_top_p = c->h_st->top_p;
  a.in_rep_penalty = c->h_st->rep_penalty;
  a.in_u = c->h_st->u;
  return launch_rc(c, launch_decode(DEC_STEP, a, c->stream, c->coop), "persistent decode kernel");
}

int run_forward(gg_ctx* c) {
  if (c->fused) {
    std::unique_lock<std::mutex> lk;
    GG_TRY(persistent_begin(c, lk));
    if (c->use_graphs) GG_HIP(c, hipGraphLaunch(c->g_ffwd, c->stream));
    else GG_TRY(record_fused_fwd(c));
    return persistent_end(c);
  }
  if (c->use_graphs) GG_HIP(c, hipGraphLaunch(c->g_fwd, c->stream));
  else GG_TRY(record_forward(c));
  return GG_OK;
}

int run_select(gg_ctx* c) {
  if (c->use_graphs) GG_HIP(c, hipGraphLaunch(c->g_sel, c->stream));
  else GG_TRY(record_select(c));
  return GG_OK;
}

// Copy the host-written head of DevState (everything before seen_count).
int push_state(gg_ctx* c, size_t from, size_t to) {
  GG_HIP(c, hipMemcpyAsync((char*)c->st + from, (char*)c->h_st + from, to - from, hipMemcpyHostToDevice,
                           c->stream));
  return GG_OK;
}

int sync(gg_ctx* c, const char* what) {
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, what);
  return GG_OK;
}


// Block tile width (128, or 144 or 96 for a C output whose width it divides)
// and K slices (up to max_ks, dividing K into whole 64-steps) that minimise
// the modelled time, in units of one block's 64-wide step on a CU of its own:
// steps per block times the load of the busiest CU, where n >= 2 co-resident
// blocks take 0.75 n of one block's time (measured on the 1B down GEMM: 144
// blocks x 108 steps 165 us, 288 x 54 124 us), times 1.2 for the 144-wide
// tile (1.125x the work per step; 85.5 us for 512 x 27 steps against 98.6 us
// for 432 x 36 steps of the 128-wide tile) or 0.96 for the 96-wide one (the
// 1B QKV GEMM, two blocks on the busiest CUs either way: 512 x 9 steps 24.7
// us against 384 x 9 steps 25.7 us), plus one unit per 2.29 M outputs of each
// slice for the consumer's read of that slice (9.4 MB in ~1.9 us at M = 2048,
// N = 1152). C must hold that many slices; the consumer adds them.
void gemm_plan(int N, int K, int M, int max_ks, bool out, int* bn_out, int* ks_out) {
  const int steps = K / 64;
  double best_cost = 0.0;
  *bn_out = 128;
  *ks_out = 1;
  for (int bn : {128, 144, 96}) {
    if (N % bn || (bn != 128 && !out)) continue;
    const int tiles = (N / bn) * ((M + 127) / 128);
    for (int ks = 1; ks <= max_ks; ++ks) {
      if (steps % ks) continue;
      const int per_cu = (tiles * ks + 255) / 256;
      const double cost = (per_cu == 1 ? 1.0 : 0.75 * per_cu) * (steps / ks) * (bn == 144 ? 1.2 : bn == 96 ? 0.96 : 1.0) +
                          (out ? ks * ((double)M * N / 2.29e6) : 0.0);
      if ((bn == 128 && ks == 1) || cost < best_cost) {
        best_cost = cost;
        *bn_out = bn;
        *ks_out = ks;
      }
    }
  }
}

GemmArgs gemm_base(const uint16_t* A, const uint16_t* W, const float* D, int N, int K, int M, float* C,
                   uint16_t* act, int max_ks = 1) {
  GemmArgs g{};
  g.A = A;
  g.W = W;
  g.D = D;
  g.M = M;
  g.N = N;
  g.K = K;
  g.C = C;
  g.act = act;
  gemm_plan(N, K, M, C ? max_ks : 1, C != nullptr, &g.bn, &g.ks);
  return g;
}

// Batched prefill of prompt rows [start, start + M): per layer QKV GEMM, k/v
// into the cache, batched attention, O GEMM, residual + norms, gate/up GEMM
// with GeGLU, down GEMM, residual + next norm; the last row ends like k_final.
int prefill_slice(gg_ctx* c, const int32_t* d_tokens, int M, int start) {
  const float eps = c->c.rms_norm_eps;
  hipStream_t s = c->stream;
  RowArgs r{};
  r.M = M;
  r.H = c->H;
  r.eps = eps;
  r.pf_start = start;
  r.tokens = d_tokens;
  r.embd = c->embd;
  r.embd_KpS = c->lay_embd.KpS;
  r.embed_scale = sqrtf((float)c->H);
  r.w_pre = c->layers[0].norm[N_ATTN];
  r.res_out = c->pf_hidden;
  r.x_out = c->pf_xn;
  GG_TRY(launch_rc(c, launch_rows_embed(r, s), "prefill embed"));
  for (int l = 0; l < c->L; ++l) {
    Layer& Ly = c->layers[l];
    const bool swa = is_swa(c->c, l);
    const GemmArgs gq = gemm_base(c->pf_xn, Ly.qkv_b, Ly.qkv_d, c->NQKV, c->H, M, c->pf_qkv, nullptr, kQkvMaxSlices);
    GG_TRY(launch_rc(c, launch_gemm(EPI_OUT, gq, s), "prefill qkv"));
    RowArgs kv{};
    kv.M = M;
    kv.pre_planes = gq.ks;
    kv.pre_stride = (size_t)M * c->NQKV;
    kv.eps = eps;
    kv.pf_start = start;
    kv.qkv = c->pf_qkv;
    kv.n_q = c->NQ;
    kv.q_norm = Ly.norm[N_QN];
    kv.k_norm = Ly.norm[N_KN];
    kv.rope = swa ? c->rope_local : c->rope_global;
    kv.k_cache = Ly.kc;
    kv.v_cache = Ly.vc;
    GG_TRY(launch_rc(c, launch_rows_kv(kv, s), "prefill kv"));
    AttnArgs at{};
    at.qkv = c->pf_qkv;
    at.n_q = c->NQ;
    at.k_cache = Ly.kc;
    at.v_cache = Ly.vc;
    at.window = swa ? c->c.sliding_window : 0;
    at.scale = (float)(1.0 / std::sqrt((double)kHeadDim));
    at.part = c->pf_part;
    at.pf_out = c->pf_attn;
    at.pf_start = start;
    at.pf_rows = M;
    at.pf_chunk = prefill_chunk(at.window, start, M);
    GG_TRY(launch_rc(c, launch_prefill_attention(at, M, s), "prefill attention"));
    const GemmArgs go = gemm_base(c->pf_attn, Ly.o_b, Ly.o_d, c->H, c->QD, M, c->pf_o, nullptr, kGemmMaxSlices);
    GG_TRY(launch_rc(c, launch_gemm(EPI_OUT, go, s), "prefill o"));
    RowArgs r1 = r;
    r1.pre = c->pf_o;
    r1.pre_planes = go.ks;
    r1.pre_stride = (size_t)M * c->H;
    r1.res = c->pf_hidden;
    r1.w_post = Ly.norm[N_POST_ATTN];
    r1.w_pre = Ly.norm[N_FFN];
    r1.res_out = c->pf_residual;
    r1.x_out = c->pf_xn;
    GG_TRY(launch_rc(c, launch_rows_resid(r1, s), "prefill post-attn"));
    GG_TRY(launch_rc(c, launch_gemm(EPI_GEGLU, gemm_base(c->pf_xn, Ly.gu_b, Ly.gu_d, 2 * c->I, c->H, M, nullptr, c->pf_act), s), "prefill gate/up"));
    const GemmArgs gd = gemm_base(c->pf_act, Ly.down_b, Ly.down_d, c->H, c->I, M, c->pf_o, nullptr, kGemmMaxSlices);
    GG_TRY(launch_rc(c, launch_gemm(EPI_OUT, gd, s), "prefill down"));
    if (l + 1 < c->L) {
      RowArgs r2 = r;
      r2.pre = c->pf_o;
      r2.pre_planes = gd.ks;
      r2.pre_stride = (size_t)M * c->H;
      r2.res = c->pf_residual;
      r2.w_post = Ly.norm[N_POST_FFW];
      r2.w_pre = c->layers[l + 1].norm[N_ATTN];
      r2.res_out = c->pf_hidden;
      r2.x_out = c->pf_xn;
      r2.last_hidden = c->hist + (size_t)l * c->H;
      GG_TRY(launch_rc(c, launch_rows_resid(r2, s), "prefill post-ffn"));
    } else {
      FinalArgs f{};
      f.pre_vec = c->pf_o + (size_t)(M - 1) * c->H;
      f.pre_planes = gd.ks;
      f.pre_stride = (size_t)M * c->H;
      f.pre_res = c->pf_residual + (size_t)(M - 1) * c->H;
      f.w_post = Ly.norm[N_POST_FFW];
      f.w_out = c->out_norm;
      f.hidden = c->hidden;
      f.hist_out = c->hist + (size_t)l * c->H;
      f.normed = c->normed;
      f.H = c->H;
      f.eps = eps;
      f.st = c->st;
      GG_TRY(launch_rc(c, launch_final(f, s), "prefill final"));
    }
  }
  return GG_OK;
}
}  // namespace

extern "C" {

gg_ctx* gg_create(const gg_config* cfg) {
  g_create_error.clear();
  if (!cfg) { set_err(nullptr, GG_ERR_INVALID, "null config"); return nullptr; }
  const gg_config& k = *cfg;
  if (k.head_dim != kHeadDim || k.num_kv_heads != 1 || k.num_q_heads < 1 || k.num_q_heads > kAttnMaxQ ||
      k.hidden_size <= 0 || k.hidden_size % 64 || k.hidden_size > 2048 || k.intermediate_size <= 0 ||
      k.intermediate_size % 64 || k.intermediate_size > kMaxK || k.vocab_size <= 0 || k.vocab_size % 64 ||
      k.num_layers <= 0 || k.context_length <= 0 || k.context_length > kMaxContext ||
      k.swa_period <= 0 || k.sliding_window < 0 || k.num_q_heads * kHeadDim > kMaxK ||
      k.prefill_batch < 0 || (k.prefill_batch > 0 && k.hidden_size % 128)) {
    set_err(nullptr, GG_ERR_INVALID,
            "unsupported config: needs head_dim 256, one KV head, <= 4 query heads, hidden/intermediate/vocab "
            "multiples of 64 (hidden <= 2048, intermediate <= 8192), context <= 65536, and for a batched "
            "prefill a hidden size that is a multiple of 128");
    return nullptr;
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
    set_err(nullptr, GG_ERR_NO_DEVICE, "no HIP device found");
    return nullptr;
  }
  int dev = 0;
  (void)hipGetDevice(&dev);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    set_err(nullptr, GG_ERR_NO_DEVICE, std::string("device is not gfx950 (MI355X): ") + prop.gcnArchName);
    return nullptr;
  }
  gg_ctx* c = new gg_ctx();
  c->c = k;
  c->device = dev;
  c->H = k.hidden_size;
  c->L = k.num_layers;
  c->NQ = k.num_q_heads;
  c->I = k.intermediate_size;
  c->V = k.vocab_size;
  c->CTX = k.context_length;
  c->QD = k.num_q_heads * kHeadDim;
  c->NQKV = c->QD + 2 * kHeadDim;
  c->layers.resize(c->L);
  auto fail = [&](int) -> gg_ctx* {  // argument: the failing gg code
    g_create_error = c->err;
    gg_destroy(c);
    return nullptr;
  };
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    c->err = "hipStreamCreate failed";
    return fail(0);
  }
  // weights: the tied embedding / LM head keeps whole 64-row groups (CI = 1,
  // also what the embedding row lookup reads); every other matrix uses 8-row
  // groups (CI = 8) so that a launch spreads over many blocks.
  c->lay_embd = q8_layout(c->V, c->H, 1);
  c->lay_qkv = q8_layout(c->NQKV, c->H, 8);
  c->lay_o = q8_layout(c->H, c->QD, 8);
  c->lay_gu = q8_layout(2 * c->I, c->H, padfree_ci(c->H / 64));
  c->lay_down = q8_layout(c->H, c->I, 8);
  if (dalloc(c, &c->embd, c->lay_embd.bytes()) || dalloc(c, &c->out_norm, (size_t)c->H * 4)) return fail(0);
  c->norm_stride = c->H > kHeadDim ? c->H : kHeadDim;
  if (dalloc(c, &c->s_qkv, c->L * c->lay_qkv.bytes()) || dalloc(c, &c->s_o, c->L * c->lay_o.bytes()) ||
      dalloc(c, &c->s_gu, c->L * c->lay_gu.bytes()) || dalloc(c, &c->s_down, c->L * c->lay_down.bytes()) ||
      dalloc(c, &c->s_norm, (size_t)c->L * N_NNORM * c->norm_stride * 4))
    return fail(0);
  // FFN copies of the persistent decode kernel, where its limits allow it
  if (c->NQ == kAttnMaxQ && c->H <= kDecMaxH && c->I % 32 == 0 &&
      c->I / 32 <= kDecMaxFBlocks) {
    c->st_guf = (size_t)(c->I / 32) * gum_group_bytes(c->H);
    c->st_dcb = (size_t)(c->I / 32) * 34 * c->H;
    if (dalloc(c, &c->s_guf, c->L * c->st_guf) || dalloc(c, &c->s_dcb, c->L * c->st_dcb)) return fail(0);
  }
  for (int l = 0; l < c->L; ++l) {
    Layer& Ly = c->layers[l];
    Ly.qkv = c->s_qkv + l * c->lay_qkv.bytes();
    Ly.o = c->s_o + l * c->lay_o.bytes();
    Ly.gu = c->s_gu + l * c->lay_gu.bytes();
    Ly.down = c->s_down + l * c->lay_down.bytes();
    for (int j = 0; j < N_NNORM; ++j) Ly.norm[j] = c->s_norm + ((size_t)l * N_NNORM + j) * c->norm_stride;
    if (c->c.prefill_batch > 0) {
      auto wcopy = [&](uint16_t** wb, float** wd, long long rows, long long K) {
        return dalloc(c, wb, (size_t)(rows * K * 2)) || dalloc(c, wd, (size_t)(rows * (K / 32) * 4));
      };
      if (wcopy(&Ly.qkv_b, &Ly.qkv_d, c->NQKV, c->H) || wcopy(&Ly.o_b, &Ly.o_d, c->H, c->QD) ||
          wcopy(&Ly.gu_b, &Ly.gu_d, 2LL * c->I, c->H) || wcopy(&Ly.down_b, &Ly.down_d, c->H, c->I))
        return fail(0);
    }
  }
  return c;
}

int gg_upload_tensor(gg_ctx* c, const char* name, uint32_t type, const uint64_t* dims, uint32_t ndims,
                     const void* bytes, size_t nbytes) {
  if (!c || !name || !bytes || (!dims && ndims)) return set_err(c, GG_ERR_INVALID, "null argument");
  if (c->lost) return set_err(c, GG_ERR_DEVICE_LOST, "device lost");
  if (c->finalized) return set_err(c, GG_ERR_INVALID, "upload after gg_finalize");
  std::string n(name);
  const std::string suf = ".weight";
  if (n.size() <= suf.size() || n.compare(n.size() - suf.size(), suf.size(), suf) != 0)
    return set_err(c, GG_ERR_INVALID, "tensor name must end in .weight: " + n);
  std::string key = n.substr(0, n.size() - suf.size());
  int layer = -1;
  if (key.compare(0, 4, "blk.") == 0) {
    size_t dot = key.find('.', 4);
    if (dot == std::string::npos) return set_err(c, GG_ERR_INVALID, "bad tensor name: " + n);
    layer = atoi(key.substr(4, dot - 4).c_str());
    if (layer < 0 || layer >= c->L) return set_err(c, GG_ERR_INVALID, "layer out of range: " + n);
    key = key.substr(dot + 1);
  }
  long long d0 = ndims > 0 ? (long long)dims[0] : 0, d1 = ndims > 1 ? (long long)dims[1] : 1;
  for (uint32_t i = 2; i < ndims; ++i) d1 *= (long long)dims[i];

  // ---- norm vectors (F32 / F16 -> f32) ----
  float* norm_dst = nullptr;
  long long norm_n = 0;
  if (layer < 0 && key == "output_norm") {
    norm_dst = c->out_norm;
    norm_n = c->H;
  } else if (layer >= 0) {
    for (int j = 0; j < N_NNORM; ++j)
      if (key == kNormNames[j]) {
        norm_dst = c->layers[layer].norm[j];
        norm_n = (j == N_QN || j == N_KN) ? kHeadDim : c->H;
        c->layers[layer].have |= 1u << (8 + j);
      }
  }
  if (norm_dst) {
    if (d0 * d1 != norm_n) return set_err(c, GG_ERR_INVALID, "wrong element count for " + n);
    std::vector<float> f((size_t)norm_n);
    if (type == GG_TYPE_F32) {
      if (nbytes != (size_t)norm_n * 4) return set_err(c, GG_ERR_INVALID, "wrong byte count for " + n);
      memcpy(f.data(), bytes, nbytes);
    } else if (type == GG_TYPE_F16) {
      if (nbytes != (size_t)norm_n * 2) return set_err(c, GG_ERR_INVALID, "wrong byte count for " + n);
      const uint8_t* b = (const uint8_t*)bytes;
      for (long long i = 0; i < norm_n; ++i) f[i] = half_to_float((uint16_t)(b[2 * i] | (b[2 * i + 1] << 8)));
    } else {
      return set_err(c, GG_ERR_INVALID, "norm tensors must be F32 or F16: " + n);
    }
    GG_HIP(c, hipMemcpy(norm_dst, f.data(), (size_t)norm_n * 4, hipMemcpyHostToDevice));
    if (layer < 0) c->have_out_norm = true;
    return GG_OK;
  }

  // ---- Q8_0 matrices ----
  uint8_t* dst = nullptr;
  const Q8Layout* lay = nullptr;
  long long rows = 0, K = 0, off = 0;
  int half = 0, bit = -1;
  if (layer < 0 && key == "token_embd") {
    dst = c->embd; rows = c->V; K = c->H; lay = &c->lay_embd;
  } else if (layer >= 0) {
    Layer& Ly = c->layers[layer];
    for (int j = 0; j < Q_NQ8; ++j)
      if (key == kQ8Names[j]) bit = j;
    switch (bit) {
      case Q_ATTN_Q: dst = Ly.qkv; rows = c->QD; K = c->H; off = 0; lay = &c->lay_qkv; break;
      case Q_ATTN_K: dst = Ly.qkv; rows = kHeadDim; K = c->H; off = c->QD; lay = &c->lay_qkv; break;
      case Q_ATTN_V: dst = Ly.qkv; rows = kHeadDim; K = c->H; off = c->QD + kHeadDim; lay = &c->lay_qkv; break;
      case Q_ATTN_O: dst = Ly.o; rows = c->H; K = c->QD; lay = &c->lay_o; break;
      case Q_GATE: dst = Ly.gu; rows = c->I; K = c->H; half = c->lay_gu.GR / 2; off = 0; lay = &c->lay_gu; break;
      case Q_UP:
        dst = Ly.gu; rows = c->I; K = c->H; half = c->lay_gu.GR / 2; off = half; lay = &c->lay_gu;
        break;
      case Q_DOWN: dst = Ly.down; rows = c->H; K = c->I; lay = &c->lay_down; break;
      default: break;
    }
  }
  if (!dst) return set_err(c, GG_ERR_INVALID, "unknown tensor: " + n);
  if (type != GG_TYPE_Q8_0) return set_err(c, GG_ERR_INVALID, "matrix tensors must be Q8_0: " + n);
  if (ndims != 2 || d0 != K || d1 != rows)
    return set_err(c, GG_ERR_INVALID, "unexpected shape for " + n);
  const size_t need = (size_t)(rows * K / 32 * 34);
  if (nbytes != need) return set_err(c, GG_ERR_INVALID, "wrong byte count for " + n);
  if (c->staging_bytes < need) {
    if (c->staging) (void)hipFree(c->staging);
    c->staging = nullptr;
    c->staging_bytes = 0;
    GG_HIP(c, hipMalloc(&c->staging, need));
    c->staging_bytes = need;
  }
  GG_HIP(c, hipMemcpy(c->staging, bytes, need, hipMemcpyHostToDevice));
  GG_TRY(launch_rc(c, launch_repack(c->staging, dst, *lay, rows, off, half, c->stream), "repack"));
  if (layer >= 0 && c->s_guf) {
    if (bit == Q_GATE || bit == Q_UP)
      GG_TRY(launch_rc(c, launch_repack_gum(c->staging, c->s_guf + layer * c->st_guf, rows, (int)K,
                                            bit == Q_UP ? 1 : 0, c->stream), "repack"));
    if (bit == Q_DOWN)
      GG_TRY(launch_rc(c, launch_repack_colblock(c->staging, c->s_dcb + layer * c->st_dcb, rows, (int)K, c->stream),
                       "repack"));
  }
  if (layer >= 0 && c->c.prefill_batch > 0) {
    Layer& Ly = c->layers[layer];
    uint16_t* wb = nullptr;
    float* wd = nullptr;
    long long boff = off;
    int bhalf = 0;
    switch (bit) {
      case Q_ATTN_Q: case Q_ATTN_K: case Q_ATTN_V: wb = Ly.qkv_b; wd = Ly.qkv_d; break;
      case Q_ATTN_O: wb = Ly.o_b; wd = Ly.o_d; break;
      case Q_GATE: wb = Ly.gu_b; wd = Ly.gu_d; boff = 0; bhalf = 16; break;
      case Q_UP: wb = Ly.gu_b; wd = Ly.gu_d; boff = 16; bhalf = 16; break;
      case Q_DOWN: wb = Ly.down_b; wd = Ly.down_d; break;
      default: break;
    }
    GG_TRY(launch_rc(c, launch_q8_bf16(c->staging, wb, wd, rows, (int)K, boff, bhalf, c->stream), "prefill weights"));
  }
  GG_TRY(sync(c, "repack"));
  if (layer < 0) c->have_embd = true;
  else c->layers[layer].have |= 1u << bit;
  return GG_OK;
}

int gg_finalize(gg_ctx* c) {
  if (!c) return GG_ERR_INVALID;
  if (c->lost) return set_err(c, GG_ERR_DEVICE_LOST, "device lost");
  if (c->finalized) return GG_OK;
  // the launches below read the runtime's last error as their status: drop
  // one that an earlier, checked-and-ignored call of this thread left (the
  // teardown of another context, for instance)
  (void)hipGetLastError();
  if (!c->have_embd) return set_err(c, GG_ERR_MISSING, "missing token_embd.weight");
  if (!c->have_out_norm) return set_err(c, GG_ERR_MISSING, "missing output_norm.weight");
  for (int l = 0; l < c->L; ++l)
    if ((c->layers[l].have & kAllLayerBits) != kAllLayerBits)
      return set_err(c, GG_ERR_MISSING, "missing tensors of blk." + std::to_string(l));
  if (c->staging) { (void)hipFree(c->staging); c->staging = nullptr; c->staging_bytes = 0; }


  const size_t kvb = (size_t)c->CTX * kHeadDim * 4;
  GG_TRY(dalloc(c, &c->s_kc, kvb * c->L));
  GG_TRY(dalloc(c, &c->s_vc, kvb * c->L));
  GG_HIP(c, hipMemset(c->s_kc, 0, kvb * c->L));
  GG_HIP(c, hipMemset(c->s_vc, 0, kvb * c->L));
  for (int l = 0; l < c->L; ++l) {
    c->layers[l].kc = c->s_kc + (size_t)l * c->CTX * kHeadDim;
    c->layers[l].vc = c->s_vc + (size_t)l * c->CTX * kHeadDim;
  }
  GG_TRY(dalloc(c, &c->qkv_out, (size_t)c->NQKV * 4));
  // decode chunk partials: o [kDecMaxChunks][kAttnMaxQ][256], then (m, l)
  GG_TRY(dalloc(c, &c->attn_part, (size_t)kDecMaxChunks * kAttnMaxQ * (2 + kHeadDim) * 4));
  GG_TRY(dalloc(c, &c->attn_out, (size_t)c->QD * 4));
  GG_TRY(dalloc(c, &c->o_out, (size_t)c->H * 4));
  GG_TRY(dalloc(c, &c->act, (size_t)c->I * 4));
  GG_TRY(dalloc(c, &c->down_out, (size_t)c->H * 4));
  GG_TRY(dalloc(c, &c->hidden, (size_t)c->H * 4));
  GG_TRY(dalloc(c, &c->residual, (size_t)c->H * 4));
  GG_TRY(dalloc(c, &c->normed, (size_t)c->H * 4));
  GG_TRY(dalloc(c, &c->normed_tmp, (size_t)c->H * 4));
  GG_TRY(dalloc(c, &c->logits, (size_t)c->V * 4));
  GG_TRY(dalloc(c, &c->hist, (size_t)c->L * c->H * 4));
  GG_TRY(dalloc(c, &c->q_dbg, (size_t)c->L * c->QD * 4));
  GG_TRY(dalloc(c, &c->rope_local, (size_t)c->CTX * kHeadDim * 4));
  GG_TRY(dalloc(c, &c->rope_global, (size_t)c->CTX * kHeadDim * 4));
  GG_TRY(dalloc(c, &c->cand_val, (size_t)kSelBlocks * 256 * 4));
  GG_TRY(dalloc(c, &c->cand_id, (size_t)kSelBlocks * 256 * 4));
  GG_TRY(dalloc(c, &c->top, 512 * 4));
  GG_TRY(dalloc(c, &c->seen, (size_t)cdiv(c->V, 32) * 4));
  GG_TRY(dalloc(c, &c->st, sizeof(DevState)));
  GG_TRY(dalloc(c, &c->tokens, (size_t)c->CTX * 4));
  GG_TRY(dalloc(c, &c->d_ids, (size_t)c->CTX * 4));
  GG_HIP(c, hipMemset(c->st, 0, sizeof(DevState)));
  if (c->c.prefill_batch > 0) {
    const int M = std::min(c->c.prefill_batch, c->CTX);
    c->pf_M = M;
    const size_t MH = (size_t)M * c->H * 4;
    GG_TRY(dalloc(c, &c->pf_hidden, MH));
    GG_TRY(dalloc(c, &c->pf_residual, MH));
    GG_TRY(dalloc(c, &c->pf_xn, MH));   // bf16 hi + lo planes: 4 bytes per element
    GG_TRY(dalloc(c, &c->pf_o, kGemmMaxSlices * MH));   // K slices of the O / down GEMMs
    GG_TRY(dalloc(c, &c->pf_qkv, (size_t)kQkvMaxSlices * M * c->NQKV * 4));   // K slices of the QKV GEMM
    GG_TRY(dalloc(c, &c->pf_attn, (size_t)M * c->QD * 4));
    GG_TRY(dalloc(c, &c->pf_act, (size_t)M * c->I * 4));
    GG_TRY(dalloc(c, &c->pf_part, (size_t)M * kPrefillChunks * kAttnMaxQ * (2 + kHeadDim) * 4));
  }
  GG_HIP(c, hipMemset(c->seen, 0, (size_t)cdiv(c->V, 32) * 4));
  GG_HIP(c, hipMemset(c->tokens, 0, (size_t)c->CTX * 4));
  GG_HIP(c, hipMemset(c->attn_out, 0, (size_t)c->QD * 4));
  GG_HIP(c, hipMemset(c->hidden, 0, (size_t)c->H * 4));
  GG_HIP(c, hipMemset(c->normed, 0, (size_t)c->H * 4));
  GG_HIP(c, hipMemset(c->logits, 0, (size_t)c->V * 4));

  // RoPE tables, computed once on the host exactly as the WGSL expressions
  // freq = 1.0 / pow(theta, f32(2i) / f32(head_dim)), angle = f32(pos) *
  // freq, cos(angle), sin(angle) (shaders.ts:457-460), for every position.
  {
    std::vector<float> tl((size_t)c->CTX * kHeadDim), tg((size_t)c->CTX * kHeadDim);
    float fl[kHeadDim / 2], fg[kHeadDim / 2];
    for (int i = 0; i < kHeadDim / 2; ++i) {
      const float e = (float)(i * 2) / (float)kHeadDim;
      fl[i] = 1.0f / powf(c->c.rope_theta_local, e);
      fg[i] = 1.0f / powf(c->c.rope_theta_global, e);
    }
    for (int p = 0; p < c->CTX; ++p)
      for (int i = 0; i < kHeadDim / 2; ++i) {
        const float al = (float)p * fl[i], ag = (float)p * fg[i];
        tl[(size_t)p * kHeadDim + i] = cosf(al);
        tl[(size_t)p * kHeadDim + kHeadDim / 2 + i] = sinf(al);
        tg[(size_t)p * kHeadDim + i] = cosf(ag);
        tg[(size_t)p * kHeadDim + kHeadDim / 2 + i] = sinf(ag);
      }
    GG_HIP(c, hipMemcpy(c->rope_local, tl.data(), tl.size() * 4, hipMemcpyHostToDevice));
    GG_HIP(c, hipMemcpy(c->rope_global, tg.data(), tg.size() * 4, hipMemcpyHostToDevice));
  }

  GG_HIP(c, hipHostMalloc((void**)&c->h_st, sizeof(DevState), hipHostMallocDefault));
  GG_HIP(c, hipHostMalloc((void**)&c->h_tokens, (size_t)c->CTX * 4, hipHostMallocDefault));
  GG_HIP(c, hipHostMalloc((void**)&c->h_out, 64, hipHostMallocMapped | hipHostMallocCoherent));
  GG_HIP(c, hipHostGetDevicePointer((void**)&c->d_out, c->h_out, 0));
  memset(c->h_out, 0, 64);
  memset(c->h_st, 0, sizeof(DevState));
  // timing events only: no system-scope fence (an L2 write-back) per record
  for (int i = 0; i < 3; ++i) GG_HIP(c, hipEventCreateWithFlags(&c->ev[i], hipEventDisableSystemFence));
  // completion of pipelined steps: the host reads each step's id from mapped
  // memory after its event, so these keep the system-scope release
  if (c->probe_kind != GG_PROBE_NONE)
    // timing-only events: no system-scope fence (cache write-back/invalidate)
    // around the bracketed launch
    for (int i = 0; i < 4; ++i) GG_HIP(c, hipEventCreateWithFlags(&c->probe_ev[i], hipEventDisableSystemFence));

  // persistent decode kernel: GG_DECODE=graph (or gg_set_decode_path) keeps
  // the per-kernel graphs for every pass
  if (c->decode_req < 0) {
    const char* dm = getenv("GG_DECODE");
    c->decode_req = (dm && strcmp(dm, "graph") == 0) ? GG_DECODE_GRAPH : GG_DECODE_FUSED;
  }
  c->fused_why = c->decode_req == GG_DECODE_FUSED ? fused_unsupported(c) : "graph path requested";
  c->fused = c->decode_req == GG_DECODE_FUSED && c->fused_why.empty();
  if (c->fused) {
    DecodeArgs& d = c->dargs;
    // hand-off words; polled buffers hold kDecThreads * (words per thread)
    const size_t w_qkv = (size_t)c->NQKV, w_part = (size_t)kAttnMaxQ * kDecChunksL * kDecPart;
    const size_t w_attn = (size_t)kAttnMaxQ * kHeadDim, w_h = kDecXW, w_dpart = (size_t)(c->I / 32) * c->H;
    const size_t w_cand = 512;
    c->xll_words = w_qkv + w_part + w_attn + 3 * w_h + w_dpart + w_cand;
    GG_TRY(dalloc(c, &c->xll, c->xll_words * 8));
    GG_HIP(c, hipMemset(c->xll, 0, c->xll_words * 8));
    d.x_qkv = c->xll;
    d.x_part = d.x_qkv + w_qkv;
    d.x_attn = d.x_part + w_part;
    d.x_o = d.x_attn + w_attn;
    d.x_down = d.x_o + w_h;   // two rows, by layer parity
    d.x_dpart = d.x_down + 2 * w_h;
    d.x_cand = d.x_dpart + w_dpart;
    d.w_qkv = c->s_qkv;
    d.w_o = c->s_o;
    d.w_guf = c->s_guf;
    d.w_dcb = c->s_dcb;
    d.st_qkv = c->lay_qkv.bytes();
    d.st_o = c->lay_o.bytes();
    d.st_guf = c->st_guf;
    d.st_dcb = c->st_dcb;
    d.norms = c->s_norm;
    d.norm_stride = c->norm_stride;
    d.kc = c->s_kc;
    d.vc = c->s_vc;
    d.kv_stride = (size_t)c->CTX * kHeadDim;
    d.rope_local = c->rope_local;
    d.rope_global = c->rope_global;
    d.swa_period = c->c.swa_period;
    d.window = c->c.sliding_window;
    d.long_ctx = c->CTX > kDecMaxCtx;
    c->fused_step = c->V % 16384 == 0 && c->V <= 262144;
    if (c->fused_step) {
      GG_TRY(dalloc(c, &c->lm_cm, c->lay_embd.bytes()));
      GG_TRY(launch_rc(c, launch_class_major(c->embd, c->lm_cm, c->V, c->lay_embd.Kp, c->stream), "class-major copy"));
      GG_TRY(sync(c, "class-major copy"));
    }
    d.L = c->L;
    d.H = c->H;
    d.I = c->I;
    d.QD = c->QD;
    d.NQKV = c->NQKV;
    d.V = c->V;
    d.kps_qkv = c->lay_qkv.KpS;
    d.kps_o = c->lay_o.KpS;
    d.kps_embd = c->lay_embd.KpS;
    d.g_f = c->I / 32;
    d.g_o = c->lay_o.rows / 8;
    d.g_down = c->lay_down.rows / 8;
    d.eps = c->c.rms_norm_eps;
    d.embed_scale = sqrtf((float)c->H);
    d.attn_scale = (float)(1.0 / std::sqrt((double)kHeadDim));
    d.embd = c->embd;
    d.lm = c->lm_cm;
    d.out_norm = c->out_norm;
    d.st = c->st;
    d.tokens = c->tokens;
    d.hidden = c->hidden;
    d.normed = c->normed;
    d.hist = c->hist;
    d.q_dbg = c->q_dbg;
    d.attn_out = c->attn_out;
    d.logits = c->logits;
    d.top = c->top;
    d.seen = c->seen;
    d.host_out = c->d_out;
    d.spin_limit = 2000000;   // 20 ms of s_memrealtime (100 MHz) per hand-off
    // GG_DEC_SPIN_LIMIT=<ticks>: a shorter bound (tests force the timeout path)
    const char* sl = getenv("GG_DEC_SPIN_LIMIT");
    if (sl && sl[0]) d.spin_limit = atoll(sl);
    // GG_DEC_COOP=1: the persistent kernel's direct launches are cooperative
    // launches (the runtime then refuses a grid that cannot be resident)
    const char* co = getenv("GG_DEC_COOP");
    c->coop = co && co[0] == '1';
    GG_HIP(c, hipEventCreateWithFlags(&c->fence_ev, hipEventDisableTiming | hipEventDisableSystemFence));
    GG_TRY(fence_register(c));
    // GG_DEC_TIMELINE=1: the persistent kernel stamps its phases (profiling)
    const char* tl = getenv("GG_DEC_TIMELINE");
    if (tl && tl[0] == '1') {
      GG_TRY(dalloc(c, &d.timeline, (size_t)kDecBlocks * c->L * kDecEvents * 8));
      GG_HIP(c, hipMemset(d.timeline, 0, (size_t)kDecBlocks * c->L * kDecEvents * 8));
      c->timeline = d.timeline;
    }
  }

  const char* ng = getenv("GG_NO_GRAPH");
  c->use_graphs = !(ng && ng[0] == '1');
  // a probe needs external event-record nodes in the captured graphs; a HIP
  // runtime that refuses them (the ROCm 7.0 runtime a process may already
  // have loaded under the same soname rejects them as an invalid value) gets
  // the same kernels launched directly, bracketed by ordinary event records
  if (c->use_graphs && c->probe_kind != GG_PROBE_NONE && !external_records_capture(c)) c->use_graphs = false;
  if (c->use_graphs) {
    GG_TRY(capture(c, record_forward, &c->g_fwd));
    GG_TRY(capture(c, record_select, &c->g_sel));
    GG_TRY(capture(c, record_step, &c->g_step));
    if (c->fused) {
      GG_TRY(capture(c, record_fused_fwd, &c->g_ffwd));
      if (!c->fused_step) GG_TRY(capture(c, record_fused_step, &c->g_fstep));
    }
  }
  c->finalized = true;
  return GG_OK;
}

int gg_prefill(gg_ctx* c, const int32_t* tokens, int32_t n, int32_t start_pos) {
  GG_TRY(check_idle(c));
  if (n < 0 || (n > 0 && !tokens) || start_pos < 0 || (long long)start_pos + n > c->CTX)
    return set_err(c, GG_ERR_INVALID, "prefill range outside the context");
  if (n == 0) return GG_OK;
  for (int i = 0; i < n; ++i) {
    if (tokens[i] < 0 || tokens[i] >= c->V) return set_err(c, GG_ERR_INVALID, "token id out of range");
    c->h_tokens[i] = tokens[i];
  }
  c->h_st->pos = start_pos;
  c->h_st->cursor = 0;
  GG_HIP(c, hipMemcpyAsync(c->tokens, c->h_tokens, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
  GG_TRY(push_state(c, 0, offsetof(DevState, temperature)));
  if (c->pf_M > 0 && n > 1) {
    for (int s0 = 0; s0 < n; s0 += c->pf_M) {
      const int M = std::min(c->pf_M, n - s0);
      GG_TRY(prefill_slice(c, c->tokens + s0, M, start_pos + s0));
    }
    c->timed = c->probed = false;
    return sync(c, "prefill");
  }
  for (;;) {
    for (int i = 0; i < n; ++i) GG_TRY(run_forward(c));
    c->timed = c->probed = false;
    GG_TRY(sync(c, "prefill"));
    const int r = check_fused(c);
    if (r != kRetry) return r;
    // after a fallback the graph path runs the prompt again from its first token
    c->h_st->pos = start_pos;
    c->h_st->cursor = 0;
    GG_TRY(push_state(c, 0, offsetof(DevState, temperature)));
  }
}

static int select_impl(gg_ctx* c, const gg_sample* s, double u, int32_t* out, bool with_forward) {
  c->h_st->temperature = s->temperature;
  c->h_st->top_p = s->top_p;
  c->h_st->rep_penalty = s->rep_penalty;
  c->h_st->u = u;
  const bool ev = c->step_timing;   // three event records cost ~9 us of device time per step
  // a persistent launch whose hand-offs timed out leaves the context on the
  // graph path (check_fused), and the selection runs again there
#define GG_CHECK_FUSED_RETRY()                                          \
  do {                                                                  \
    const int r_ = check_fused(c);                                      \
    if (r_ == kRetry) return select_impl(c, s, u, out, with_forward);   \
    if (r_ != GG_OK) return r_;                                         \
  } while (0)
  if (with_forward && !ev) {
    if (c->fused) {
      std::unique_lock<std::mutex> lk;
      GG_TRY(persistent_begin(c, lk));
      if (c->fused_step) GG_TRY(launch_fused_step(c));
      else if (c->use_graphs) GG_HIP(c, hipGraphLaunch(c->g_fstep, c->stream));
      else GG_TRY(record_fused_step(c));
      GG_TRY(persistent_end(c));
    } else {
      if (c->use_graphs) GG_HIP(c, hipGraphLaunch(c->g_step, c->stream));
      else GG_TRY(record_step(c));
    }
    GG_TRY(sync(c, "step"));
    GG_CHECK_FUSED_RETRY();
    c->logits_cm = c->fused_step;
    c->timed = false;
    c->probed = true;
    *out = c->h_out[0];
    return GG_OK;
  }
  if (with_forward && c->fused && c->fused_step) {
    // timed persistent step: the whole token is one launch (forward, LM
    // head and selection), reported as the forward time with select 0
    {
      std::unique_lock<std::mutex> lk;
      GG_TRY(persistent_begin(c, lk));
      GG_HIP(c, hipEventRecord(c->ev[0], c->stream));
      GG_TRY(launch_fused_step(c));
      GG_HIP(c, hipEventRecord(c->ev[1], c->stream));
      GG_HIP(c, hipEventRecord(c->ev[2], c->stream));
      GG_TRY(persistent_end(c));
    }
    GG_TRY(sync(c, "step"));
    GG_CHECK_FUSED_RETRY();
    c->logits_cm = true;
    c->timed = true;
    c->probed = true;
    *out = c->h_out[0];
    return GG_OK;
  }
  if (with_forward) {
    GG_TRY(push_state(c, 0, offsetof(DevState, seen_count)));
    if (ev) GG_HIP(c, hipEventRecord(c->ev[0], c->stream));
    GG_TRY(run_forward(c));
  } else {
    GG_TRY(push_state(c, offsetof(DevState, temperature), offsetof(DevState, seen_count)));
    if (ev) GG_HIP(c, hipEventRecord(c->ev[0], c->stream));
  }
  if (ev) GG_HIP(c, hipEventRecord(c->ev[1], c->stream));
  GG_TRY(run_select(c));
  if (ev) GG_HIP(c, hipEventRecord(c->ev[2], c->stream));
  // the selector stores the token straight into the mapped host word
  GG_TRY(sync(c, with_forward ? "step" : "select"));
  GG_CHECK_FUSED_RETRY();
#undef GG_CHECK_FUSED_RETRY
  c->logits_cm = false;
  c->timed = ev;
  c->probed = true;
  *out = c->h_out[0];
  return GG_OK;
}

int gg_select(gg_ctx* c, const gg_sample* s, double u, int32_t* out_token) {
  GG_TRY(check_idle(c));
  if (!s || !out_token) return set_err(c, GG_ERR_INVALID, "null argument");
  GG_TRY(select_impl(c, s, u, out_token, false));
  c->have_prev = true;
  c->last_tok = *out_token;
  c->sel_id = *out_token;
  return GG_OK;
}

static int step_impl(gg_ctx* c, int32_t token, int32_t pos, const gg_sample* s, double u, int32_t* out_token) {
  if (!s || !out_token) return set_err(c, GG_ERR_INVALID, "null argument");
  if (token < 0 || token >= c->V) return set_err(c, GG_ERR_INVALID, "token id out of range");
  if (pos < 0 || pos >= c->CTX) return set_err(c, GG_ERR_INVALID, "position outside the context");
  c->h_st->pos = pos;
  c->h_st->cursor = -1;   // embed DevState.token: one state upload per step
  c->h_st->token = token;
  GG_TRY(select_impl(c, s, u, out_token, true));
  c->have_prev = true;
  c->last_tok = *out_token;
  c->sel_id = *out_token;
  return GG_OK;
}

int gg_step(gg_ctx* c, int32_t token, int32_t pos, const gg_sample* s, double u, int32_t* out_token) {
  GG_TRY(check_idle(c));
  return step_impl(c, token, pos, s, u, out_token);
}

// A queued persistent step stores its id (or raises its timeout flag) in
// mapped host memory; the host waits for either with plain loads. No runtime
// call in the normal wait: a stream query or event wait would put a marker
// between the queued launches. Past 100 ms the stream is queried, so a
// launch that ended without an id, or a device error, is reported.
int wait_step_id(gg_ctx* c, int slot) {
  const auto t0 = std::chrono::steady_clock::now();
  for (unsigned n = 1;; ++n) {
    if (__atomic_load_n(&c->h_out[4 + slot], __ATOMIC_ACQUIRE) != kNoId ||
        __atomic_load_n(&c->h_out[12 + slot], __ATOMIC_ACQUIRE) != 0)
      return GG_OK;
    if ((n & 4095) == 0 && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(100)) {
      const hipError_t q = hipStreamQuery(c->stream);
      if (q != hipSuccess && q != hipErrorNotReady) return hip_fail(c, q, "persistent decode kernel");
      if (q == hipSuccess && __atomic_load_n(&c->h_out[4 + slot], __ATOMIC_ACQUIRE) == kNoId &&
          __atomic_load_n(&c->h_out[12 + slot], __ATOMIC_ACQUIRE) == 0)
        return set_err(c, GG_ERR_HIP, "persistent decode kernel ended without an id");
    }
  }
}

int gg_step_submit(gg_ctx* c, int32_t token, int32_t pos, const gg_sample* s, double u) {
  GG_TRY(check_ready(c));
  if (!s) return set_err(c, GG_ERR_INVALID, "null argument");
  if (token >= c->V) return set_err(c, GG_ERR_INVALID, "token id out of range");
  if (token < 0 && !c->have_prev) return set_err(c, GG_ERR_INVALID, "no selected id to take: select or step first");
  if (pos < 0 || pos >= c->CTX) return set_err(c, GG_ERR_INVALID, "position outside the context");
  if (c->pipe_n >= 2) return set_err(c, GG_ERR_INVALID, "two steps outstanding: gg_step_collect first");
  const int slot = (c->pipe_head + c->pipe_n) & 1;
  if (c->fused && c->fused_step) {
    // one launch, queued behind the previous one; with token < 0 it embeds
    // the id that launch selects (DevState::out_token, read on the device)
    std::unique_lock<std::mutex> lk;
    GG_TRY(persistent_begin(c, lk));
    DecodeArgs a = c->dargs;
    a.in_use = 1;
    a.in_pos = pos;
    a.in_token = token;
    a.in_temperature = s->temperature;
    a.in_top_p = s->top_p;
    a.in_rep_penalty = s->rep_penalty;
    a.in_u = u;
    a.out_slot = 4 + slot;
    // the launch stores its id into this mapped word; no event is recorded
    // behind it (a record between two queued launches idles the GPU ~6 us at
    // every launch boundary)
    __atomic_store_n(&c->h_out[4 + slot], kNoId, __ATOMIC_RELEASE);
    GG_TRY(launch_rc(c, launch_decode(DEC_STEP, a, c->stream, c->coop), "persistent decode kernel"));
    GG_TRY(persistent_end(c));
    c->pipe_args[slot] = {token, pos, *s, u};
    c->pipe_launched[slot] = true;
    c->logits_cm = true;
    c->timed = false;
    c->probed = true;
  } else {
    // no single-launch step here: run it now, keep its id for the collect
    int32_t tok = 0;
    GG_TRY(step_impl(c, token < 0 ? c->last_tok : token, pos, s, u, &tok));
    c->pipe_tok[slot] = tok;
    c->pipe_launched[slot] = false;
  }
  c->have_prev = true;
  c->pipe_n += 1;
  return GG_OK;
}

int gg_step_collect(gg_ctx* c, int32_t* out_token) {
  GG_TRY(check_ready(c));
  if (!out_token) return set_err(c, GG_ERR_INVALID, "null argument");
  if (c->pipe_n == 0) return set_err(c, GG_ERR_INVALID, "no step outstanding");
  const int slot = c->pipe_head;
  c->pipe_head ^= 1;
  c->pipe_n -= 1;
  if (c->pipe_launched[slot]) {
    GG_TRY(wait_step_id(c, slot));
    if (c->h_out[12 + slot] != 0) {
      // this step's launch timed out, and a step queued behind it took its
      // id on the device: switch to the graph path and run both again there
      // with the ids the host now has
      const int nxt = slot ^ 1;
      const bool redo_next = c->pipe_n > 0 && c->pipe_launched[nxt];
      const int r = fall_back_to_graphs(c);
      if (r != kRetry) return r;
      const gg_ctx::PipeArgs pa = c->pipe_args[slot], pb = c->pipe_args[nxt];
      GG_TRY(step_impl(c, pa.token >= 0 ? pa.token : c->sel_id, pa.pos, &pa.s, pa.u, out_token));
      if (redo_next) {
        GG_TRY(step_impl(c, pb.token >= 0 ? pb.token : *out_token, pb.pos, &pb.s, pb.u, &c->pipe_tok[nxt]));
        c->pipe_launched[nxt] = false;
      }
      c->sel_id = *out_token;
      return GG_OK;
    }
    *out_token = c->h_out[4 + slot];
    if (c->pipe_n == 0) c->last_tok = *out_token;
  } else {
    *out_token = c->pipe_tok[slot];
  }
  c->sel_id = *out_token;
  return GG_OK;
}

int gg_penalty_reset(gg_ctx* c) {
  GG_TRY(check_idle(c));
  GG_HIP(c, hipMemsetAsync(c->seen, 0, (size_t)cdiv(c->V, 32) * 4, c->stream));
  GG_HIP(c, hipMemsetAsync((char*)c->st + offsetof(DevState, seen_count), 0, 4, c->stream));
  return sync(c, "penalty reset");
}

int gg_penalty_add(gg_ctx* c, const int32_t* ids, int32_t n) {
  GG_TRY(check_idle(c));
  if (n < 0 || n > c->CTX || (n > 0 && !ids)) return set_err(c, GG_ERR_INVALID, "bad id list");
  if (n == 0) return GG_OK;
  for (int i = 0; i < n; ++i) c->h_tokens[i] = ids[i];
  GG_HIP(c, hipMemcpyAsync(c->d_ids, c->h_tokens, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
  GG_TRY(launch_rc(c, launch_seen_add(c->seen, c->st, c->d_ids, n, c->V, c->stream), "penalty add"));
  return sync(c, "penalty add");
}

int gg_reset_kv(gg_ctx* c) {
  GG_TRY(check_idle(c));
  const size_t kvb = (size_t)c->CTX * kHeadDim * 4;
  for (Layer& Ly : c->layers) {
    GG_HIP(c, hipMemsetAsync(Ly.kc, 0, kvb, c->stream));
    GG_HIP(c, hipMemsetAsync(Ly.vc, 0, kvb, c->stream));
  }
  return sync(c, "reset kv");
}

int gg_read(gg_ctx* c, int32_t what, int32_t layer, void* dst, size_t nbytes) {
  GG_TRY(check_idle(c));
  if (!dst) return set_err(c, GG_ERR_INVALID, "null destination");
  const void* src = nullptr;
  size_t sz = 0;
  const bool lay_ok = layer >= 0 && layer < c->L;
  switch (what) {
    case GG_READ_HIDDEN: src = c->hidden; sz = (size_t)c->H * 4; break;
    case GG_READ_NORMED: src = c->normed; sz = (size_t)c->H * 4; break;
    case GG_READ_LOGITS: src = c->logits; sz = (size_t)c->V * 4; break;
    case GG_READ_TOPK256: src = c->top; sz = 512 * 4; break;
    case GG_READ_LAYER_HIDDEN:
      if (!lay_ok) return set_err(c, GG_ERR_INVALID, "layer out of range");
      src = c->hist + (size_t)layer * c->H; sz = (size_t)c->H * 4; break;
    case GG_READ_K_CACHE:
    case GG_READ_V_CACHE:
      if (!lay_ok) return set_err(c, GG_ERR_INVALID, "layer out of range");
      src = what == GG_READ_K_CACHE ? c->layers[layer].kc : c->layers[layer].vc;
      sz = (size_t)c->CTX * kHeadDim * 4; break;
    case GG_READ_Q:
      if (!lay_ok) return set_err(c, GG_ERR_INVALID, "layer out of range");
      src = c->q_dbg + (size_t)layer * c->QD; sz = (size_t)c->QD * 4; break;
    case GG_READ_ATTN_OUT: src = c->attn_out; sz = (size_t)c->QD * 4; break;
    case GG_READ_EMBED:
      if (layer < 0 || layer >= c->V) return set_err(c, GG_ERR_INVALID, "token out of range");
      GG_TRY(launch_rc(c, launch_embed_row(c->embd, c->lay_embd.KpS, sqrtf((float)c->H), layer, c->H, c->normed_tmp,
                                           c->stream), "embedding row"));
      src = c->normed_tmp;
      sz = (size_t)c->H * 4;
      break;
    default: return set_err(c, GG_ERR_INVALID, "unknown read target");
  }
  if (nbytes < sz) sz = nbytes;
  GG_TRY(sync(c, "read"));
  if (what == GG_READ_LOGITS && c->logits_cm) {
    // the persistent kernel's LM head leaves class-major logits:
    // row c + 256 k at c * (V / 256) + k
    std::vector<float> cm((size_t)c->V);
    GG_HIP(c, hipMemcpy(cm.data(), src, (size_t)c->V * 4, hipMemcpyDeviceToHost));
    const int R = c->V / 256;
    float* o = (float*)dst;
    const size_t n = sz / 4;
    for (size_t r = 0; r < n; ++r) o[r] = cm[(r & 255) * R + (r >> 8)];
    return GG_OK;
  }
  GG_HIP(c, hipMemcpy(dst, src, sz, hipMemcpyDeviceToHost));
  return GG_OK;
}

int gg_set_timing(gg_ctx* c, int32_t on) {
  GG_TRY(check_ready(c));
  c->step_timing = on != 0;
  c->timed = false;
  return GG_OK;
}

int gg_last_timing(gg_ctx* c, float* forward_ms, float* select_ms) {
  GG_TRY(check_ready(c));
  if (!c->timed) return set_err(c, GG_ERR_INVALID, "no timed step yet (gg_set_timing off, or no step since)");
  float a = 0.f, b = 0.f;
  GG_HIP(c, hipEventElapsedTime(&a, c->ev[0], c->ev[1]));
  GG_HIP(c, hipEventElapsedTime(&b, c->ev[1], c->ev[2]));
  if (forward_ms) *forward_ms = a;
  if (select_ms) *select_ms = b;
  return GG_OK;
}

int gg_set_probe(gg_ctx* c, int32_t kind, int32_t layer) {
  if (!c) return GG_ERR_INVALID;
  if (c->finalized) return set_err(c, GG_ERR_INVALID, "gg_set_probe must precede gg_finalize");
  if (kind < GG_PROBE_NONE || kind > GG_PROBE_SELECT || layer < 0 || layer >= c->L)
    return set_err(c, GG_ERR_INVALID, "bad probe");
  c->probe_kind = kind;
  c->probe_layer = layer;
  return GG_OK;
}

int gg_probe_elapsed(gg_ctx* c, float* ms) {
  GG_TRY(check_ready(c));
  if (c->probe_kind == GG_PROBE_NONE || !ms) return set_err(c, GG_ERR_INVALID, "no probe set");
  if (!c->probed) return set_err(c, GG_ERR_INVALID, "no step yet");
  GG_HIP(c, hipEventElapsedTime(ms, c->probe_ev[0], c->probe_ev[1]));
  return GG_OK;
}
int gg_probe_overhead(gg_ctx* c, float* ms) {
  GG_TRY(check_ready(c));
  if (c->probe_kind == GG_PROBE_NONE || !ms) return set_err(c, GG_ERR_INVALID, "no probe set");
  if (!c->probed) return set_err(c, GG_ERR_INVALID, "no step yet");
  GG_HIP(c, hipEventElapsedTime(ms, c->probe_ev[2], c->probe_ev[3]));
  return GG_OK;
}

int gg_set_decode_path(gg_ctx* c, int32_t path) {
  if (!c) return GG_ERR_INVALID;
  if (c->finalized) return set_err(c, GG_ERR_INVALID, "gg_set_decode_path must precede gg_finalize");
  if (path != GG_DECODE_GRAPH && path != GG_DECODE_FUSED) return set_err(c, GG_ERR_INVALID, "unknown decode path");
  c->decode_req = path;
  return GG_OK;
}

int gg_decode_timeline(gg_ctx* c, int64_t* dst, size_t n) {
  GG_TRY(check_ready(c));
  if (!c->timeline || !dst) return set_err(c, GG_ERR_INVALID, "no timeline (GG_DEC_TIMELINE=1 at finalize)");
  const size_t total = (size_t)kDecBlocks * c->L * kDecEvents;
  GG_TRY(sync(c, "timeline"));
  GG_HIP(c, hipMemcpy(dst, c->timeline, (n < total ? n : total) * 8, hipMemcpyDeviceToHost));
  return GG_OK;
}

int gg_decode_path(gg_ctx* c) {
  GG_TRY(check_ready(c));
  return c->fused ? GG_DECODE_FUSED : GG_DECODE_GRAPH;
}

const char* gg_last_error(const gg_ctx* c) { return c ? c->err.c_str() : g_create_error.c_str(); }

void gg_destroy(gg_ctx* c) {
  if (!c) return;
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  fence_unregister(c);
  if (c->fence_ev) (void)hipEventDestroy(c->fence_ev);
  if (c->g_fwd) (void)hipGraphExecDestroy(c->g_fwd);
  if (c->g_sel) (void)hipGraphExecDestroy(c->g_sel);
  if (c->g_step) (void)hipGraphExecDestroy(c->g_step);
  if (c->g_ffwd) (void)hipGraphExecDestroy(c->g_ffwd);
  if (c->g_fstep) (void)hipGraphExecDestroy(c->g_fstep);
  for (hipEvent_t e : c->ev)
    if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->probe_ev)
    if (e) (void)hipEventDestroy(e);
  for (void* p : c->allocs) (void)hipFree(p);
  if (c->staging) (void)hipFree(c->staging);
  if (c->h_st) (void)hipHostFree(c->h_st);
  if (c->h_tokens) (void)hipHostFree(c->h_tokens);
  if (c->h_out) (void)hipHostFree(c->h_out);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
  (void)hipGetLastError();   // teardown errors are not the next call's
}

// ---- kernel-level entry points --------------------------------------------

size_t gg_q8_0_packed_size(int64_t rows, int64_t k) {
  if (rows <= 0 || k <= 0 || rows % 64 || k % 64 || rows > (1LL << 30) || k > kMaxK) return 0;
  return q8_layout((int)rows, (int)k).bytes();
}

int gg_q8_0_repack(const void* src, void* dst, int64_t rows, int64_t k, void* stream) {
  if (!src || !dst || !gg_q8_0_packed_size(rows, k)) return GG_ERR_INVALID;
  const Q8Layout L = q8_layout((int)rows, (int)k);
  return launch_repack((const uint8_t*)src, (uint8_t*)dst, L, rows, 0, 0, stream) ? GG_ERR_HIP : GG_OK;
}

int gg_q8_0_gemv(const void* w, const float* x, float* y, int64_t rows, int64_t k, void* stream) {
  if (!w || !x || !y || !gg_q8_0_packed_size(rows, k)) return GG_ERR_INVALID;
  const Q8Layout L = q8_layout((int)rows, (int)k);
  GemvArgs a = gemv_base((const uint8_t*)w, L, y);
  a.x = x;
  return launch_gemv(PRO_NONE, EPI_OUT, L.CI, a, stream) ? GG_ERR_HIP : GG_OK;
}

int gg_q8_0_dequant(const void* src, float* out, int64_t n, void* stream) {
  if (!src || !out || n <= 0 || n % 32) return GG_ERR_INVALID;
  return launch_dequant((const uint8_t*)src, out, n, stream) ? GG_ERR_HIP : GG_OK;
}

// workspace: DevState | cand_val | cand_id | top
size_t gg_select_workspace_size(int32_t n) {
  (void)n;
  return 256 + (size_t)kSelBlocks * 256 * 8 + 512 * 4;
}

}  // extern "C"

// Token selection with the workspace at ws (DevState | cand_val | cand_id |
// top, gg_select_workspace_size bytes): shared by gg_select_logits and
// gg_select_logits_noalloc.
static int select_with_workspace(const float* logits, int32_t n, const uint32_t* seen, const gg_sample* s,
                                 double u, char* ws, void* topk_out, int32_t* out_token, hipStream_t hs) {
  DevState h{};
  h.temperature = s->temperature;
  h.top_p = s->top_p;
  h.rep_penalty = s->rep_penalty;
  h.u = u;
  h.seen_count = seen ? 1 : 0;
  SelectArgs a{};
  a.logits = logits;
  a.V = n;
  a.st = (DevState*)ws;
  a.cand_val = (float*)(ws + 256);
  a.cand_id = (uint32_t*)(ws + 256 + (size_t)kSelBlocks * 256 * 4);
  a.top = topk_out ? (uint32_t*)topk_out : (uint32_t*)(ws + 256 + (size_t)kSelBlocks * 256 * 8);
  a.seen = seen ? (uint32_t*)seen : (uint32_t*)ws;  // never read when seen_count == 0
  a.auto_add = 0;
  if (hipMemcpyAsync(ws, &h, sizeof(h), hipMemcpyHostToDevice, hs) != hipSuccess) return GG_ERR_HIP;
  if (launch_select(a, hs)) return GG_ERR_HIP;
  DevState back{};
  if (hipMemcpyAsync(&back, ws, sizeof(back), hipMemcpyDeviceToHost, hs) != hipSuccess) return GG_ERR_HIP;
  if (hipStreamSynchronize(hs) != hipSuccess) return GG_ERR_HIP;
  *out_token = back.out_token;
  return GG_OK;
}

// Workspace of gg_select_logits_noalloc: one copy per device, held until the
// process ends. Host code never passes `scratch` itself to a kernel or copy
// (on the host it names a stand-in, not device memory); it uses the device
// address hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocScratchBytes = 256 + (size_t)kSelBlocks * 256 * 8 + 512 * 4;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

// The current device's address of `scratch`, looked up on the first call on
// that device.
static int scratch_address(char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return GG_ERR_NO_DEVICE;
  if (dev < 0 || dev >= kMaxScratchDevices) return GG_ERR_INVALID;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return GG_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = (char*)g_scratch_ptr[dev];
  return GG_OK;
}

extern "C" {

int gg_select_logits(const float* logits, int32_t n, const uint32_t* seen, const gg_sample* s, double u,
                     void* workspace, void* topk_out, int32_t* out_token, void* stream) {
  if (!logits || n <= 0 || !s || !workspace || !out_token) return GG_ERR_INVALID;
  return select_with_workspace(logits, n, seen, s, u, (char*)workspace, topk_out, out_token, (hipStream_t)stream);
}

int gg_select_logits_noalloc(const float* logits, int32_t n, const uint32_t* seen, const gg_sample* s, double u,
                             void* topk_out, int32_t* out_token, void* stream) {
  if (!logits || n <= 0 || !s || !out_token) return GG_ERR_INVALID;
  if (gg_select_workspace_size(n) > kNoAllocScratchBytes) {
    std::fprintf(stderr, "gg_select_logits_noalloc: %d logits need a %zu-byte workspace, above the %zu-byte "
                 "static one\n", n, gg_select_workspace_size(n), kNoAllocScratchBytes);
    return GG_ERR_INVALID;
  }
  char* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != GG_OK) return rc;
  return select_with_workspace(logits, n, seen, s, u, ws, topk_out, out_token, (hipStream_t)stream);
}

}  // extern "C"

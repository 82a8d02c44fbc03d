/* gg_napi.c -- Node-API binding of libgg.so for the JavaScript host.
 *
 * Replaces the WebGPU device layer of the reference engine (engine.ts:124-949,
 * 1039-1077) with calls into the C-ABI of include/gg.h. One binding call per
 * reference method:
 *   create(config)                       initWebGPU + createUniformBuffers
 *   upload(ctx, name, type, dims, bytes) uploadWeights* (GGUF bytes as stored)
 *   finalize(ctx)                        createWorkBuffers + createBindGroups
 *   prefill(ctx, ids, startPos)          prefillBatched            -> Promise
 *   select(ctx, T, topP, rep, u)         getFirstTokenAfterPrefill -> Promise<id>
 *   step(ctx, id, pos, T, topP, rep, u)  forwardPassAndGetToken    -> Promise<id>
 *   stepSubmit(ctx, id, pos, T, topP, rep, u), stepCollect(ctx) -> Promise<id>
 *                                        the same step queued ahead (id -1:
 *                                        the previous step's, on the device)
 *   penaltyReset(ctx), penaltyAdd(ctx, ids)   the per-turn Set(allTokens)
 *   resetKV(ctx)                         resetKVCaches
 *   read(ctx, what, layer, typedArray)   debug readbacks
 *   destroy(ctx)                         dispose
 * prefill/select/step run on the libuv thread pool (napi_async_work) so the
 * JavaScript generate() loop stays asynchronous. A context runs one call at a
 * time: while a prefill/select/step is in flight every other call on that
 * context throws / rejects with GG_ERR_INVALID ("busy"), and destroy() (or the
 * garbage collector's finalizer) only marks the context; the last job's
 * completion callback then calls gg_destroy, so a worker thread never runs on
 * a destroyed context. Failures reject / throw an Error whose `code` is the
 * GG_ERR_* name; GG_ERR_DEVICE_LOST maps to the reference's deviceLost state.
 */
#include <node_api.h>
#include <stdlib.h>
#include <string.h>

#include "gg.h"

#define CHECK(env, call)                                                      \
  do {                                                                        \
    if ((call) != napi_ok) {                                                  \
      napi_throw_error((env), "GG_ERR_NAPI", "Node-API call failed: " #call); \
      return NULL;                                                            \
    }                                                                         \
  } while (0)

static const char* code_name(int rc) {
  switch (rc) {
    case GG_ERR_INVALID: return "GG_ERR_INVALID";
    case GG_ERR_NO_DEVICE: return "GG_ERR_NO_DEVICE";
    case GG_ERR_HIP: return "GG_ERR_HIP";
    case GG_ERR_DEVICE_LOST: return "GG_ERR_DEVICE_LOST";
    case GG_ERR_MISSING: return "GG_ERR_MISSING";
    case GG_ERR_OOM: return "GG_ERR_OOM";
  }
  return "GG_ERR";
}

static napi_value make_error(napi_env env, int rc, const char* msg) {
  napi_value code, text, err;
  napi_create_string_utf8(env, code_name(rc), NAPI_AUTO_LENGTH, &code);
  napi_create_string_utf8(env, msg ? msg : "unknown error", NAPI_AUTO_LENGTH, &text);
  napi_create_error(env, code, text, &err);
  return err;
}

static napi_value throw_rc(napi_env env, gg_ctx* ctx, int rc) {
  napi_throw(env, make_error(env, rc, gg_last_error(ctx)));
  return NULL;
}

/* ---- argument helpers ---------------------------------------------------- */
/* The JavaScript external's payload. Every field is read and written on the
 * JavaScript thread only (binding calls, job completion, the finalizer); the
 * worker thread sees the gg_ctx* copied into its job when the job was queued. */
typedef struct {
  gg_ctx* ctx;          /* NULL once destroyed */
  int busy;             /* a prefill/select/step job is in flight */
  int destroy_pending;  /* destroy() or the finalizer ran while busy */
  int orphaned;         /* the finalizer ran: the job's completion frees this */
} handle_t;

static void finalize_handle(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  handle_t* h = (handle_t*)data;
  if (h->busy) {
    h->destroy_pending = 1;
    h->orphaned = 1;
    return;
  }
  if (h->ctx) gg_destroy(h->ctx);
  free(h);
}

/* The handle behind argument v when it names a live context that is not
 * running a job; otherwise throws GG_ERR_INVALID and returns NULL. */
static handle_t* get_handle(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_error(env, "GG_ERR_INVALID", "not an engine context");
    return NULL;
  }
  handle_t* h = (handle_t*)p;
  if (!h->ctx || h->destroy_pending) {
    napi_throw_error(env, "GG_ERR_INVALID", "the engine context was destroyed");
    return NULL;
  }
  if (h->busy) {
    napi_throw_error(env, "GG_ERR_INVALID", "the engine context is busy with another prefill/select/step call");
    return NULL;
  }
  return h;
}

static gg_ctx* get_ctx(napi_env env, napi_value v) {
  handle_t* h = get_handle(env, v);
  return h ? h->ctx : NULL;
}

static int get_f64(napi_env env, napi_value obj, const char* key, double* out) {
  napi_value v;
  bool has = false;
  if (napi_has_named_property(env, obj, key, &has) != napi_ok || !has) return 0;
  if (napi_get_named_property(env, obj, key, &v) != napi_ok) return 0;
  return napi_get_value_double(env, v, out) == napi_ok;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok || argc < want) {
    napi_throw_type_error(env, "GG_ERR_INVALID", "missing arguments");
    return 0;
  }
  return 1;
}

/* An Int32Array argument copied into malloc'd memory (owned by the caller). */
static int32_t* copy_ids(napi_env env, napi_value v, size_t* n) {
  napi_typedarray_type type;
  size_t len;
  void* data;
  napi_value ab;
  size_t off;
  if (napi_get_typedarray_info(env, v, &type, &len, &data, &ab, &off) != napi_ok || type != napi_int32_array) {
    napi_throw_type_error(env, "GG_ERR_INVALID", "token ids must be an Int32Array");
    return NULL;
  }
  int32_t* out = (int32_t*)malloc(len ? len * sizeof(int32_t) : 1);
  if (!out) {
    napi_throw_error(env, "GG_ERR_OOM", "host allocation failed");
    return NULL;
  }
  memcpy(out, data, len * sizeof(int32_t));
  *n = len;
  return out;
}

/* ---- synchronous calls --------------------------------------------------- */
static napi_value Create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  gg_config c;
  memset(&c, 0, sizeof(c));
  double v;
#define FIELD_I(name)                                          \
  if (get_f64(env, argv[0], #name, &v)) c.name = (int32_t)v;
#define FIELD_F(name)                                          \
  if (get_f64(env, argv[0], #name, &v)) c.name = (float)v;
  FIELD_I(hidden_size)
  FIELD_I(num_layers)
  FIELD_I(num_q_heads)
  FIELD_I(num_kv_heads)
  FIELD_I(head_dim)
  FIELD_I(intermediate_size)
  FIELD_I(vocab_size)
  FIELD_I(context_length)
  FIELD_F(rms_norm_eps)
  FIELD_F(rope_theta_global)
  FIELD_F(rope_theta_local)
  FIELD_I(swa_period)
  FIELD_I(sliding_window)
  FIELD_I(attention_mode)
  FIELD_I(prefill_batch)
#undef FIELD_I
#undef FIELD_F
  gg_ctx* ctx = gg_create(&c);
  if (!ctx) {
    const char* msg = gg_last_error(NULL);
    int rc = (msg && strstr(msg, "device")) ? GG_ERR_NO_DEVICE : GG_ERR_INVALID;
    return throw_rc(env, NULL, rc);
  }
  handle_t* h = (handle_t*)calloc(1, sizeof(handle_t));
  if (!h) {
    gg_destroy(ctx);
    napi_throw_error(env, "GG_ERR_OOM", "host allocation failed");
    return NULL;
  }
  h->ctx = ctx;
  napi_value ext;
  CHECK(env, napi_create_external(env, h, finalize_handle, NULL, &ext));
  return ext;
}

static napi_value Upload(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  char name[256];
  size_t nlen;
  CHECK(env, napi_get_value_string_utf8(env, argv[1], name, sizeof(name), &nlen));
  uint32_t type;
  CHECK(env, napi_get_value_uint32(env, argv[2], &type));
  uint32_t ndims;
  CHECK(env, napi_get_array_length(env, argv[3], &ndims));
  if (ndims < 1 || ndims > 4) {
    napi_throw_range_error(env, "GG_ERR_INVALID", "tensor rank must be 1..4");
    return NULL;
  }
  uint64_t dims[4];
  for (uint32_t i = 0; i < ndims; ++i) {
    napi_value e;
    double d;
    CHECK(env, napi_get_element(env, argv[3], i, &e));
    CHECK(env, napi_get_value_double(env, e, &d));
    dims[i] = (uint64_t)d;
  }
  void* bytes;
  size_t nbytes;
  bool is_buf = false;
  CHECK(env, napi_is_buffer(env, argv[4], &is_buf));
  if (is_buf) {
    CHECK(env, napi_get_buffer_info(env, argv[4], &bytes, &nbytes));
  } else {
    napi_typedarray_type t;
    size_t len, off;
    napi_value ab;
    CHECK(env, napi_get_typedarray_info(env, argv[4], &t, &len, &bytes, &ab, &off));
    nbytes = len * (t == napi_float32_array || t == napi_int32_array || t == napi_uint32_array ? 4 :
                    t == napi_uint16_array || t == napi_int16_array ? 2 : 1);
  }
  int rc = gg_upload_tensor(ctx, name, type, dims, ndims, bytes, nbytes);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

static napi_value Finalize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  int rc = gg_finalize(ctx);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

static napi_value PenaltyReset(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  int rc = gg_penalty_reset(ctx);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

static napi_value PenaltyAdd(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  size_t n = 0;
  int32_t* ids = copy_ids(env, argv[1], &n);
  if (!ids) return NULL;
  int rc = gg_penalty_add(ctx, ids, (int32_t)n);
  free(ids);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

static napi_value ResetKV(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  int rc = gg_reset_kv(ctx);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

static napi_value Read(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  int32_t what, layer;
  CHECK(env, napi_get_value_int32(env, argv[1], &what));
  CHECK(env, napi_get_value_int32(env, argv[2], &layer));
  napi_typedarray_type t;
  size_t len, off;
  void* data;
  napi_value ab;
  CHECK(env, napi_get_typedarray_info(env, argv[3], &t, &len, &data, &ab, &off));
  if (t != napi_float32_array && t != napi_uint32_array) {
    napi_throw_type_error(env, "GG_ERR_INVALID", "read needs a Float32Array or Uint32Array");
    return NULL;
  }
  int rc = gg_read(ctx, what, layer, data, len * 4);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

static napi_value Destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  void* p = NULL;
  CHECK(env, napi_get_value_external(env, argv[0], &p));
  handle_t* h = (handle_t*)p;
  if (!h || !h->ctx) return NULL;
  if (h->busy) {
    h->destroy_pending = 1;  /* the running job's completion destroys it */
    return NULL;
  }
  gg_destroy(h->ctx);
  h->ctx = NULL;
  return NULL;
}

/* decodePath(ctx): 1 while forward passes run on the persistent kernel
 * (stepSubmit queues a launch and returns), 0 on the graph path (stepSubmit
 * runs the step before it returns; gg_decode_path). */
static napi_value DecodePath(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  int p = gg_decode_path(ctx);
  if (p < 0) return throw_rc(env, ctx, p);
  napi_value r;
  CHECK(env, napi_create_int32(env, p, &r));
  return r;
}

/* stepSubmit(ctx, id, pos, T, topP, rep, u): queues a step and returns
 * without waiting (gg_step_submit); stepCollect awaits it. */
static napi_value StepSubmit(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!get_args(env, info, 7, argv)) return NULL;
  gg_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return NULL;
  int32_t token = 0, pos = 0;
  gg_sample s;
  double u = 0.0;
  if (napi_get_value_int32(env, argv[1], &token) != napi_ok || napi_get_value_int32(env, argv[2], &pos) != napi_ok ||
      napi_get_value_double(env, argv[3], &s.temperature) != napi_ok ||
      napi_get_value_double(env, argv[4], &s.top_p) != napi_ok ||
      napi_get_value_double(env, argv[5], &s.rep_penalty) != napi_ok || napi_get_value_double(env, argv[6], &u) != napi_ok) {
    napi_throw_type_error(env, "GG_ERR_INVALID", "step arguments must be numbers");
    return NULL;
  }
  int rc = gg_step_submit(ctx, token, pos, &s, u);
  if (rc != GG_OK) return throw_rc(env, ctx, rc);
  return NULL;
}

/* ---- asynchronous calls (prefill / select / step / stepCollect) --------- */
enum { OP_PREFILL, OP_SELECT, OP_STEP, OP_COLLECT };
typedef struct {
  int op;
  handle_t* h;
  gg_ctx* ctx;
  int32_t* ids;
  size_t n;
  int32_t token, pos;
  gg_sample s;
  double u;
  int32_t out;
  int rc;
  char err[512];
  napi_deferred deferred;
  napi_async_work work;
} job_t;

static void job_execute(napi_env env, void* data) {
  (void)env;
  job_t* j = (job_t*)data;
  switch (j->op) {
    case OP_PREFILL: j->rc = gg_prefill(j->ctx, j->ids, (int32_t)j->n, j->pos); break;
    case OP_SELECT: j->rc = gg_select(j->ctx, &j->s, j->u, &j->out); break;
    case OP_STEP: j->rc = gg_step(j->ctx, j->token, j->pos, &j->s, j->u, &j->out); break;
    case OP_COLLECT: j->rc = gg_step_collect(j->ctx, &j->out); break;
  }
  if (j->rc != GG_OK) {
    const char* m = gg_last_error(j->ctx);
    strncpy(j->err, m ? m : "", sizeof(j->err) - 1);
    j->err[sizeof(j->err) - 1] = 0;
  }
}

/* Runs on the JavaScript thread after job_execute. The handle is released
 * (and a deferred destroy carried out) before the promise settles, because
 * settling it may run the caller's continuation, which can start the next
 * call on the same context. */
static void job_complete(napi_env env, napi_status status, void* data) {
  job_t* j = (job_t*)data;
  handle_t* h = j->h;
  h->busy = 0;
  if (h->destroy_pending && h->ctx) {
    gg_destroy(h->ctx);
    h->ctx = NULL;
  }
  if (h->orphaned) free(h);
  napi_deferred d = j->deferred;
  napi_value v;
  int ok = 0;
  if (status != napi_ok) {
    v = make_error(env, GG_ERR_INVALID, "job cancelled");
  } else if (j->rc != GG_OK) {
    v = make_error(env, j->rc, j->err);
  } else {
    ok = 1;
    if (j->op == OP_PREFILL) napi_get_undefined(env, &v);
    else napi_create_int32(env, j->out, &v);
  }
  napi_delete_async_work(env, j->work);
  free(j->ids);
  free(j);
  if (ok) napi_resolve_deferred(env, d, v);
  else napi_reject_deferred(env, d, v);
}

/* Queues job j on handle h (live and idle, checked by get_handle) and marks
 * h busy until job_complete runs. */
static napi_value queue_job(napi_env env, handle_t* h, job_t* j) {
  napi_value promise, name;
  j->h = h;
  j->ctx = h->ctx;
  j->work = NULL;
  if (napi_create_promise(env, &j->deferred, &promise) != napi_ok ||
      napi_create_string_utf8(env, "gg", NAPI_AUTO_LENGTH, &name) != napi_ok ||
      napi_create_async_work(env, NULL, name, job_execute, job_complete, j, &j->work) != napi_ok ||
      napi_queue_async_work(env, j->work) != napi_ok) {
    if (j->work) napi_delete_async_work(env, j->work);
    free(j->ids);
    free(j);
    napi_throw_error(env, "GG_ERR_NAPI", "could not queue the call");
    return NULL;
  }
  h->busy = 1;
  return promise;
}

static int read_sample(napi_env env, napi_value* argv, job_t* j) {
  return napi_get_value_double(env, argv[0], &j->s.temperature) == napi_ok &&
         napi_get_value_double(env, argv[1], &j->s.top_p) == napi_ok &&
         napi_get_value_double(env, argv[2], &j->s.rep_penalty) == napi_ok &&
         napi_get_value_double(env, argv[3], &j->u) == napi_ok;
}

static napi_value Prefill(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  handle_t* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = (job_t*)calloc(1, sizeof(job_t));
  if (!j) {
    napi_throw_error(env, "GG_ERR_OOM", "host allocation failed");
    return NULL;
  }
  j->op = OP_PREFILL;
  j->ids = copy_ids(env, argv[1], &j->n);
  if (!j->ids || napi_get_value_int32(env, argv[2], &j->pos) != napi_ok) {
    free(j->ids);
    free(j);
    return NULL;
  }
  return queue_job(env, h, j);
}

static napi_value Select(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  handle_t* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = (job_t*)calloc(1, sizeof(job_t));
  if (!j) {
    napi_throw_error(env, "GG_ERR_OOM", "host allocation failed");
    return NULL;
  }
  j->op = OP_SELECT;
  if (!read_sample(env, argv + 1, j)) {
    free(j);
    napi_throw_type_error(env, "GG_ERR_INVALID", "sampling options must be numbers");
    return NULL;
  }
  return queue_job(env, h, j);
}

static napi_value Step(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!get_args(env, info, 7, argv)) return NULL;
  handle_t* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = (job_t*)calloc(1, sizeof(job_t));
  if (!j) {
    napi_throw_error(env, "GG_ERR_OOM", "host allocation failed");
    return NULL;
  }
  j->op = OP_STEP;
  if (napi_get_value_int32(env, argv[1], &j->token) != napi_ok || napi_get_value_int32(env, argv[2], &j->pos) != napi_ok ||
      !read_sample(env, argv + 3, j)) {
    free(j);
    napi_throw_type_error(env, "GG_ERR_INVALID", "step arguments must be numbers");
    return NULL;
  }
  return queue_job(env, h, j);
}

static napi_value StepCollect(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle_t* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = (job_t*)calloc(1, sizeof(job_t));
  if (!j) {
    napi_throw_error(env, "GG_ERR_OOM", "host allocation failed");
    return NULL;
  }
  j->op = OP_COLLECT;
  return queue_job(env, h, j);
}

static napi_value Init(napi_env env, napi_value exports) {
  struct {
    const char* name;
    napi_callback cb;
  } fns[] = {{"create", Create},   {"upload", Upload},         {"finalize", Finalize}, {"prefill", Prefill},
             {"select", Select},   {"step", Step},             {"stepSubmit", StepSubmit},
             {"stepCollect", StepCollect}, {"decodePath", DecodePath}, {"penaltyReset", PenaltyReset},
             {"penaltyAdd", PenaltyAdd}, {"resetKV", ResetKV}, {"read", Read},         {"destroy", Destroy}};
  for (size_t i = 0; i < sizeof(fns) / sizeof(fns[0]); ++i) {
    napi_value f;
    CHECK(env, napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].cb, NULL, &f));
    CHECK(env, napi_set_named_property(env, exports, fns[i].name, f));
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)

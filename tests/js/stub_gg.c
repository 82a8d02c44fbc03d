/* stub_gg.c -- a CPU stand-in for libgg.so that exercises the Node-API
 * binding's context lifetime without a GPU. gg_prefill/gg_select/gg_step sleep
 * so JavaScript can call destroy() or start a second job while one runs. Each
 * context carries a magic word that gg_destroy overwrites (the memory is then
 * freed, so an AddressSanitizer build of the binding also sees any later
 * access); every call checks the word on entry and again after its sleep and
 * aborts with "USE AFTER DESTROY" when it changed, and aborts with
 * "CONCURRENT CALL" when two calls overlap on one context. Events go to stderr
 * as "stub: <event> <context id>" lines for the test to check their order. */
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "gg.h"

#define LIVE 0x6767c0deu
#define DEAD 0xdeadbeefu

struct gg_ctx {
  volatile uint32_t magic;
  int id;
  int in_call;
};

static int g_next_id = 1;

static void note(const char* what, const gg_ctx* c) {
  fprintf(stderr, "stub: %s %d\n", what, c->id);
  fflush(stderr);
}

static void enter(gg_ctx* c, const char* what) {
  if (c->magic != LIVE) {
    fprintf(stderr, "USE AFTER DESTROY in %s\n", what);
    abort();
  }
  if (__atomic_fetch_add(&c->in_call, 1, __ATOMIC_SEQ_CST) != 0) {
    fprintf(stderr, "CONCURRENT CALL in %s\n", what);
    abort();
  }
  note(what, c);
}

static void leave(gg_ctx* c, const char* what, int sleep_ms) {
  struct timespec ts = {sleep_ms / 1000, (long)(sleep_ms % 1000) * 1000000L};
  nanosleep(&ts, NULL);
  if (c->magic != LIVE) {
    fprintf(stderr, "USE AFTER DESTROY in %s\n", what);
    abort();
  }
  char buf[64];
  snprintf(buf, sizeof(buf), "%s-end", what);
  note(buf, c);
  __atomic_fetch_sub(&c->in_call, 1, __ATOMIC_SEQ_CST);
}

gg_ctx* gg_create(const gg_config* cfg) {
  (void)cfg;
  gg_ctx* c = (gg_ctx*)calloc(1, sizeof(gg_ctx));
  c->magic = LIVE;
  c->id = g_next_id++;
  note("create", c);
  return c;
}

void gg_destroy(gg_ctx* c) {
  if (!c) return;
  if (c->magic != LIVE) {
    fprintf(stderr, "USE AFTER DESTROY in gg_destroy (double destroy)\n");
    abort();
  }
  if (c->in_call) {
    fprintf(stderr, "USE AFTER DESTROY: gg_destroy while a call runs\n");
    abort();
  }
  note("destroy", c);
  c->magic = DEAD;
  free(c);
}

const char* gg_last_error(const gg_ctx* c) {
  (void)c;
  return "stub error";
}

int gg_upload_tensor(gg_ctx* c, const char* name, uint32_t type, const uint64_t* dims, uint32_t ndims,
                     const void* data, size_t nbytes) {
  (void)name, (void)type, (void)dims, (void)ndims, (void)data, (void)nbytes;
  enter(c, "upload");
  leave(c, "upload", 0);
  return GG_OK;
}

int gg_finalize(gg_ctx* c) {
  enter(c, "finalize");
  leave(c, "finalize", 0);
  return GG_OK;
}

int gg_penalty_reset(gg_ctx* c) {
  enter(c, "penalty_reset");
  leave(c, "penalty_reset", 0);
  return GG_OK;
}

int gg_penalty_add(gg_ctx* c, const int32_t* ids, int32_t n) {
  (void)ids, (void)n;
  enter(c, "penalty_add");
  leave(c, "penalty_add", 0);
  return GG_OK;
}

int gg_reset_kv(gg_ctx* c) {
  enter(c, "reset_kv");
  leave(c, "reset_kv", 0);
  return GG_OK;
}

int gg_read(gg_ctx* c, int32_t what, int32_t layer, void* dst, size_t nbytes) {
  (void)what, (void)layer;
  enter(c, "read");
  memset(dst, 0, nbytes);
  leave(c, "read", 0);
  return GG_OK;
}

int gg_prefill(gg_ctx* c, const int32_t* ids, int32_t n, int32_t start_pos) {
  (void)ids, (void)n, (void)start_pos;
  enter(c, "prefill");
  leave(c, "prefill", 150);
  return GG_OK;
}

int gg_select(gg_ctx* c, const gg_sample* s, double u, int32_t* out) {
  (void)s, (void)u;
  enter(c, "select");
  leave(c, "select", 150);
  *out = 7;
  return GG_OK;
}

int gg_step(gg_ctx* c, int32_t token, int32_t pos, const gg_sample* s, double u, int32_t* out) {
  (void)pos, (void)s, (void)u;
  enter(c, "step");
  leave(c, "step", 300);
  *out = token + 1;
  return GG_OK;
}

/* pipelined steps: submit records the id, collect sleeps like a step */
static int32_t g_pending = -1;
int gg_step_submit(gg_ctx* c, int32_t token, int32_t pos, const gg_sample* s, double u) {
  (void)pos, (void)s, (void)u;
  enter(c, "step_submit");
  leave(c, "step_submit", 0);
  g_pending = token < 0 ? g_pending + 1 : token + 1;
  return GG_OK;
}

int gg_step_collect(gg_ctx* c, int32_t* out) {
  enter(c, "step_collect");
  leave(c, "step_collect", 300);
  *out = g_pending;
  return GG_OK;
}

/* the stub queues its steps like the persistent decode kernel */
int gg_decode_path(gg_ctx* c) { return c ? GG_DECODE_FUSED : GG_ERR_INVALID; }

// libana's effects for Bend: the handlers behind bend/AnaIo.bend.
//
// Bend's runtime compiles this file as it compiles the reference's
// effs/bulk.c (/root/reference/bend/effs/bulk.c), so the runtime's own
// types and calls are in scope here: Env, Term, IoWork, u32, u64, u32a,
// f32, io_eff, CID, io_cbuf, io_tup, err_fail, f32_unbox and the block
// accessors blk_ptr, blk_loc, blk_cls. Only those are used, each the way
// bulk.c uses it (io_cbuf's four arguments as at bulk.c:2502, a handler's
// registration as at bulk.c:2590-2592, a cell's address as at bulk.c:41-43).
// Bend is not installed where this file was written, so it has not been
// compiled.
//
// libana is opened with dlopen at the first call, as bulk.c opens cuBLAS
// (bulk.c:124-166): ANA_LIB names the library (default "libana.so"),
// ANA_DEVICE the HIP device (default 0). The build needs only
// include/ana.h, for the plain C types of the interface.

#include <dlfcn.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/ana.h"

enum { AN_MAX = 16 };   // contexts open at once

static struct {
  int loaded;
  int (*open)(const char*, const ana_opts*, struct ana_ctx**);
  int (*config_of)(const struct ana_ctx*, ana_config*, uint64_t*);
  int (*reset)(struct ana_ctx*, uint32_t);
  int (*feed)(struct ana_ctx*, uint32_t, const uint32_t*, const uint32_t*, const uint32_t*);
  int (*feeds)(struct ana_ctx*, uint32_t, uint32_t, const uint32_t*, uint32_t);
  int (*logits)(struct ana_ctx*, uint32_t, const uint32_t*, float*);
  int (*top)(struct ana_ctx*, uint32_t, const uint32_t*, uint32_t*);
  int (*pick)(struct ana_ctx*, uint32_t, const uint32_t*, const ana_sampling*, uint64_t*, uint32_t*);
  int (*score_n)(struct ana_ctx*, uint32_t, const uint32_t*, const uint32_t*, const uint32_t*,
                 const uint32_t*, float*);
  const char* (*error)(const struct ana_ctx*);
  struct ana_ctx* ctx[AN_MAX];
  uint32_t vocab[AN_MAX];
} AN;

// one call into the library at a time: a context is not safe to share
// between threads, and the effects of one program may run on several
static pthread_mutex_t an_mu = PTHREAD_MUTEX_INITIALIZER;

static void an_die(const char* what) {
  static char msg[512];
  snprintf(msg, sizeof msg, "ana: %s", what ? what : "unknown error");
  pthread_mutex_unlock(&an_mu);
  err_fail(msg);
}

static void* an_sym(void* lib, const char* name) {
  void* p = dlsym(lib, name);
  if (p == NULL) {
    an_die(name);
  }
  return p;
}

// (called with an_mu held)
static void an_load(void) {
  if (AN.loaded) {
    return;
  }
  const char* so = getenv("ANA_LIB");
  void* lib = dlopen(so != NULL ? so : "libana.so", RTLD_NOW | RTLD_LOCAL);
  if (lib == NULL) {
    an_die(dlerror());
  }
  AN.open = (int (*)(const char*, const ana_opts*, struct ana_ctx**))an_sym(lib, "ana_open");
  AN.config_of = (int (*)(const struct ana_ctx*, ana_config*, uint64_t*))an_sym(lib, "ana_config_of");
  AN.reset = (int (*)(struct ana_ctx*, uint32_t))an_sym(lib, "ana_reset");
  AN.feed = (int (*)(struct ana_ctx*, uint32_t, const uint32_t*, const uint32_t*, const uint32_t*))
    an_sym(lib, "ana_feed");
  AN.feeds = (int (*)(struct ana_ctx*, uint32_t, uint32_t, const uint32_t*, uint32_t))an_sym(lib, "ana_feeds");
  AN.logits = (int (*)(struct ana_ctx*, uint32_t, const uint32_t*, float*))an_sym(lib, "ana_logits");
  AN.top = (int (*)(struct ana_ctx*, uint32_t, const uint32_t*, uint32_t*))an_sym(lib, "ana_top");
  AN.pick = (int (*)(struct ana_ctx*, uint32_t, const uint32_t*, const ana_sampling*, uint64_t*, uint32_t*))
    an_sym(lib, "ana_pick");
  AN.score_n = (int (*)(struct ana_ctx*, uint32_t, const uint32_t*, const uint32_t*, const uint32_t*,
                        const uint32_t*, float*))an_sym(lib, "ana_score_n");
  AN.error = (const char* (*)(const struct ana_ctx*))an_sym(lib, "ana_error");
  AN.loaded = 1;
}

// the context a handle names (called with an_mu held)
static struct ana_ctx* an_ctx(Term h) {
  u32 i = (u32)h;
  if (i >= AN_MAX || AN.ctx[i] == NULL) {
    an_die("no open context has that handle");
  }
  return AN.ctx[i];
}

// a failed call ends the program with the library's own message (the
// reference's wording where it has one: "checkpoint: short read", ...)
static void an_check(struct ana_ctx* c, int rc) {
  if (rc != 0) {
    an_die(AN.error(c));
  }
}

// cell i of an Array<F32> block (indices wrap, as Array.set's do): the
// runtime's block address, as bulk.c's ft_cell forms it
static u32a* an_cell(Env e, Term a, u32 i) {
  return blk_ptr(e.mem, blk_loc(e.mem, a), i & (u32)((1ull << blk_cls(a)) - 1));
}

static f32 an_get(Env e, Term a, u32 i) {
  return f32_unbox((u64)*an_cell(e, a, i));
}

static void an_put(Env e, Term a, u32 i, float v) {
  u32 b;
  memcpy(&b, &v, 4);
  *an_cell(e, a, i) = b;
}

// n ids held as F32 values in cells at .. at + n (a malloc'd copy; called
// without an_mu)
static uint32_t* an_ids(Env e, Term a, u32 at, u32 n) {
  uint32_t* t = (uint32_t*)malloc(4 * (size_t)(n ? n : 1));
  if (t == NULL) {
    err_fail("ana: out of host memory");
  }
  for (u32 i = 0; i < n; i += 1) {
    t[i] = (uint32_t)an_get(e, a, at + i);
  }
  return t;
}

#ifdef CID(ana.open)
Term ana_open_run(Env e, Term* f, IoWork* w) {
  (void)w;
  u64 n = 0;
  char* t = io_cbuf(e, f[0], &n, CID(SCon));
  char* path = (char*)malloc((size_t)n + 1);
  if (path == NULL) {
    err_fail("ana: out of host memory");
  }
  memcpy(path, t, (size_t)n);
  path[n] = 0;
  free(t);
  ana_opts o;
  const char* dev = getenv("ANA_DEVICE");
  o.device = dev != NULL ? atoi(dev) : 0;
  o.numerics = (int)(u32)f[1];
  o.max_seqs = (u32)f[2];
  o.prefill_chunk = (u32)f[3];
  pthread_mutex_lock(&an_mu);
  an_load();
  u32 s = 0;
  while (s < AN_MAX && AN.ctx[s] != NULL) {
    s += 1;
  }
  if (s == AN_MAX) {
    an_die("too many open contexts");
  }
  struct ana_ctx* c = NULL;
  if (AN.open(path, &o, &c) != 0) {
    an_die(AN.error(NULL));
  }
  ana_config k;
  an_check(c, AN.config_of(c, &k, NULL));
  AN.ctx[s] = c;
  AN.vocab[s] = k.vocab;
  pthread_mutex_unlock(&an_mu);
  free(path);
  return (Term)s;
}
static void __attribute__((constructor)) ana_open_use(void) {
  io_eff(CID(ana.open), ana_open_run);
}
#endif

#ifdef CID(ana.step)
Term ana_step_run(Env e, Term* f, IoWork* w) {
  (void)e;
  (void)w;
  ana_config k;
  uint64_t step = 0;
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.config_of(c, &k, &step));
  pthread_mutex_unlock(&an_mu);
  return (Term)(u32)step;
}
static void __attribute__((constructor)) ana_step_use(void) {
  io_eff(CID(ana.step), ana_step_run);
}
#endif

#ifdef CID(ana.reset)
Term ana_reset_run(Env e, Term* f, IoWork* w) {
  (void)e;
  (void)w;
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.reset(c, (u32)f[1]));
  pthread_mutex_unlock(&an_mu);
  return (Term)0;
}
static void __attribute__((constructor)) ana_reset_use(void) {
  io_eff(CID(ana.reset), ana_reset_run);
}
#endif

#ifdef CID(ana.feed)
Term ana_feed_run(Env e, Term* f, IoWork* w) {
  (void)e;
  (void)w;
  uint32_t seq = (u32)f[1], pos = (u32)f[2], tok = (u32)f[3];
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.feed(c, 1, &seq, &pos, &tok));
  pthread_mutex_unlock(&an_mu);
  return (Term)0;
}
static void __attribute__((constructor)) ana_feed_use(void) {
  io_eff(CID(ana.feed), ana_feed_run);
}
#endif

#ifdef CID(ana.feeds)
Term ana_feeds_run(Env e, Term* f, IoWork* w) {
  (void)w;
  u32 n = (u32)f[5];
  uint32_t* ids = an_ids(e, f[3], (u32)f[4], n);
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.feeds(c, (u32)f[1], (u32)f[2], ids, n));
  pthread_mutex_unlock(&an_mu);
  free(ids);
  return f[3];
}
static void __attribute__((constructor)) ana_feeds_use(void) {
  io_eff(CID(ana.feeds), ana_feeds_run);
}
#endif

#ifdef CID(ana.logits)
Term ana_logits_run(Env e, Term* f, IoWork* w) {
  (void)w;
  uint32_t seq = (u32)f[1];
  u32 at = (u32)f[3];
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  u32 v = AN.vocab[(u32)f[0]];
  float* lg = (float*)malloc(4 * (size_t)v);
  if (lg == NULL) {
    an_die("out of host memory");
  }
  an_check(c, AN.logits(c, 1, &seq, lg));
  pthread_mutex_unlock(&an_mu);
  for (u32 i = 0; i < v; i += 1) {
    an_put(e, f[2], at + i, lg[i]);
  }
  free(lg);
  return f[2];
}
static void __attribute__((constructor)) ana_logits_use(void) {
  io_eff(CID(ana.logits), ana_logits_run);
}
#endif

#ifdef CID(ana.top)
Term ana_top_run(Env e, Term* f, IoWork* w) {
  (void)e;
  (void)w;
  uint32_t seq = (u32)f[1], tok = 0;
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.top(c, 1, &seq, &tok));
  pthread_mutex_unlock(&an_mu);
  return (Term)tok;
}
static void __attribute__((constructor)) ana_top_use(void) {
  io_eff(CID(ana.top), ana_top_run);
}
#endif

#ifdef CID(ana.pick)
// the Rng's words from 8 cells: cell at + 2 i holds the high half of word
// i and cell at + 2 i + 1 its low half, each as F32 bits (N.U64{hi, lo})
Term ana_pick_run(Env e, Term* f, IoWork* w) {
  (void)w;
  uint32_t seq = (u32)f[1], tok = 0;
  u32 at = (u32)f[6];
  ana_sampling s;
  s.temperature = f32_unbox((u64)f[2]);
  s.top_k = (u32)f[3];
  s.top_p = f32_unbox((u64)f[4]);
  uint64_t rng[4];
  for (u32 i = 0; i < 4; i += 1) {
    uint64_t hi = (u32)*an_cell(e, f[5], at + 2 * i);
    uint64_t lo = (u32)*an_cell(e, f[5], at + 2 * i + 1);
    rng[i] = (hi << 32) | lo;
  }
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.pick(c, 1, &seq, &s, rng, &tok));
  pthread_mutex_unlock(&an_mu);
  for (u32 i = 0; i < 4; i += 1) {
    *an_cell(e, f[5], at + 2 * i) = (u32)(rng[i] >> 32);
    *an_cell(e, f[5], at + 2 * i + 1) = (u32)rng[i];
  }
  return io_tup(e, (Term)tok, f[5]);
}
static void __attribute__((constructor)) ana_pick_use(void) {
  io_eff(CID(ana.pick), ana_pick_run);
}
#endif

#ifdef CID(ana.score)
// window.go over one window of n ids in cells at .. at + n: n - 1 summands
// G.lse(logits) - logits[next id], written over cells at .. at + n - 1
Term ana_score_run(Env e, Term* f, IoWork* w) {
  (void)w;
  u32 n = (u32)f[5], at = (u32)f[4];
  if (n < 2) {
    return f[3];
  }
  uint32_t* ids = an_ids(e, f[3], at, n);
  float* ce = (float*)malloc(4 * (size_t)(n - 1));
  if (ce == NULL) {
    err_fail("ana: out of host memory");
  }
  uint32_t seq = (u32)f[1], pos = (u32)f[2], len = n;
  pthread_mutex_lock(&an_mu);
  struct ana_ctx* c = an_ctx(f[0]);
  an_check(c, AN.score_n(c, 1, &seq, &pos, &len, ids, ce));
  pthread_mutex_unlock(&an_mu);
  for (u32 i = 0; i + 1 < n; i += 1) {
    an_put(e, f[3], at + i, ce[i]);
  }
  free(ce);
  free(ids);
  return f[3];
}
static void __attribute__((constructor)) ana_score_use(void) {
  io_eff(CID(ana.score), ana_score_run);
}
#endif

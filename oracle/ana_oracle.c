/*
 * ana_oracle -- TEST INFRASTRUCTURE ONLY (see ana_oracle.h for scope and
 * for how each part is pinned). A CPU restatement of ana's dense decoder
 * (bend/Dense/Decode.bend over bend/effs/bulk.c's CPU numerics), of its tree
 * meaning (bend/Model.bend) and of its sampler (bend/Sample.bend).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -mavx2, no -mfma).
 */
#define _GNU_SOURCE
#include "ana_oracle.h"

#include <errno.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define OR_AVX2 1
#else
#define OR_AVX2 0
#endif

/* ------------------------------------------------------------------------ */
/* F32 steps of the reference (bulk.c:1012-1040: libm through double)        */

static inline float f32exp(float x) { return (float)exp((double)x); }
static inline float f32log(float x) { return (float)log((double)x); }
static inline float f32sqrt(float x) { return (float)sqrt((double)x); }
static inline float fabs32(float x) { return (float)fabs((double)x); }
/* Ex.max / Ex.min of bend/Dense/Ex.bend:126-131: max a b = (a < b ? b : a) */
static inline float exmax(float a, float b) { return a < b ? b : a; }
static inline float exmin(float a, float b) { return a < b ? a : b; }

/* sigmoid as a select (bend/Dense/Ex.bend:148-150) */
static float ex_sigmoid(float z) {
  if (0.0f <= z) return 1.0f / (1.0f + f32exp(-z));
  float e = f32exp(z);
  return e / (1.0f + e);
}
static float ex_silu(float z) { return z * ex_sigmoid(z); }
/* log1p with Goldberg's trick (bend/Dense/Ex.bend:141-143) */
static float ex_log1p(float u) {
  float w = 1.0f + u;
  float eq = (w <= 1.0f ? 1.0f : 0.0f) * (1.0f <= w ? 1.0f : 0.0f);
  if (eq != 0.0f) return u;
  return (f32log(w) * u) / (w - 1.0f);
}
/* bend/Dense/Ex.bend:145-146 */
static float ex_log_sigmoid(float z) {
  return -(exmax(-z, 0.0f) + ex_log1p(f32exp(-fabs32(z))));
}
#define OR_CAP (-1.0e-4f)
/* bend/Dense/Ex.bend:158-162 */
static float ex_rglru_log_gate(float z, float lam) {
  return exmin(OR_CAP, (8.0f * ex_sigmoid(z)) * ex_log_sigmoid(lam));
}
static float ex_rglru_write_scale(float la) {
  return f32sqrt(1.0f - f32exp(2.0f * exmin(OR_CAP, la)));
}
/* rms_scale (bend/Dense/Ex.bend:165-166) */
static float ex_rms_scale(float ss, float n) {
  return 1.0f / f32sqrt((ss / n) + 1.0e-5f);
}

/* ------------------------------------------------------------------------ */
/* Config and layout (bend/Config.bend:213-253, bend/Dense/Layout.bend:627-686) */

static int is_softmax(uint32_t i) { return i % 4 == 3; }

uint64_t or_params(const or_config* c) {
  uint64_t d = c->d, f = c->f, v = c->vocab, L = c->layers, h = c->heads;
  uint64_t hd = c->heads ? d / h : 0;
  uint64_t sm = L / 4, gla = L - sm;
  uint64_t p = v * d + L * (4 * d * d + 3 * f * d + 2 * d) + gla * d * d;
  if (c->rglru) p += gla * d;
  if (c->qk) p += sm * 2 * hd;
  if (c->sinks) p += sm * h;
  p += d;
  if (!c->tied) p += v * d;
  return p;
}

size_t or_model_id(const or_config* c, char* buf, size_t cap) {
  int n = snprintf(buf, cap,
    "formal-transformer-futhark-hybrid-gla-v3:Config {vocabSize = %u, contextSize = %u, "
    "modelDim = %u, ffDim = %u, layerCount = %u, headCount = %u, gateKind = %s, "
    "qkNorm = %s, headSinks = %s, tiedHead = %s}",
    c->vocab, c->ctx, c->d, c->f, c->layers, c->heads, c->rglru ? "GateRgLru" : "GateSigmoid",
    c->qk ? "True" : "False", c->sinks ? "True" : "False", c->tied ? "True" : "False");
  return n < 0 ? 0 : (size_t)n;
}

typedef struct {
  int gla;
  uint64_t ra, wq, wk, wv, wo, wa, lam, gq, gk, sink, rf, wg, wu, wd, size;
} blk;

static void layout(const or_config* c, blk* b, uint64_t* fin) {
  uint64_t d = c->d, f = c->f, dd = d * d, hd = d / c->heads;
  uint64_t o = (uint64_t)c->vocab * d;
  for (uint32_t i = 0; i < c->layers; i++) {
    blk* x = &b[i];
    memset(x, 0, sizeof *x);
    x->gla = !is_softmax(i);
    x->ra = o;
    uint64_t q = o + d;
    x->wq = q; x->wk = q + dd; x->wv = q + 2 * dd; x->wo = q + 3 * dd;
    if (x->gla) {
      x->wa = q + 4 * dd;
      x->lam = q + 5 * dd;
      x->rf = x->lam + (c->rglru ? d : 0);
    } else {
      x->gq = q + 4 * dd;
      x->gk = x->gq + (c->qk ? hd : 0);
      x->sink = x->gk + (c->qk ? hd : 0);
      x->rf = x->sink + (c->sinks ? c->heads : 0);
    }
    x->wg = x->rf + d;
    x->wu = x->wg + f * d;
    x->wd = x->wg + 2 * f * d;
    x->size = x->wd + d * f - o;
    o += x->size;
  }
  *fin = o;
}

/* ------------------------------------------------------------------------ */
/* Thread pool for the matrix products: threads are distinct outputs, so the
 * bits do not depend on the thread count (bulk.c:196-208).                   */

typedef void (*or_job)(void* arg, int lo, int hi);
static struct {
  int n;                    /* worker threads beside the caller */
  pthread_t th[64];
  pthread_barrier_t start, done;
  or_job fn;
  void* arg;
  int rows, quit;
} P = {0};
static int g_threads = 1;

static void* pool_main(void* a) {
  int id = (int)(intptr_t)a;
  for (;;) {
    pthread_barrier_wait(&P.start);
    if (P.quit) return NULL;
    int t = P.n + 1, per = (P.rows + t - 1) / t;
    int lo = per * id, hi = lo + per > P.rows ? P.rows : lo + per;
    if (lo < hi) P.fn(P.arg, lo, hi);
    pthread_barrier_wait(&P.done);
  }
}

static void pool_stop(void) {
  if (P.n == 0) return;
  P.quit = 1;
  pthread_barrier_wait(&P.start);
  for (int i = 0; i < P.n; i++) pthread_join(P.th[i], NULL);
  pthread_barrier_destroy(&P.start);
  pthread_barrier_destroy(&P.done);
  P.n = 0;
  P.quit = 0;
}

void or_set_threads(int n) {
  if (n < 1) n = 1;
  if (n > 64) n = 64;
  pool_stop();
  g_threads = n;
  if (n == 1) return;
  P.n = n - 1;
  pthread_barrier_init(&P.start, NULL, (unsigned)n);
  pthread_barrier_init(&P.done, NULL, (unsigned)n);
  for (int i = 0; i < P.n; i++) pthread_create(&P.th[i], NULL, pool_main, (void*)(intptr_t)(i + 1));
}

static void par_for(or_job fn, void* arg, int rows) {
  if (g_threads == 1 || rows < 64) { fn(arg, 0, rows); return; }
  P.fn = fn; P.arg = arg; P.rows = rows;
  pthread_barrier_wait(&P.start);
  int t = P.n + 1, per = (rows + t - 1) / t;
  if (per > rows) per = rows;
  fn(arg, 0, per);
  pthread_barrier_wait(&P.done);
}

/* ------------------------------------------------------------------------ */
/* Model: parameters, plus 8-row panels of every matrix for the AVX2 product
 * (panel p holds rows 8p..8p+7 k-major: W[8p+r][q] at p*8K + 8q + r).       */

struct or_model {
  or_config c;
  uint64_t P, step, fin;
  blk* b;
  float* w;      /* P floats */
  float* pk;     /* panels, indexed by matrix offset map below */
  uint64_t* pk_off; /* per matrix: offset into pk; indexed through mat_id() */
  uint64_t pk_n;
};

/* matrices: 0 = embedding (head), then per layer: qkv(3d), wa, wo, gu(2f), wd */
enum { M_QKV, M_WA, M_WO, M_GU, M_WD, M_PER };

static uint64_t panels_of(uint64_t rows, uint64_t k) { return ((rows + 7) / 8) * 8 * k; }

static void pack(const float* W, uint64_t rows, uint64_t k, float* out) {
  for (uint64_t p = 0; p < (rows + 7) / 8; p++)
    for (uint64_t q = 0; q < k; q++)
      for (uint64_t r = 0; r < 8; r++) {
        uint64_t row = p * 8 + r;
        out[p * 8 * k + q * 8 + r] = row < rows ? W[row * k + q] : 0.0f;
      }
}

static void model_pack(or_model* m) {
  const or_config* c = &m->c;
  uint64_t d = c->d, f = c->f, v = c->vocab;
  uint64_t nm = 1 + (uint64_t)c->layers * M_PER;
  m->pk_off = calloc(nm, sizeof(uint64_t));
  uint64_t tot = panels_of(v, d);
  for (uint32_t l = 0; l < c->layers; l++) {
    tot += panels_of(3 * d, d) + (m->b[l].gla ? panels_of(d, d) : 0) + panels_of(d, d)
         + panels_of(2 * f, d) + panels_of(d, f);
  }
  m->pk = malloc(tot * sizeof(float));
  m->pk_n = tot;
  uint64_t o = 0;
  m->pk_off[0] = o; pack(m->w, v, d, m->pk + o); o += panels_of(v, d);
  for (uint32_t l = 0; l < c->layers; l++) {
    const blk* b = &m->b[l];
    uint64_t* po = &m->pk_off[1 + l * M_PER];
    po[M_QKV] = o; pack(m->w + b->wq, 3 * d, d, m->pk + o); o += panels_of(3 * d, d);
    if (b->gla) { po[M_WA] = o; pack(m->w + b->wa, d, d, m->pk + o); o += panels_of(d, d); }
    po[M_WO] = o; pack(m->w + b->wo, d, d, m->pk + o); o += panels_of(d, d);
    po[M_GU] = o; pack(m->w + b->wg, 2 * f, d, m->pk + o); o += panels_of(2 * f, d);
    po[M_WD] = o; pack(m->w + b->wd, d, f, m->pk + o); o += panels_of(d, f);
  }
}

static or_model* model_new(const or_config* c, float* w, uint64_t step) {
  or_model* m = calloc(1, sizeof *m);
  m->c = *c;
  m->P = or_params(c);
  m->step = step;
  m->b = calloc(c->layers ? c->layers : 1, sizeof(blk));
  layout(c, m->b, &m->fin);
  m->w = w;
  model_pack(m);
  return m;
}

or_model* or_from_params(const or_config* c, const float* params) {
  uint64_t n = or_params(c);
  float* w = malloc(n * sizeof(float));
  memcpy(w, params, n * sizeof(float));
  return model_new(c, w, 0);
}

void or_model_free(or_model* m) {
  if (!m) return;
  free(m->w); free(m->pk); free(m->pk_off); free(m->b); free(m);
}
void or_model_config(const or_model* m, or_config* out) { *out = m->c; }
const float* or_model_params(const or_model* m) { return m->w; }
uint64_t or_model_step(const or_model* m) { return m->step; }

/* y[o] = sum_q x[q] * W[o][q], q ascending from 0.0f (bulk.c:49-71) */
typedef struct { const float* x; const float* pk; uint64_t k; float* y; uint64_t rows; } gemv_a;

static void gemv_job(void* a_, int lo, int hi) {
  gemv_a* a = a_;
  uint64_t k = a->k;
  for (int p = lo; p < hi; p++) {
    const float* pw = a->pk + (uint64_t)p * 8 * k;
    float out[8];
#if OR_AVX2
    __m256 s = _mm256_setzero_ps();
    for (uint64_t q = 0; q < k; q++) {
      __m256 t = _mm256_mul_ps(_mm256_set1_ps(a->x[q]), _mm256_loadu_ps(pw + q * 8));
      s = _mm256_add_ps(s, t);
    }
    _mm256_storeu_ps(out, s);
#else
    for (int r = 0; r < 8; r++) {
      float s = 0.0f;
      for (uint64_t q = 0; q < k; q++) s = s + a->x[q] * pw[q * 8 + r];
      out[r] = s;
    }
#endif
    for (int r = 0; r < 8; r++) {
      uint64_t row = (uint64_t)p * 8 + r;
      if (row < a->rows) a->y[row] = out[r];
    }
  }
}

static void gemv(const float* x, const float* pk, uint64_t rows, uint64_t k, float* y) {
  gemv_a a = {x, pk, k, y, rows};
  par_for(gemv_job, &a, (int)((rows + 7) / 8));
}

/* ------------------------------------------------------------------------ */
/* FTC2 (bend/Checkpoint.bend, bend/Dense/Ckpt.bend:12-110)                  */

typedef struct { const uint8_t* p; size_t n, at; int bad; } cur;

static uint64_t rd_be(cur* c, int k) {
  if (c->at + (size_t)k > c->n) { c->bad = 1; return 0; }
  uint64_t v = 0;
  for (int i = 0; i < k; i++) v = (v << 8) | c->p[c->at + i];
  c->at += (size_t)k;
  return v;
}
/* Load.nat: an Int64's low word */
static uint32_t rd_nat(cur* c) { return (uint32_t)rd_be(c, 8); }
/* Load.string: Int64 character count, then UTF-8 characters */
static void rd_string(cur* c, char* out, size_t cap) {
  uint32_t n = rd_nat(c);
  size_t o = 0;
  for (uint32_t i = 0; i < n && !c->bad; i++) {
    uint32_t b = (uint32_t)rd_be(c, 1);
    int extra = b < 128 ? 0 : b < 224 ? 1 : b < 240 ? 2 : 3;
    if (o + 1 < cap) out[o++] = (char)b;
    for (int j = 0; j < extra; j++) {
      uint32_t x = (uint32_t)rd_be(c, 1);
      if (o + 1 < cap) out[o++] = (char)x;
    }
  }
  if (cap) out[o < cap ? o : cap - 1] = 0;
}
/* Load.double: Integer then Int64 (the value is not needed, only skipped) */
static void rd_double(cur* c) {
  uint32_t tag = (uint32_t)rd_be(c, 1);
  if (tag == 0) rd_be(c, 4);
  else { rd_be(c, 1); uint32_t n = rd_nat(c); for (uint32_t i = 0; i < n && !c->bad; i++) rd_be(c, 1); }
  rd_be(c, 8);
}

static void set_err(char* err, size_t cap, const char* msg) {
  if (err && cap) snprintf(err, cap, "%s", msg);
}

or_model* or_open(const char* path, char* err, size_t errcap) {
  FILE* fp = fopen(path, "rb");
  if (!fp) { set_err(err, errcap, strerror(errno)); return NULL; }
  fseek(fp, 0, SEEK_END);
  long sz = ftell(fp);
  fseek(fp, 0, SEEK_SET);
  uint8_t* buf = malloc((size_t)sz > 0 ? (size_t)sz : 1);
  if (fread(buf, 1, (size_t)sz, fp) != (size_t)sz) { fclose(fp); free(buf); set_err(err, errcap, "checkpoint: short read"); return NULL; }
  fclose(fp);
  cur c = {buf, (size_t)sz, 0, 0};
  if ((uint32_t)rd_be(&c, 4) != 1179927346u || c.bad) {
    free(buf); set_err(err, errcap, "not a compact checkpoint (magic is not FTC2)"); return NULL;
  }
  uint32_t version = (uint32_t)rd_be(&c, 4);
  or_config cf;
  cf.vocab = rd_nat(&c); cf.ctx = rd_nat(&c); cf.d = rd_nat(&c); cf.f = rd_nat(&c);
  cf.layers = rd_nat(&c); cf.heads = rd_nat(&c);
  cf.rglru = rd_be(&c, 1) != 0; cf.qk = rd_be(&c, 1) != 0; cf.sinks = rd_be(&c, 1) != 0; cf.tied = rd_be(&c, 1) != 0;
  uint32_t count = rd_nat(&c);
  char lay[256], mid[1024], tid[1024], did[1024];
  rd_string(&c, lay, sizeof lay);
  uint32_t lv = (uint32_t)rd_be(&c, 4);
  for (int i = 0; i < 5; i++) rd_double(&c);
  rd_nat(&c); rd_nat(&c);
  if (rd_be(&c, 1)) rd_double(&c);
  rd_string(&c, mid, sizeof mid);
  rd_string(&c, tid, sizeof tid);
  rd_string(&c, did, sizeof did);
  rd_double(&c);
  rd_be(&c, 1);
  if (c.bad) { free(buf); set_err(err, errcap, "checkpoint: short read"); return NULL; }
  size_t h = c.at;
  char want[1024];
  or_model_id(&cf, want, sizeof want);
  const char* why = NULL;
  if (version != 4) why = "checkpoint: unsupported checkpoint manifest version (this branch reads version 4)";
  else if (strcmp(lay, "hybrid-gla-decoder-flat-parameters") != 0) why = "checkpoint: unsupported checkpoint model layout identity";
  else if (lv != 3) why = "checkpoint: unsupported checkpoint model layout version";
  else if ((uint64_t)count != or_params(&cf)) why = "checkpoint: manifest parameter count does not match config";
  else if (strcmp(mid, want) != 0) why = "checkpoint: checkpoint model identity is not supported by this host";
  else if (!cf.tied) why = "checkpoint: the dense decoder needs a tied head";
  if (why) { free(buf); set_err(err, errcap, why); return NULL; }
  uint64_t P = or_params(&cf);
  size_t par = h + 8, stp = par + 4 * P;
  if (stp + 16 > c.n) { free(buf); set_err(err, errcap, "checkpoint: short read"); return NULL; }
  c.at = h;
  uint32_t pc = (uint32_t)rd_be(&c, 8);
  if (pc != (uint32_t)P) { free(buf); set_err(err, errcap, "checkpoint: checkpoint parameter vector length is not the parameter count"); return NULL; }
  float* w = malloc(P * sizeof(float));
  for (uint64_t i = 0; i < P; i++) {
    const uint8_t* q = buf + par + 4 * i;
    uint32_t u = ((uint32_t)q[0] << 24) | ((uint32_t)q[1] << 16) | ((uint32_t)q[2] << 8) | q[3];
    memcpy(&w[i], &u, 4);
  }
  c.at = stp;
  uint64_t step = rd_be(&c, 8);
  free(buf);
  return model_new(&cf, w, (uint32_t)step);
}

/* ------------------------------------------------------------------------ */
/* The dense step (bend/Dense/Decode.bend dd.feed at n = 1)                   */

struct or_state {
  const or_model* m;
  float** lay;     /* per layer: GLA S [h][hd][hd] or K ring then V ring [2][ctx][d] */
  size_t* lay_n;
  float* x;        /* residual row */
  /* workspace */
  float *nrm, *qkv, *z, *qh, *kh0, *la, *kh, *al, *o, *oi, *y1, *xa, *nrm2, *gu, *hh, *y2, *s, *e;
  float *m1, *mm, *se, *den;
};

or_state* or_state_new(const or_model* m) {
  const or_config* c = &m->c;
  or_state* s = calloc(1, sizeof *s);
  s->m = m;
  uint32_t d = c->d, f = c->f, h = c->heads, hd = d / h;
  s->lay = calloc(c->layers, sizeof(float*));
  s->lay_n = calloc(c->layers, sizeof(size_t));
  for (uint32_t l = 0; l < c->layers; l++) {
    s->lay_n[l] = m->b[l].gla ? (size_t)h * hd * hd : (size_t)2 * c->ctx * d;
    s->lay[l] = calloc(s->lay_n[l], sizeof(float));
  }
  s->x = calloc(d, 4);
  s->nrm = calloc(d, 4); s->qkv = calloc(3 * d, 4); s->z = calloc(d, 4); s->qh = calloc(d, 4);
  s->kh0 = calloc(d, 4); s->la = calloc(d, 4); s->kh = calloc(d, 4); s->al = calloc(d, 4);
  s->o = calloc(d, 4); s->oi = calloc(d, 4); s->y1 = calloc(d, 4); s->xa = calloc(d, 4);
  s->nrm2 = calloc(d, 4); s->gu = calloc(2 * f, 4); s->hh = calloc(f, 4); s->y2 = calloc(d, 4);
  s->s = calloc((size_t)h * c->ctx, 4); s->e = calloc((size_t)h * c->ctx, 4);
  s->m1 = calloc(h, 4); s->mm = calloc(h, 4); s->se = calloc(h, 4); s->den = calloc(h, 4);
  return s;
}

/* a copy of s's states and residual row (workspace is scratch, not copied) */
or_state* or_state_clone(const or_state* s) {
  or_state* t = or_state_new(s->m);
  for (uint32_t l = 0; l < s->m->c.layers; l++) memcpy(t->lay[l], s->lay[l], s->lay_n[l] * sizeof(float));
  memcpy(t->x, s->x, (size_t)s->m->c.d * sizeof(float));
  return t;
}

void or_state_free(or_state* s) {
  if (!s) return;
  for (uint32_t l = 0; l < s->m->c.layers; l++) free(s->lay[l]);
  free(s->lay); free(s->lay_n); free(s->x);
  float* ws[] = {s->nrm, s->qkv, s->z, s->qh, s->kh0, s->la, s->kh, s->al, s->o, s->oi, s->y1, s->xa,
                 s->nrm2, s->gu, s->hh, s->y2, s->s, s->e, s->m1, s->mm, s->se, s->den};
  for (size_t i = 0; i < sizeof ws / sizeof ws[0]; i++) free(ws[i]);
  free(s);
}

void or_reset(or_state* s) {
  for (uint32_t l = 0; l < s->m->c.layers; l++) memset(s->lay[l], 0, s->lay_n[l] * sizeof(float));
}

const float* or_state_layer(const or_state* s, uint32_t layer, size_t* n) {
  if (layer >= s->m->c.layers) { if (n) *n = 0; return NULL; }
  if (n) *n = s->lay_n[layer];
  return s->lay[layer];
}
const float* or_state_x(const or_state* s) { return s->x; }

/* M.norm (bend/Dense/Model.bend:27-30): ss = sum x*x, then (x*scale)*g */
static void norm(uint32_t d, const float* x, const float* g, float* y) {
  float ss = 0.0f;
  for (uint32_t j = 0; j < d; j++) ss = ss + x[j] * x[j];
  float sc = ex_rms_scale(ss, (float)d);
  for (uint32_t j = 0; j < d; j++) y[j] = (x[j] * sc) * g[j];
}

/* M.tail (bend/Dense/Model.bend:48-60) */
static void tail(const or_model* m, or_state* s, uint32_t l) {
  const or_config* c = &m->c;
  const blk* b = &m->b[l];
  uint32_t d = c->d, f = c->f;
  const uint64_t* po = &m->pk_off[1 + l * M_PER];
  gemv(s->o, m->pk + po[M_WO], d, d, s->y1);
  for (uint32_t j = 0; j < d; j++) s->xa[j] = s->x[j] + s->y1[j];
  norm(d, s->xa, m->w + b->rf, s->nrm2);
  gemv(s->nrm2, m->pk + po[M_GU], 2 * f, d, s->gu);
  for (uint32_t j = 0; j < f; j++) s->hh[j] = ex_silu(s->gu[j]) * s->gu[f + j];
  gemv(s->hh, m->pk + po[M_WD], d, f, s->y2);
  for (uint32_t j = 0; j < d; j++) s->x[j] = s->xa[j] + s->y2[j];
}

/* dd.gla (bend/Dense/Decode.bend:242-292) */
static void gla_layer(const or_model* m, or_state* s, uint32_t l) {
  const or_config* c = &m->c;
  const blk* b = &m->b[l];
  uint32_t d = c->d, h = c->heads, hd = d / h;
  const uint64_t* po = &m->pk_off[1 + l * M_PER];
  norm(d, s->x, m->w + b->ra, s->nrm);
  gemv(s->nrm, m->pk + po[M_QKV], 3 * d, d, s->qkv);
  gemv(s->nrm, m->pk + po[M_WA], d, d, s->z);
  /* M.l2 (bend/Dense/Model.bend:33-36) on q then on k */
  for (int which = 0; which < 2; which++) {
    const float* src = s->qkv + which * d;
    float* y = which ? s->kh0 : s->qh;
    for (uint32_t hh = 0; hh < h; hh++) {
      float sq = 0.0f;
      for (uint32_t k = 0; k < hd; k++) sq = sq + src[hh * hd + k] * src[hh * hd + k];
      for (uint32_t k = 0; k < hd; k++) y[hh * hd + k] = src[hh * hd + k] / f32sqrt(1.0e-6f + sq);
    }
  }
  const float* key;
  if (c->rglru) {
    const float* lam = m->w + b->lam;
    for (uint32_t j = 0; j < d; j++) s->la[j] = ex_rglru_log_gate(s->z[j], lam[j]);
    for (uint32_t j = 0; j < d; j++) s->kh[j] = s->kh0[j] * ex_rglru_write_scale(s->la[j]);
    for (uint32_t j = 0; j < d; j++) s->al[j] = f32exp(s->la[j]);
    key = s->kh;
  } else {
    for (uint32_t j = 0; j < d; j++) s->al[j] = ex_sigmoid(s->z[j]);
    key = s->kh0;
  }
  /* dd.gla.tok: S' = al*S + kh*v in place, then o = qh^T S' */
  float* S = s->lay[l];
  const float* v = s->qkv + 2 * d;
  for (uint32_t hh = 0; hh < h; hh++)
    for (uint32_t a = 0; a < hd; a++)
      for (uint32_t bb = 0; bb < hd; bb++) {
        float* p = &S[(size_t)hh * hd * hd + a * hd + bb];
        *p = (s->al[hh * hd + a] * *p) + (key[hh * hd + a] * v[hh * hd + bb]);
      }
  for (uint32_t hh = 0; hh < h; hh++)
    for (uint32_t bb = 0; bb < hd; bb++) {
      float acc = 0.0f;
      for (uint32_t a = 0; a < hd; a++) acc = acc + s->qh[hh * hd + a] * S[(size_t)hh * hd * hd + a * hd + bb];
      s->o[hh * hd + bb] = acc;
    }
  tail(m, s, l);
}

/* dd.sm (bend/Dense/Decode.bend:294-353,422-437) */
static void sm_layer(const or_model* m, or_state* s, uint32_t l, uint32_t slot, uint32_t npos) {
  const or_config* c = &m->c;
  const blk* b = &m->b[l];
  uint32_t d = c->d, h = c->heads, hd = d / h, t = c->ctx;
  const uint64_t* po = &m->pk_off[1 + l * M_PER];
  norm(d, s->x, m->w + b->ra, s->nrm);
  gemv(s->nrm, m->pk + po[M_QKV], 3 * d, d, s->qkv);
  const float *qo = s->qkv, *ko = s->qkv + d, *v = s->qkv + 2 * d;
  if (c->qk) {
    /* M.qkn (bend/Dense/Model.bend:39-42) */
    for (int which = 0; which < 2; which++) {
      const float* src = s->qkv + which * d;
      const float* g = m->w + (which ? b->gk : b->gq);
      float* y = which ? s->kh0 : s->qh;
      for (uint32_t hh = 0; hh < h; hh++) {
        float sq = 0.0f;
        for (uint32_t k = 0; k < hd; k++) sq = sq + src[hh * hd + k] * src[hh * hd + k];
        float sc = ex_rms_scale(sq, (float)hd);
        for (uint32_t k = 0; k < hd; k++) y[hh * hd + k] = (src[hh * hd + k] * sc) * (1.0f + g[k]);
      }
    }
    qo = s->qh; ko = s->kh0;
  }
  float* K = s->lay[l];
  float* V = K + (size_t)t * d;
  /* dd.sm.write */
  memcpy(K + (size_t)slot * d, ko, d * sizeof(float));
  memcpy(V + (size_t)slot * d, v, d * sizeof(float));
  /* dd.sm.attend */
  float sc = 1.0f / f32sqrt((float)hd);
  for (uint32_t hh = 0; hh < h; hh++)
    for (uint32_t tp = 0; tp < t; tp++) {
      float acc = 0.0f;
      for (uint32_t k = 0; k < hd; k++) acc = acc + qo[hh * hd + k] * K[(size_t)tp * d + hh * hd + k];
      s->s[(size_t)hh * t + tp] = acc;
    }
  for (uint32_t hh = 0; hh < h; hh++) {
    float r = -INFINITY;
    for (uint32_t tp = 0; tp < t; tp++) {
      float x = ((float)tp <= (float)npos) ? sc * s->s[(size_t)hh * t + tp] : -INFINITY;
      r = x > r ? x : r;
    }
    s->m1[hh] = r;
  }
  const float* mo = s->m1;
  if (c->sinks) {
    const float* sink = m->w + b->sink;
    for (uint32_t hh = 0; hh < h; hh++) s->mm[hh] = exmax(s->m1[hh], sink[hh]);
    mo = s->mm;
  }
  for (uint32_t hh = 0; hh < h; hh++)
    for (uint32_t tp = 0; tp < t; tp++)
      s->e[(size_t)hh * t + tp] = ((float)tp <= (float)npos) ? f32exp((sc * s->s[(size_t)hh * t + tp]) - mo[hh]) : 0.0f;
  for (uint32_t hh = 0; hh < h; hh++) {
    float r = 0.0f;
    for (uint32_t tp = 0; tp < t; tp++) r = r + s->e[(size_t)hh * t + tp];
    s->se[hh] = r;
  }
  const float* deno = s->se;
  if (c->sinks) {
    const float* sink = m->w + b->sink;
    for (uint32_t hh = 0; hh < h; hh++) s->den[hh] = s->se[hh] + f32exp(sink[hh] - mo[hh]);
    deno = s->den;
  }
  for (uint32_t hh = 0; hh < h; hh++)
    for (uint32_t k = 0; k < hd; k++) {
      float acc = 0.0f;
      for (uint32_t tp = 0; tp < t; tp++) acc = acc + s->e[(size_t)hh * t + tp] * V[(size_t)tp * d + hh * hd + k];
      s->oi[hh * hd + k] = acc;
    }
  for (uint32_t hh = 0; hh < h; hh++)
    for (uint32_t k = 0; k < hd; k++) s->o[hh * hd + k] = (1.0f / deno[hh]) * s->oi[hh * hd + k];
  tail(m, s, l);
}

void or_feed(const or_model* m, or_state* s, uint32_t pos, uint32_t tok) {
  const or_config* c = &m->c;
  uint32_t slot = pos % c->ctx, npos = pos < c->ctx - 1 ? pos : c->ctx - 1;
  memcpy(s->x, m->w + (size_t)tok * c->d, c->d * sizeof(float));    /* dd.embed */
  for (uint32_t l = 0; l < c->layers; l++) {
    if (m->b[l].gla) gla_layer(m, s, l);
    else sm_layer(m, s, l, slot, npos);
  }
}

/* head (bend/Dense/Decode.bend:514): final norm, then the tied embedding */
void or_logits(const or_model* m, const or_state* s, float* out) {
  const or_config* c = &m->c;
  float* fv = malloc(c->d * sizeof(float));
  norm(c->d, s->x, m->w + m->fin, fv);
  gemv(fv, m->pk + m->pk_off[0], c->vocab, c->d, out);
  free(fv);
}

/* dd.pick (bend/Dense/Decode.bend:481-484) */
uint32_t or_top(uint32_t v, const float* lg) {
  float top = -INFINITY;
  for (uint32_t i = 0; i < v; i++) top = lg[i] > top ? lg[i] : top;
  float r = -INFINITY;
  for (uint32_t i = 0; i < v; i++) {
    float t = (top <= lg[i]) ? ((float)v - (float)i) : 0.0f;
    r = t > r ? t : r;
  }
  return v - (uint32_t)r;
}

/* ------------------------------------------------------------------------ */
/* Trees (bend/Tensor.bend): a vector of n present components in a
 * left-packed tree of depth depth(n); absent subtrees are VZ.               */

static int tdepth(uint64_t n) { int d = 0; while ((1ull << d) < n) d++; return d; }

/* V.sum / V.sumsq / V.dot: VZ counts 0.0 */
static float t_sum(const float* x, uint32_t n, uint32_t base, int p) {
  if (base >= n) return 0.0f;
  if (p == 0) return x[base];
  return t_sum(x, n, base, p - 1) + t_sum(x, n, base + (1u << (p - 1)), p - 1);
}
static float t_sumsq(const float* x, uint32_t n, uint32_t base, int p) {
  if (base >= n) return 0.0f;
  if (p == 0) return x[base] * x[base];
  return t_sumsq(x, n, base, p - 1) + t_sumsq(x, n, base + (1u << (p - 1)), p - 1);
}
static float t_dot(const float* a, const float* b, uint32_t n, uint32_t base, int p) {
  if (base >= n) return 0.0f;
  if (p == 0) return a[base] * b[base];
  return t_dot(a, b, n, base, p - 1) + t_dot(a, b, n, base + (1u << (p - 1)), p - 1);
}
/* V.max: VZ is -3e38, F32.max a b = (a < b ? b : a) */
static float t_max(const float* x, uint32_t n, uint32_t base, int p) {
  if (base >= n) return -3.0e38f;
  if (p == 0) return x[base];
  return exmax(t_max(x, n, base, p - 1), t_max(x, n, base + (1u << (p - 1)), p - 1));
}

float or_tree_sum(uint32_t n, const float* x) { return t_sum(x, n, 0, tdepth(n)); }

/* Evaluate.bend's summand (window.go, bend/Evaluate.bend:33-44):
   G.lse(l) - l[y], with G.lse l = V.max l + F32.log (V.sum_exp (V.max l) l)
   (bend/Train/Grad.bend:795-797), V.max and V.sum_exp the tree reductions
   of bend/Tensor.bend:170-177,292-299 over the depth-dv tree of the logits */
float or_ce(uint32_t vocab, const float* logits, uint32_t y) {
  int dv = tdepth(vocab);
  float m = t_max(logits, vocab, 0, dv);
  float* e = (float*)malloc(sizeof(float) * (vocab ? vocab : 1));
  for (uint32_t i = 0; i < vocab; i++) e[i] = f32exp(logits[i] - m);
  float sum = t_sum(e, vocab, 0, dv);
  free(e);
  return (m + f32log(sum)) - logits[y];
}

static void t_matvec(const float* W, uint32_t rows, uint32_t cols, const float* x, float* y) {
  int dc = tdepth(cols);
  for (uint32_t r = 0; r < rows; r++) y[r] = t_dot(W + (size_t)r * cols, x, cols, 0, dc);
}

/* Ops.rms_norm: ((1/sqrt(sumsq/n + 1e-5)) * x) * gain */
static void t_rms(uint32_t d, const float* x, const float* g, float* y) {
  float sc = 1.0f / f32sqrt((t_sumsq(x, d, 0, tdepth(d)) / (float)d) + 1.0e-5f);
  for (uint32_t j = 0; j < d; j++) y[j] = (sc * x[j]) * g[j];
}

struct or_tree {
  uint32_t layers;
  float** lay;      /* GLA S [h][hd][hd] or K ring then V ring */
  uint8_t** here;   /* softmax: slot written */
};

or_tree* or_tree_new(const or_model* m) {
  const or_config* c = &m->c;
  or_tree* t = calloc(1, sizeof *t);
  uint32_t d = c->d, h = c->heads, hd = d / h;
  t->layers = c->layers;
  t->lay = calloc(c->layers, sizeof(float*));
  t->here = calloc(c->layers, sizeof(uint8_t*));
  for (uint32_t l = 0; l < c->layers; l++) {
    if (m->b[l].gla) t->lay[l] = calloc((size_t)h * hd * hd, 4);
    else { t->lay[l] = calloc((size_t)2 * c->ctx * d, 4); t->here[l] = calloc(c->ctx, 1); }
  }
  return t;
}

void or_tree_free(or_tree* t) {
  if (!t) return;
  for (uint32_t l = 0; l < t->layers; l++) { free(t->lay[l]); free(t->here[l]); }
  free(t->lay); free(t->here); free(t);
}

/* absent-skipping pairwise tree over slots (M trees with MZ, add.pad/maxpad):
 * returns 0 when the whole subtree is absent */
typedef struct { float v; int here; } pv;
static pv pv_join_add(pv a, pv b) {
  if (!a.here) return b;
  if (!b.here) return a;
  pv r = {a.v + b.v, 1};
  return r;
}
static pv pv_join_max(pv a, pv b) {
  if (!a.here) return b;
  if (!b.here) return a;
  pv r = {exmax(a.v, b.v), 1};
  return r;
}

typedef struct { const float* val; const uint8_t* here; uint32_t stride; } slots;

static pv t_slot_red(const slots* s, uint32_t n, uint32_t base, int p, int is_max) {
  if (base >= n) { pv z = {0.0f, 0}; return z; }
  if (p == 0) { pv r = {s->val[(size_t)base * s->stride], s->here[base] != 0}; return r; }
  pv a = t_slot_red(s, n, base, p - 1, is_max);
  pv b = t_slot_red(s, n, base + (1u << (p - 1)), p - 1, is_max);
  return is_max ? pv_join_max(a, b) : pv_join_add(a, b);
}

void or_tree_step(const or_model* m, or_tree* tr, uint32_t pos, uint32_t tok, float* logits) {
  const or_config* c = &m->c;
  uint32_t d = c->d, f = c->f, h = c->heads, hd = d / h, ctx = c->ctx;
  int dhd = tdepth(hd), dcx = tdepth(ctx);
  uint32_t slot = pos % ctx;
  float* x = malloc(d * 4), *nrm = malloc(d * 4), *q = malloc(d * 4), *k = malloc(d * 4), *v = malloc(d * 4);
  float* z = malloc(d * 4), *att = malloc(d * 4), *xa = malloc(d * 4), *g = malloc(f * 4), *u = malloc(f * 4);
  float* hh = malloc(f * 4), *y = malloc(d * 4);
  float* sc_ = malloc((size_t)ctx * h * 4), *e = malloc((size_t)ctx * h * 4);
  memcpy(x, m->w + (size_t)tok * d, d * 4);
  for (uint32_t l = 0; l < c->layers; l++) {
    const blk* b = &m->b[l];
    t_rms(d, x, m->w + b->ra, nrm);
    t_matvec(m->w + b->wq, d, d, nrm, q);
    t_matvec(m->w + b->wk, d, d, nrm, k);
    t_matvec(m->w + b->wv, d, d, nrm, v);
    if (b->gla) {
      t_matvec(m->w + b->wa, d, d, nrm, z);
      /* l2_heads on q and k (bend/Ops.bend l2_head) */
      for (int which = 0; which < 2; which++) {
        float* a = which ? k : q;
        for (uint32_t i = 0; i < h; i++) {
          float n = f32sqrt(1.0e-6f + t_sumsq(a + i * hd, hd, 0, dhd));
          for (uint32_t j = 0; j < hd; j++) a[i * hd + j] = a[i * hd + j] / n;
        }
      }
      float* al = malloc(d * 4), *kh = malloc(d * 4);
      for (uint32_t j = 0; j < d; j++) {
        if (c->rglru) {
          float la = ex_rglru_log_gate(z[j], m->w[b->lam + j]);
          al[j] = f32exp(la);
          kh[j] = k[j] * ex_rglru_write_scale(la);
        } else {
          al[j] = ex_sigmoid(z[j]);
          kh[j] = k[j];
        }
      }
      float* S = tr->lay[l];
      for (uint32_t i = 0; i < h; i++)
        for (uint32_t a = 0; a < hd; a++)
          for (uint32_t bb = 0; bb < hd; bb++) {
            float* p = &S[(size_t)i * hd * hd + a * hd + bb];
            *p = (al[i * hd + a] * *p) + (kh[i * hd + a] * v[i * hd + bb]);
          }
      /* gla.out: vecmat, rows combined by add.pad in tree order */
      float* col = malloc(hd * 4);
      uint8_t* ones = malloc(hd);
      memset(ones, 1, hd);
      for (uint32_t i = 0; i < h; i++)
        for (uint32_t bb = 0; bb < hd; bb++) {
          for (uint32_t a = 0; a < hd; a++) col[a] = q[i * hd + a] * S[(size_t)i * hd * hd + a * hd + bb];
          slots s = {col, ones, 1};
          att[i * hd + bb] = t_slot_red(&s, hd, 0, dhd, 0).v;
        }
      free(col); free(ones); free(al); free(kh);
    } else {
      if (c->qk) {
        for (int which = 0; which < 2; which++) {
          float* a = which ? k : q;
          const float* gw = m->w + (which ? b->gk : b->gq);
          for (uint32_t i = 0; i < h; i++) {
            float scl = 1.0f / f32sqrt((t_sumsq(a + i * hd, hd, 0, dhd) / (float)hd) + 1.0e-5f);
            for (uint32_t j = 0; j < hd; j++) a[i * hd + j] = (scl * a[i * hd + j]) * (1.0f + gw[j]);
          }
        }
      }
      float* K = tr->lay[l];
      float* V = K + (size_t)ctx * d;
      memcpy(K + (size_t)slot * d, k, d * 4);
      memcpy(V + (size_t)slot * d, v, d * 4);
      tr->here[l][slot] = 1;
      float scl = 1.0f / f32sqrt((float)hd);
      for (uint32_t t = 0; t < ctx; t++)
        for (uint32_t i = 0; i < h; i++)
          sc_[(size_t)t * h + i] = tr->here[l][t] ? scl * t_dot(q + i * hd, K + (size_t)t * d + i * hd, hd, 0, dhd) : 0.0f;
      for (uint32_t i = 0; i < h; i++) {
        slots s = {sc_ + i, tr->here[l], h};
        float mx = t_slot_red(&s, ctx, 0, dcx, 1).v;
        if (c->sinks) mx = exmax(mx, m->w[b->sink + i]);
        for (uint32_t t = 0; t < ctx; t++) e[(size_t)t * h + i] = tr->here[l][t] ? f32exp(sc_[(size_t)t * h + i] - mx) : 0.0f;
        slots se = {e + i, tr->here[l], h};
        float den = t_slot_red(&se, ctx, 0, dcx, 0).v;
        if (c->sinks) den = den + f32exp(m->w[b->sink + i] - mx);
        float* mixv = malloc((size_t)ctx * 4);
        for (uint32_t j = 0; j < hd; j++) {
          for (uint32_t t = 0; t < ctx; t++) mixv[t] = tr->here[l][t] ? e[(size_t)t * h + i] * V[(size_t)t * d + i * hd + j] : 0.0f;
          slots sm = {mixv, tr->here[l], 1};
          att[i * hd + j] = (1.0f / den) * t_slot_red(&sm, ctx, 0, dcx, 0).v;
        }
        free(mixv);
      }
    }
    /* Model.bend tail */
    t_matvec(m->w + b->wo, d, d, att, y);
    for (uint32_t j = 0; j < d; j++) xa[j] = x[j] + y[j];
    t_rms(d, xa, m->w + b->rf, nrm);
    t_matvec(m->w + b->wg, f, d, nrm, g);
    t_matvec(m->w + b->wu, f, d, nrm, u);
    for (uint32_t j = 0; j < f; j++) hh[j] = ex_silu(g[j]) * u[j];
    t_matvec(m->w + b->wd, d, f, hh, y);
    for (uint32_t j = 0; j < d; j++) x[j] = xa[j] + y[j];
  }
  t_rms(d, x, m->w + m->fin, nrm);
  t_matvec(m->w, c->vocab, d, nrm, logits);
  free(x); free(nrm); free(q); free(k); free(v); free(z); free(att); free(xa); free(g); free(u);
  free(hh); free(y); free(sc_); free(e);
}

/* ------------------------------------------------------------------------ */
/* Sampler (bend/Sample.bend)                                                 */

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

typedef struct { uint64_t z, s; } mix;
static mix splitmix(uint64_t s) {
  uint64_t s2 = s + 0x9E3779B97F4A7C15ull;
  uint64_t z1 = (s2 ^ (s2 >> 30)) * 0xBF58476D1CE4E5B9ull;
  uint64_t z2 = (z1 ^ (z1 >> 27)) * 0x94D049BB133111EBull;
  mix r = {z2 ^ (z2 >> 31), s2};
  return r;
}

void or_rng_seeded(uint64_t seed, uint64_t r[4]) {
  mix m1 = splitmix(seed), m2 = splitmix(m1.s), m3 = splitmix(m2.s), m4 = splitmix(m3.s);
  r[0] = m1.z; r[1] = m2.z; r[2] = m3.z; r[3] = m4.z;
}

/* Rng.next (bend/Sample.bend:57-66), the file's transition */
uint64_t or_rng_next(uint64_t r[4]) {
  uint64_t s0 = r[0], s1 = r[1], s2 = r[2], s3 = r[3];
  uint64_t t = s1 << 17;
  uint64_t w = rotl64(s1 * 5, 7) * 9;
  r[0] = (s0 ^ s3) ^ (s1 ^ s2);
  r[1] = s1 ^ s2;
  r[2] = (s2 ^ s0) ^ t;
  r[3] = rotl64(s3 ^ s1, 45);
  return w;
}

int or_u64_read(const char* s, uint64_t* out) {
  if (!s || !*s) return 0;
  uint64_t v = 0;
  int ok = 1;
  for (; *s; s++) {
    if (*s < '0' || *s > '9') ok = 0;
    else v = v * 10 + (uint64_t)(*s - '0');
  }
  if (ok) *out = v;
  return ok;
}

/* Sample.argmax: pairwise, later wins only when strictly greater */
typedef struct { float v; uint32_t i; } best;
static best t_argmax(const float* x, uint32_t n, uint32_t base, int p) {
  if (base >= n) { best z = {-3.0e38f, 0}; return z; }
  if (p == 0) { best b = {x[base], base}; return b; }
  best a = t_argmax(x, n, base, p - 1), b = t_argmax(x, n, base + (1u << (p - 1)), p - 1);
  return b.v > a.v ? b : a;
}
uint32_t or_tree_argmax(uint32_t v, const float* lg) { return t_argmax(lg, v, 0, tdepth(v)).i; }

/* dc.prob.of (bend/Decode.bend:199-202) and al.stat (bend/Agent/Loop.bend:
 * 284-288): m = T.V.max, z = T.V.sum_exp(m, lg) (bend/Tensor.bend:292-299),
 * p = F32.exp(l[x] - m) / z; a = Sample.argmax of lg with l[x] set to
 * -3e38 (T.V.set), pa = F32.exp(l[a] - m) / z */
void or_stat(uint32_t vocab, const float* logits, uint32_t x, float* p, uint32_t* a, float* pa) {
  int dv = tdepth(vocab);
  float m = t_max(logits, vocab, 0, dv);
  float* e = (float*)calloc(vocab ? vocab : 1, sizeof(float));
  for (uint32_t i = 0; i < vocab; i++) e[i] = f32exp(logits[i] - m);
  float z = t_sum(e, vocab, 0, dv);
  for (uint32_t i = 0; i < vocab; i++) e[i] = i == x ? -3.0e38f : logits[i];
  uint32_t r = t_argmax(e, vocab, 0, dv).i;
  free(e);
  *p = f32exp(logits[x] - m) / z;
  *a = r;
  *pa = f32exp(logits[r] - m) / z;
}


static float t_count_ge(const float* x, uint32_t n, uint32_t base, int p, float t) {
  if (base >= n) return 0.0f;
  if (p == 0) return x[base] >= t ? 1.0f : 0.0f;
  return t_count_ge(x, n, base, p - 1, t) + t_count_ge(x, n, base + (1u << (p - 1)), p - 1, t);
}
static float t_mass_ge(const float* x, uint32_t n, uint32_t base, int p, float t) {
  if (base >= n) return 0.0f;
  if (p == 0) return x[base] >= t ? x[base] : 0.0f;
  return t_mass_ge(x, n, base, p - 1, t) + t_mass_ge(x, n, base + (1u << (p - 1)), p - 1, t);
}

float or_topk_threshold(uint32_t v, const float* lg, uint32_t topk) {
  int dv = tdepth(v);
  float peak = t_max(lg, v, 0, dv);
  float need = (float)topk, lo = peak - 100.0f, hi = peak;
  for (int i = 0; i < 40; i++) {
    float mid = 0.5f * (lo + hi);
    if (t_count_ge(lg, v, 0, dv, mid) >= need) lo = mid; else hi = mid;
  }
  return lo;
}

float or_topp_threshold(uint32_t v, const float* w, float topp) {
  int dv = tdepth(v);
  float need = topp * t_sum(w, v, 0, dv), lo = 0.0f, hi = 1.0f;
  for (int i = 0; i < 40; i++) {
    float mid = 0.5f * (lo + hi);
    if (t_mass_ge(w, v, 0, dv, mid) >= need) lo = mid; else hi = mid;
  }
  return lo;
}

/* draw.go: the first index whose running mass exceeds u, walking the tree */
static uint32_t t_draw(const float* w, uint32_t n, uint32_t base, int p, float u) {
  if (base >= n) return base;
  if (p == 0) return base;
  uint32_t half = 1u << (p - 1);
  float ml = t_sum(w, n, base, p - 1);
  int right_absent = base + half >= n;
  int left = (u < ml) || right_absent;
  if (left) return t_draw(w, n, base, p - 1, u);
  return t_draw(w, n, base + half, p - 1, u - ml);
}

uint32_t or_pick(uint32_t v, const float* lg, float temp, uint32_t topk, float topp, uint64_t rng[4]) {
  if (temp <= 0.0f) return or_tree_argmax(v, lg);
  int dv = tdepth(v);
  float* w = malloc((size_t)v * 4);
  float peak = t_max(lg, v, 0, dv);
  if (topk < v) {
    float t = or_topk_threshold(v, lg, topk);
    for (uint32_t i = 0; i < v; i++) w[i] = lg[i] >= t ? lg[i] : -3.0e38f;
  } else {
    memcpy(w, lg, (size_t)v * 4);
  }
  for (uint32_t i = 0; i < v; i++) w[i] = f32exp((w[i] - peak) / temp);
  if (topp < 1.0f) {
    float t = or_topp_threshold(v, w, topp);
    for (uint32_t i = 0; i < v; i++) w[i] = w[i] >= t ? w[i] : 0.0f;
  }
  uint64_t word = or_rng_next(rng);
  float unit = (float)(uint32_t)((word >> 32) >> 8) / 16777216.0f;
  float u = unit * t_sum(w, v, 0, dv);
  uint32_t tok = t_draw(w, v, 0, dv, u);
  free(w);
  return tok;
}

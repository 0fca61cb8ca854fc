// libana: the C ABI of include/ana.h over the kernels.
//
// One context = one checkpoint on one device, one HIP stream, and state for
// max_seqs sequences. A sequence's states are one contiguous region (per
// layer: the GLA S of heads x hd x hd floats, or the softmax K ring then V
// ring of ctx x d floats each), followed in a separate array by the residual
// row of its last fed token, which the head reads (the store's x cell in
// bend/Dense/Decode.bend).
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ana_internal.h"

using namespace ana;

struct ana_ctx {
  int device = 0;
  hipStream_t st = nullptr;
  ana_config cfg{};
  uint64_t P = 0, step = 0, fin = 0;
  std::vector<Blk> blk;
  std::vector<uint64_t> layer_off;   // floats from a sequence's state start
  uint64_t seq_stride = 0;           // floats per sequence
  uint32_t max_seqs = 1, chunk = 64, wb = 1;
  uint32_t rows = 1;                 // capacity of the row workspaces (a prefill batch)
  int mode = ANA_EXACT_FP32;         // numerics
  float* W = nullptr;                // parameters [P]
  uint16_t* Wh = nullptr;            // ANA_BF16: the parameters as bfloat16 [P]
  uint16_t* Wp = nullptr;            // ANA_BF16: the persistent kernel's bf16 matrices that start off 16 bytes in Wh, on 16 bytes
  // ANA_BF16 keeps the first block's matrices in fp32: parameters in
  // [fp32_lo, fp32_hi) are read as fp32 in every mode (the first block's
  // rounding dominates the bf16 logits' error: alone it gives ~1.3e-2 of the
  // ~1.4e-2 all blocks give at 115M)
  uint64_t fp32_lo = 0, fp32_hi = 0;
  float* state = nullptr;            // [max_seqs][seq_stride]
  float* xs = nullptr;               // [max_seqs][d]
  // workspace, wb rows
  float *X = nullptr, *XA = nullptr, *XN = nullptr, *QKV = nullptr, *Z = nullptr, *O = nullptr,
        *HH = nullptr;
  float* LG = nullptr;               // [max_seqs][vocab]
  uint32_t *d_seq = nullptr, *d_pos = nullptr, *d_tok = nullptr, *d_pick = nullptr, *d_out = nullptr,
           *d_step = nullptr;
  uint64_t* d_rng = nullptr;
  unsigned long long* d_amax = nullptr;  // [wb] greedy argmax keys
  float *d_ss = nullptr, *d_pm = nullptr; // split attention scratch
  float* d_part = nullptr;           // fast attention's per-split partials
  size_t part_cap = 0;               // their floats
  float* SC = nullptr;               // scoring: the head's logits for up to sc_rows rows
  uint32_t sc_rows = 1;
  uint32_t* d_tgt = nullptr;         // scoring: each row's target token
  float* d_stat = nullptr;           // ana_stats: each row's p and rival p, then the rivals
  float* d_ce = nullptr;             // scoring: each row's G.lse - logit[target]
  __bf16* d_sah = nullptr;   // ANA_BF16 prefill: a product's activations in bf16
  __bf16* d_hh = nullptr;    // ANA_BF16 prefill: gate|up's outputs in bf16, down's input
  bool hh_bf = false;        // d_hh holds the last gate|up's outputs
  float* d_rsc = nullptr;                      // and its rows' norm scales
  // ANA_BF16 prefill, the operands producers leave for the next product
  // (k_split's work done in their epilogues): d_oh the mixes' outputs in
  // bf16 (Wo's operand) when oh_ok; d_nxh a residual product's outputs times
  // the next norm's gain in bf16, with d_ssp its rows' partial sums of
  // squares (nx_n a row), for the product that reads nx_of with gain nx_g
  __bf16* d_oh = nullptr;
  bool oh_ok = false;
  __bf16* d_nxh = nullptr;
  float* d_ssp = nullptr;
  const float* nx_of = nullptr;
  const float* nx_g = nullptr;
  uint32_t nx_n = 0;
  // fast modes: every layer product's weights packed for k_gemm_pk (fp32, or
  // bf16 in ANA_BF16; the norm gains folded in), found by the product's first
  // weight row; the entry keeps the segment shape and gains it was packed for
  void* PK = nullptr;
  unsigned long long* d_hpc = nullptr;  // the fused head and sampler's arrival counters
  uint32_t* d_hpctl = nullptr;          // and its ran-out flag
  struct PkEnt {
    uint64_t off;
    uint32_t rows0, rows1, nseg, mode, K;
    const float* ng;
    int bf;                          // packed as bf16 (else fp32)
  };
  std::unordered_map<const float*, PkEnt> pk;
  // the persistent one-sequence decode (every mode; the exact build in ANA_EXACT_FP32): its layer table,
  // exchange entries (two sets of ll_par), control words, grid and the
  // epoch its next launch starts from
  bool persist = false, persist_off = false;
  uint32_t pG = 0, pnp = 0;
  PLayer* d_play = nullptr;
  unsigned long long* d_ll = nullptr;   // uncached (uc_take), never freed
  uint64_t ll_par = 0, e_key = 0, ll_bytes = 0;
  uint32_t* d_ctl = nullptr;
  uint32_t epoch = 0;
  uint64_t p_tmo = 0;                // a wait's limit in the device clock's ticks (2 s)
  uint32_t* d_trace = nullptr;       // ana_trace's phase stamps, when armed
  uint32_t trace_steps = 0, trace_phases = 0;
  float* d_gla = nullptr;            // fast prefill's GLA scan scratch
  GlaScratch gla{};                  // its regions
  GlaSub* d_gtab = nullptr;          // a prefill step's sub-chunk table
  GlaRun* d_grun = nullptr;          // and its chunk table
  uint32_t *d_rseq = nullptr, *d_rpos = nullptr;  // a prefill step's per-row sequence, position
  uint32_t* d_rcp = nullptr;   // a prefill step's (last row, sequence) pairs for the residual rows
  uint32_t seg_cap = 1, gsub_cap = 1; // chunks a prefill step holds; table entries
  AttnTile* d_atab = nullptr;        // a prefill step's attention tiles
  uint32_t atab_cap = 1;
  // host copies of the step tables, kept until the step's synchronize
  std::vector<AttnTile> h_atab;
  std::vector<GlaSub> h_gtab;
  std::vector<GlaRun> h_grun;
  std::vector<uint32_t> h_rseq, h_rpos;
  std::string err;
  // ana_generate's decode step captured as HIP graphs, replayed per step:
  // one step, and kGraphSteps steps back to back (a graph launch costs tens
  // of microseconds on the host side, so several steps share one)
  hipGraphExec_t gexec = nullptr, gexec_n = nullptr;
  // what the captured steps depend on (not the step count: each row's
  // picks go to the step-major d_out at its own step counter)
  struct GKey {
    uint32_t n;
    float temp, topp;
    uint32_t topk;
    const uint32_t* out;
    bool split;
    bool operator==(const GKey& o) const {
      return n == o.n && temp == o.temp && topp == o.topp && topk == o.topk && out == o.out && split == o.split;
    }
  } gkey{};
  // decode steps above kSmallB rows split each row's attention over
  // kRowsSplit-slot pieces (set per call from the rows' positions)
  bool attn_split = false;
  std::vector<uint32_t> h_out;       // step-major picks of the last ana_generate
  // kernel timing (ana_prof)
  bool prof = false;
  double attn_bytes = 0.0;           // per softmax-layer launch of the current step
  std::vector<hipEvent_t> ev;        // pool, two per recorded launch
  struct Rec { uint32_t kind; double bytes; bool attn; };
  std::vector<Rec> recs;
  uint64_t acc_n[ANA_K_KINDS] = {};
  double acc_ms[ANA_K_KINDS] = {}, acc_bytes[ANA_K_KINDS] = {};
};

static const uint32_t kGraphSteps = 8;
// steps of every row d_out holds: ana_generate runs longer calls in pieces
static const uint32_t kOutSteps = 1024;

static const size_t kProfMax = 16384;

// bracket one launch with events on the context's stream
// (ext: the launch itself records the pair, hipExtLaunchKernelGGL's start
// and stop events, which bracket exactly the kernel's execution)
struct ProfScope {
  ana_ctx* c;
  uint32_t kind;
  double bytes;
  bool on, ext;
  ProfScope(ana_ctx* c_, uint32_t k, double b, bool ext_ = false)
      : c(c_), kind(k), bytes(b), on(false), ext(ext_) {
    if (!c->prof || c->recs.size() >= kProfMax) return;
    const size_t i = c->recs.size();
    if (c->ev.size() < 2 * (i + 1)) {
      hipEvent_t a, e;
      if (hipEventCreate(&a) != hipSuccess) return;
      if (hipEventCreate(&e) != hipSuccess) { (void)hipEventDestroy(a); return; }
      c->ev.push_back(a);
      c->ev.push_back(e);
    }
    if (!ext && hipEventRecord(c->ev[2 * i], c->st) != hipSuccess) return;
    on = true;
  }
  hipEvent_t start() const { return on && ext ? c->ev[2 * c->recs.size()] : nullptr; }
  hipEvent_t stop() const { return on && ext ? c->ev[2 * c->recs.size() + 1] : nullptr; }
  ~ProfScope() {
    if (!on) return;
    const size_t i = c->recs.size();
    if (ext || hipEventRecord(c->ev[2 * i + 1], c->st) == hipSuccess)
      c->recs.push_back({kind, bytes, kind == ANA_K_ATTN});
  }
};

static thread_local std::string g_open_err;

static int fail(ana_ctx* c, int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  else g_open_err = buf;
  return code;
}

#define HIPCHK(ctx, x)                                                                  \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess)                                                               \
      return fail(ctx, ANA_EDEVICE, "device fault: %s (%s:%d)", hipGetErrorString(e_), \
                  __FILE__, __LINE__);                                                  \
  } while (0)

template <class T>
static hipError_t dalloc(T** p, size_t n) {
  return hipMalloc((void**)p, std::max<size_t>(n, 1) * sizeof(T));
}

// The persistent kernel's exchange entries live in uncached device memory:
// its device-coherent stores and polls then skip the L2s, and an
// all-gather of 768 entries over 256 workgroups took 1.49 us against 1.99
// us in ordinary device memory (measured alone, on MI355X). Uncached memory
// that a kernel has read is never freed before the process ends (a block
// freed after such use left later allocations holding wrong values on these
// machines), so a closed context's block returns to a per-device pool that
// later contexts reuse, the smallest block that fits first.
struct UcBlock {
  int dev;
  void* p;
  size_t bytes;
};
static std::mutex g_uc_mu;
static std::vector<UcBlock> g_uc_free;
static hipError_t uc_take(int dev, size_t bytes, void** p) {
  {
    std::lock_guard<std::mutex> lock(g_uc_mu);
    size_t best = g_uc_free.size();
    for (size_t i = 0; i < g_uc_free.size(); i++)
      if (g_uc_free[i].dev == dev && g_uc_free[i].bytes >= bytes &&
          (best == g_uc_free.size() || g_uc_free[i].bytes < g_uc_free[best].bytes))
        best = i;
    if (best < g_uc_free.size()) {
      *p = g_uc_free[best].p;
      g_uc_free.erase(g_uc_free.begin() + best);
      return hipSuccess;
    }
  }
  return hipExtMallocWithFlags(p, std::max<size_t>(bytes, 256), hipDeviceMallocUncached);
}
static void uc_give(int dev, void* p, size_t bytes) {
  if (!p) return;
  std::lock_guard<std::mutex> lock(g_uc_mu);
  g_uc_free.push_back({dev, p, std::max<size_t>(bytes, 256)});
}

static void release(ana_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
  if (c->gexec_n) (void)hipGraphExecDestroy(c->gexec_n);
  uc_give(c->device, c->d_ll, c->ll_bytes);
  void* ps[] = {c->d_play, c->d_ctl, c->d_trace, c->W, c->Wh, c->Wp, c->d_part, c->d_gla, c->state, c->xs, c->X, c->XA, c->XN, c->QKV, c->Z, c->O, c->HH, c->LG,
                c->d_seq, c->d_pos, c->d_tok, c->d_pick, c->d_out, c->d_step, c->d_rng, c->d_amax,
                c->d_ss, c->d_pm, c->d_gtab, c->d_grun, c->d_atab, c->d_rseq, c->d_rpos, c->SC, c->d_tgt, c->d_ce, c->d_stat, c->d_rcp,
                c->d_sah, c->d_hh, c->d_rsc, c->PK, c->d_hpc, c->d_hpctl, c->d_oh, c->d_nxh, c->d_ssp};
  for (void* p : ps)
    if (p) (void)hipFree(p);
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  if (c->st) (void)hipStreamDestroy(c->st);
}

static StateRef sref(const ana_ctx* c, uint32_t l) {
  return StateRef{c->state, c->seq_stride, c->layer_off[l]};
}

// what the kernels require of a configuration
static const char* unsupported(const ana_config& c) {
  if (c.heads == 0 || c.d % c.heads) return "model dim is not a multiple of the head count";
  const uint32_t hd = c.d / c.heads;
  if (hd > 64) return "head dimension above 64";
  if (c.d % 4 || c.f % 4 || hd % 4) return "model, MLP and head dimensions must be multiples of 4";
  if (c.sinks && c.heads % 4) return "with head sinks the head count must be a multiple of 4";
  if (c.ctx == 0 || c.ctx > 4096) return "context above 4096 slots";
  if (c.vocab < 2 || c.vocab > 65536) return "vocabulary outside 2..65536";
  return nullptr;
}

extern "C" void ana_rng_seeded(uint64_t seed, uint64_t r[4]) {
  // Rng.seeded: four SplitMix64 draws (bend/Sample.bend:68-93)
  uint64_t s = seed;
  for (int i = 0; i < 4; i++) {
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = (s ^ (s >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    r[i] = z ^ (z >> 31);
  }
}

static hipError_t pack_weights(ana_ctx* c);
static hipError_t persist_setup(ana_ctx* c);
static void resolve_scratch(int device);

extern "C" int ana_open(const char* path, const ana_opts* opts, ana_ctx** out) {
  if (!path || !out) return fail(nullptr, ANA_EINVAL, "ana_open: null argument");
  *out = nullptr;
  ana_opts o{};
  o.max_seqs = 1;
  if (opts) o = *opts;
  if (o.numerics != ANA_EXACT_FP32 && o.numerics != ANA_FAST_FP32 && o.numerics != ANA_BF16)
    return fail(nullptr, ANA_EUNSUP, "ana_open: unknown numerics mode %d", o.numerics);
  if (o.max_seqs == 0) o.max_seqs = 1;
  if (o.prefill_chunk == 0) o.prefill_chunk = 64;
  Ftc2 ck;
  std::string why = read_ftc2(path, &ck);
  if (!why.empty()) return fail(nullptr, ANA_ECKPT, "%s", why.c_str());
  if (const char* u = unsupported(ck.cfg)) return fail(nullptr, ANA_EUNSUP, "ana_open: %s", u);
  ana_ctx* c = new ana_ctx();
  c->device = o.device;
  c->mode = o.numerics;
  c->cfg = ck.cfg;
  c->step = ck.step;
  c->P = params_of(ck.cfg);
  c->blk = layout_of(ck.cfg, &c->fin);
  if (!c->blk.empty()) {
    c->fp32_lo = c->blk[0].ra;
    c->fp32_hi = c->blk[0].end;
  }
  c->max_seqs = o.max_seqs;
  c->chunk = o.prefill_chunk;
  c->wb = std::max(c->max_seqs, c->chunk);
  // a batched prefill's step holds every sequence's chunk, up to 8192 rows
  c->rows = std::max<uint32_t>(c->wb, (uint32_t)std::min<uint64_t>((uint64_t)c->max_seqs * c->chunk, 8192));
  // a step holds at most kMaxSegs chunks (each at least one row), and so
  // at most rows / kGlaSub + seg_cap sub-chunks
  c->seg_cap = std::min({c->max_seqs, c->rows, kMaxSegs});
  c->gsub_cap = c->rows / kGlaSub + c->seg_cap;
  c->atab_cap = c->rows / kFlashQ + c->seg_cap;
  c->sc_rows = std::min(c->rows, kScoreRows);
  const ana_config& cf = c->cfg;
  const uint32_t d = cf.d, hd = d / cf.heads;
  uint64_t off = 0;
  for (uint32_t l = 0; l < cf.layers; l++) {
    c->layer_off.push_back(off);
    off += c->blk[l].gla ? (uint64_t)cf.heads * hd * hd : 2ull * cf.ctx * d;
  }
  c->seq_stride = off;
  auto bad = [&](hipError_t e) {
    int r = fail(nullptr, e == hipErrorOutOfMemory ? ANA_ENOMEM : ANA_EDEVICE, "device fault: %s",
                 hipGetErrorString(e));
    release(c);
    delete c;
    return r;
  };
  hipError_t e;
  if ((e = hipSetDevice(c->device)) != hipSuccess) return bad(e);
  resolve_scratch(c->device);
  if ((e = hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking)) != hipSuccess) return bad(e);
  const uint64_t wb = c->wb;
  if ((e = dalloc(&c->W, c->P)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->state, c->seq_stride * c->max_seqs)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->xs, (uint64_t)d * c->max_seqs)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->X, (uint64_t)c->rows * d)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->XA, (uint64_t)c->rows * d)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->XN, (uint64_t)c->rows * d)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_step, wb)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_out, wb * kOutSteps)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_amax, wb * kAmaxPerRow)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_ss, wb * cf.heads * cf.ctx)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_pm, wb * cf.heads * ((cf.ctx + kAttnTS - 1) / kAttnTS))) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->QKV, (uint64_t)c->rows * 3 * d)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->Z, (uint64_t)c->rows * d)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->O, (uint64_t)c->rows * d)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->HH, (uint64_t)c->rows * cf.f)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->LG, (uint64_t)c->max_seqs * cf.vocab)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_seq, wb)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_pos, wb)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_tok, c->rows)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_pick, wb)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->d_rng, 4 * wb)) != hipSuccess) return bad(e);
  if ((e = dalloc(&c->SC, (uint64_t)c->sc_rows * cf.vocab)) != hipSuccess ||
      (e = dalloc(&c->d_tgt, c->rows)) != hipSuccess || (e = dalloc(&c->d_ce, c->rows)) != hipSuccess ||
      (e = dalloc(&c->d_stat, 3 * (uint64_t)c->max_seqs)) != hipSuccess)
    return bad(e);
  // a prefill step's residual-row pairs (every mode)
  if ((e = dalloc(&c->d_rcp, 2 * (uint64_t)c->rows)) != hipSuccess) return bad(e);
  if (c->mode != ANA_EXACT_FP32) {
    // the fast kernels' scratch: attention partials for every row of a step,
    // the GLA scan's regions and tables
    c->part_cap = attn_fast_part_floats(c->rows, cf.heads, cf.ctx, hd);
    if ((e = dalloc(&c->d_part, c->part_cap)) != hipSuccess ||
        (e = dalloc(&c->d_gla, gla_scan_floats(c->rows, c->gsub_cap, c->seg_cap, d, cf.heads))) != hipSuccess ||
        (e = dalloc(&c->d_gtab, c->gsub_cap)) != hipSuccess || (e = dalloc(&c->d_grun, c->seg_cap)) != hipSuccess ||
        (e = dalloc(&c->d_atab, c->atab_cap)) != hipSuccess ||
        (e = dalloc(&c->d_rseq, c->rows)) != hipSuccess || (e = dalloc(&c->d_rpos, c->rows)) != hipSuccess)
      return bad(e);
    c->gla = gla_scan_carve(c->d_gla, c->rows, c->gsub_cap, c->seg_cap, d, cf.heads);
  }
  if (c->mode == ANA_BF16) {
    const uint64_t kmax = std::max(d, cf.f);
    if ((e = dalloc(&c->Wh, c->P)) != hipSuccess || (e = dalloc(&c->d_sah, (uint64_t)c->rows * kmax)) != hipSuccess ||
        (e = dalloc(&c->d_hh, (uint64_t)c->rows * cf.f)) != hipSuccess || (e = dalloc(&c->d_rsc, c->rows)) != hipSuccess ||
        (e = dalloc(&c->d_oh, (uint64_t)c->rows * d)) != hipSuccess ||
        (e = dalloc(&c->d_nxh, (uint64_t)c->rows * d)) != hipSuccess ||
        (e = dalloc(&c->d_ssp, (uint64_t)c->rows * (d / 48 + 1))) != hipSuccess)
      return bad(e);
  }
  if ((e = hipMemcpyAsync(c->W, ck.raw.data(), 4 * c->P, hipMemcpyHostToDevice, c->st)) != hipSuccess) return bad(e);
  if ((e = launch_bswap(reinterpret_cast<uint32_t*>(c->W), c->P, c->st)) != hipSuccess) return bad(e);
  if (c->Wh && (e = launch_to_bf16(c->W, c->Wh, c->P, c->st)) != hipSuccess) return bad(e);
  if (c->mode != ANA_EXACT_FP32 && (e = pack_weights(c)) != hipSuccess) return bad(e);
  if (c->mode != ANA_EXACT_FP32) {
    // the fused head and sampler's counters (one per 32-row block, only
    // ever added to) and flag start at zero
    const size_t blocks = (c->max_seqs + 31) / 32;
    if ((e = dalloc(&c->d_hpc, blocks)) != hipSuccess || (e = dalloc(&c->d_hpctl, 1)) != hipSuccess ||
        (e = hipMemsetAsync(c->d_hpc, 0, 8 * blocks, c->st)) != hipSuccess ||
        (e = hipMemsetAsync(c->d_hpctl, 0, 4, c->st)) != hipSuccess)
      return bad(e);
  }
  if ((e = persist_setup(c)) != hipSuccess) return bad(e);
  // ANA_PERSIST=0 keeps one-sequence decode on the captured graphs
  if (const char* pv = getenv("ANA_PERSIST")) c->persist_off = strcmp(pv, "0") == 0;
  if ((e = launch_zero(c->state, c->seq_stride * c->max_seqs, c->st)) != hipSuccess) return bad(e);
  if ((e = launch_zero(c->xs, (uint64_t)d * c->max_seqs, c->st)) != hipSuccess) return bad(e);
  if ((e = hipStreamSynchronize(c->st)) != hipSuccess) return bad(e);
  *out = c;
  return ANA_OK;
}

extern "C" int ana_config_of(const ana_ctx* c, ana_config* out, uint64_t* step) {
  if (!c || !out) return ANA_EINVAL;
  *out = c->cfg;
  if (step) *step = c->step;
  return ANA_OK;
}

extern "C" const char* ana_error(const ana_ctx* c) { return c ? c->err.c_str() : g_open_err.c_str(); }

extern "C" int ana_manifest_read(const char* path, ana_manifest* out) {
  if (!path || !out) return fail(nullptr, ANA_EINVAL, "ana_manifest_read: null argument");
  const std::string why = read_manifest(path, out);
  if (!why.empty()) return fail(nullptr, ANA_ECKPT, "%s", why.c_str());
  return ANA_OK;
}

extern "C" void ana_close(ana_ctx* c) {
  if (!c) return;
  (void)hipStreamSynchronize(c->st);
  release(c);
  delete c;
}

extern "C" int ana_reset(ana_ctx* c, uint32_t seq) {
  if (!c) return ANA_EINVAL;
  if (seq >= c->max_seqs) return fail(c, ANA_EINVAL, "ana_reset: sequence %u outside 0..%u", seq, c->max_seqs - 1);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, launch_zero(c->state + (uint64_t)seq * c->seq_stride, c->seq_stride, c->st));
  HIPCHK(c, launch_zero(c->xs + (uint64_t)seq * c->cfg.d, c->cfg.d, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

// ------------------------------------------------------------------ the step

// algorithmic bytes of a product: weights once, activations in and out
static double gemv_bytes(const GemvArgs& g) {
  double rows = g.seg[0].rows + (g.nseg > 1 ? g.seg[1].rows : 0);
  double out_rows = g.mode == GM_SILU ? g.seg[0].rows : rows;
  double b = 4.0 * rows * g.K + 4.0 * g.B * g.K + 4.0 * g.B * out_rows;
  if (g.mode == GM_RESID) b += 4.0 * g.B * out_rows;
  return b;
}

// The fast modes: decode steps of B <= kSmallB sequences stream bf16
// (ANA_BF16) or fp32 rows with split-K sums and take the reassociated GLA and
// attention kernels. Prefill steps of more than kSmallB rows, and the layer
// products and head of decode steps of more sequences, run on the matrix
// cores (below 128 rows over packed weights). The decode steps of more
// sequences keep the exact GLA and attention, and prefill steps of kSmallB
// rows or fewer the exact kernels: the fast GLA and attention above kSmallB
// decode rows were on in a first test that faulted the GPU and stay off
// until its cause is found.
static bool fast_mode(const ana_ctx* c) { return c->mode != ANA_EXACT_FP32; }
static bool fast_path(const ana_ctx* c, uint32_t B) { return fast_mode(c) && B <= kSmallB; }
// a decode call's attention above kSmallB rows goes in kRowsSplit-slot
// pieces once some row reaches 2 kRowsSplit live slots (one workgroup a row
// would stream the whole window alone: at B = 32 and 1930 slots, 96 us a
// layer for 379 MB), while its (head, row) pairs are fewer than
// kRowsSplitPairs. With more pairs than that, one workgroup each already
// gives every CU two or more, and the pieces only add partials and the
// combine: at B = 64 and ~1950 live slots the whole-window grid ran the step
// 0.991 -> 0.944 ms, and B = 256 at 512-767 slots 157.8k -> 161.7k tok/s
constexpr uint64_t kRowsSplitPairs = 512;
static bool split_attention(const ana_ctx* c, uint32_t n, const uint32_t* pos, uint32_t steps) {
  uint64_t top = 0;
  for (uint32_t i = 0; i < n; i++) top = std::max<uint64_t>(top, (uint64_t)pos[i] + steps);
  return n > kSmallB && top >= 2ull * kRowsSplit && (uint64_t)n * c->cfg.heads < kRowsSplitPairs;
}
// decode steps below this many rows take the products over packed weights
// (the prefill products' 128-row tiles would leave most CUs idle: at 256
// rows gate|up is 64 workgroups)
static const uint32_t kPwMaxB = 1024;

// the packed weights of product g, when they were packed for its shape and gains
static const ana_ctx::PkEnt* find_pk(const ana_ctx* c, const GemvArgs& g) {
  const auto it = c->pk.find(g.seg[0].W);
  if (it == c->pk.end()) return nullptr;
  const ana_ctx::PkEnt& pe = it->second;
  const bool same = pe.rows0 == g.seg[0].rows && pe.nseg == g.nseg && (g.nseg < 2 || pe.rows1 == g.seg[1].rows) &&
                    pe.mode == (g.mode == GM_SILU ? 1u : 0u) && pe.K == g.K && pe.ng == g.ng;
  return same ? &pe : nullptr;
}

// whether product g reads bfloat16 weights (ANA_BF16, outside the fp32 block)
static bool reads_bf16(const ana_ctx* c, const GemvArgs& g) {
  if (!c->Wh) return false;
  const uint64_t o = (uint64_t)(g.seg[0].W - c->W);
  return !(o >= c->fp32_lo && o < c->fp32_hi);
}

// next_gain: the norm gain of the product that reads this one's outputs
// next (a prefill step's residual products), for a producer-side bf16 copy
static hipError_t gemv_timed(ana_ctx* c, const GemvArgs& g0, uint32_t kind, bool chunk = false,
                             const float* next_gain = nullptr) {
  const bool small = g0.B <= kSmallB;
  // the operands producers left: each serves the one product it was made
  // for, and goes stale when that product (or another) has run
  const bool nx_here = c->nx_of && g0.X == c->nx_of && g0.ng == c->nx_g;
  const bool oh_here = c->oh_ok && g0.X == c->O && !g0.ng;
  c->nx_of = nullptr;
  c->oh_ok = false;
  // (d_hh holds this gate|up's outputs only if the path below writes them)
  const bool hh_was = c->hh_bf;
  if (g0.mode == GM_SILU) c->hh_bf = false;
  // the hidden rows exist only in bf16 after a gate|up that wrote d_hh, so
  // down must take the path that reads them there
  const bool hh_only = (g0.X == c->HH && hh_was) || oh_here;   // (or O, when the mix left it in bf16 only)
  const bool pk_ok = gemm_pk_fits(g0) || (kind == ANA_K_HEAD && head_pw_fits(g0));
  const ana_ctx::PkEnt* pe =
      fast_mode(c) && !small && g0.B < (chunk ? 128u : kPwMaxB) && pk_ok ? find_pk(c, g0) : nullptr;
  // the head of a decode step of kPwMaxB rows or more takes the prefill
  // products too (greedy picks then read the stored logits)
  if (pe || (fast_mode(c) && (small ? !chunk : (chunk || kind != ANA_K_HEAD || g0.B >= kPwMaxB)))) {
    GemvArgs g = g0;
    // prefill steps on the big tiles read every block's weights in bf16
    // (decode keeps the first block in fp32)
    const bool bf = reads_bf16(c, g) || (c->Wh && chunk && g.B >= 128);
    if (bf) {
      g.Wh0 = c->Wh + (g.seg[0].W - c->W);
      g.Wh1 = g.nseg > 1 ? c->Wh + (g.seg[1].W - c->W) : nullptr;
    }
    double by = gemv_bytes(g);
    if (bf) by -= 2.0 * (g.seg[0].rows + (g.nseg > 1 ? g.seg[1].rows : 0)) * g.K;
    if (hh_only && (small || pe)) return hipErrorInvalidValue;
    ProfScope ps(c, kind, by, true);
    if (small) return launch_gemv_fast(g, c->st, ps.start(), ps.stop());
    if (pe && kind == ANA_K_HEAD && head_pw_fits(g))
      return launch_head_pw(g, static_cast<const char*>(c->PK) + pe->off, pe->bf, c->st, ps.start(), ps.stop());
    if (pe)
      return launch_gemm_pk(g, static_cast<const char*>(c->PK) + pe->off, pe->bf, c->st, ps.start(), ps.stop());
    if (g.B >= 128 && c->d_sah && bf && g.K % 64 == 0 && g.B <= c->rows) {
      // gate|up leaves its outputs in bf16 only, and down reads them there
      // instead of splitting them again
      if (g.mode == GM_SILU && c->d_hh && gemm_wide_takes(g)) g.Yh = c->d_hh;
      if (g.X == c->HH && hh_was && !g.ng && g.K == c->cfg.f) g.Xh = c->d_hh;
      if (nx_here && g.K == c->cfg.d) {
        g.Xh = c->d_nxh;
        g.sspi = c->d_ssp;
        g.nspi = c->nx_n;
      }
      if (oh_here) {
        if (g.K != c->cfg.d) return hipErrorInvalidValue;
        g.Xh = c->d_oh;
      }
      // a residual product of one segment on k_gemm_dl's full tiles also
      // leaves the next product's operand
      const bool fold = next_gain && g.Xh != c->d_nxh && g.nseg == 1 && g.mode != GM_SILU && g.B % 128 == 0 &&
                        g.seg[0].rows == c->cfg.d && g.seg[0].rows % gemm_dl_cols(g) == 0 && !gemm_wide_takes(g);
      if (fold) {
        g.Yn = c->d_nxh;
        g.gn = next_gain;
        g.ssp = c->d_ssp;
      }
      const hipError_t e = launch_gemm_dl(g, c->d_sah, c->d_rsc, c->rows, c->st, ps.start(), ps.stop());
      if (g.mode == GM_SILU) c->hh_bf = g.Yh != nullptr && e == hipSuccess;
      if (fold && e == hipSuccess) {
        c->nx_of = g.seg[0].Y;
        c->nx_g = next_gain;
        c->nx_n = g.seg[0].rows / (gemm_dl_cols(g) / 2);
      }
      return e;
    }
    if (hh_only) return hipErrorInvalidValue;
    if (g.B >= 128) return launch_gemm_big(g, c->st, ps.start(), ps.stop());
    return launch_gemm_mfma(g, c->st, ps.start(), ps.stop());
  }
  if (hh_only) return hipErrorInvalidValue;
  ProfScope ps(c, kind, gemv_bytes(g0), true);
  return launch_gemv(g0, c->st, ps.start(), ps.stop());
}

static GemvArgs gemv1(const float* X, uint32_t ldx, uint32_t K, const float* W, uint32_t rows,
                      float* Y, uint32_t ldy, uint32_t B) {
  GemvArgs a{};
  a.X = X; a.ldx = ldx; a.K = K;
  a.seg[0] = GemvSeg{W, rows, Y, ldy};
  a.nseg = 1;
  a.mode = GM_PLAIN;
  a.B = B;
  return a;
}

// The weight side of layer l's four products, with the workspaces they run
// on (norm, then q|k|v, + the gate's z in GLA layers; Wo with the residual;
// norm, then gate|up with SiLU; down with the residual); B left 0 for the
// caller.
enum { P_QKV = 0, P_WO = 1, P_GU = 2, P_WD = 3 };
static void layer_products(const ana_ctx* c, uint32_t l, GemvArgs p[4]) {
  const ana_config& cf = c->cfg;
  const uint32_t d = cf.d, f = cf.f;
  const float* W = c->W;
  const Blk& b = c->blk[l];
  p[P_QKV] = gemv1(c->X, d, d, W + b.wq, 3 * d, c->QKV, 3 * d, 0);
  p[P_QKV].ng = W + b.ra;
  if (b.gla) {
    p[P_QKV].seg[1] = GemvSeg{W + b.wa, d, c->Z, d};
    p[P_QKV].nseg = 2;
  }
  p[P_WO] = gemv1(c->O, d, d, W + b.wo, d, c->XA, d, 0);
  p[P_WO].mode = GM_RESID; p[P_WO].R = c->X; p[P_WO].ldr = d;
  p[P_GU] = gemv1(c->XA, d, d, W + b.wg, f, c->HH, f, 0);
  p[P_GU].seg[1] = GemvSeg{W + b.wu, f, c->HH, f};
  p[P_GU].nseg = 2;
  p[P_GU].mode = GM_SILU;
  p[P_GU].ng = W + b.rf;
  p[P_WD] = gemv1(c->HH, f, f, W + b.wd, d, c->X, d, 0);
  p[P_WD].mode = GM_RESID; p[P_WD].R = c->XA; p[P_WD].ldr = d;
}

// The persistent one-sequence decode's tables, when the kernel takes this
// model on this device's CUs (one workgroup a CU): each layer's parameter
// offsets and exchange slots, two sets of exchange entries, control words.
static hipError_t persist_setup(ana_ctx* c) {
  const ana_config& cf = c->cfg;
  hipDeviceProp_t pr;
  hipError_t e = hipGetDeviceProperties(&pr, c->device);
  if (e != hipSuccess) return e;
  int coop = 0;
  if ((e = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, c->device)) != hipSuccess) return e;
  const uint32_t G = (uint32_t)std::min(pr.multiProcessorCount, 256);
  const bool exact = c->mode == ANA_EXACT_FP32;
  if (!coop || !decode1_fits(cf, G, exact)) return hipSuccess;
  int rate_khz = 0;   // the constant-rate clock the kernel's waits are timed by
  if ((e = hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, c->device)) != hipSuccess) return e;
  if (rate_khz <= 0) return hipSuccess;
  c->p_tmo = (uint64_t)rate_khz * 2000ull;
  const uint32_t d = cf.d, f = cf.f, hd = d / cf.heads, np = decode1_pieces(cf, G);
  // bf16 pieces are 16 bytes of eight values: rows start on 16 bytes when
  // d and f are multiples of 8 and the matrix does
  if (c->Wh && (d % 8 || f % 8)) return hipSuccess;
  std::vector<PLayer> t(cf.layers);
  uint64_t en = 0;
  for (uint32_t l = 0; l < cf.layers; l++) {
    const Blk& b = c->blk[l];
    PLayer& P = t[l];
    P.ra = b.ra; P.wq = b.wq; P.wa = b.wa; P.lam = b.lam; P.gq = b.gq; P.gk = b.gk; P.sink = b.sink;
    P.wo = b.wo; P.rf = b.rf; P.wg = b.wg; P.wd = b.wd;
    P.soff = c->layer_off[l];
    P.gla = b.gla ? 1u : 0u;
    P.e_qkv = en; en += (b.gla ? 4ull : 3ull) * d;
    // the attention's partials (a piece's max, sum and hd columns; exact:
    // the piece's raw scores)
    if (!b.gla) { P.e_part = en; en += (uint64_t)cf.heads * np * std::max(hd + 2, (cf.ctx + np - 1) / np); }
    P.e_o = en; en += d;
    P.e_xa = en; en += d;
    P.e_hh = en; en += f;
    P.e_x = en; en += d;
  }
  if (c->Wh) {
    // the bf16 matrices past the first layer: in place where they start on
    // 16 bytes, else copied into Wp on 16 bytes (in the 115M's layout the
    // attention layers' 12 sinks shift every later matrix by 8 bytes)
    struct Mat { uint64_t off, n, *at; };
    std::vector<Mat> ms;
    for (uint32_t l = 1; l < cf.layers; l++) {
      const Blk& b = c->blk[l];
      PLayer& P = t[l];
      ms.push_back({b.wq, 3ull * d * d, &P.hq});
      if (b.gla) ms.push_back({b.wa, (uint64_t)d * d, &P.ha});
      ms.push_back({b.wo, (uint64_t)d * d, &P.ho});
      ms.push_back({b.wg, 2ull * f * d, &P.hg});
      ms.push_back({b.wd, (uint64_t)d * f, &P.hd});
    }
    uint64_t need = 0;
    for (const Mat& m : ms)
      if (m.off % 8) need += (m.n + 7) & ~7ull;
    if (need && (e = dalloc(&c->Wp, need)) != hipSuccess) return e;
    uint64_t at = 0;
    for (const Mat& m : ms) {
      if (m.off % 8 == 0) {
        *m.at = (uint64_t)(uintptr_t)(c->Wh + m.off);
        continue;
      }
      if ((e = hipMemcpyAsync(c->Wp + at, c->Wh + m.off, 2 * m.n, hipMemcpyDeviceToDevice, c->st)) != hipSuccess)
        return e;
      *m.at = (uint64_t)(uintptr_t)(c->Wp + at);
      at += (m.n + 7) & ~7ull;
    }
  }
  c->e_key = en;
  en += G;
  c->ll_par = (en + 63) & ~63ull;
  if ((e = dalloc(&c->d_play, cf.layers)) != hipSuccess) return e;
  c->ll_bytes = 2 * c->ll_par * sizeof(unsigned long long);
  if ((e = uc_take(c->device, c->ll_bytes, (void**)&c->d_ll)) != hipSuccess) {
    c->d_ll = nullptr;
    return e;
  }
  if ((e = dalloc(&c->d_ctl, 4)) != hipSuccess) return e;
  if ((e = hipMemcpyAsync(c->d_play, t.data(), sizeof(PLayer) * t.size(), hipMemcpyHostToDevice, c->st)) != hipSuccess)
    return e;
  if ((e = launch_zero_u64(c->d_ll, (uint32_t)(2 * c->ll_par), c->st)) != hipSuccess) return e;
  c->pG = G;
  c->pnp = np;
  c->persist = true;
  return hipSuccess;
}

// algorithmic bytes of one decode step of one sequence: every weight once
// (the head reads all of the tied embedding; in ANA_BF16 two bytes a weight
// outside the fp32 block), the GLA states read and written, the live K and
// V rows read and the new ones written
static double step_bytes(const ana_ctx* c, uint64_t pos) {
  const ana_config& cf = c->cfg;
  const double hd = (double)cf.d / cf.heads;
  double b = c->Wh ? 2.0 * (double)(c->P + cf.d) + 2.0 * (double)(c->fp32_hi - c->fp32_lo)
                   : 4.0 * (double)(c->P + cf.d);
  const uint64_t live = std::min<uint64_t>(pos, cf.ctx - 1) + 1;
  for (uint32_t l = 0; l < cf.layers; l++)
    b += c->blk[l].gla ? 8.0 * cf.heads * hd * hd : 4.0 * cf.d * (2.0 * live + 2.0);
  return b;
}

// every layer product's packed weights and the head's (final norm, tied
// embedding), in one allocation
static hipError_t pack_weights(ana_ctx* c) {
  const ana_config& cf = c->cfg;
  uint64_t total = 0;
  std::vector<GemvArgs> all;
  for (uint32_t l = 0; l <= cf.layers; l++) {
    GemvArgs p[4];
    uint32_t np = 4;
    if (l < cf.layers) {
      layer_products(c, l, p);
    } else {
      p[0] = gemv1(c->X, cf.d, cf.d, c->W, cf.vocab, c->LG, cf.vocab, 0);
      p[0].ng = c->W + c->fin;
      np = 1;
    }
    for (uint32_t i = 0; i < np; i++) {
      const GemvArgs& g = p[i];
      if (g.K % 128) continue;
      const int bf = reads_bf16(c, g);
      c->pk[g.seg[0].W] = ana_ctx::PkEnt{total, g.seg[0].rows, g.nseg > 1 ? g.seg[1].rows : 0u, g.nseg,
                                         g.mode == GM_SILU ? 1u : 0u, g.K, g.ng, bf};
      total += (pack_bytes(g, bf) + 255) & ~255ull;
      all.push_back(g);
    }
  }
  if (all.empty()) return hipSuccess;
  hipError_t e = hipMalloc(&c->PK, total);
  if (e != hipSuccess) return e;
  for (const GemvArgs& g : all) {
    const ana_ctx::PkEnt& pe = c->pk[g.seg[0].W];
    if ((e = launch_pack(g, static_cast<char*>(c->PK) + pe.off, pe.bf, c->st)) != hipSuccess) return e;
  }
  return hipSuccess;
}

// RMSNorm(X; g) then the product: inside the product for small batches,
// else a norm kernel into XN first
static int norm_gemv(ana_ctx* c, const float* X, const float* g, GemvArgs a, uint32_t kind,
                     bool chunk = false) {
  a.X = X;
  a.ldx = c->cfg.d;
  a.ng = g;
  HIPCHK(c, gemv_timed(c, a, kind, chunk));
  return ANA_OK;
}

// A prefill chunk of one sequence inside a batch of rows: sequence seq at
// positions pos0.., rows row0 .. row0 + T of the workspaces.
struct Seg {
  uint32_t seq, pos0, row0, T;
};

// every layer for B rows of X (embedded already). Decode (segs == nullptr):
// row b is sequence seq[b] at position pos[b] (device arrays). Prefill:
// the rows are chunks of several sequences (segs); the products run over all
// B rows at once (row-wise the same as one chunk at a time), the GLA and
// attention per chunk.
static int run_layers(ana_ctx* c, uint32_t B, const uint32_t* seq, const uint32_t* pos,
                      const std::vector<Seg>* segs) {
  const ana_config& cf = c->cfg;
  const uint32_t d = cf.d, f = cf.f;
  const float* W = c->W;
  const bool chunk = segs != nullptr;
  // ANA_BF16 prefill steps whose products run on the bf16 tiles: the mixes
  // write Wo's operand in bf16 and the residual products the next norm's
  c->nx_of = nullptr;
  c->oh_ok = false;
  const bool bf_ops = c->d_oh && chunk && B >= 128 && B <= c->rows && d % 64 == 0;
  // a fast mode's prefill step: the GLA scan's sub-chunk table and each row's
  // sequence and position, uploaded once for every layer
  uint32_t nsub = 0;
  bool fresh_all = true, gla_run = true;
  if (chunk && fast_mode(c)) {
    if (segs->size() > c->seg_cap) return fail(c, ANA_EINVAL, "prefill step of %zu chunks (at most %u)", segs->size(), c->seg_cap);
    c->h_gtab.clear();
    c->h_grun.clear();
    c->h_atab.clear();
    // attention tile rows: 128 on the bf16 flash kernel, else 64
    const uint32_t fq = attn_flash_tile_rows(c->mode == ANA_BF16, d / cf.heads);
    c->h_rseq.resize(B);
    c->h_rpos.resize(B);
    for (uint32_t si = 0; si < segs->size(); si++) {
      const Seg& sg = (*segs)[si];
      const uint32_t ns = (sg.T + kGlaSub - 1) / kGlaSub;
      for (uint32_t j = 0; j < ns; j++)
        c->h_gtab.push_back(GlaSub{sg.row0 + j * kGlaSub, std::min(kGlaSub, sg.T - j * kGlaSub), j, ns, sg.seq, si, 0, 0});
      c->h_grun.push_back(GlaRun{sg.row0, sg.T, sg.seq, 0});
      if (sg.T > kGlaRunMaxT) gla_run = false;
      for (uint32_t t = 0; t < sg.T; t++) {
        c->h_rseq[sg.row0 + t] = sg.seq;
        c->h_rpos[sg.row0 + t] = sg.pos0 + t;
      }
      for (uint32_t t = 0; t < sg.T; t += fq)
        c->h_atab.push_back(AttnTile{sg.seq, sg.pos0 + t, sg.row0 + t, std::min(fq, sg.T - t)});
      const uint64_t last = (uint64_t)sg.pos0 + sg.T - 1;
      if (last >= cf.ctx) fresh_all = false;
    }
    nsub = (uint32_t)c->h_gtab.size();
    if (nsub > c->gsub_cap) return fail(c, ANA_EINVAL, "prefill step of %u sub-chunks (at most %u)", nsub, c->gsub_cap);
    if (c->h_atab.size() > c->atab_cap) return fail(c, ANA_EINVAL, "prefill step of %zu attention tiles (at most %u)", c->h_atab.size(), c->atab_cap);
    if (fresh_all && !c->h_atab.empty())
      HIPCHK(c, hipMemcpyAsync(c->d_atab, c->h_atab.data(), sizeof(AttnTile) * c->h_atab.size(), hipMemcpyHostToDevice, c->st));
    if (gla_run)
      HIPCHK(c, hipMemcpyAsync(c->d_grun, c->h_grun.data(), sizeof(GlaRun) * c->h_grun.size(), hipMemcpyHostToDevice, c->st));
    else
      HIPCHK(c, hipMemcpyAsync(c->d_gtab, c->h_gtab.data(), sizeof(GlaSub) * nsub, hipMemcpyHostToDevice, c->st));
    HIPCHK(c, hipMemcpyAsync(c->d_rseq, c->h_rseq.data(), 4 * (size_t)B, hipMemcpyHostToDevice, c->st));
    HIPCHK(c, hipMemcpyAsync(c->d_rpos, c->h_rpos.data(), 4 * (size_t)B, hipMemcpyHostToDevice, c->st));
  }
  for (uint32_t l = 0; l < cf.layers; l++) {
    const Blk& b = c->blk[l];
    GemvArgs p[4];
    layer_products(c, l, p);
    for (GemvArgs& g : p) g.B = B;
    // norm, then q|k|v (+ the gate's z): dd.gla / dd.sm `pre`
    if (int r = norm_gemv(c, c->X, W + b.ra, p[P_QKV], ANA_K_GEMV, chunk)) return r;
    if (b.gla && !chunk) {
      // S read and written once per sequence, q|k|v|z in, o out
      ProfScope ps(c, ANA_K_GLA, (double)B * (8.0 * cf.heads * (d / cf.heads) * (d / cf.heads) + 4.0 * 5 * d));
      if (fast_path(c, B))
        HIPCHK(c, launch_gla_fast(c->QKV, c->Z, cf.rglru ? W + b.lam : nullptr, sref(c, l), seq,
                                  c->O, d, cf.heads, cf.rglru, B, c->st));
      else if (fast_mode(c) && d == 64 * cf.heads)
        HIPCHK(c, launch_gla_wfast(c->QKV, c->Z, cf.rglru ? W + b.lam : nullptr, sref(c, l), seq,
                                   c->O, d, cf.heads, cf.rglru, B, c->st));
      else
        HIPCHK(c, launch_gla_step(c->QKV, c->Z, cf.rglru ? W + b.lam : nullptr, sref(c, l), seq,
                                  c->O, d, cf.heads, cf.rglru, B, c->st));
    } else if (b.gla && fast_mode(c)) {
      // every chunk of the step at once: a workgroup per (head, chunk)
      // through its sub-chunks, or the closed-form chunked scan
      if (gla_run) {
        HIPCHK(c, launch_gla_run(c->QKV, c->Z, cf.rglru ? W + b.lam : nullptr, sref(c, l), c->O,
                                 bf_ops ? c->d_oh : nullptr, c->d_grun, (uint32_t)c->h_grun.size(), c->rows, d,
                                 cf.heads, cf.rglru, c->st));
        c->oh_ok = bf_ops;
      } else
        HIPCHK(c, launch_gla_scan(c->QKV, c->Z, cf.rglru ? W + b.lam : nullptr, sref(c, l), c->O, c->gla,
                                  c->d_gtab, nsub, d, cf.heads, cf.rglru, c->st));
    } else if (b.gla) {
      for (const Seg& sg : *segs) {
        float* S = c->state + (uint64_t)sg.seq * c->seq_stride + c->layer_off[l];
        HIPCHK(c, launch_gla_chunk(c->QKV + (size_t)sg.row0 * 3 * d, c->Z + (size_t)sg.row0 * d,
                                   cf.rglru ? W + b.lam : nullptr, S, c->O + (size_t)sg.row0 * d, d,
                                   cf.heads, cf.rglru, sg.T, c->st));
      }
    } else {
      AttnArgs a{};
      a.gq = cf.qk ? W + b.gq : nullptr;
      a.gk = cf.qk ? W + b.gk : nullptr;
      a.sink = cf.sinks ? W + b.sink : nullptr;
      a.KV = sref(c, l);
      a.d = d; a.heads = cf.heads; a.ctx = cf.ctx;
      a.ss = c->d_ss; a.pm = c->d_pm; a.ss_rows = c->wb;
      a.part_cap = c->part_cap;
      if (!chunk) {
        // each sequence's write, then its attention (dd.sm.write, dd.sm.attend)
        a.QKV = c->QKV; a.O = c->O; a.B = B; a.seq = seq; a.pos = pos; a.write_kv = 1;
        ProfScope ps(c, ANA_K_ATTN, c->attn_bytes);
        if (fast_path(c, B)) {
          a.part = c->d_part;
          HIPCHK(c, launch_attn_fast(a, c->st));
        } else if (fast_mode(c)) {
          a.part = c->d_part;
          HIPCHK(c, launch_attn_rows(a, c->attn_split || cf.ctx > kAttnRowsMaxCtx, c->st));
        } else {
          HIPCHK(c, launch_attn(a, c->st));
        }
      } else if (fast_mode(c) && fresh_all) {
        // no chunk reaches the ring's wrap: every row's write, then every
        // row's attention over the splits up to the step's last position
        a.QKV = c->QKV; a.O = c->O; a.B = B; a.seq = c->d_rseq; a.pos = c->d_rpos; a.write_kv = 0;
        HIPCHK(c, launch_kv_write_fast(a, c->st));
        a.Oh = bf_ops ? c->d_oh : nullptr;
        HIPCHK(c, launch_attn_flash(a, c->d_atab, (uint32_t)c->h_atab.size(), c->mode == ANA_BF16, c->st));
        c->oh_ok = bf_ops;
      } else {
        for (const Seg& sg : *segs) {
          const bool fresh = (uint64_t)sg.pos0 + sg.T <= cf.ctx;
          const bool fast_chunk = fast_mode(c) && sg.T > kSmallB;
          if (fresh) {
            // before the ring wraps: every row's write, then every row's
            // attention (dd.sm.writes, then dd.sm.rows)
            a.QKV = c->QKV + (size_t)sg.row0 * 3 * d; a.O = c->O + (size_t)sg.row0 * d; a.B = sg.T;
            a.seq = nullptr; a.seq0 = sg.seq; a.pos = nullptr; a.pos0 = sg.pos0; a.write_kv = 0;
            HIPCHK(c, launch_kv_write(a, c->st));
            if (fast_chunk) {
              a.part = c->d_part;
              HIPCHK(c, launch_attn_fast(a, c->st));
            } else {
              HIPCHK(c, launch_attn(a, c->st));
            }
          } else {
            // past the wrap: each token's write and attention in turn (dd.sm.toks)
            for (uint32_t t = 0; t < sg.T; t++) {
              a.QKV = c->QKV + (size_t)(sg.row0 + t) * 3 * d; a.O = c->O + (size_t)(sg.row0 + t) * d;
              a.seq = nullptr; a.seq0 = sg.seq; a.pos = nullptr; a.pos0 = sg.pos0 + t; a.B = 1;
              a.write_kv = 1;
              HIPCHK(c, launch_attn(a, c->st));
            }
          }
        }
      }
    }
    // M.tail: xa = x + Wo o; hh = silu(g) * u on norm(xa); x = xa + Wd hh
    HIPCHK(c, gemv_timed(c, p[P_WO], ANA_K_GEMV, chunk, bf_ops ? W + b.rf : nullptr));
    if (int r = norm_gemv(c, c->XA, W + b.rf, p[P_GU], ANA_K_GEMV, chunk)) return r;
    HIPCHK(c, gemv_timed(c, p[P_WD], ANA_K_GEMV, chunk, bf_ops && l + 1 < cf.layers ? W + c->blk[l + 1].ra : nullptr));
  }
  return ANA_OK;
}

// head on B rows of src: final RMSNorm, then the tied embedding. With
// `greedy`, small batches also leave dd.pick's argmax keys in d_amax (the
// caller cleared them), larger ones dd.top's picks in d_pick.
// the head's product over B rows of src (final norm, tied embedding)
static GemvArgs head_args(const ana_ctx* c, const float* src, uint32_t B) {
  const ana_config& cf = c->cfg;
  GemvArgs h = gemv1(src, cf.d, cf.d, c->W, cf.vocab, c->LG, cf.vocab, B);
  h.ng = c->W + c->fin;
  return h;
}

// Greedy picks from the head's argmax keys (dd.pick's order, no pass over
// the stored logits): small batches, and the fast modes' wide head over
// packed weights (5 .. kPwMaxB - 1 rows); else k_top over the logits.
static bool head_keys(const ana_ctx* c, const float* src, uint32_t B) {
  if (B <= kSmallB) return true;
  if (!fast_mode(c) || B >= kPwMaxB) return false;
  GemvArgs h = head_args(c, src, B);
  h.amax = c->d_amax;
  return head_pw_fits(h) && find_pk(c, h) != nullptr;
}

static int run_head(ana_ctx* c, const float* src, uint32_t B, bool greedy) {
  GemvArgs h = head_args(c, src, B);
  const bool keys = greedy && head_keys(c, src, B);
  if (keys) h.amax = c->d_amax;
  if (int r = norm_gemv(c, src, c->W + c->fin, h, ANA_K_HEAD)) return r;
  if (greedy && !keys) HIPCHK(c, launch_top(c->LG, c->cfg.vocab, B, c->d_pick, c->st));
  return ANA_OK;
}

// algorithmic bytes of one softmax layer's attention for rows at these
// positions: the live K and V rows read, the new k and v written, q in, o out
static double attn_bytes_of(const ana_ctx* c, const uint32_t* pos, uint32_t n, uint32_t plus) {
  const ana_config& cf = c->cfg;
  double b = 0.0;
  for (uint32_t i = 0; i < n; i++) {
    const uint64_t p = (uint64_t)pos[i] + plus;
    const uint64_t live = std::min<uint64_t>(p, cf.ctx - 1) + 1;
    b += 4.0 * cf.d * (2.0 * live + 2.0 + 3.0 + 1.0);
  }
  return b;
}

static int check_seqs(ana_ctx* c, const char* fn, uint32_t n, const uint32_t* seq) {
  if (n == 0 || n > c->max_seqs || !seq) return fail(c, ANA_EINVAL, "%s: %u sequences (1..%u)", fn, n, c->max_seqs);
  std::vector<uint8_t> seen(c->max_seqs, 0);
  for (uint32_t i = 0; i < n; i++) {
    if (seq[i] >= c->max_seqs) return fail(c, ANA_EINVAL, "%s: sequence %u outside 0..%u", fn, seq[i], c->max_seqs - 1);
    if (seen[seq[i]]++) return fail(c, ANA_EINVAL, "%s: sequence %u listed twice", fn, seq[i]);
  }
  return ANA_OK;
}

extern "C" int ana_feed(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                        const uint32_t* tok) {
  if (!c) return ANA_EINVAL;
  if (int r = check_seqs(c, "ana_feed", n, seq)) return r;
  if (!pos || !tok) return fail(c, ANA_EINVAL, "ana_feed: null argument");
  for (uint32_t i = 0; i < n; i++)
    if (tok[i] >= c->cfg.vocab) return fail(c, ANA_EINVAL, "ana_feed: token %u outside the vocabulary", tok[i]);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(c->d_seq, seq, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, hipMemcpyAsync(c->d_pos, pos, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, hipMemcpyAsync(c->d_tok, tok, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, launch_embed(c->W, c->d_tok, c->cfg.d, n, c->X, nullptr, c->st));
  if (c->prof) c->attn_bytes = attn_bytes_of(c, pos, n, 0);
  c->attn_split = split_attention(c, n, pos, 1);
  if (int r = run_layers(c, n, c->d_seq, c->d_pos, nullptr)) return r;
  HIPCHK(c, launch_scatter_rows(c->X, c->d_seq, n, c->cfg.d, c->xs, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

// dd.feeds (bend/Dense/Decode.bend:561-639) for n sequences at once. Step j
// feeds tokens [jC, (j+1)C) of every sequence that has them (C the prefill
// chunk): their rows go through each product together, the GLA and the
// attention chunk by chunk, so each sequence ends as n separate dd.feeds
// would leave it (bit for bit in ANA_EXACT_FP32: products are row-wise the
// same for any number of rows).
// the head over rows r0 .. r0 + g of X into SC, for scoring: in exact mode
// the exact product (row-wise the bits of ana_logits' head), in the fast
// modes the 128 x 128 matrix-core tiles
static int score_head(ana_ctx* c, uint32_t r0, uint32_t g) {
  const ana_config& cf = c->cfg;
  GemvArgs h = gemv1(c->X + (size_t)r0 * cf.d, cf.d, cf.d, c->W, cf.vocab, c->SC, cf.vocab, g);
  h.ng = c->W + c->fin;
  if (fast_mode(c)) {
    h.Wh0 = c->Wh;
    // ANA_BF16 at 128 rows or more: the bf16 matrix-core tiles, as the
    // layer products of a prefill step (activations rounded to bf16 with
    // the final norm's gain, as the decode head rounds them)
    if (c->Wh && c->d_sah && g >= 128 && cf.d % 64 == 0)
      HIPCHK(c, launch_gemm_dl(h, c->d_sah, c->d_rsc, c->rows, c->st));
    else
      HIPCHK(c, launch_gemm_big(h, c->st));
  } else {
    HIPCHK(c, launch_gemv(h, c->st));
  }
  return ANA_OK;
}

// With ce (scoring, Evaluate.bend's window.go): sequence i feeds its first
// len[i] - 1 tokens, and after each fed token t the head's G.lse minus the
// logit of token t + 1 goes to ce (len[i] - 1 values a sequence, in order).
static int feeds_n(ana_ctx* c, const char* fn, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                   const uint32_t* len, const uint32_t* toks, float* ce = nullptr) {
  if (n == 0) return ANA_OK;
  if (!seq || !pos || !len || !toks) return fail(c, ANA_EINVAL, "%s: null argument", fn);
  std::vector<uint8_t> seen(c->max_seqs, 0);
  std::vector<uint64_t> off(n), coff(n);
  std::vector<uint32_t> flen(n);
  uint64_t total = 0, ctot = 0;
  uint32_t maxlen = 0;
  for (uint32_t i = 0; i < n; i++) {
    if (seq[i] >= c->max_seqs) return fail(c, ANA_EINVAL, "%s: sequence %u outside 0..%u", fn, seq[i], c->max_seqs - 1);
    if (seen[seq[i]]++) return fail(c, ANA_EINVAL, "%s: sequence %u listed twice", fn, seq[i]);
    off[i] = total;
    total += len[i];
    flen[i] = ce ? (len[i] ? len[i] - 1 : 0) : len[i];
    coff[i] = ctot;
    ctot += ce ? flen[i] : 0;
    maxlen = std::max(maxlen, flen[i]);
  }
  for (uint64_t i = 0; i < total; i++)
    if (toks[i] >= c->cfg.vocab) return fail(c, ANA_EINVAL, "%s: token %u outside the vocabulary", fn, toks[i]);
  HIPCHK(c, hipSetDevice(c->device));
  const uint32_t d = c->cfg.d;
  std::vector<Seg> segs;
  std::vector<uint32_t> rows, tg, rcp;
  std::vector<uint64_t> cix;
  std::vector<float> hce;
  auto flush = [&]() -> int {
    if (segs.empty()) return ANA_OK;
    const uint32_t M = (uint32_t)rows.size();
    // each sequence's residual row is its last row of the step: the
    // (row, sequence) pairs go up with the step's tokens, and one copy
    // kernel moves every row after the layers
    rcp.clear();
    if (segs.size() > c->rows) return fail(c, ANA_EINVAL, "%s: %zu sequences in one step", fn, segs.size());
    for (const Seg& sg : segs) {
      rcp.push_back(sg.row0 + sg.T - 1);
      rcp.push_back(sg.seq);
    }
    HIPCHK(c, hipMemcpyAsync(c->d_tok, rows.data(), 4 * (size_t)M, hipMemcpyHostToDevice, c->st));
    HIPCHK(c, hipMemcpyAsync(c->d_rcp, rcp.data(), 4 * rcp.size(), hipMemcpyHostToDevice, c->st));
    HIPCHK(c, launch_embed(c->W, c->d_tok, d, M, c->X, nullptr, c->st));
    if (int r = run_layers(c, M, nullptr, nullptr, &segs)) return r;
    HIPCHK(c, launch_copy_rows(c->X, c->d_rcp, (uint32_t)segs.size(), d, c->xs, c->st));
    if (ce) {
      HIPCHK(c, hipMemcpyAsync(c->d_tgt, tg.data(), 4 * (size_t)M, hipMemcpyHostToDevice, c->st));
      for (uint32_t r0 = 0; r0 < M; r0 += c->sc_rows) {
        const uint32_t g = std::min(c->sc_rows, M - r0);
        if (int r = score_head(c, r0, g)) return r;
        HIPCHK(c, launch_ce(c->SC, c->cfg.vocab, g, c->d_tgt + r0, c->d_ce + r0, c->st));
      }
      hce.resize(M);
      HIPCHK(c, hipMemcpyAsync(hce.data(), c->d_ce, 4 * (size_t)M, hipMemcpyDeviceToHost, c->st));
    }
    // the host rows are read by the copies above before they change
    HIPCHK(c, hipStreamSynchronize(c->st));
    if (ce)
      for (uint32_t r = 0; r < M; r++) ce[cix[r]] = hce[r];
    segs.clear();
    rows.clear();
    tg.clear();
    cix.clear();
    return ANA_OK;
  };
  for (uint32_t t0 = 0; t0 < maxlen; t0 += c->chunk) {
    for (uint32_t i = 0; i < n; i++) {
      if (flen[i] <= t0) continue;
      const uint32_t T = std::min(c->chunk, flen[i] - t0);
      if (rows.size() + T > c->rows || segs.size() == c->seg_cap)
        if (int r = flush()) return r;
      segs.push_back(Seg{seq[i], pos[i] + t0, (uint32_t)rows.size(), T});
      rows.insert(rows.end(), toks + off[i] + t0, toks + off[i] + t0 + T);
      if (ce)
        for (uint32_t t = t0; t < t0 + T; t++) {
          tg.push_back(toks[off[i] + t + 1]);
          cix.push_back(coff[i] + t);
        }
    }
    // the next step's chunks start from the states this step leaves
    if (int r = flush()) return r;
  }
  return ANA_OK;
}

extern "C" int ana_feeds(ana_ctx* c, uint32_t seq, uint32_t pos, const uint32_t* toks, uint32_t len) {
  if (!c) return ANA_EINVAL;
  if (seq >= c->max_seqs) return fail(c, ANA_EINVAL, "ana_feeds: sequence %u outside 0..%u", seq, c->max_seqs - 1);
  if (len == 0) return ANA_OK;
  if (!toks) return fail(c, ANA_EINVAL, "ana_feeds: null tokens");
  return feeds_n(c, "ana_feeds", 1, &seq, &pos, &len, toks);
}

extern "C" int ana_feeds_n(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                           const uint32_t* len, const uint32_t* toks) {
  if (!c) return ANA_EINVAL;
  return feeds_n(c, "ana_feeds_n", n, seq, pos, len, toks);
}

extern "C" int ana_score_n(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                           const uint32_t* len, const uint32_t* toks, float* ce) {
  if (!c) return ANA_EINVAL;
  if (!ce && n) return fail(c, ANA_EINVAL, "ana_score_n: null output");
  return feeds_n(c, "ana_score_n", n, seq, pos, len, toks, ce);
}

static int head_of(ana_ctx* c, const char* fn, uint32_t n, const uint32_t* seq) {
  if (int r = check_seqs(c, fn, n, seq)) return r;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(c->d_seq, seq, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, launch_gather_rows(c->xs, c->d_seq, n, c->cfg.d, c->X, c->st));
  return ANA_OK;
}

extern "C" int ana_logits(ana_ctx* c, uint32_t n, const uint32_t* seq, float* out) {
  if (!c) return ANA_EINVAL;
  if (!out) return fail(c, ANA_EINVAL, "ana_logits: null output");
  if (int r = head_of(c, "ana_logits", n, seq)) return r;
  if (int r = run_head(c, c->X, n, false)) return r;
  HIPCHK(c, hipMemcpyAsync(out, c->LG, (size_t)4 * n * c->cfg.vocab, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

extern "C" int ana_stats(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* tok, float* prob,
                         uint32_t* alt, float* alt_prob) {
  if (!c) return ANA_EINVAL;
  if (!tok || !prob || !alt || !alt_prob) return fail(c, ANA_EINVAL, "ana_stats: null argument");
  if (int r = head_of(c, "ana_stats", n, seq)) return r;
  for (uint32_t i = 0; i < n; i++)
    if (tok[i] >= c->cfg.vocab) return fail(c, ANA_EINVAL, "ana_stats: token %u outside the vocabulary", tok[i]);
  if (int r = run_head(c, c->X, n, false)) return r;
  float* dp = c->d_stat;
  float* dpa = dp + c->max_seqs;
  uint32_t* dalt = reinterpret_cast<uint32_t*>(dp + 2 * (size_t)c->max_seqs);
  HIPCHK(c, hipMemcpyAsync(c->d_tgt, tok, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, launch_stats(c->LG, c->cfg.vocab, n, c->d_tgt, dp, dalt, dpa, c->st));
  HIPCHK(c, hipMemcpyAsync(prob, dp, 4 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipMemcpyAsync(alt, dalt, 4 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipMemcpyAsync(alt_prob, dpa, 4 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

extern "C" int ana_top(ana_ctx* c, uint32_t n, const uint32_t* seq, uint32_t* tok) {
  if (!c) return ANA_EINVAL;
  if (!tok) return fail(c, ANA_EINVAL, "ana_top: null output");
  if (int r = head_of(c, "ana_top", n, seq)) return r;
  HIPCHK(c, launch_zero_u64(c->d_amax, (uint32_t)(n * kAmaxPerRow), c->st));
  if (int r = run_head(c, c->X, n, true)) return r;
  if (head_keys(c, c->X, n)) HIPCHK(c, launch_keys_to_tok(c->d_amax, c->cfg.vocab, n, c->d_pick, c->st));
  HIPCHK(c, hipMemcpyAsync(tok, c->d_pick, 4 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

static PickArgs pick_args(ana_ctx* c, uint32_t n, const ana_sampling* s, uint32_t store_first) {
  PickArgs p{};
  p.logits = c->LG;
  p.vocab = c->cfg.vocab;
  p.B = n;
  p.temp = s ? s->temperature : 0.0f;
  p.topk = s ? s->top_k : 0xFFFFFFFFu;
  p.topp = s ? s->top_p : 1.0f;
  p.rng = c->d_rng;
  p.tok = c->d_pick;
  p.store_first = store_first;
  return p;
}

extern "C" int ana_pick(ana_ctx* c, uint32_t n, const uint32_t* seq, const ana_sampling* s,
                        uint64_t* rng, uint32_t* tok) {
  if (!c) return ANA_EINVAL;
  if (!s || !tok) return fail(c, ANA_EINVAL, "ana_pick: null argument");
  const bool greedy = s->temperature <= 0.0f;
  if (!greedy && !rng) return fail(c, ANA_EINVAL, "ana_pick: sampling needs rng state");
  if (int r = head_of(c, "ana_pick", n, seq)) return r;
  if (int r = run_head(c, c->X, n, false)) return r;
  if (!greedy) HIPCHK(c, hipMemcpyAsync(c->d_rng, rng, 32 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, launch_pick(pick_args(c, n, s, 0), c->st));
  HIPCHK(c, hipMemcpyAsync(tok, c->d_pick, 4 * n, hipMemcpyDeviceToHost, c->st));
  if (!greedy) HIPCHK(c, hipMemcpyAsync(rng, c->d_rng, 32 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

// one decode step of the token loop: embed the current tokens, every
// layer, the head, the pick, then advance (pos + 1, tok = pick, record the
// pick at out[step[b] * n + b] and count the row's step)
// A sampled step's LM head and pick as one launch (launch_head_pick) where
// the fused form applies: above kSmallB rows (at or below it the head is
// the one-wave GEMV over every CU, 27 us a step faster at B = 1 than the
// fused form's head on 128 workgroups), the fast modes' head over packed
// weights, a grid the GPU holds at once. 1: launched; 0: run them apart;
// < 0: an error.
static int head_pick(ana_ctx* c, uint32_t n, const PickArgs& pa) {
  if (!fast_mode(c) || !c->d_hpc || n <= kSmallB) return 0;
  GemvArgs h = head_args(c, c->X, n);
  const ana_ctx::PkEnt* pe = head_pw_fits(h) ? find_pk(c, h) : nullptr;
  if (!pe) return 0;
  double by = gemv_bytes(h);
  if (pe->bf) by -= 2.0 * h.seg[0].rows * h.K;
  ProfScope ps(c, ANA_K_HEAD, by, true);
  const hipError_t e = launch_head_pick(h, static_cast<const char*>(c->PK) + pe->off, pe->bf,
                                        HeadPick{pa, c->d_hpc, c->d_hpctl}, c->st, ps.start(), ps.stop());
  if (e == hipErrorNotSupported) return 0;
  if (e != hipSuccess) return -fail(c, ANA_EDEVICE, "launch_head_pick: %s", hipGetErrorString(e));
  return 1;
}

// after a sampled call's last synchronisation: whether a fused sampler's
// wait for its head ran out (its picks then never landed)
static int head_pick_check(ana_ctx* c, const char* fn) {
  if (!c->d_hpctl) return ANA_OK;
  uint32_t f = 0;
  HIPCHK(c, hipMemcpy(&f, c->d_hpctl, 4, hipMemcpyDeviceToHost));
  if (!f) return ANA_OK;
  HIPCHK(c, hipMemset(c->d_hpctl, 0, 4));
  return fail(c, ANA_EDEVICE, "%s: a sampler's wait for the LM head ran out", fn);
}

static int gen_step(ana_ctx* c, uint32_t n, const PickArgs& pa, bool greedy, uint32_t* out, uint32_t* step) {
  HIPCHK(c, launch_embed(c->W, c->d_tok, c->cfg.d, n, c->X, c->d_amax, c->st));
  if (int r = run_layers(c, n, c->d_seq, c->d_pos, nullptr)) return r;
  const int fused = greedy ? 0 : head_pick(c, n, pa);
  if (fused < 0) return -fused;
  if (!fused) {
    if (int r = run_head(c, c->X, n, greedy)) return r;
    if (!greedy) {
      ProfScope ps(c, ANA_K_PICK, 4.0 * n * c->cfg.vocab);
      HIPCHK(c, launch_pick(pa, c->st));
    }
  }
  AdvanceArgs ad{};
  ad.logits = c->LG;
  ad.vocab = c->cfg.vocab;
  ad.B = n;
  ad.amax = greedy && head_keys(c, c->X, n) ? c->d_amax : nullptr;
  ad.pick = c->d_pick;
  ad.greedy = greedy;
  ad.pos = c->d_pos;
  ad.tok = c->d_tok;
  ad.out = out;
  ad.step = step;
  ProfScope ps(c, ANA_K_PICK, 16.0 * n);
  HIPCHK(c, launch_advance(ad, c->st));
  return ANA_OK;
}

// ana_generate's checks, with no heap allocation (a 64k-bit bitset on the
// stack finds a sequence listed twice)
static int check_generate(ana_ctx* c, const char* fn, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                          const uint32_t* tok, uint32_t steps, const ana_sampling* s, const uint64_t* rng,
                          const uint32_t* out) {
  if (n == 0 || n > c->max_seqs || !seq) return fail(c, ANA_EINVAL, "%s: %u sequences (1..%u)", fn, n, c->max_seqs);
  if (c->max_seqs > 65536) return fail(c, ANA_EUNSUP, "%s: more than 65536 sequence slots", fn);
  uint64_t seen[1024] = {};
  for (uint32_t i = 0; i < n; i++) {
    const uint32_t q = seq[i];
    if (q >= c->max_seqs) return fail(c, ANA_EINVAL, "%s: sequence %u outside 0..%u", fn, q, c->max_seqs - 1);
    if (seen[q >> 6] >> (q & 63) & 1) return fail(c, ANA_EINVAL, "%s: sequence %u listed twice", fn, q);
    seen[q >> 6] |= 1ull << (q & 63);
  }
  if (!pos || !tok || (steps && !out)) return fail(c, ANA_EINVAL, "%s: null argument", fn);
  const bool greedy = !s || s->temperature <= 0.0f;
  if (!greedy && !rng) return fail(c, ANA_EINVAL, "%s: sampling needs rng state", fn);
  for (uint32_t i = 0; i < n; i++)
    if (tok[i] >= c->cfg.vocab) return fail(c, ANA_EINVAL, "%s: token %u outside the vocabulary", fn, tok[i]);
  return ANA_OK;
}

// the rows' sequence, position and token (and RNG words) into the context
static int gen_inputs(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos, const uint32_t* tok,
                      bool greedy, const uint64_t* rng) {
  HIPCHK(c, hipMemcpyAsync(c->d_seq, seq, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, hipMemcpyAsync(c->d_pos, pos, 4 * n, hipMemcpyHostToDevice, c->st));
  HIPCHK(c, hipMemcpyAsync(c->d_tok, tok, 4 * n, hipMemcpyHostToDevice, c->st));
  if (!greedy) HIPCHK(c, hipMemcpyAsync(c->d_rng, rng, 32 * n, hipMemcpyHostToDevice, c->st));
  return ANA_OK;
}

// ana_generate of one greedy sequence in the fast fp32 mode: the token
// loop as persistent launches (pieces of kOutSteps steps; a step whose
// logits have no maximum ends a launch, and k_advance picks it by
// Sample.argmax before the next). Returns ANA_EUNSUP, having run nothing,
// when the launch itself is refused (the caller then takes the graphs).
static int generate_persist(ana_ctx* c, const uint32_t* pos, uint32_t steps, uint32_t* out) {
  uint32_t ctl[4];
  for (uint32_t k0 = 0; k0 < steps; k0 += kOutSteps) {
    const uint32_t m = std::min(kOutSteps, steps - k0);
    HIPCHK(c, launch_zero_u32(c->d_step, 1, c->st));
    uint32_t done = 0;
    while (done < m) {
      HIPCHK(c, launch_zero_u32(c->d_ctl, 4, c->st));
      PersistArgs pa{};
      pa.W = c->W;
      pa.Wh = c->Wh;
      pa.lay = c->d_play;
      pa.L = c->cfg.layers; pa.d = c->cfg.d; pa.f = c->cfg.f; pa.heads = c->cfg.heads; pa.ctx = c->cfg.ctx;
      pa.vocab = c->cfg.vocab; pa.rglru = c->cfg.rglru; pa.qk = c->cfg.qk; pa.sinks = c->cfg.sinks;
      pa.np = c->pnp;
      pa.exact = c->mode == ANA_EXACT_FP32 ? 1u : 0u;
      pa.fin = c->fin;
      pa.state = c->state; pa.seq_stride = c->seq_stride;
      pa.X = c->X; pa.LG = c->LG;
      pa.seq = c->d_seq; pa.pos = c->d_pos; pa.tok = c->d_tok; pa.out = c->d_out; pa.step = c->d_step;
      pa.pick = c->d_pick;
      pa.steps = m - done;
      pa.ll = c->d_ll; pa.ll_par = c->ll_par; pa.e_key = c->e_key;
      pa.epoch0 = c->epoch;
      pa.ctl = c->d_ctl;
      pa.tmo = c->p_tmo;
      pa.trace = c->d_trace;
      pa.trace_steps = c->trace_steps;
      pa.trace_phases = c->trace_phases;
      hipError_t e;
      {
        double by = 0.0;
        if (c->prof)
          for (uint32_t k = done; k < m; k++) by += step_bytes(c, (uint64_t)pos[0] + k0 + k);
        ProfScope ps(c, ANA_K_STEP, by);
        e = launch_decode1(pa, c->pG, c->st);
      }
      if (e != hipSuccess) {
        if (k0 == 0 && done == 0) {
          (void)hipGetLastError();
          return ANA_EUNSUP;
        }
        return fail(c, ANA_EDEVICE, "device fault: %s (persistent decode launch)", hipGetErrorString(e));
      }
      HIPCHK(c, hipMemcpyAsync(ctl, c->d_ctl, sizeof ctl, hipMemcpyDeviceToHost, c->st));
      HIPCHK(c, hipStreamSynchronize(c->st));
      // the next launch's entries never carry an epoch this one wrote
      c->epoch += (m - done) + 2;
      if (ctl[0] || ctl[1])
        return fail(c, ANA_ETIME,
                    "persistent decode: a wait between workgroups passed its 2 s limit at step %u of the call; "
                    "the sequence's state is partly advanced: reset it before feeding it again",
                    k0 + done + ctl[2]);
      done += ctl[2];
      if (ctl[3]) {
        // no logit reached the maximum: Sample.argmax over the stored logits
        AdvanceArgs ad{};
        ad.logits = c->LG;
        ad.vocab = c->cfg.vocab;
        ad.B = 1;
        ad.pick = c->d_pick;
        ad.greedy = 1;
        ad.pos = c->d_pos;
        ad.tok = c->d_tok;
        ad.out = c->d_out;
        ad.step = c->d_step;
        HIPCHK(c, launch_advance(ad, c->st));
        done += 1;
      }
    }
    c->h_out.resize(m);
    HIPCHK(c, hipMemcpyAsync(c->h_out.data(), c->d_out, 4 * (size_t)m, hipMemcpyDeviceToHost, c->st));
    HIPCHK(c, hipStreamSynchronize(c->st));
    for (uint32_t k = 0; k < m; k++) out[k0 + k] = c->h_out[k];
  }
  HIPCHK(c, launch_scatter_rows(c->X, c->d_seq, 1, c->cfg.d, c->xs, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

extern "C" int ana_generate(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                            const uint32_t* tok, uint32_t steps, const ana_sampling* s,
                            uint64_t* rng, uint32_t* out) {
  if (!c) return ANA_EINVAL;
  if (int r = check_generate(c, "ana_generate", n, seq, pos, tok, steps, s, rng, out)) return r;
  if (steps == 0) return ANA_OK;
  const bool greedy = !s || s->temperature <= 0.0f;
  HIPCHK(c, hipSetDevice(c->device));
  if (int r = gen_inputs(c, n, seq, pos, tok, greedy, rng)) return r;
  if (n == 1 && greedy && c->persist && !c->persist_off) {
    const int r = generate_persist(c, pos, steps, out);
    if (r != ANA_EUNSUP) return r;
    c->persist = false;   // refused (resources): the graphs from now on
  }
  c->attn_split = split_attention(c, n, pos, steps);
  const PickArgs pa = pick_args(c, n, greedy ? nullptr : s, 1);
  // capture `count` steps into a graph
  auto capture = [&](uint32_t count, hipGraphExec_t* ex) -> int {
    hipGraph_t g = nullptr;
    HIPCHK(c, hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
    int r = 0;
    for (uint32_t i = 0; i < count && !r; i++) r = gen_step(c, n, pa, greedy, c->d_out, c->d_step);
    const hipError_t ec = hipStreamEndCapture(c->st, &g);
    if (r) { if (g) (void)hipGraphDestroy(g); return r; }
    HIPCHK(c, ec);
    const hipError_t ei = hipGraphInstantiate(ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIPCHK(c, ei);
    return ANA_OK;
  };
  if (!c->prof) {
    ana_ctx::GKey key{n, pa.temp, pa.topp, pa.topk, c->d_out, c->attn_split};
    if (!c->gexec || !(c->gkey == key)) {
      if (c->gexec) { HIPCHK(c, hipGraphExecDestroy(c->gexec)); c->gexec = nullptr; }
      if (c->gexec_n) { HIPCHK(c, hipGraphExecDestroy(c->gexec_n)); c->gexec_n = nullptr; }
      if (int r = capture(1, &c->gexec)) return r;
      c->gkey = key;
    }
    // the kGraphSteps graph only for a call that replays it (one-step calls,
    // an agent loop's, never do)
    if (steps >= kGraphSteps && !c->gexec_n)
      if (int r = capture(kGraphSteps, &c->gexec_n)) return r;
  }
  // pieces of at most kOutSteps steps: d_out (allocated at ana_open) holds
  // one piece's picks, step-major; each piece's picks go to the caller
  // before the next piece starts over at step 0
  for (uint32_t k0 = 0; k0 < steps; k0 += kOutSteps) {
    const uint32_t m = std::min(kOutSteps, steps - k0);
    HIPCHK(c, launch_zero_u32(c->d_step, n, c->st));
    if (c->prof) {
      // launch by launch, each product timed by its own start/stop events
      for (uint32_t k = 0; k < m; k++) {
        c->attn_bytes = attn_bytes_of(c, pos, n, k0 + k);
        if (int r = gen_step(c, n, pa, greedy, c->d_out, c->d_step)) return r;
      }
    } else {
      uint32_t k = 0;
      for (; k + kGraphSteps <= m; k += kGraphSteps) HIPCHK(c, hipGraphLaunch(c->gexec_n, c->st));
      for (; k < m; k++) HIPCHK(c, hipGraphLaunch(c->gexec, c->st));
    }
    c->h_out.resize((size_t)n * m);
    HIPCHK(c, hipMemcpyAsync(c->h_out.data(), c->d_out, 4 * (size_t)n * m, hipMemcpyDeviceToHost, c->st));
    HIPCHK(c, hipStreamSynchronize(c->st));
    // step-major on the device, row-major for the caller
    for (uint32_t k = 0; k < m; k++)
      for (uint32_t b = 0; b < n; b++) out[(size_t)b * steps + k0 + k] = c->h_out[(size_t)k * n + b];
  }
  HIPCHK(c, launch_scatter_rows(c->X, c->d_seq, n, c->cfg.d, c->xs, c->st));
  if (!greedy) HIPCHK(c, hipMemcpyAsync(rng, c->d_rng, 32 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  if (!greedy) return head_pick_check(c, "ana_generate");
  return ANA_OK;
}

// ------------------------------------------------------------------ no-allocation token loop
//
// ana_generate_noalloc's scratch: the rows' step counters, the step-major
// picks and their row-major copy, in one file-scope device array that each
// GPU holds for the life of the process. Host code uses its address as
// hipGetSymbolAddress gives it on each device (g_scratch), never the
// array's name.
static constexpr uint32_t kNoAllocWords = 1u << 18;   // 1 MB of uint32
static __device__ __align__(256) uint32_t scratch[kNoAllocWords];
static constexpr int kMaxDevices = 64;
static uint32_t* g_scratch[kMaxDevices] = {};
static std::mutex g_scratch_mu;
// held by a call for its whole use of a device's array, from clearing the
// counters to the final synchronisation, so calls on one GPU from several
// threads (several contexts) take the array in turn instead of racing
static std::mutex g_scratch_use[kMaxDevices];

// once per device, with that device current (ana_open): scratch's device
// address; an error here leaves only ana_generate_noalloc unavailable
static void resolve_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device]) return;
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch[device] = static_cast<uint32_t*>(p);
}

extern "C" int ana_generate_noalloc(ana_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                                    const uint32_t* tok, uint32_t steps, const ana_sampling* s,
                                    uint64_t* rng, uint32_t* out) {
  if (!c) return ANA_EINVAL;
  const char* fn = "ana_generate_noalloc";
  if (int r = check_generate(c, fn, n, seq, pos, tok, steps, s, rng, out)) return r;
  if (steps == 0) return ANA_OK;
  const uint64_t cnt_words = ((uint64_t)n + 63) & ~63ull;
  const uint64_t need = cnt_words + 2ull * n * steps;
  if (need > kNoAllocWords)
    return fail(c, ANA_EINVAL, "%s: %u sequences x %u steps need %llu scratch words, at most %u", fn, n, steps,
                (unsigned long long)need, kNoAllocWords);
  uint32_t* base = c->device >= 0 && c->device < kMaxDevices ? g_scratch[c->device] : nullptr;
  if (!base) return fail(c, ANA_EDEVICE, "%s: no scratch address on device %d", fn, c->device);
  uint32_t* d_step = base;
  uint32_t* d_sm = base + cnt_words;
  uint32_t* d_rm = d_sm + (size_t)n * steps;
  const bool greedy = !s || s->temperature <= 0.0f;
  std::lock_guard<std::mutex> use(g_scratch_use[c->device]);
  HIPCHK(c, hipSetDevice(c->device));
  if (int r = gen_inputs(c, n, seq, pos, tok, greedy, rng)) return r;
  // the counters start at zero (the array keeps the last call's contents)
  HIPCHK(c, launch_zero_u32(d_step, n, c->st));
  c->attn_split = split_attention(c, n, pos, steps);
  const PickArgs pa = pick_args(c, n, greedy ? nullptr : s, 1);
  // no graphs and no timing events here: launch by launch
  const bool prof = c->prof;
  c->prof = false;
  int r = ANA_OK;
  for (uint32_t k = 0; k < steps && !r; k++) r = gen_step(c, n, pa, greedy, d_sm, d_step);
  c->prof = prof;
  if (r) return r;
  HIPCHK(c, launch_scatter_rows(c->X, c->d_seq, n, c->cfg.d, c->xs, c->st));
  HIPCHK(c, launch_picks_rows(d_sm, n, steps, d_rm, c->st));
  HIPCHK(c, hipMemcpyAsync(out, d_rm, 4 * (size_t)n * steps, hipMemcpyDeviceToHost, c->st));
  if (!greedy) HIPCHK(c, hipMemcpyAsync(rng, c->d_rng, 32 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  if (!greedy) return head_pick_check(c, "ana_generate_noalloc");
  return ANA_OK;
}

extern "C" int ana_prof(ana_ctx* c, int on) {
  if (!c) return ANA_EINVAL;
  HIPCHK(c, hipStreamSynchronize(c->st));
  c->prof = on != 0;
  c->recs.clear();
  for (uint32_t k = 0; k < ANA_K_KINDS; k++) {
    c->acc_n[k] = 0;
    c->acc_ms[k] = 0.0;
    c->acc_bytes[k] = 0.0;
  }
  return ANA_OK;
}

extern "C" int ana_prof_read(ana_ctx* c, uint32_t kind, uint64_t* launches, double* ms,
                             double* bytes) {
  if (!c || kind >= ANA_K_KINDS) return ANA_EINVAL;
  HIPCHK(c, hipStreamSynchronize(c->st));
  uint64_t n = c->acc_n[kind];
  double t = c->acc_ms[kind], by = c->acc_bytes[kind];
  for (size_t i = 0; i < c->recs.size(); i++) {
    if (c->recs[i].kind != kind) continue;
    float e = 0.0f;
    HIPCHK(c, hipEventElapsedTime(&e, c->ev[2 * i], c->ev[2 * i + 1]));
    n++;
    t += e;
    by += c->recs[i].bytes;
  }
  if (launches) *launches = n;
  if (ms) *ms = t;
  if (bytes) *bytes = by;
  return ANA_OK;
}

extern "C" int ana_trace(ana_ctx* c, uint32_t steps) {
  if (!c) return ANA_EINVAL;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->st));
  if (c->d_trace) (void)hipFree(c->d_trace);
  c->d_trace = nullptr;
  c->trace_steps = c->trace_phases = 0;
  if (steps == 0) return ANA_OK;
  if (!c->persist) return fail(c, ANA_EUNSUP, "ana_trace: this context has no persistent decode kernel");
  if (steps > 64) return fail(c, ANA_EINVAL, "ana_trace: %u steps, at most 64", steps);
  const uint32_t ph = decode1_phases(c->cfg);
  const size_t n = (size_t)steps * ph * c->pG * 4;
  if (c->cfg.layers > 32) return fail(c, ANA_EUNSUP, "ana_trace: %u layers, at most 32", c->cfg.layers);
  if (hipMalloc(&c->d_trace, 4 * n) != hipSuccess) {
    (void)hipGetLastError();
    c->d_trace = nullptr;
    return fail(c, ANA_ENOMEM, "ana_trace: out of device memory");
  }
  HIPCHK(c, launch_zero_u32(c->d_trace, (uint32_t)n, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  c->trace_steps = steps;
  c->trace_phases = ph;
  return ANA_OK;
}

extern "C" int ana_trace_read(ana_ctx* c, uint32_t* out, size_t cap, uint32_t dims[3]) {
  if (!c || !dims) return ANA_EINVAL;
  dims[0] = c->trace_steps;
  dims[1] = c->trace_phases;
  dims[2] = c->trace_steps ? c->pG : 0;
  const size_t n = (size_t)dims[0] * dims[1] * dims[2] * 4;
  if (n == 0 || !out) return ANA_OK;   // (no buffer: the extents only)
  if (cap < n) return fail(c, ANA_EINVAL, "ana_trace_read: %zu stamps, room for %zu", n, cap);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(out, c->d_trace, 4 * n, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

// a streaming read of n4 float4s, grid-stride (16-byte loads, a wave's
// loads 1 KB contiguous); the sum keeps the loads, and the store never
// happens for the zero-filled buffer the probe reads
__global__ __launch_bounds__(256) void k_stream_read(const float4* __restrict__ p, size_t n4, float* sink) {
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
    const float4 v = p[i];
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  const float sum = (acc.x + acc.y) + (acc.z + acc.w);
  if (sum != 0.0f) sink[0] = sum;
}

extern "C" int ana_probe_reread(int device, uint64_t bytes, uint32_t reps, double* gbs) {
  if (!gbs || reps == 0 || bytes < 4096 || bytes % 16) return ANA_EINVAL;
  if (hipSetDevice(device) != hipSuccess) return ANA_EDEVICE;
  void* buf = nullptr;
  float* sink = nullptr;
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int r = ANA_EDEVICE;
  if (hipMalloc(&buf, bytes) != hipSuccess) return ANA_ENOMEM;
  if (hipMalloc(reinterpret_cast<void**>(&sink), 16) == hipSuccess && hipStreamCreate(&st) == hipSuccess &&
      hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess &&
      hipMemsetAsync(buf, 0, bytes, st) == hipSuccess) {
    const size_t n4 = bytes / 16;
    // one untimed pass brings the buffer into whatever cache holds it
    hipLaunchKernelGGL(k_stream_read, dim3(8192), dim3(256), 0, st, static_cast<const float4*>(buf), n4, sink);
    bool ok = hipGetLastError() == hipSuccess && hipEventRecord(e0, st) == hipSuccess;
    for (uint32_t i = 0; ok && i < reps; i++) {
      hipLaunchKernelGGL(k_stream_read, dim3(8192), dim3(256), 0, st, static_cast<const float4*>(buf), n4, sink);
      ok = hipGetLastError() == hipSuccess;
    }
    float ms = 0.0f;
    if (ok && hipEventRecord(e1, st) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
        hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0.0f) {
      *gbs = (double)bytes * reps / (ms * 1e-3) / 1e9;
      r = ANA_OK;
    }
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (st) {
    (void)hipStreamSynchronize(st);
    (void)hipStreamDestroy(st);
  }
  if (sink) (void)hipFree(sink);
  (void)hipFree(buf);
  return r;
}

extern "C" int ana_state(ana_ctx* c, uint32_t seq, uint32_t layer, float* out, size_t n) {
  if (!c || !out) return ANA_EINVAL;
  if (seq >= c->max_seqs || layer > c->cfg.layers) return fail(c, ANA_EINVAL, "ana_state: no such sequence or layer");
  const float* src;
  size_t cnt;
  if (layer == c->cfg.layers) {
    src = c->xs + (uint64_t)seq * c->cfg.d;
    cnt = c->cfg.d;
  } else {
    src = c->state + (uint64_t)seq * c->seq_stride + c->layer_off[layer];
    const uint64_t end = layer + 1 < c->cfg.layers ? c->layer_off[layer + 1] : c->seq_stride;
    cnt = end - c->layer_off[layer];
  }
  if (n != cnt) return fail(c, ANA_EINVAL, "ana_state: layer %u holds %zu floats, not %zu", layer, cnt, n);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(out, src, 4 * cnt, hipMemcpyDeviceToHost, c->st));
  HIPCHK(c, hipStreamSynchronize(c->st));
  return ANA_OK;
}

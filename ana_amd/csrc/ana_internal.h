// Internal declarations shared by libana's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/ana.h"

namespace ana {

// One layer's parameter offsets in the FTC2 vector (BP of
// bend/Dense/Layout.bend:99-100, placed by BP.gla.at / BP.sm.at, 627-655).
struct Blk {
  bool gla;
  uint64_t ra, wq, wk, wv, wo, wa, lam, gq, gk, sink, rf, wg, wu, wd, end;
};

uint64_t params_of(const ana_config& c);                       // Config.params
std::string model_id_of(const ana_config& c);                  // Config.model_id
std::vector<Blk> layout_of(const ana_config& c, uint64_t* fin); // BP.list, blocks.end

// A checkpoint read from disk: config, step, and the parameter bytes exactly
// as stored (big-endian f32), so the device does the byte swap.
struct Ftc2 {
  ana_config cfg;
  uint64_t step = 0;
  std::vector<uint8_t> raw;   // P * 4 bytes, big-endian
};
// Returns "" on success, else the reference's message.
std::string read_ftc2(const char* path, Ftc2* out);
// the manifest alone ("" or the reason it could not be read)
std::string read_manifest(const char* path, ana_manifest* out);

// ---------------------------------------------------------------- kernels
// Every kernel computes in IEEE f32 with products and sums rounded
// separately (compiled with -ffp-contract=off) and exp/log through double,
// so each output takes the reference's F32 steps in the reference's order.

// A matrix-vector product over a batch of rows, y[b][o] = sum_q x[b][q] W[o][q]
// (q ascending from 0.0f), over up to two row segments.
struct GemvSeg {
  const float* W;     // [rows][K] row-major
  uint32_t rows;
  float* Y;           // output rows: Y[b * ldy + o]
  uint32_t ldy;
};
enum GemvMode : uint32_t {
  GM_PLAIN = 0,       // y = s
  GM_RESID = 1,       // y = r + s (add2 of bend/Dense/Model.bend:44-45)
  GM_SILU = 2,        // seg0 gate rows, seg1 up rows: y = silu(g) * u
};
struct GemvArgs {
  const float* X;     // [B][ldx]
  uint32_t ldx;
  uint32_t K;
  GemvSeg seg[2];
  uint32_t nseg;
  uint32_t mode;
  const float* R;     // GM_RESID: residual rows R[b * ldr + o]
  uint32_t ldr;
  uint32_t B;         // batch rows
  const float* ng;    // RMSNorm gains over K, applied to X first
  unsigned long long* amax;  // per batch row (amax_at): argmax keys of seg 0's outputs
                             // (small batches only)
  const uint16_t* Wh0;       // fast products: the segments' rows as bfloat16
  const uint16_t* Wh1;       // (nullptr: read the fp32 rows)
  __bf16* Yh;                // ANA_BF16 prefill, SiLU: the outputs in bf16 only (seg0.Y not
                             // written), [B][seg0.rows]
  const __bf16* Xh;          // ANA_BF16 prefill: X already in bf16, [B][K] (with a norm: the
                             // gain applied, the scales from sspi)
  __bf16* Yn;                // ANA_BF16 prefill, k_gemm_dl on full tiles, one segment: the
                             // outputs times gn in bf16 too, [B][seg0.rows] (the next
                             // product's operand, k_split's work done here)
  const float* gn;           // that next product's norm gain
  float* ssp;                // the rows' partial sums of the outputs' squares, [B][nsp]: one
                             // a (128-column tile, 64-column half), nsp = seg0.rows / 64
  const float* sspi;         // with Xh and a norm: the producer's partials, nspi a row, the
  uint32_t nspi;             // norm scale 1 / sqrt(their sum / K + 1e-5)
};
// The two row segments as plain values (a runtime index into GemvArgs.seg
// would send every lookup through memory).
struct Segs {
  const float* W0;
  const float* W1;
  uint32_t rows0, rows1, nseg, silu, K;
  __device__ __forceinline__ explicit Segs(const GemvArgs& a)
      : W0(a.seg[0].W), W1(a.seg[1].W), rows0(a.seg[0].rows), rows1(a.seg[1].rows), nseg(a.nseg),
        silu(a.mode == GM_SILU), K(a.K) {}
  // weight row of tile row r of workgroup tile t (R rows per tile; with
  // silu the first R/2 rows are gate rows j, the rest up rows j); written
  // with selects only, so loads that depend on it stay in straight-line code
  __device__ __forceinline__ bool row(uint32_t R, uint32_t t, uint32_t r, const float** w,
                                      uint32_t* seg, uint32_t* lr) const {
    const uint32_t half = R >> 1;
    const uint32_t vs = t * R + r;
    const uint32_t sg_s = r >= half ? 1u : 0u;
    const uint32_t j_s = t * half + r - sg_s * half;
    const uint32_t sg_p = vs >= rows0 ? 1u : 0u;
    const uint32_t j_p = vs - sg_p * rows0;
    const uint32_t sg = silu ? sg_s : sg_p;
    const uint32_t j = silu ? j_s : j_p;
    const bool ok = j < (sg ? rows1 : rows0) && (sg == 0 || nseg > 1);
    *w = (sg ? W1 : W0) + (size_t)j * K;
    *seg = sg;
    *lr = j;
    return ok;
  }
};

// small-batch products take the norm and the argmax inside (B <= 4)
constexpr uint32_t kSmallB = 4;
// e0/e1: optional start/stop events recorded by the launch itself
hipError_t launch_gemv(const GemvArgs& a, hipStream_t st, hipEvent_t e0 = nullptr,
                       hipEvent_t e1 = nullptr);

// Greedy argmax keys: each batch row has kAmaxSlots keys, kAmaxStride
// apart (separate cache lines), and a workgroup raises slot
// blockIdx.x % kAmaxSlots, so thousands of workgroups do not queue on one
// address; the pick is the max over a row's slots.
constexpr uint32_t kAmaxSlots = 32, kAmaxStride = 16;
__host__ __device__ inline size_t amax_at(uint32_t b, uint32_t slot) {
  return ((size_t)b * kAmaxSlots + slot) * kAmaxStride;
}
constexpr size_t kAmaxPerRow = (size_t)kAmaxSlots * kAmaxStride;

// dd.pick as a key: larger value wins, then the lower index; -0 counts as
// +0 and NaN never enters (key 0 = no candidate)
__host__ __device__ inline unsigned long long argmax_key(float v, uint32_t i) {
  if (v != v) return 0ull;
  if (v == 0.0f) v = 0.0f;
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)o << 32) | (0xFFFFFFFFu - i);
}

// M.norm (bend/Dense/Model.bend:27-30) on B rows of d: y = (x * s) * g with
// s = 1 / sqrt((sum x*x) / d + 1e-5), the sum in index order
hipError_t launch_rmsnorm(const float* X, const float* g, uint32_t d, uint32_t B, float* Y,
                          hipStream_t st);

// Per-sequence state addressing: a sequence's states start at
// base + seq * seq_stride; a layer's at + layer_off.
struct StateRef {
  float* base;
  uint64_t seq_stride;
  uint64_t layer_off;
};

// X[b] = E[tok[b]]; also clears amax[b] (nullptr: nothing to clear)
hipError_t launch_embed(const float* E, const uint32_t* tok, uint32_t d, uint32_t B, float* X,
                        unsigned long long* amax, hipStream_t st);
hipError_t launch_bswap(uint32_t* w, uint64_t n, hipStream_t st);

// GLA decode step for B sequences (one token each): per-head L2 norms, the
// gate, S' = al S + kh v^T in place, o = qh^T S'.
hipError_t launch_gla_step(const float* QKV, const float* Z, const float* lam, StateRef S,
                           const uint32_t* seq, float* O, uint32_t d, uint32_t heads,
                           uint32_t rglru, uint32_t B, hipStream_t st);
// GLA over T tokens of one sequence, token after token (S kept on chip).
hipError_t launch_gla_chunk(const float* QKV, const float* Z, const float* lam, float* S,
                            float* O, uint32_t d, uint32_t heads, uint32_t rglru, uint32_t T,
                            hipStream_t st);

// Softmax attention over the ring for B (seq, pos) rows. write_kv: each
// row writes its own k (qk-normed) and v into its slot first (the decode
// step); else the slots were written before (launch_kv_write, a chunk before
// the ring wraps).
struct AttnArgs {
  const float* QKV;     // [B][3d]
  const float* gq;      // qk-norm gains (nullptr when off)
  const float* gk;
  const float* sink;    // per-head sink logits (nullptr when off)
  StateRef KV;          // K ring [ctx][d] then V ring [ctx][d]
  const uint32_t* seq;  // per row: state slot (nullptr: all rows seq0)
  uint32_t seq0;
  const uint32_t* pos;  // per row position (device)
  uint32_t pos0;        // when pos is nullptr: row b is at pos0 + b
  float* O;             // [B][d]
  __bf16* Oh;           // k_attn_flash(_bf): the outputs in bf16 only (nullptr: O)
  uint32_t d, heads, ctx, B, write_kv;
  float* ss;            // scratch [B][heads][ctx]: sc * score
  float* pm;            // scratch [B][heads][ctx / kAttnTS]: partial maxima
  uint32_t ss_rows;     // rows ss and pm hold
  float* part;          // fast attention: per split (m, l, o[hd])
  size_t part_cap;      // floats at part (the launchers reject grids that need more)
  uint32_t nsp;         // fast attention: splits in the grid, those holding
                        // slots 0 .. nsp * kFastTS - 1 (0: the whole ring)
};
// ring slots per split of the fast attention
constexpr uint32_t kFastTS = 64;
// slots per workgroup in the split attention's score pass
constexpr uint32_t kAttnTS = 128;
hipError_t launch_attn(const AttnArgs& a, hipStream_t st);
// each row's k (qk-normed when gk) and v into slot pos mod ctx (dd.sm.write)
hipError_t launch_kv_write(const AttnArgs& a, hipStream_t st);

// dd.pick over B logit rows: least index reaching the max, vocab on NaN
hipError_t launch_top(const float* logits, uint32_t vocab, uint32_t B, uint32_t* tok,
                      hipStream_t st);
// S.pick over B logit rows
struct PickArgs {
  const float* logits;  // [B][vocab]
  uint32_t vocab, B;
  float temp;
  uint32_t topk;
  float topp;
  uint64_t* rng;        // [B][4]
  uint32_t* tok;
  uint32_t store_first; // greedy as the dense engine picks: dd.top, and
                        // Sample.argmax only when dd.top answers vocab
};
hipError_t launch_pick(const PickArgs& a, hipStream_t st);
// per row b of B logit rows: G.lse(row) - row[tgt[b]] in the tree's order
// (Evaluate.bend's scoring summand)
// dc.prob.of and al.stat for B rows of logits: each row's token probability,
// its likeliest rival and the rival's probability
hipError_t launch_stats(const float* logits, uint32_t vocab, uint32_t B, const uint32_t* tok, float* p,
                        uint32_t* alt, float* palt, hipStream_t st);
hipError_t launch_ce(const float* logits, uint32_t vocab, uint32_t B, const uint32_t* tgt, float* ce,
                     hipStream_t st);

// small helpers for the token loop
hipError_t launch_gather_rows(const float* src, const uint32_t* idx, uint32_t n, uint32_t d,
                              float* dst, hipStream_t st);
hipError_t launch_scatter_rows(const float* src, const uint32_t* idx, uint32_t n, uint32_t d,
                               float* dst, hipStream_t st);
// dst row pairs[2 b + 1] = src row pairs[2 b] for b < n (pairs on the device)
hipError_t launch_copy_rows(const float* src, const uint32_t* pairs, uint32_t n, uint32_t d, float* dst,
                            hipStream_t st);
// The token loop's step end for B sequences: the pick (from the sampler's
// pick[b], or greedy: the amax key or top[b] of dd.pick, falling back to
// Sample.argmax over the logits when there is none), recorded at
// out[step[b] * B + b] (step-major), fed next (tok = pick, pos + 1); then
// step[b] + 1.
// The step indices (one a row) live in device memory, so one captured step
// serves every iteration.
struct AdvanceArgs {
  const float* logits;              // [B][vocab]
  uint32_t vocab, B;
  const unsigned long long* amax;   // greedy, keys (or nullptr)
  const uint32_t* pick;             // sampled picks, or greedy dd.pick results
  uint32_t greedy;
  uint32_t* pos;
  uint32_t* tok;
  uint32_t* out;
  uint32_t* step;                   // [B]
  uint32_t* last;                   // [B]: the pick, for ana_top-like readers
};
hipError_t launch_advance(const AdvanceArgs& a, hipStream_t st);
// n x steps step-major picks (step k, row b at sm[k * n + b]) to row-major rm
hipError_t launch_picks_rows(const uint32_t* sm, uint32_t n, uint32_t steps, uint32_t* rm, hipStream_t st);
// greedy picks from amax keys (dd.top), vocab where there is none
hipError_t launch_keys_to_tok(const unsigned long long* amax, uint32_t vocab, uint32_t B,
                              uint32_t* tok, hipStream_t st);
hipError_t launch_zero(float* p, uint64_t n, hipStream_t st);

// ---------------------------------------------------------------- fast modes
// Reassociated (tree / fused multiply-add) versions of the decode step's
// kernels for ANA_FAST_FP32 and ANA_BF16, B <= kSmallB rows (launch_gla_fast
// and launch_attn_fast reject decode steps of more rows: those paths are
// off above kSmallB).
hipError_t launch_to_bf16(const float* w, uint16_t* h, uint64_t n, hipStream_t st);
hipError_t launch_gemv_fast(const GemvArgs& a, hipStream_t st, hipEvent_t e0 = nullptr,
                            hipEvent_t e1 = nullptr);
hipError_t launch_gla_fast(const float* QKV, const float* Z, const float* lam, StateRef S,
                           const uint32_t* seq, float* O, uint32_t d, uint32_t heads,
                           uint32_t rglru, uint32_t B, hipStream_t st);
hipError_t launch_attn_fast(const AttnArgs& a, hipStream_t st);
// the fast modes' GLA step above kSmallB decode rows: one wave a (head,
// row), hd 64 (k_gla_w's layout, the fast mode's arithmetic)
hipError_t launch_gla_wfast(const float* QKV, const float* Z, const float* lam, StateRef S, const uint32_t* seq,
                            float* O, uint32_t d, uint32_t heads, uint32_t rglru, uint32_t B, hipStream_t st);
// a fast-mode prefill step's K/V ring writes (dd.sm.write over every row,
// the qk-norm's sums reassociated): hd 16, 32 or 64
hipError_t launch_kv_write_fast(const AttnArgs& a, hipStream_t st);
// Decode attention of more than kSmallB rows in the fast modes (hd 16, 32
// or 64): one workgroup per (head, row) over every live slot (ctx <=
// kAttnRowsMaxCtx: the scores stay in LDS), or with `split` one per (head,
// row, kRowsSplit slots) and a combine (a.part holds the partials: rows x
// heads x ctx / kRowsSplit x (hd + 2) floats)
constexpr uint32_t kAttnRowsMaxCtx = 8192, kRowsSplit = 256;
hipError_t launch_attn_rows(const AttnArgs& a, bool split, hipStream_t st);
// GLA over the prefill chunks of one step as a chunked scan: kGlaSub-token
// sub-chunks in parallel, then their states carried across. The table holds
// one entry per sub-chunk, those of one chunk consecutive.
constexpr uint32_t kGlaSub = 32;
// chunks a batched prefill step holds at most
constexpr uint32_t kMaxSegs = 256;
// rows the scoring head runs at once (its logits workspace)
constexpr uint32_t kScoreRows = 512;
struct GlaSub {
  uint32_t row;   // first workspace row
  uint32_t n;     // tokens (1 .. kGlaSub)
  uint32_t j;     // index inside its chunk
  uint32_t nsub;  // sub-chunks of its chunk
  uint32_t seq;   // state slot of the chunk's sequence
  uint32_t seg;   // the chunk's index in the step (its entering-state copy)
  uint32_t pad0, pad1;
};
// scratch: qt per row, D and U per (sub-chunk, head), the entering states
// per (chunk, head)
struct GlaScratch {
  float *Qt, *Dj, *Uj, *S0;
  uint32_t rows_cap, nsub_cap, nseg_cap;  // what the regions were carved for
};
// One chunk of a prefill step for k_gla_run: one workgroup per (head,
// chunk) walks its sub-chunks in order, the state in LDS. Chunks of at most
// kGlaRunMaxT tokens take it (a few sequential sub-chunks, and a tenth of
// the scan's traffic); longer ones the scan.
struct GlaRun {
  uint32_t row;   // first workspace row
  uint32_t T;     // tokens
  uint32_t seq;   // state slot
  uint32_t pad;
};
constexpr uint32_t kGlaRunMaxT = 8 * kGlaSub;
// (rows: the workspace rows QKV and Z hold)
// (Oh: the outputs in bf16 only, for a bf16 Wo operand)
hipError_t launch_gla_run(const float* QKV, const float* Z, const float* lam, StateRef S, float* O, __bf16* Oh,
                          const GlaRun* runs, uint32_t nrun, uint32_t rows, uint32_t d, uint32_t heads,
                          uint32_t rglru, hipStream_t st);
size_t gla_scan_floats(uint32_t rows, uint32_t nsub, uint32_t nseg, uint32_t d, uint32_t heads);
GlaScratch gla_scan_carve(float* p, uint32_t rows, uint32_t nsub, uint32_t nseg, uint32_t d,
                          uint32_t heads);
hipError_t launch_gla_scan(const float* QKV, const float* Z, const float* lam, StateRef S, float* O,
                           const GlaScratch& g, const GlaSub* tab, uint32_t nsub, uint32_t d,
                           uint32_t heads, uint32_t rglru, hipStream_t st);
// batched products (B > kSmallB) on the matrix cores whose K the packed
// GEMM does not take (K % 128 != 0 or K > 2048): bf16 when Wh0 is set, else
// fp32; no argmax epilogue
hipError_t launch_gemm_mfma(const GemvArgs& a, hipStream_t st, hipEvent_t e0 = nullptr,
                            hipEvent_t e1 = nullptr);
// A product's weights packed for k_gemm_pk (fp32, or bf16 with bf; the
// gains of ng folded in): pack_bytes of device memory at dst.
uint64_t pack_bytes(const GemvArgs& a, int bf);
hipError_t launch_pack(const GemvArgs& a, void* dst, int bf, hipStream_t st);
// The decode-batch GEMM over packed weights (packed with the same ng, which
// here only turns the norm scale on): K % 128 == 0, K <= 2048, X 16-byte
// aligned (gemm_pk_fits)
bool gemm_pk_fits(const GemvArgs& a);
hipError_t launch_gemm_pk(const GemvArgs& a, const void* pk, int bf, hipStream_t st, hipEvent_t e0,
                          hipEvent_t e1);
// The LM head fused with the seeded sampler (k_head_pw with PICK): the
// head's workgroups write their logits through to the level every XCD
// reads and count themselves in per 32-row block; the last `rows` of a
// block to arrive wait for the rest and run S.pick on one row each. Only
// for grids the GPU holds at once with at least as many workgroups a block
// as rows (launch_head_pick answers hipErrorNotSupported otherwise, and for
// vocabularies whose sampler geometry has no fused form).
struct HeadPick {
  PickArgs pa;                // pa.logits: the head's output rows
  unsigned long long* cnt;    // per 32-row block: arrivals, only ever added to
  uint32_t* ctl;              // set when a wait ran out
};
constexpr uint32_t kPickPollMax = 1u << 20;   // polls before a sampler's wait gives up
hipError_t launch_head_pick(const GemvArgs& a, const void* pk, int bf, const HeadPick& hp, hipStream_t st,
                            hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
// The wide form for the LM head (plain products, K % 256 == 0,
// K <= kHeadMaxK): 32 batch rows in LDS per workgroup, 16 weight tiles each
constexpr uint32_t kHeadMaxK = 1024;
bool head_pw_fits(const GemvArgs& a);
hipError_t launch_head_pw(const GemvArgs& a, const void* pk, int bf, hipStream_t st, hipEvent_t e0,
                          hipEvent_t e1);
// the same for 128 rows or more, 128 x 128 tiles
hipError_t launch_gemm_big(const GemvArgs& a, hipStream_t st, hipEvent_t e0 = nullptr,
                           hipEvent_t e1 = nullptr);
// ANA_BF16 at 128 rows or more: the activations (times the norm's gain)
// rounded to bf16 (Ah: B x K; rsc: B norm scales), then the product with
// both operands streamed straight into LDS (K a multiple of 64)
// (cap_rows: the rows Ah and rsc hold; larger batches are rejected)
// whether launch_gemm_dl takes product a on the 256 x 256 wide-wave tiles
// (gemm_wide.hip), the only ones that write Yh
bool gemm_wide_takes(const GemvArgs& a);
// the wide-wave tiles alone (A in bf16, rsc the norm scales with a gain)
hipError_t launch_gemm_wide(const GemvArgs& a, const __bf16* Ah, const float* rsc, hipStream_t st);
// k_gemm_dl's tile width for a product (96 or 128 columns); a row's
// partial sums of squares from its epilogue (Yn) come one per half tile
uint32_t gemm_dl_cols(const GemvArgs& a);
hipError_t launch_gemm_dl(const GemvArgs& a, __bf16* Ah, float* rsc, uint32_t cap_rows,
                          hipStream_t st, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
size_t attn_fast_part_floats(uint32_t B, uint32_t heads, uint32_t ctx, uint32_t hd);
// causal attention of fresh prefill rows on the matrix cores: one workgroup
// per (head, tile of up to kFlashQ rows of one sequence), the rows' k and v
// already in the ring
constexpr uint32_t kFlashQ = 64, kFlashQBf = 128;
struct AttnTile {
  uint32_t seq, pos0, row0, n;  // sequence, first row's position and workspace row, rows
};
// bf: the products on the bf16 matrix cores (ANA_BF16; hd 32 or 64, else
// the fp32 ones); the tiles hold up to attn_flash_tile_rows(bf, hd) rows
// (kFlashQBf on the bf16 kernel, else kFlashQ)
uint32_t attn_flash_tile_rows(bool bf, uint32_t hd);
hipError_t launch_attn_flash(const AttnArgs& a, const AttnTile* tab, uint32_t ntiles, bool bf, hipStream_t st);
hipError_t launch_zero_u32(uint32_t* p, uint32_t n, hipStream_t st);
hipError_t launch_zero_u64(unsigned long long* p, uint32_t n, hipStream_t st);

// ---------------------------------------------------------------- persistent B = 1 decode
// The fast fp32 token loop of one sequence in one cooperative launch: one
// workgroup a CU runs every phase of every step, phases exchanging their
// outputs as 8-byte (value, epoch) entries. Per layer: parameter offsets
// (floats into the parameter vector), the layer's offset in a sequence's
// state, and its exchange slots (entries into one parity's set).
struct PLayer {
  uint64_t ra, wq, wa, lam, gq, gk, sink, wo, rf, wg, wd;
  // the bf16 matrices' device addresses, each on 16 bytes (q|k|v, z, Wo,
  // gate|up, down), or 0 where the layer reads fp32
  uint64_t hq, ha, ho, hg, hd;
  uint64_t soff;
  uint64_t e_qkv, e_part, e_o, e_xa, e_hh, e_x;
  uint32_t gla, pad;
};
struct PersistArgs {
  const float* W;
  const uint16_t* Wh;       // bf16 weights (past the first layer: PLayer's h* addresses; the head: the
                            // tied embedding here, on 16 bytes), or null for fp32
  const PLayer* lay;        // [L], device
  uint32_t L, d, f, heads, ctx, vocab, rglru, qk, sinks, np;  // np: attention pieces a head
  uint32_t exact;           // the exact build (ANA_EXACT_FP32; fp32 weights)
  uint64_t fin;             // the final norm's gains
  float* state;
  uint64_t seq_stride;
  float* X;                 // out: the last fed token's residual row
  float* LG;                // out: the last step's logits
  const uint32_t* seq;      // [1]
  uint32_t *pos, *tok, *out, *step, *pick;   // as ana_generate's step (out step-major)
  uint32_t steps;
  unsigned long long* ll;   // two sets of ll_par entries
  uint64_t ll_par, e_key;   // entries a set; the head's keys (one a workgroup)
  uint32_t epoch0;          // step k of the launch tags its entries epoch0 + k + 1
  uint32_t* ctl;            // [0] a wait timed out, [1] abort, [2] steps picked, [3] stopped on NaN
  uint64_t tmo;             // a wait's limit, in ticks of the device's constant-rate clock
  uint32_t* trace;          // phase stamps [trace_steps][trace_phases][G][4], or null
  uint32_t trace_steps, trace_phases;
};
// pieces of the ring a head's attention takes (one workgroup each)
uint32_t decode1_pieces(const ana_config& c, uint32_t G);
// whether the persistent kernel takes this configuration on G workgroups
bool decode1_fits(const ana_config& c, uint32_t G, bool exact);
hipError_t launch_decode1(const PersistArgs& a, uint32_t G, hipStream_t st);
// phases a step of the persistent kernel takes (the trace's second extent)
uint32_t decode1_phases(const ana_config& c);

}  // namespace ana

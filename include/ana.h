/*
 * libana -- MI355X (gfx950) decoder token loop for hhefesto/ana checkpoints.
 *
 * A plain C ABI over hand-written HIP kernels. It replaces the dense engine
 * seam of bend/Decode.bend (EDense, driven through Dd.dd.{load, feed, feeds,
 * logits, top, reset} of bend/Dense/Decode.bend:531-699) at engine
 * granularity: one call runs a whole decode step (every layer), not one
 * bulk op.
 *
 * Conventions
 *   - Every int-returning function answers 0 on success, or a nonzero
 *     ANA_E* code; ana_error(ctx) (or ana_error(NULL) after a failed
 *     ana_open) then holds the message, using the reference's wording where
 *     the reference has one (e.g. "checkpoint: short read").
 *   - Host buffers are the caller's, read or written only during the call.
 *     Device memory is the library's.
 *   - A context is single-threaded: the caller serialises calls on it, as
 *     the reference serialises the GPU with FT.mu (bend/effs/bulk.c:79-92).
 *     Every call returns after its device work has completed.
 *   - Sequences are slots 0 .. max_seqs-1 of a context; each keeps its own
 *     recurrent state (GLA S per layer and head, softmax K/V rings) and the
 *     residual row of the last token fed, as one dense store does for one
 *     sequence in the reference.
 *   - Positions count tokens from 0 per sequence; the softmax ring slot is
 *     pos mod ctx and the last live slot min(pos, ctx-1)
 *     (bend/Dense/Decode.bend:540-545).
 */
#ifndef ANA_H
#define ANA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANA_ABI_VERSION 1

/* error codes */
#define ANA_OK 0
#define ANA_EINVAL 1     /* bad argument (sequence, position, token, size) */
#define ANA_ECKPT 2      /* checkpoint rejected (Manifest.problem, short read, ...) */
#define ANA_EDEVICE 3    /* HIP error: "device fault" */
#define ANA_ENOMEM 4     /* device allocation failed */
#define ANA_EUNSUP 5     /* configuration outside what the kernels handle */
#define ANA_ETOK 6       /* tokenizer artifact unreadable or rejected (Bpe.parse) */
#define ANA_ETIME 7      /* a wait between the persistent decode kernel's workgroups passed
                            its time limit (a stalled or heavily shared GPU): the call's
                            sequence is partly advanced and must be reset (ana_reset)
                            before it is fed again */

/* numerics modes */
#define ANA_EXACT_FP32 0 /* bit-exact with the reference's CPU kernels */
#define ANA_FAST_FP32 1  /* fp32, sums reassociated (split-K, fused multiply-add):
                            logits within 1e-4 of the reference, relative to their
                            largest magnitude */
#define ANA_BF16 2       /* matrices read as bfloat16 (rounded once at load); fp32
                            activations, accumulation and state: logits within 2e-2 */

/* bend/Config.bend:7-10 */
typedef struct {
  uint32_t vocab, ctx, d, f, layers, heads;
  uint32_t rglru, qk, sinks, tied;
} ana_config;

typedef struct {
  int device;              /* HIP device ordinal */
  int numerics;            /* ANA_EXACT_FP32, ANA_FAST_FP32 or ANA_BF16 */
  uint32_t max_seqs;       /* sequences the context keeps state for (>= 1) */
  uint32_t prefill_chunk;  /* tokens per prefill chunk; 0 = 64, as ANA_PREFILL_CHUNK */
} ana_opts;

/* the decoding settings of bend/Decode.bend:147-148,546-548 */
typedef struct {
  float temperature;       /* <= 0: greedy (argmax, least index on ties) */
  uint32_t top_k;          /* on when < vocab (0xFFFFFFFF = off) */
  float top_p;             /* on when < 1 */
} ana_sampling;

/* Open an FTC2 checkpoint on a device.
 * Replaces dc.loaded.dense + Dd.dd.of.n + Dd.dd.load
 * (bend/Decode.bend:501-520, bend/Dense/Decode.bend:492-518,689-699): the
 * manifest is validated as Manifest.problem (bend/Checkpoint.bend:162-170),
 * the parameter count and a tied head are required, and the P big-endian
 * floats are read into device memory. All sequences start reset. */
int ana_open(const char* ftc2_path, const ana_opts* opts, struct ana_ctx** out);

/* The checkpoint's config and the Adam step it was saved at. */
int ana_config_of(const struct ana_ctx* ctx, ana_config* out, uint64_t* step);

/* Zero one sequence's states: dd.reset (bend/Dense/Decode.bend:534-538). */
int ana_reset(struct ana_ctx* ctx, uint32_t seq);

/* One token into each of n sequences (distinct seq[i]), no head:
 * dd.feed (bend/Dense/Decode.bend:548-551) for n sequences at once. */
int ana_feed(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const uint32_t* pos,
             const uint32_t* tok);

/* len tokens into one sequence from pos, a chunk at a time: dd.feeds
 * (bend/Dense/Decode.bend:637-639). In ANA_EXACT_FP32 the states and the
 * residual row are bit-identical to len ana_feed calls. */
int ana_feeds(struct ana_ctx* ctx, uint32_t seq, uint32_t pos, const uint32_t* toks, uint32_t len);

/* dd.feeds for n sequences at once (distinct seq[i]): sequence seq[i] takes
 * len[i] tokens from pos[i]; toks holds the sequences' tokens one after
 * another. A chunk step feeds every sequence's next chunk together, so the
 * products run over all their rows at once (the reference prefills one
 * sequence per process and has no counterpart; its meaning is n ana_feeds
 * calls, and in ANA_EXACT_FP32 the states are bit-identical to them). */
int ana_feeds_n(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                const uint32_t* len, const uint32_t* toks);

/* Window scoring, Evaluate.bend's window.go (bend/Evaluate.bend:33-44) for
 * n sequences: sequence seq[i] feeds its first len[i] - 1 tokens from
 * pos[i] (as ana_feeds_n would), and after each fed token t, ce receives
 * G.lse(logits) - logits[token t + 1] (bend/Train/Grad.bend:795-797: the
 * tree max, plus F32.log of the tree sum of F32.exp(x - max)). ce holds
 * len[i] - 1 values per sequence, one sequence after another. In
 * ANA_EXACT_FP32 each value has the bits of ana_feed + ana_logits + that
 * lse; the fast modes are within their tolerance. The caller forms window
 * means and bits per byte from them (window.mean, report). */
int ana_score_n(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                const uint32_t* len, const uint32_t* toks, float* ce);

/* The head on each listed sequence's last fed token: n x vocab floats,
 * dd.logits (bend/Dense/Decode.bend:641-646). */
int ana_logits(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, float* out);

/* The model's own probability of a token after each listed sequence's
 * last fed token, and its likeliest rival: dc.prob.of
 * (bend/Decode.bend:199-202, the prob= of SAMPLE_STATS's lines,
 * bend/Generate.bend:40-49) and al.stat (bend/Agent/Loop.bend:284-288, the
 * agent's pass along a failed term). The head runs on the device and only
 * the three answers come back: with m the logits' tree max and z the tree
 * sum of F32.exp(x - m), prob[i] = exp(l[tok[i]] - m) / z; alt[i] is
 * Sample.argmax of the logits with l[tok[i]] set to -3e38, and alt_prob[i]
 * its probability the same way. Bit-exact with those formulas on the
 * reference's logits in ANA_EXACT_FP32. */
int ana_stats(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const uint32_t* tok, float* prob,
              uint32_t* alt, float* alt_prob);

/* Greedy's pick on the device: dd.top (bend/Dense/Decode.bend:475-484,
 * 648-660), the least index reaching the maximum logit; vocab when no logit
 * does (a NaN maximum), where the caller falls back to ana_pick. */
int ana_top(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, uint32_t* tok);

/* S.pick (bend/Sample.bend:246-254) on the device: greedy (tree argmax)
 * when temperature <= 0, else temperature, top-k and top-p by 40-step
 * bisections and one inverse-CDF draw in tree order. rng holds n x 4 u64
 * xoshiro words (bend/Sample.bend:49-93), advanced in place by one draw for
 * each sampled sequence (untouched when greedy). */
int ana_pick(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const ana_sampling* s,
             uint64_t* rng, uint32_t* tok);

/* Rng.seeded (bend/Sample.bend:68-93): the 4 words for a seed. */
void ana_rng_seeded(uint64_t seed, uint64_t rng[4]);

/* The token loop of bend/Generate.bend:39-51 on the device, for n sequences
 * at once: steps times, feed each sequence's current token at its position,
 * run the head and pick (greedy when s is NULL or temperature <= 0), and
 * feed the pick back. tok[i] is sequence i's first token at pos[i]; out
 * receives n x steps picks (row i = sequence i). EOS does not stop the loop;
 * a caller wanting Generate's stop truncates each row after its first 1.
 * rng as ana_pick (NULL when greedy). One greedy sequence (n = 1) runs as
 * one persistent launch a call in every mode where the device and the model
 * allow it (the environment's ANA_PERSIST=0 keeps it on the step graphs);
 * its results are those of the graphs (bit for bit in ANA_EXACT_FP32), and
 * it can fail with ANA_ETIME. */
int ana_generate(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                 const uint32_t* tok, uint32_t steps, const ana_sampling* s, uint64_t* rng,
                 uint32_t* out);

/* ana_generate for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. Same arguments, semantics and results
 * as ana_generate, but the call allocates nothing: it calls no hipMalloc or
 * hipFree, captures no graph and records no timing events (kernels are
 * launched one by one), and its scratch (the rows' step counters and
 * picks) lives in a fixed device array of 2^18 words that each GPU holds
 * until the process ends. A call needs 64 * ceil(n / 64) + 2 * n * steps
 * words of it; larger calls fail with ANA_EINVAL. Every call on one GPU
 * shares that array, whatever the context, so calls on one GPU from several
 * threads run one at a time: each holds a per-device lock from clearing its
 * counters to its final synchronisation. */
int ana_generate_noalloc(struct ana_ctx* ctx, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                         const uint32_t* tok, uint32_t steps, const ana_sampling* s, uint64_t* rng,
                         uint32_t* out);

/* Copy one sequence's state out (for parity checks): layer l's GLA S
 * (heads x hd x hd floats) or K ring then V ring (2 x ctx x d floats); l ==
 * layers gives the residual row (d floats). n is the float count of out. */
int ana_state(struct ana_ctx* ctx, uint32_t seq, uint32_t layer, float* out, size_t n);

/* Kernel timing (no counterpart in the reference; for benchmarks and
 * profiling). While on, every launch of the listed kinds is bracketed by HIP
 * events on the context's stream and its algorithmic bytes are counted;
 * ana_prof_read sums them since the last ana_prof(ctx, 1). */
#define ANA_K_GEMV 0     /* the layers' matrix-vector products */
#define ANA_K_HEAD 1     /* the LM head's product */
#define ANA_K_ATTN 2     /* softmax attention over the ring */
#define ANA_K_GLA 3      /* the GLA state update and readout */
#define ANA_K_PICK 4     /* greedy pick / sampler */
#define ANA_K_STEP 5     /* whole decode steps in one persistent launch (one greedy
                            sequence, any mode): every kind above at once */
#define ANA_K_KINDS 6
int ana_prof(struct ana_ctx* ctx, int on);
int ana_prof_read(struct ana_ctx* ctx, uint32_t kind, uint64_t* launches, double* ms,
                  double* bytes);

/* Phase stamps of the persistent one-sequence decode kernel (no counterpart
 * in the reference; for profiling the exchange between its workgroups).
 * ana_trace(ctx, steps) with 1 <= steps <= 64 arms it (allocating the
 * stamps' buffer; ANA_EUNSUP where the context has no persistent kernel or
 * more than 32 layers); steps == 0 disarms it. While armed, each persistent
 * launch records its first `steps` steps: per (step, phase, workgroup), four
 * readings of the device's constant-rate clock (100 MHz on gfx950; its low
 * 32 bits, so differences are taken modulo 2^32) taken by the
 * workgroup's first thread: the phase's start, all of its inputs seen, its
 * weights landed in LDS, its outputs published. A step's phases are, per
 * layer, q|k|v(|z), the mix (GLA; or the attention pieces, then their
 * combination), Wo, gate|up and down, then the head and the pick.
 * ana_trace_read copies the last launch's stamps, [steps][phases]
 * [workgroups][4], into out (cap entries) and their extents into dims;
 * with out NULL it gives the extents only. */
int ana_trace(struct ana_ctx* ctx, uint32_t steps);
int ana_trace_read(struct ana_ctx* ctx, uint32_t* out, size_t cap, uint32_t dims[3]);

/* A measurement probe with no counterpart in the reference (no context):
 * the rate of re-reading one zero-filled device buffer of `bytes` (at least
 * 4096, a multiple of 16) `reps` times with a streaming float4 read over
 * 8192 x 256 threads, after one untimed pass, in GB/s (HIP events). Where
 * the buffer fits a cache level (the XCDs' L2s, the Infinity Cache), the
 * rate is that level's; past it, HBM's. It allocates and frees its buffer. */
int ana_probe_reread(int device, uint64_t bytes, uint32_t reps, double* gbs);

/* The last error on ctx, or of the last failed ana_open when ctx is NULL. */
const char* ana_error(const struct ana_ctx* ctx);

void ana_close(struct ana_ctx* ctx);

typedef struct ana_ctx ana_ctx;

/* ---- the FTC2 manifest (bend/Checkpoint.bend:19-136) ----
 * Every field of Load.header's Manifest; the doubles as the reference forms
 * them in F32 (Load.double). Strings are UTF-8, NUL-terminated, cut at
 * ANA_MANIFEST_STR - 1 bytes. tokenizer_id names the tokenizer a caller
 * finds by identity (dc.tok.of). */
#define ANA_MANIFEST_STR 1024
typedef struct ana_manifest {
  uint32_t version;
  ana_config cfg;
  uint32_t count;                       /* the parameter count field */
  char layout[ANA_MANIFEST_STR];
  uint32_t layout_version;
  float lr, beta1, beta2, eps, weight_decay;   /* AdamW */
  uint32_t warmup, total_steps;
  uint32_t has_muon;
  float muon;
  char model_id[ANA_MANIFEST_STR], tokenizer_id[ANA_MANIFEST_STR], dataset_id[ANA_MANIFEST_STR];
  float clip;
  uint32_t numerics;
} ana_manifest;

/* Load.header's manifest of an FTC2 file, without Manifest.problem's
 * verdict (ana_open applies that): ANA_ECKPT and ana_error(NULL) on an
 * unreadable file, a wrong magic or a short header. */
int ana_manifest_read(const char* path, ana_manifest* out);

/* ---- the fast BPE tokenizer (bend/Tokenizer.bend), host side ----
 * Tokens: 0 = BOS, 1 = EOS, 2..257 the bytes, then one per merge in id
 * order. The GPU path sees ids only; these serve the prompts and the
 * outputs around it (dc.tok.of, Bpe.encode, Bpe.decode). */
struct ana_bpe;

/* Bpe.parse of a .bpe artifact ("BPE <vocab> [v2]", then "a b new" rows,
 * ids contiguous from 258): ANA_ETOK when unreadable or rejected. */
int ana_bpe_open(const char* path, struct ana_bpe** out);
/* the byte tokenizer (no merges, V2 rule; dc.tok.btc, bend/Decode.bend:264-268) */
int ana_bpe_bytes(struct ana_bpe** out);
void ana_bpe_close(struct ana_bpe* t);
uint32_t ana_bpe_vocab(const struct ana_bpe* t);
/* Bpe.identity (bend/Tokenizer.bend:330-336): "fastbpe-word-v1:bos=0:eos=1:
 * bytes=2..257:pretoken=<rule>:vocab=<v>:sha256=<digest of the merges>",
 * NUL-terminated into buf (ANA_EINVAL if cap is too small) */
int ana_bpe_identity(const struct ana_bpe* t, char* buf, size_t cap);
/* Bpe.encode (bend/Tokenizer.bend:631-634): pretokenize, then BPE per
 * word; *nids receives the count, ids the ids when cap holds them
 * (ANA_EINVAL otherwise, *nids still set) */
int ana_bpe_encode(const struct ana_bpe* t, const uint8_t* bytes, size_t n, uint32_t* ids, size_t cap,
                   size_t* nids);
/* Bpe.decode of each id, concatenated (BOS and EOS give no bytes) */
int ana_bpe_decode(const struct ana_bpe* t, const uint32_t* ids, size_t n, uint8_t* bytes, size_t cap,
                   size_t* nbytes);
/* H.sha256 (bend/Sha256.bend): 64 lowercase hex digits and a NUL */
int ana_sha256_hex(const uint8_t* bytes, size_t n, char* out65);

#ifdef __cplusplus
}
#endif
#endif

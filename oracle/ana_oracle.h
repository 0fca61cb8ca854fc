/*
 * ana_oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement, in plain C, of hhefesto/ana's dense decoder token loop
 * (the path bend/Dense/Decode.bend runs through bend/effs/bulk.c's CPU
 * kernels), of its tree "meaning" (bend/Model.bend) and of its sampler
 * (bend/Sample.bend). It exists to check the HIP library in ana_amd/csrc and
 * to time the reference's algorithm on host cores; nothing in the product
 * links it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Numerics contract (bend/effs/bulk.c:30-71, 845-849, 979-1088): every
 * reduction runs in index order from 0 (sum) or -inf (max, as t > r ? t : r),
 * products and sums are separate roundings (compile with -ffp-contract=off),
 * exp/log/sqrt go through double and are rounded to float.
 *
 * Parity pinning (what holds each part of this restatement):
 *   dense step      -- within 1e-5 relative of the tree meaning, which is a
 *                      separate restatement of bend/Model.bend (the law of
 *                      bend/tests/decode-dense.bend:13-22); reset => same bits;
 *                      closed forms on hand-built weights (tests/test_oracle.py)
 *   store pick      -- tie vectors of bend/tests/decode-dense.bend:199-220
 *   sampler         -- U64 KATs of bend/tests/num.bend:4-11; closed forms
 *                      (top-k 1 => argmax, top-p floor => argmax, bisection
 *                      thresholds against brute force); the RNG transition is
 *                      the file's (bend/Sample.bend:57-66), not textbook
 *                      xoshiro, checked against a hand expansion
 *   host F32 exp in the sampler -- assumed (float)exp((double)x): the Bend
 *                      runtime's host F32 primitives are not in the reference
 *                      tree, so this one choice is "parity unpinned"
 *   FTC2 reader     -- round trip with ana_amd/ckpt.py's writer and the
 *                      reference's error strings (bend/Checkpoint.bend:162-170,
 *                      bend/Dense/Decode.bend:671-699)
 */
#ifndef ANA_ORACLE_H
#define ANA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bend/Config.bend:7-10 */
typedef struct {
  uint32_t vocab, ctx, d, f, layers, heads;
  uint32_t rglru, qk, sinks, tied;
} or_config;

typedef struct or_model or_model;
typedef struct or_state or_state;

/* Config.params (bend/Config.bend:243-253) */
uint64_t or_params(const or_config* c);
/* Config.model_id (bend/Config.bend:262-277) into buf; returns its length */
size_t or_model_id(const or_config* c, char* buf, size_t cap);

/* FTC2 load (bend/Dense/Decode.bend:689-699). NULL on failure, with the
 * reference's message in err. */
or_model* or_open(const char* path, char* err, size_t errcap);
/* a model over parameters given in memory (P floats in namedLayout order) */
or_model* or_from_params(const or_config* c, const float* params);
void or_model_free(or_model* m);
void or_model_config(const or_model* m, or_config* out);
const float* or_model_params(const or_model* m);
uint64_t or_model_step(const or_model* m);
/* threads used by the matrix products (1 = scalar, the definition) */
void or_set_threads(int n);

/* dense engine: one sequence's states (GLA S, softmax K/V rings) + residual */
or_state* or_state_new(const or_model* m);
or_state* or_state_clone(const or_state* s);                 /* same states, own storage */
void or_state_free(or_state* s);
void or_reset(or_state* s);                                  /* dd.reset */
void or_feed(const or_model* m, or_state* s, uint32_t pos, uint32_t tok); /* dd.feed */
void or_logits(const or_model* m, const or_state* s, float* out);         /* dd.logits */
/* dd.pick / dd.top on a logit vector: the least index reaching the max, or
 * vocab when no logit does (NaN) */
uint32_t or_top(uint32_t vocab, const float* logits);
/* raw state access for parity checks: layer l's GLA S (h*hd*hd floats) or
 * K ring then V ring (2*ctx*d floats); residual x (d floats) */
const float* or_state_layer(const or_state* s, uint32_t layer, size_t* n);
const float* or_state_x(const or_state* s);

/* the meaning (bend/Model.bend decode): tree-order sums; one token */
typedef struct or_tree or_tree;
or_tree* or_tree_new(const or_model* m);
void or_tree_free(or_tree* t);
void or_tree_step(const or_model* m, or_tree* t, uint32_t pos, uint32_t tok, float* logits);

/* Sampler (bend/Sample.bend) */
void or_rng_seeded(uint64_t seed, uint64_t rng[4]);          /* Rng.seeded */
uint64_t or_rng_next(uint64_t rng[4]);                       /* Rng.next: word, state advanced */
int or_u64_read(const char* s, uint64_t* out);               /* U64.read: 1 ok, 0 None */
uint32_t or_tree_argmax(uint32_t vocab, const float* logits); /* Sample.argmax */
/* S.pick: greedy iff temp <= 0 (rng untouched), else one draw */
uint32_t or_pick(uint32_t vocab, const float* logits, float temp, uint32_t topk,
                 float topp, uint64_t rng[4]);
/* the thresholds sample.topk / sample.topp find (for tests) */
float or_topk_threshold(uint32_t vocab, const float* logits, uint32_t topk);
float or_topp_threshold(uint32_t vocab, const float* w, float topp);
float or_tree_sum(uint32_t n, const float* x);
/* G.lse(logits) - logits[y] in the tree's order (Evaluate.bend's summand) */
float or_ce(uint32_t vocab, const float* logits, uint32_t y);
/* dc.prob.of and al.stat: token x's probability, its likeliest rival a
 * (Sample.argmax with l[x] = -3e38) and a's probability */
void or_stat(uint32_t vocab, const float* logits, uint32_t x, float* p, uint32_t* a, float* pa);

#ifdef __cplusplus
}
#endif
#endif

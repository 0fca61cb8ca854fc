// The sampler's kernels: S.pick a row per workgroup (k_pick, its body in
// pick_row.h), the token loop's step end (k_advance), the scoring summand
// (k_ce) and their launchers.
#include <type_traits>

#include "ana_internal.h"
#include "numerics.h"
#include "pick_row.h"

#pragma clang fp contract(off)

namespace ana {

template <int LPT>
__global__ __launch_bounds__(1024) void k_pick(PickArgs a, uint32_t NT, uint32_t dv) {
  pick_row<LPT>(a, blockIdx.x, NT, dv);
}

// the token loop's step end (see AdvanceArgs): row b's pick (from the
// head's argmax keys, wave 0 reading a slot a lane; from the stored logits
// when no key reaches the max, a NaN row), recorded at out[b][step[b]];
// every row keeps its own step count, so no row waits on another
template <int LPT>
__global__ __launch_bounds__(1024) void k_advance(AdvanceArgs a, uint32_t NT) {
  __shared__ float red[16];
  __shared__ uint32_t redi[16];
  __shared__ uint32_t cand_s;
  const uint32_t b = blockIdx.x, tid = threadIdx.x, v = a.vocab;
  uint32_t t;
  if (a.greedy) {
    if (tid < 64) {
      uint32_t cand;
      if (a.amax) {
        unsigned long long key = tid < kAmaxSlots ? a.amax[amax_at(b, tid)] : 0ull;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
          const unsigned long long o = __shfl_xor(key, m, 64);
          key = o > key ? o : key;
        }
        cand = key ? 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull) : v;
      } else {
        cand = a.pick[b];
      }
      if (tid == 0) cand_s = cand;
    }
    __syncthreads();
    const uint32_t cand = cand_s;
    if (cand < v) {
      t = cand;
    } else {
      // no logit reaches the max (NaN): Sample.argmax over the tree
      const uint32_t base = tid * LPT;
      const bool active = tid < NT;
      const float* lg = a.logits + (size_t)b * v;
      float x[LPT];
      load_run<LPT>(lg, base, v, active, x);
      t = tree_argmax<LPT>(x, base, v, red, redi, tid, NT);
    }
  } else {
    t = a.pick[b];
  }
  if (tid == 0) {
    const uint32_t k = a.step[b];
    a.out[(size_t)k * a.B + b] = t;
    a.tok[b] = t;
    a.pos[b] = a.pos[b] + 1;
    if (a.last) a.last[b] = t;
    a.step[b] = k + 1;
  }
}

hipError_t launch_advance(const AdvanceArgs& a, hipStream_t st) {
  uint32_t dv = 0;
  while ((1ull << dv) < a.vocab) dv++;
  const uint64_t vpad = 1ull << dv;
  const uint32_t lpt = vpad > 1024 ? (uint32_t)(vpad / 1024) : 1u;
  const uint32_t NT = (uint32_t)(vpad / lpt);
  switch (lpt) {
#define ANA_ADV(L) \
  case L: hipLaunchKernelGGL(k_advance<L>, dim3(a.B), dim3(1024), 0, st, a, NT); break;
    ANA_ADV(1) ANA_ADV(2) ANA_ADV(4) ANA_ADV(8) ANA_ADV(16) ANA_ADV(32) ANA_ADV(64)
#undef ANA_ADV
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// step-major picks (step k, row b at k * n + b) to row-major (b * steps + k)
__global__ __launch_bounds__(256) void k_picks_rows(const uint32_t* __restrict__ sm, uint32_t n, uint32_t steps,
                                                    uint32_t* __restrict__ rm) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)n * steps) return;
  const uint32_t b = (uint32_t)(i / steps), k = (uint32_t)(i % steps);
  rm[i] = sm[(size_t)k * n + b];
}

hipError_t launch_picks_rows(const uint32_t* sm, uint32_t n, uint32_t steps, uint32_t* rm, hipStream_t st) {
  const uint64_t total = (uint64_t)n * steps;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_picks_rows, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, st, sm, n, steps, rm);
  return hipGetLastError();
}

// Evaluate.bend's summand (window.go, bend/Evaluate.bend:33-44): G.lse of
// the logits minus the target's logit, G.lse = V.max + F32.log(V.sum_exp)
// (bend/Train/Grad.bend:795-797; bend/Tensor.bend:170-177,292-299) over the
// logits' tree, one workgroup per row
template <int LPT>
__global__ __launch_bounds__(1024) void k_ce(const float* __restrict__ logits, uint32_t vocab,
                                             const uint32_t* __restrict__ tgt, float* __restrict__ ce,
                                             uint32_t NT) {
  __shared__ float red[16];
  const uint32_t b = blockIdx.x, tid = threadIdx.x, base = tid * LPT;
  const bool active = tid < NT;
  const float* lg = logits + (size_t)b * vocab;
  float x[LPT], pm[LPT];
  load_run<LPT>(lg, base, vocab, active, x);
#pragma unroll
  for (int i = 0; i < LPT; i++) pm[i] = (active && base + i < vocab) ? x[i] : -3.0e38f;
  const float m = tree_up(local_reduce<LPT>(pm, Max()), Max(), red, tid, NT);
  float e[LPT];
#pragma unroll
  for (int i = 0; i < LPT; i++) e[i] = (active && base + i < vocab) ? dexp(x[i] - m) : 0.0f;
  const float s = tree_up(local_reduce<LPT>(e, Add()), Add(), red, tid, NT);
  if (tid == 0) ce[b] = (m + dlog(s)) - lg[tgt[b]];
}

// The model's own probability of a token and its likeliest rival, from one
// row of logits: dc.prob.of (bend/Decode.bend:199-202; SAMPLE_STATS's prob)
// and al.stat (bend/Agent/Loop.bend:284-288). With m the tree max and z the
// tree sum of F32.exp(x - m): p = exp(l[t] - m) / z, a = Sample.argmax of
// the row with l[t] set to -3e38, pa = exp(l[a] - m) / z. One workgroup per
// row, the reductions in the logits' tree order.
template <int LPT>
__global__ __launch_bounds__(1024) void k_stats(const float* __restrict__ logits, uint32_t vocab,
                                                const uint32_t* __restrict__ tok, float* __restrict__ p,
                                                uint32_t* __restrict__ alt, float* __restrict__ palt, uint32_t NT) {
  __shared__ float red[16];
  __shared__ uint32_t redi[16];
  const uint32_t b = blockIdx.x, tid = threadIdx.x, base = tid * LPT;
  const bool active = tid < NT;
  const float* lg = logits + (size_t)b * vocab;
  const uint32_t t = tok[b];
  float x[LPT], pm[LPT];
  load_run<LPT>(lg, base, vocab, active, x);
#pragma unroll
  for (int i = 0; i < LPT; i++) pm[i] = (active && base + i < vocab) ? x[i] : -3.0e38f;
  const float m = tree_up(local_reduce<LPT>(pm, Max()), Max(), red, tid, NT);
  float e[LPT];
#pragma unroll
  for (int i = 0; i < LPT; i++) e[i] = (active && base + i < vocab) ? dexp(x[i] - m) : 0.0f;
  const float z = tree_up(local_reduce<LPT>(e, Add()), Add(), red, tid, NT);
#pragma unroll
  for (int i = 0; i < LPT; i++)
    if (base + i == t) x[i] = -3.0e38f;
  const uint32_t a = tree_argmax<LPT>(x, base, vocab, red, redi, tid, NT);
  if (tid == 0) {
    p[b] = dexp(lg[t] - m) / z;
    alt[b] = a;
    palt[b] = dexp(lg[a] - m) / z;
  }
}

hipError_t launch_stats(const float* logits, uint32_t vocab, uint32_t B, const uint32_t* tok, float* p,
                        uint32_t* alt, float* palt, hipStream_t st) {
  if (B == 0) return hipSuccess;
  uint32_t dv = 0;
  while ((1ull << dv) < vocab) dv++;
  const uint64_t vpad = 1ull << dv;
  const uint32_t lpt = vpad > 1024 ? (uint32_t)(vpad / 1024) : 1u;
  const uint32_t NT = (uint32_t)(vpad / lpt);
  switch (lpt) {
#define ANA_ST(L) \
  case L: hipLaunchKernelGGL(k_stats<L>, dim3(B), dim3(1024), 0, st, logits, vocab, tok, p, alt, palt, NT); break;
    ANA_ST(1) ANA_ST(2) ANA_ST(4) ANA_ST(8) ANA_ST(16) ANA_ST(32) ANA_ST(64)
#undef ANA_ST
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ce(const float* logits, uint32_t vocab, uint32_t B, const uint32_t* tgt, float* ce,
                     hipStream_t st) {
  if (B == 0) return hipSuccess;
  uint32_t dv = 0;
  while ((1ull << dv) < vocab) dv++;
  const uint64_t vpad = 1ull << dv;
  const uint32_t lpt = vpad > 1024 ? (uint32_t)(vpad / 1024) : 1u;
  const uint32_t NT = (uint32_t)(vpad / lpt);
  switch (lpt) {
#define ANA_CE(L) \
  case L: hipLaunchKernelGGL(k_ce<L>, dim3(B), dim3(1024), 0, st, logits, vocab, tgt, ce, NT); break;
    ANA_CE(1) ANA_CE(2) ANA_CE(4) ANA_CE(8) ANA_CE(16) ANA_CE(32) ANA_CE(64)
#undef ANA_CE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_pick(const PickArgs& a, hipStream_t st) {
  uint32_t dv = 0;
  while ((1ull << dv) < a.vocab) dv++;
  const uint64_t vpad = 1ull << dv;
  uint32_t lpt = vpad > 1024 ? (uint32_t)(vpad / 1024) : 1u;
  const uint32_t NT = (uint32_t)(vpad / lpt);
  switch (lpt) {
#define ANA_PICK(L) \
  case L: hipLaunchKernelGGL(k_pick<L>, dim3(a.B), dim3(1024), 0, st, a, NT, dv); break;
    ANA_PICK(1) ANA_PICK(2) ANA_PICK(4) ANA_PICK(8) ANA_PICK(16) ANA_PICK(32) ANA_PICK(64)
#undef ANA_PICK
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ana

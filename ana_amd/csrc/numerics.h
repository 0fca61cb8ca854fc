// The reference's scalar F32 steps as device functions.
//
// bend/effs/bulk.c evaluates einsum expressions with separate F32 roundings
// and with exp/log/sqrt through double (bulk.c:1012-1040); bend/Dense/Ex.bend
// builds those expressions (sigmoid as a select, log1p with Goldberg's trick,
// the RG-LRU gate). Each function below is one such expression tree.
#pragma once

#include <hip/hip_runtime.h>

#pragma clang fp contract(off)

namespace ana {

__device__ __forceinline__ float dexp(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float dlog(float x) { return (float)log((double)x); }
// sqrt through double, rounded once more to float: equal to the correctly
// rounded float square root (53 >= 2*24 + 2)
__device__ __forceinline__ float csqrt(float x) { return (float)sqrt((double)x); }

// Ex max / min (bend/Dense/Ex.bend:126-131): max a b = (a < b ? b : a)
__device__ __forceinline__ float ex_max(float a, float b) { return a < b ? b : a; }
__device__ __forceinline__ float ex_min(float a, float b) { return a < b ? a : b; }

// bend/Dense/Ex.bend:148-150
__device__ __forceinline__ float ex_sigmoid(float z) {
  if (0.0f <= z) return 1.0f / (1.0f + dexp(-z));
  const float e = dexp(z);
  return e / (1.0f + e);
}

// bend/Dense/Ex.bend:152-153
__device__ __forceinline__ float ex_silu(float z) { return z * ex_sigmoid(z); }

// bend/Dense/Ex.bend:141-143: w == 1 ? u : (log w * u) / (w - 1)
__device__ __forceinline__ float ex_log1p(float u) {
  const float w = 1.0f + u;
  const float eq = (w <= 1.0f ? 1.0f : 0.0f) * (1.0f <= w ? 1.0f : 0.0f);
  if (eq != 0.0f) return u;
  return (dlog(w) * u) / (w - 1.0f);
}

// bend/Dense/Ex.bend:145-146: -(max(-z, 0) + log1p(exp(-|z|)))
__device__ __forceinline__ float ex_log_sigmoid(float z) {
  return -(ex_max(-z, 0.0f) + ex_log1p(dexp(-fabsf(z))));
}

#define ANA_CAP (-1.0e-4f)

// bend/Dense/Ex.bend:158-159: min(cap, (8 * sigmoid z) * log_sigmoid lam)
__device__ __forceinline__ float ex_rglru_log_gate(float z, float lam) {
  return ex_min(ANA_CAP, (8.0f * ex_sigmoid(z)) * ex_log_sigmoid(lam));
}

// bend/Dense/Ex.bend:161-162: sqrt(1 - exp(2 * min(cap, la)))
__device__ __forceinline__ float ex_rglru_write_scale(float la) {
  return csqrt(1.0f - dexp(2.0f * ex_min(ANA_CAP, la)));
}

// bend/Dense/Ex.bend:165-166: 1 / sqrt(ss / n + 1e-5)
__device__ __forceinline__ float ex_rms_scale(float ss, float n) {
  return 1.0f / csqrt((ss / n) + 1.0e-5f);
}

}  // namespace ana

namespace ana {

// s + f(v(0).x) + f(v(0).y) + ... + f(v(n4 - 1).w) in order, the float4s
// read from LDS by the accessor. Blocks of eight float4 in turn: a block's
// reads are issued before the adds of the block before it, and one wait
// (the LDS counter down to eight: the older block landed) precedes each
// block's 32 adds. A wait for each float4, which the compiler places by
// itself, holds the chain back every few adds: about 11 cycles a dependent
// add against 6.5 this way, measured on one gfx950 wave with every lane
// adding.
template <class A, class F>
__device__ __forceinline__ float chain4_lds(float s, uint32_t n4, A at, F f) {
  auto add8 = [&](const float4 (&b)[8]) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      s = s + f(b[u].x);
      s = s + f(b[u].y);
      s = s + f(b[u].z);
      s = s + f(b[u].w);
    }
  };
  auto load8 = [&](float4 (&b)[8], uint32_t i) {
#pragma unroll
    for (int u = 0; u < 8; u++) b[u] = at(i + u);
  };
  // s_waitcnt lgkmcnt(k) alone (vector-memory and export counters not
  // waited on), fenced so that neither the reads nor the adds move across it
#define ANA_LGKM_WAIT(k)                                 \
  do {                                                   \
    __builtin_amdgcn_sched_barrier(0);                   \
    __builtin_amdgcn_s_waitcnt(0xC07F | ((k) << 8));     \
    __builtin_amdgcn_sched_barrier(0);                   \
  } while (0)
  uint32_t i = 0;
  if (n4 >= 8) {
    float4 a[8], b[8];
    load8(a, 0);
    for (i = 8; i + 16 <= n4; i += 16) {
      load8(b, i);
      ANA_LGKM_WAIT(8);
      add8(a);
      load8(a, i + 8);
      ANA_LGKM_WAIT(8);
      add8(b);
    }
    if (i + 8 <= n4) {
      load8(b, i);
      ANA_LGKM_WAIT(8);
      add8(a);
      ANA_LGKM_WAIT(0);
      add8(b);
      i += 8;
    } else {
      ANA_LGKM_WAIT(0);
      add8(a);
    }
  }
#undef ANA_LGKM_WAIT
  for (; i < n4; i++) {
    const float4 v = at(i);
    s = s + f(v.x);
    s = s + f(v.y);
    s = s + f(v.z);
    s = s + f(v.w);
  }
  return s;
}

// s = (((s + f(p[0])) + f(p[1])) + ...) + f(p[n-1]): one in-order chain
// over LDS (p 16-byte aligned)
template <class F>
__device__ __forceinline__ float chain_lds(float s, const float* __restrict__ p, uint32_t n, F f) {
  const float4* q = reinterpret_cast<const float4*>(p);
  s = chain4_lds(s, n >> 2, [&](uint32_t i) { return q[i]; }, f);
  for (uint32_t j = n & ~3u; j < n; j++) s = s + f(p[j]);
  return s;
}

// s = (((s + p[0]) + p[1]) + ...) + p[n-1]
__device__ __forceinline__ float chain_sum_lds(float s, const float* __restrict__ p, uint32_t n) {
  return chain_lds(s, p, n, [](float x) { return x; });
}

// s = s + x0*x0 + x1*x1 ... in order (M.norm's sum of squares)
__device__ __forceinline__ float chain_sumsq_lds(float s, const float* __restrict__ p, uint32_t n) {
  return chain_lds(s, p, n, [](float x) { return x * x; });
}

}  // namespace ana

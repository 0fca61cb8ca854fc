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

// s = (((s + f(b[0].x)) + f(b[0].y)) + ...) + f(b[7].w), in order
template <class F>
__device__ __forceinline__ float chain_add8(float s, const float4 (&b)[8], F f) {
#pragma unroll
  for (int u = 0; u < 8; u++) {
    s = s + f(b[u].x);
    s = s + f(b[u].y);
    s = s + f(b[u].z);
    s = s + f(b[u].w);
  }
  return s;
}

// s = (((s + f(p[0])) + f(p[1])) + ...) + f(p[n-1]): one in-order chain
// over LDS (p 16-byte aligned). Two sets of 8 float4 take turns: a set is
// loaded again as soon as its 32 adds are issued, so its loads are in
// flight while the other set's 32 adds run, and no set is copied into
// another (a rotation through copies put the next loads behind a wait for
// the current ones).
template <class F>
__device__ __forceinline__ float chain_lds(float s, const float* __restrict__ p, uint32_t n, F f) {
  const float4* q = reinterpret_cast<const float4*>(p);
  const uint32_t n4 = n >> 2;
  uint32_t i = 0;
  if (n4 >= 16) {
    float4 a[8], b[8];
#pragma unroll
    for (int u = 0; u < 8; u++) a[u] = q[u];
#pragma unroll
    for (int u = 0; u < 8; u++) b[u] = q[8 + u];
    // a holds float4s i - 16 .. i - 9, b i - 8 .. i - 1
    for (i = 16; i + 16 <= n4; i += 16) {
      s = chain_add8(s, a, f);
#pragma unroll
      for (int u = 0; u < 8; u++) a[u] = q[i + u];
      s = chain_add8(s, b, f);
#pragma unroll
      for (int u = 0; u < 8; u++) b[u] = q[i + 8 + u];
    }
    s = chain_add8(s, a, f);
    if (i + 8 <= n4) {
#pragma unroll
      for (int u = 0; u < 8; u++) a[u] = q[i + u];
      s = chain_add8(s, b, f);
      s = chain_add8(s, a, f);
      i += 8;
    } else {
      s = chain_add8(s, b, f);
    }
  }
  if (i + 8 <= n4) {
    float4 a[8];
#pragma unroll
    for (int u = 0; u < 8; u++) a[u] = q[i + u];
    s = chain_add8(s, a, f);
    i += 8;
  }
  for (; i < n4; i++) {
    const float4 v = q[i];
    s = s + f(v.x);
    s = s + f(v.y);
    s = s + f(v.z);
    s = s + f(v.w);
  }
  for (uint32_t j = n4 << 2; j < n; j++) s = s + f(p[j]);
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

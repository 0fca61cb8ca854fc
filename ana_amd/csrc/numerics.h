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

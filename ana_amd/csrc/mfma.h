// Matrix-core helpers shared by the fast product kernels (gfx950): operand
// vectors, the LDS address type of global_load_lds, explicit wait counts,
// the SiLU of the gate|up epilogues and the XCD-grouped tile order.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace ana {

// MFMA operand and accumulator vectors
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
// an LDS address for global_load_lds
typedef __attribute__((address_space(3))) void lds_void;
// vmcnt(n) alone (expcnt and lgkmcnt at their maxima)
#define ANA_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))
// lgkmcnt(0) alone (vmcnt and expcnt at their maxima)
#define ANA_LGKMCNT0() __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4))

// (the hardware reciprocal, ~1 ulp, as the exponential beside it: an IEEE
// division is ten instructions, and the SiLU epilogues take thousands a
// lane)
__device__ __forceinline__ float fast_silu(float z) { return z * __builtin_amdgcn_rcpf(1.0f + __expf(-z)); }

// a row's RMSNorm scale from its producer's n partial sums of squares, in
// order (K: the row's length)
__device__ __forceinline__ float norm_from_partials(const float* p, uint32_t n, uint32_t K) {
  float s = 0.0f;
  for (uint32_t i = 0; i < n; i++) s += p[i];
  return 1.0f / sqrtf(s / (float)K + 1.0e-5f);
}

// Workgroup -> (n tile, m tile) so that the workgroups one XCD runs (ids
// equal mod 8) take consecutive tiles, n fastest: the A rows those n tiles
// share stay in that XCD's L2.
__device__ __forceinline__ void xcd_tile(uint32_t* nt, uint32_t* mt) {
  const uint32_t NT = gridDim.x, total = gridDim.x * gridDim.y;
  const uint32_t L = blockIdx.x + blockIdx.y * NT;
  const uint32_t x = L % 8, idx = L / 8, per = total / 8, rem = total % 8;
  const uint32_t g = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + idx;
  *nt = g % NT;
  *mt = g / NT;
}

}  // namespace ana

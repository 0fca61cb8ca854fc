// Wave-level helpers shared by the kernels: DPP lane moves and the sums
// and maxima they build (gfx950, 64-lane waves of four 16-lane rows).
#pragma once
#include <hip/hip_runtime.h>

namespace ana {

// a DPP move of v (lane permutation dpp_ctrl within each row of 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// the sum over each row of 16 lanes, in every lane of the row: lane ^ 1 and
// lane ^ 2 (quad_perm), then the mirrored quad (row_half_mirror), then the
// mirrored half-row (row_mirror)
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}
// the rows' values carried into lane 63: row_bcast:15 adds row r - 1's
// lane 15 into rows 1 and 3, row_bcast:31 lane 31 into rows 2 and 3; rows
// outside ROWS take 0 (with op +) or keep v (with op max)
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float v, float other) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, other), __builtin_bit_cast(int, v),
                                                              CTRL, ROWS, 0xF, false));
}
// the maximum over each row of 16 lanes, in every lane of the row
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// the sum over the wave (every lane gets it): the rows' sums by DPP, then
// the four rows' into lane 63 by row broadcasts, (r3 + r2) + (r1 + r0):
// the same float as (r0 + r1) + (r2 + r3), each add being commutative.
// (Four lane reads and three adds for the last step took about 0.2 us for
// four values at once, a fifth of a small product's phase.)
__device__ __forceinline__ float wsum(float v) {
  v = row16_sum(v);
  v += dpp_rows<0x142, 0xA>(v, 0.0f);
  v += dpp_rows<0x143, 0xC>(v, 0.0f);
  return lane_f(v, 63);
}
// wsum of N values at once, each summed in wsum's order (so each result is
// wsum's): every DPP step of all N before the next, so the steps of one
// fill the others' DPP wait states instead of s_nop
template <int N>
__device__ __forceinline__ void wsum_n(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0xB1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0x4E>(v[i]);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0x141>(v[i]);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0x140>(v[i]);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp_rows<0x142, 0xA>(v[i], 0.0f);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp_rows<0x143, 0xC>(v[i], 0.0f);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = lane_f(v[i], 63);
}
// the maximum over the wave, the same way
__device__ __forceinline__ float wmax(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, dpp_rows<0x142, 0xA>(v, v));
  v = fmaxf(v, dpp_rows<0x143, 0xC>(v, v));
  return lane_f(v, 63);
}

// the sum over each group of G consecutive lanes (G = 16, 32 or 64), in
// every lane of the group
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 16 || G == 32 || G == 64, "rows, half waves or the wave");
  v = row16_sum(v);
  if constexpr (G == 16) {
    return v;
  } else if constexpr (G == 32) {
    const float lo = lane_f(v, 0) + lane_f(v, 16), hi = lane_f(v, 32) + lane_f(v, 48);
    return (threadIdx.x & 32) ? hi : lo;
  } else {
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
  }
}

}  // namespace ana

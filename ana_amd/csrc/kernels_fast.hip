// Fast decode kernels (ANA_FAST_FP32, ANA_BF16) for gfx950.
//
// The same decode step as the exact kernels, with the reductions split
// across lanes and reassociated (tree sums, fused multiply-adds), so that the
// weights stream at HBM rate instead of waiting on one lane's in-order chain.
// Results are within a stated tolerance of the reference rather than equal
// to it. ANA_BF16 reads the matrices as bfloat16 (rounded to nearest even
// once, at load); activations, accumulation and recurrent state stay fp32.
#include <hip/hip_ext.h>

#include <type_traits>
#include <utility>

#include "ana_internal.h"
#include "mfma.h"
#include "numerics.h"
#include "pick_row.h"
#include "wave.h"

namespace ana {

// ------------------------------------------------------------------ weights

// fp32 bits -> bfloat16, round to nearest even; NaN stays a quiet NaN
__global__ void k_to_bf16(const uint32_t* __restrict__ w, uint16_t* __restrict__ h, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t u = w[i];
    uint16_t r;
    if ((u & 0x7fffffffu) > 0x7f800000u) r = (uint16_t)((u >> 16) | 0x40u);
    else r = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    h[i] = r;
  }
}

hipError_t launch_to_bf16(const float* w, uint16_t* h, uint64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_to_bf16, dim3(4096), dim3(256), 0, st, reinterpret_cast<const uint32_t*>(w), h, n);
  return hipGetLastError();
}

// four consecutive weights of a row as floats
template <int WT> struct WLoad;
template <> struct WLoad<0> {
  using V = float4;
  __device__ static __forceinline__ V load(const float* f, const uint16_t*, uint32_t k) {
    return *reinterpret_cast<const float4*>(f + k);
  }
  __device__ static __forceinline__ float4 f4(const V& v) { return v; }
};
template <> struct WLoad<1> {
  using V = uint2;
  __device__ static __forceinline__ V load(const float*, const uint16_t* h, uint32_t k) {
    return *reinterpret_cast<const uint2*>(h + k);
  }
  __device__ static __forceinline__ float4 f4(const V& v) {
    return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                       __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
  }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// ------------------------------------------------------------------ products

// Small batches (B <= 4): one wave per workgroup, RW rows of the product.
// Lane l covers k = 4 (l + 64 j), j < NF, of every row (split K): it loads
// its slices of the BT activation rows first, then all RW x NF weight
// slices at once (so they stream while the activations are normalised),
// multiplies with fused multiply-adds and the wave sums each row's 64
// partial dot products. Epilogues as the exact product's: plain, residual,
// SiLU gate (tile rows [0, RW/2) gate, RW/2 further their up rows) and the
// greedy argmax key.
template <int WT, int BT, int RW, int NF>
__global__ __launch_bounds__(64) void k_gemv_fast(GemvArgs a) {
  using WL = WLoad<WT>;
  __shared__ float4 xs[BT][NF * 64];
  const uint32_t lane = threadIdx.x, K = a.K;
  const uint32_t nb = a.B < (uint32_t)BT ? a.B : (uint32_t)BT;
  const Segs sgs(a);
  // activations (and the norm's gains) first: their wait leaves the weight
  // loads issued after them in flight
  float4 xv[BT][NF], gv[NF];
#pragma unroll
  for (int b = 0; b < BT; b++)
#pragma unroll
    for (int j = 0; j < NF; j++) {
      const uint32_t k = 4 * (lane + 64 * j);
      const bool in = k < K && (uint32_t)b < nb;
      xv[b][j] = *reinterpret_cast<const float4*>(a.X + (size_t)(in ? b : 0) * a.ldx + (in ? k : 0));
    }
  if (a.ng) {
#pragma unroll
    for (int j = 0; j < NF; j++) {
      const uint32_t k = 4 * (lane + 64 * j);
      gv[j] = *reinterpret_cast<const float4*>(a.ng + (k < K ? k : 0));
    }
  }
  typename WL::V wv[RW][NF];
  uint32_t lr[RW], sg[RW];
  bool rok[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const float* w;
    rok[r] = sgs.row(RW, blockIdx.x, r, &w, &sg[r], &lr[r]);
    const uint16_t* wh = (sg[r] ? a.Wh1 : a.Wh0) + (size_t)lr[r] * K;
    if (!rok[r]) {
      w = sgs.W0;
      wh = a.Wh0;
    }
#pragma unroll
    for (int j = 0; j < NF; j++) {
      const uint32_t k = 4 * (lane + 64 * j);
      wv[r][j] = WL::load(w, wh, k < K ? k : 0);
    }
  }
  // the residual this lane's output adds, loaded with the weights (not after
  // the reduction, which would add a dependent memory round trip)
  float res = 0.0f;
  if (a.mode == GM_RESID && lane < (uint32_t)(RW * BT)) {
    const uint32_t rr = lane / BT, bb = lane % BT;
    uint32_t rl = 0;
    bool ok = false;
#pragma unroll
    for (int r = 0; r < RW; r++)
      if ((uint32_t)r == rr) {
        rl = lr[r];
        ok = rok[r];
      }
    if (ok && bb < nb) res = a.R[(size_t)bb * a.ldr + rl];
  }
  // M.norm on the lane's slices: ss over the row by a wave sum
#pragma unroll
  for (int b = 0; b < BT; b++) {
    float4 x4[NF];
#pragma unroll
    for (int j = 0; j < NF; j++) {
      const uint32_t k = 4 * (lane + 64 * j);
      x4[j] = (k < K && (uint32_t)b < nb) ? xv[b][j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (a.ng) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < NF; j++) ss += x4[j].x * x4[j].x + x4[j].y * x4[j].y + x4[j].z * x4[j].z + x4[j].w * x4[j].w;
      ss = wave_sum(ss);
      const float rs = 1.0f / sqrtf(ss / (float)K + 1.0e-5f);
#pragma unroll
      for (int j = 0; j < NF; j++) {
        x4[j].x = (x4[j].x * rs) * gv[j].x;
        x4[j].y = (x4[j].y * rs) * gv[j].y;
        x4[j].z = (x4[j].z * rs) * gv[j].z;
        x4[j].w = (x4[j].w * rs) * gv[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < NF; j++) xs[b][j * 64 + lane] = x4[j];
  }
  float acc[RW][BT];
#pragma unroll
  for (int r = 0; r < RW; r++) {
#pragma unroll
    for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;
#pragma unroll
    for (int j = 0; j < NF; j++) {
      const float4 w4 = WL::f4(wv[r][j]);
#pragma unroll
      for (int b = 0; b < BT; b++) {
        const float4 x4 = xs[b][j * 64 + lane];
        acc[r][b] = fmaf(w4.x, x4.x, acc[r][b]);
        acc[r][b] = fmaf(w4.y, x4.y, acc[r][b]);
        acc[r][b] = fmaf(w4.z, x4.z, acc[r][b]);
        acc[r][b] = fmaf(w4.w, x4.w, acc[r][b]);
      }
    }
#pragma unroll
    for (int b = 0; b < BT; b++) acc[r][b] = wave_sum(acc[r][b]);
  }
  if (a.mode == GM_SILU) {
#pragma unroll
    for (int r = 0; r < RW / 2; r++)
#pragma unroll
      for (int b = 0; b < BT; b++)
        if (lane == (uint32_t)(r * BT + b) && rok[r] && (uint32_t)b < nb)
          a.seg[0].Y[(size_t)b * a.seg[0].ldy + lr[r]] = fast_silu(acc[r][b]) * acc[r + RW / 2][b];
    return;
  }
#pragma unroll
  for (int r = 0; r < RW; r++)
#pragma unroll
    for (int b = 0; b < BT; b++)
      if (lane == (uint32_t)(r * BT + b) && rok[r] && (uint32_t)b < nb) {
        float y = acc[r][b];
        if (a.mode == GM_RESID) y = res + y;
        if (sg[r]) a.seg[1].Y[(size_t)b * a.seg[1].ldy + lr[r]] = y;
        else a.seg[0].Y[(size_t)b * a.seg[0].ldy + lr[r]] = y;
      }
  if (a.amax && lane < (uint32_t)BT && lane < nb) {
    unsigned long long k = 0;
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
      for (int b = 0; b < BT; b++)
        if ((uint32_t)b == lane && rok[r] && sg[r] == 0) {
          const unsigned long long kk = argmax_key(acc[r][b], lr[r]);
          k = kk > k ? kk : k;
        }
    if (k) atomicMax(&a.amax[amax_at(lane, blockIdx.x % kAmaxSlots)], k);
  }
}

#define ANA_LAUNCH_F(K, GRID, BLOCK, LDS, ST, E0, E1, ...)                               \
  do {                                                                                  \
    if (E0) hipExtLaunchKernelGGL(K, GRID, BLOCK, LDS, ST, E0, E1, 0, __VA_ARGS__);      \
    else hipLaunchKernelGGL(K, GRID, BLOCK, LDS, ST, __VA_ARGS__);                      \
  } while (0)

template <int WT, int BT, int RW, int NF>
static hipError_t gemv_fast_go(const GemvArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  const uint32_t per = a.mode == GM_SILU ? RW / 2 : RW;
  const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
  ANA_LAUNCH_F((k_gemv_fast<WT, BT, RW, NF>), dim3(tiles), dim3(64), 0, st, e0, e1, a);
  return hipGetLastError();
}

template <int WT, int BT>
static hipError_t gemv_fast_nf(const GemvArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const uint32_t nf = (a.K + 255) / 256;
  if (nf <= 1) return gemv_fast_go<WT, BT, 8, 1>(a, st, e0, e1);
  if (nf <= 2) return gemv_fast_go<WT, BT, 8, 2>(a, st, e0, e1);
  if (nf <= 3) return gemv_fast_go<WT, BT, 4, 3>(a, st, e0, e1);
  if (nf <= 4) return gemv_fast_go<WT, BT, 4, 4>(a, st, e0, e1);
  if constexpr (BT <= 4) {
    if (nf <= 6) return gemv_fast_go<WT, BT, 2, 6>(a, st, e0, e1);
  }
  if constexpr (BT <= 2) {
    if (nf <= 8) return gemv_fast_go<WT, BT, 2, 8>(a, st, e0, e1);
    if (nf <= 12) return gemv_fast_go<WT, BT, 2, 12>(a, st, e0, e1);
  }
  return hipErrorInvalidValue;
}

// the widest batch tile whose activation slices fit the registers
static uint32_t fast_bt(uint32_t K, uint32_t B) {
  const uint32_t nf = (K + 255) / 256;
  const uint32_t cap = nf <= 6 ? 4 : nf <= 12 ? 2 : 0;
  const uint32_t bt = B <= 1 ? 1 : B <= 2 ? 2 : 4;
  return bt < cap ? bt : cap;
}

hipError_t launch_gemv_fast(const GemvArgs& a0, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  if (a0.B == 0 || a0.B > kSmallB || (a0.K & 3) || fast_bt(a0.K, 1) == 0) return hipErrorInvalidValue;
  const bool bf = a0.Wh0 != nullptr;
  if (bf && a0.nseg > 1 && !a0.Wh1) return hipErrorInvalidValue;
  const uint32_t BT = fast_bt(a0.K, a0.B);
  // batch rows in tiles of BT; one launch per tile (the events bracket the
  // first and the last)
  for (uint32_t b0 = 0; b0 < a0.B; b0 += BT) {
    GemvArgs a = a0;
    a.B = a0.B - b0 < BT ? a0.B - b0 : BT;
    a.X += (size_t)b0 * a.ldx;
    a.seg[0].Y += (size_t)b0 * a.seg[0].ldy;
    a.seg[1].Y += (size_t)b0 * a.seg[1].ldy;
    if (a.R) a.R += (size_t)b0 * a.ldr;
    if (a.amax) a.amax += b0 * kAmaxPerRow;
    hipEvent_t s0 = b0 == 0 ? e0 : nullptr, s1 = b0 + BT >= a0.B ? e1 : nullptr;
    hipError_t e;
    if (s0 && !s1) {
      (void)hipEventRecord(s0, st);
      s0 = nullptr;
    }
    if (!s0 && s1) {
      // start recorded already (or by the first tile): stop after this launch
      if (bf) e = BT == 1 ? gemv_fast_nf<1, 1>(a, st, nullptr, nullptr) : BT == 2 ? gemv_fast_nf<1, 2>(a, st, nullptr, nullptr) : gemv_fast_nf<1, 4>(a, st, nullptr, nullptr);
      else e = BT == 1 ? gemv_fast_nf<0, 1>(a, st, nullptr, nullptr) : BT == 2 ? gemv_fast_nf<0, 2>(a, st, nullptr, nullptr) : gemv_fast_nf<0, 4>(a, st, nullptr, nullptr);
      if (e != hipSuccess) return e;
      (void)hipEventRecord(s1, st);
      continue;
    }
    if (bf) e = BT == 1 ? gemv_fast_nf<1, 1>(a, st, s0, s1) : BT == 2 ? gemv_fast_nf<1, 2>(a, st, s0, s1) : gemv_fast_nf<1, 4>(a, st, s0, s1);
    else e = BT == 1 ? gemv_fast_nf<0, 1>(a, st, s0, s1) : BT == 2 ? gemv_fast_nf<0, 2>(a, st, s0, s1) : gemv_fast_nf<0, 4>(a, st, s0, s1);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ------------------------------------------------------------------ GLA

// One decode token of dd.gla for one head, one block of CB state columns:
// L2 norms of q and k (wave sums), the gate (Ex.bend's expressions in float
// arithmetic), S' = al*S + kh v^T on the block, and o over the block's
// columns = qh^T S' (per-thread partials, then lane shuffles and LDS).
__device__ __forceinline__ float f_sigmoid(float z) {
  if (0.0f <= z) return 1.0f / (1.0f + expf(-z));
  const float e = expf(z);
  return e / (1.0f + e);
}
__device__ __forceinline__ float f_log_sigmoid(float z) {
  return -(fmaxf(-z, 0.0f) + log1pf(expf(-fabsf(z))));
}

template <int HD>
__global__ __launch_bounds__(256) void k_gla_fast(const float* __restrict__ QKV,
                                                   const float* __restrict__ Z,
                                                   const float* __restrict__ lam, StateRef S,
                                                   const uint32_t* __restrict__ seq,
                                                   float* __restrict__ O, uint32_t d,
                                                   uint32_t rglru) {
  constexpr int CB = 16, C4 = CB / 4;
  constexpr int RPP = 256 / C4;           // state rows per pass (64)
  constexpr int NP = (HD + RPP - 1) / RPP;
  __shared__ float al[HD], kh[HD], qh[HD], v[CB], sq[2];
  __shared__ float4 part[4][C4];
  const uint32_t h = blockIdx.x, cb = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const uint32_t sl = seq[b];
  float* Sg = S.base + (size_t)sl * S.seq_stride + S.layer_off + (size_t)h * HD * HD + cb * CB;
  const float* x = QKV + (size_t)b * 3 * d;
  // the block of S first: it does not depend on this token
  const uint32_t c4 = tid % C4, r0 = tid / C4;
  float4 sv[NP];
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const uint32_t r = r0 + RPP * p;
    sv[p] = *reinterpret_cast<const float4*>(Sg + (size_t)(r < HD ? r : 0) * HD + 4 * c4);
  }
  float qv = 0.0f, kv = 0.0f, zv = 0.0f, lv = 0.0f;
  if ((int)tid < HD) {
    qv = x[h * HD + tid];
    kv = x[d + h * HD + tid];
    zv = Z[(size_t)b * d + h * HD + tid];
    if (rglru) lv = lam[h * HD + tid];
  }
  if (tid < 64) {
    const float s0 = wave_sum(qv * qv), s1 = wave_sum(kv * kv);
    if (tid == 0) {
      sq[0] = s0;
      sq[1] = s1;
    }
  }
  if (tid < CB) v[tid] = x[2 * d + h * HD + cb * CB + tid];
  __syncthreads();
  if ((int)tid < HD) {
    qh[tid] = qv / sqrtf(1.0e-6f + sq[0]);
    const float kn = kv / sqrtf(1.0e-6f + sq[1]);
    if (rglru) {
      // dd.gate's RG-LRU arm (bend/Dense/Ex.bend:158-162)
      const float la = fminf(ANA_CAP, (8.0f * f_sigmoid(zv)) * f_log_sigmoid(lv));
      kh[tid] = kn * sqrtf(1.0f - expf(2.0f * la));
      al[tid] = expf(la);
    } else {
      al[tid] = f_sigmoid(zv);
      kh[tid] = kn;
    }
  }
  __syncthreads();
  float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const uint32_t r = r0 + RPP * p;
    if (r < HD) {
      const float a_ = al[r], k_ = kh[r], q_ = qh[r];
      float4 s = sv[p];
      s.x = fmaf(a_, s.x, k_ * v[4 * c4 + 0]);
      s.y = fmaf(a_, s.y, k_ * v[4 * c4 + 1]);
      s.z = fmaf(a_, s.z, k_ * v[4 * c4 + 2]);
      s.w = fmaf(a_, s.w, k_ * v[4 * c4 + 3]);
      *reinterpret_cast<float4*>(Sg + (size_t)r * HD + 4 * c4) = s;
      o.x = fmaf(q_, s.x, o.x);
      o.y = fmaf(q_, s.y, o.y);
      o.z = fmaf(q_, s.z, o.z);
      o.w = fmaf(q_, s.w, o.w);
    }
  }
  // sum over the rows: lanes differing in bits 2..5 share a column quad
#pragma unroll
  for (int m = 4; m < 64; m <<= 1) {
    o.x += __shfl_xor(o.x, m, 64);
    o.y += __shfl_xor(o.y, m, 64);
    o.z += __shfl_xor(o.z, m, 64);
    o.w += __shfl_xor(o.w, m, 64);
  }
  if ((tid & 63) < (uint32_t)C4) part[tid >> 6][tid & 63] = o;
  __syncthreads();
  if (tid < CB) {
    const uint32_t c = tid / 4, e = tid % 4;
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float4 p4 = part[w][c];
      acc += e == 0 ? p4.x : e == 1 ? p4.y : e == 2 ? p4.z : p4.w;
    }
    O[(size_t)b * d + h * HD + cb * CB + tid] = acc;
  }
}

hipError_t launch_gla_fast(const float* QKV, const float* Z, const float* lam, StateRef S,
                           const uint32_t* seq, float* O, uint32_t d, uint32_t heads,
                           uint32_t rglru, uint32_t B, hipStream_t st) {
  const uint32_t hd = d / heads;
  // off above kSmallB rows (those decode steps take the exact one-wave step)
  if (hd % 16 || B > kSmallB) return hipErrorInvalidValue;
#define L_(H) hipLaunchKernelGGL(k_gla_fast<H>, dim3(heads, H / 16, B), dim3(256), 0, st, QKV, Z, lam, S, seq, O, d, rglru)
  switch (hd) {
    case 64: L_(64); break;
    case 32: L_(32); break;
    case 16: L_(16); break;
    default: return hipErrorInvalidValue;
  }
#undef L_
  return hipGetLastError();
}

// The GLA step of a fast-mode decode batch above kSmallB rows (dd.gla.tok,
// bend/Dense/Decode.bend): one wave per (head, row) as the exact k_gla_w
// lays it out (lane b holds column b of S, the 64 rows in registers, loaded
// and stored as coalesced rows, the rows issued before this token's q|k|v|z
// since they do not depend on it), with the fast mode's arithmetic: the
// norms' sums by DPP over the wave, the hardware's reciprocal square root,
// the gates in float, S' = al_a S_ab + kh_a v_b as one fused multiply-add
// and o_b = sum_a qh_a S'_ab in four interleaved partial sums. (The exact
// kernel's in-order chains, double-precision gates and IEEE divisions held
// it at 8 us a layer at B = 64.)
__global__ __launch_bounds__(64) void k_gla_wf(const float* __restrict__ QKV, const float* __restrict__ Z,
                                               const float* __restrict__ lam, StateRef S,
                                               const uint32_t* __restrict__ seq, float* __restrict__ O,
                                               uint32_t d, uint32_t rglru) {
  constexpr int HD = 64;
  __shared__ __align__(16) float al[HD], kh[HD], qh[HD];
  const uint32_t h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  float* Sg = S.base + (size_t)seq[b] * S.seq_stride + S.layer_off + (size_t)h * HD * HD;
  float s[HD];
#pragma unroll
  for (int a = 0; a < HD; a++) s[a] = Sg[a * HD + lane];
  const float* x = QKV + (size_t)b * 3 * d;
  const float qv = x[h * HD + lane], kv = x[d + h * HD + lane], vv = x[2 * d + h * HD + lane];
  const float zv = Z[(size_t)b * d + h * HD + lane];
  const float lv = rglru ? lam[h * HD + lane] : 0.0f;
  const float s0 = wsum(qv * qv), s1 = wsum(kv * kv);
  const float kn = kv * __builtin_amdgcn_rsqf(1.0e-6f + s1);
  qh[lane] = qv * __builtin_amdgcn_rsqf(1.0e-6f + s0);
  if (rglru) {
    // dd.gate's RG-LRU arm (bend/Dense/Ex.bend:158-162)
    const float la = fminf(ANA_CAP, (8.0f * f_sigmoid(zv)) * f_log_sigmoid(lv));
    kh[lane] = kn * sqrtf(1.0f - expf(2.0f * la));
    al[lane] = expf(la);
  } else {
    al[lane] = f_sigmoid(zv);
    kh[lane] = kn;
  }
  __syncthreads();
  const float4* al4 = reinterpret_cast<const float4*>(al);
  const float4* kh4 = reinterpret_cast<const float4*>(kh);
  const float4* qh4 = reinterpret_cast<const float4*>(qh);
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int a4 = 0; a4 < HD / 4; a4++) {
    const float4 A = al4[a4], K = kh4[a4], Q = qh4[a4];
    const float an[4] = {A.x, A.y, A.z, A.w}, kn4[4] = {K.x, K.y, K.z, K.w}, qn[4] = {Q.x, Q.y, Q.z, Q.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int a = 4 * a4 + e;
      const float sa = fmaf(an[e], s[a], kn4[e] * vv);
      Sg[a * HD + lane] = sa;
      o[e] = fmaf(qn[e], sa, o[e]);
    }
  }
  O[(size_t)b * d + h * HD + lane] = (o[0] + o[1]) + (o[2] + o[3]);
}

hipError_t launch_gla_wfast(const float* QKV, const float* Z, const float* lam, StateRef S, const uint32_t* seq,
                            float* O, uint32_t d, uint32_t heads, uint32_t rglru, uint32_t B, hipStream_t st) {
  if (heads == 0 || d / heads != 64 || d % heads) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gla_wf, dim3(heads, B), dim3(64), 0, st, QKV, Z, lam, S, seq, O, d, rglru);
  return hipGetLastError();
}

// ------------------------------------------------------------------ attention

// Split softmax attention (flash decoding). Pass 1, per (head, split of
// kFastTS ring slots, row): qk-norm of q (and of k for the row's own slot,
// which the split holding it writes to the ring first), the scores, the
// split's max m, l = sum exp(s - m) and o = sum exp(s - m) v. Pass 2 folds
// the splits and the sink: m* = max(m_i, sink), den = sum l_i e^(m_i - m*)
// + e^(sink - m*), o = sum o_i e^(m_i - m*) / den.

template <int HD>
__global__ __launch_bounds__(256) void k_attn_fast_part(AttnArgs a) {
  constexpr int C4 = HD / 4;       // column quads
  constexpr int QD = HD / 4;       // dims per score lane (4 lanes a slot)
  __shared__ float q[HD], kk[HD], vs[HD], es[kFastTS], red[4], nrm[2];
  __shared__ float4 op[4][C4];
  const uint32_t h = blockIdx.x, sp = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const uint32_t d = a.d, ctx = a.ctx, ns = gridDim.y;
  // a decode row (its sequence and position), or row b of a chunk of one
  // sequence at positions pos0 + b
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t slot = pos % ctx, npos = pos < ctx - 1 ? pos : ctx - 1;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  float* Kr = a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off;
  float* Vr = Kr + (size_t)ctx * d;
  const uint32_t t0 = sp * kFastTS;
  float* out = a.part + (((size_t)b * a.heads + h) * ns + sp) * (HD + 2);
  // a split past the row's last live slot holds nothing (nor the row's own
  // slot, which is live); the combine reads only live splits
  if (t0 > npos) return;
  const bool mine = a.write_kv && slot >= t0 && slot < t0 + kFastTS;
  const uint32_t nt = min(kFastTS, npos + 1 - t0);
  // score lanes: slot i = tid / 4, dims [qq * QD, (qq + 1) * QD)
  const uint32_t i = tid >> 2, qq = tid & 3, t = t0 + i;
  const bool live = i < nt;
  // V lanes: column quad c4, slots g, g + 256 / C4, ...
  constexpr int GS = 256 / C4;
  const uint32_t c4 = tid % C4, g = tid / C4;
  float4 kv[QD / 4], vv[(kFastTS + GS - 1) / GS];
  {
    const float4* k4 = reinterpret_cast<const float4*>(Kr + (size_t)(live ? t : t0) * d + h * HD + qq * QD);
#pragma unroll
    for (int u = 0; u < QD / 4; u++) kv[u] = k4[u];
#pragma unroll
    for (int j = 0; j < (int)((kFastTS + GS - 1) / GS); j++) {
      const uint32_t ii = g + GS * j;
      vv[j] = *reinterpret_cast<const float4*>(Vr + (size_t)(t0 + (ii < nt ? ii : 0)) * d + h * HD + 4 * c4);
    }
  }
  const float* x = a.QKV + (size_t)b * 3 * d;
  if (tid < 64) {
    const float qv = (int)tid < HD ? x[h * HD + tid] : 0.0f;
    if ((int)tid < HD) q[tid] = qv;
    if (a.gq) {
      const float s2 = wave_sum(qv * qv);
      if (tid == 0) nrm[0] = 1.0f / sqrtf(s2 / (float)HD + 1.0e-5f);
    }
  } else if (tid < 128 && mine) {
    const uint32_t e = tid - 64;
    const float kx = (int)e < HD ? x[d + h * HD + e] : 0.0f;
    if ((int)e < HD) {
      kk[e] = kx;
      vs[e] = x[2 * d + h * HD + e];
    }
    if (a.gk) {
      const float s2 = wave_sum(kx * kx);
      if (e == 0) nrm[1] = 1.0f / sqrtf(s2 / (float)HD + 1.0e-5f);
    }
  }
  __syncthreads();
  if (a.gq && (int)tid < HD) q[tid] = (q[tid] * nrm[0]) * (1.0f + a.gq[tid]);
  if (mine && tid >= 64 && (int)(tid - 64) < HD) {
    const uint32_t e = tid - 64;
    if (a.gk) kk[e] = (kk[e] * nrm[1]) * (1.0f + a.gk[e]);
    Kr[(size_t)slot * d + h * HD + e] = kk[e];
    Vr[(size_t)slot * d + h * HD + e] = vs[e];
  }
  __syncthreads();
  const float sc = 1.0f / sqrtf((float)HD);
  float acc = 0.0f;
  if (mine && t == slot) {
#pragma unroll
    for (int c = 0; c < QD; c++) acc = fmaf(q[qq * QD + c], kk[qq * QD + c], acc);
  } else {
#pragma unroll
    for (int u = 0; u < QD / 4; u++) {
      const uint32_t c = qq * QD + 4 * u;
      acc = fmaf(q[c + 0], kv[u].x, acc);
      acc = fmaf(q[c + 1], kv[u].y, acc);
      acc = fmaf(q[c + 2], kv[u].z, acc);
      acc = fmaf(q[c + 3], kv[u].w, acc);
    }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  const float y = live ? sc * acc : -INFINITY;
  // split max, then exp and its sum
  float m = y;
#pragma unroll
  for (int s2 = 32; s2 >= 4; s2 >>= 1) {
    const float o = __shfl_xor(m, s2, 64);
    m = o > m ? o : m;
  }
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float e = live ? __expf(y - m) : 0.0f;
  if (qq == 0) es[i] = e;
  const float ls = wave_sum(qq == 0 ? e : 0.0f);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = ls;
  float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int j = 0; j < (int)((kFastTS + GS - 1) / GS); j++) {
    const uint32_t ii = g + GS * j;
    if (ii < nt) {
      float4 v4 = vv[j];
      if (mine && t0 + ii == slot) v4 = make_float4(vs[4 * c4], vs[4 * c4 + 1], vs[4 * c4 + 2], vs[4 * c4 + 3]);
      const float ev = es[ii];
      o.x = fmaf(ev, v4.x, o.x);
      o.y = fmaf(ev, v4.y, o.y);
      o.z = fmaf(ev, v4.z, o.z);
      o.w = fmaf(ev, v4.w, o.w);
    }
  }
  // sum over the slot groups: lanes differing above the column-quad bits
#pragma unroll
  for (int s2 = C4; s2 < 64; s2 <<= 1) {
    o.x += __shfl_xor(o.x, s2, 64);
    o.y += __shfl_xor(o.y, s2, 64);
    o.z += __shfl_xor(o.z, s2, 64);
    o.w += __shfl_xor(o.w, s2, 64);
  }
  if ((tid & 63) < (uint32_t)C4) op[tid >> 6][tid & 63] = o;
  __syncthreads();
  if ((int)tid < HD) {
    const uint32_t c = tid / 4, e4 = tid % 4;
    float s2 = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float4 p4 = op[w][c];
      s2 += e4 == 0 ? p4.x : e4 == 1 ? p4.y : e4 == 2 ? p4.z : p4.w;
    }
    out[2 + tid] = s2;
  }
  if (tid == 0) {
    out[0] = m;
    out[1] = red[0] + red[1] + red[2] + red[3];
  }
}

// the row's live splits, at most 64 (one lane each), of ns in the grid
template <int HD>
__global__ __launch_bounds__(64) void k_attn_fast_comb(AttnArgs a, uint32_t ns) {
  __shared__ float wgt[64];
  __shared__ float den_s;
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t npos = pos < a.ctx - 1 ? pos : a.ctx - 1;
  const uint32_t nl = min(ns, npos / kFastTS + 1);
  const float* p = a.part + ((size_t)b * a.heads + h) * ns * (HD + 2);
  // every split's (m, l) at once, one lane each
  const float mi = tid < nl ? p[tid * (HD + 2)] : -INFINITY;
  const float li = tid < nl ? p[tid * (HD + 2) + 1] : 0.0f;
  float m = mi;
#pragma unroll
  for (int s2 = 32; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2, 64));
  float sink = 0.0f;
  if (a.sink) {
    sink = a.sink[h];
    m = fmaxf(m, sink);
  }
  const float w = mi == -INFINITY ? 0.0f : __expf(mi - m);
  wgt[tid] = w;
  const float den = wave_sum(li * w);
  if (tid == 0) den_s = a.sink ? den + __expf(sink - m) : den;
  __syncthreads();
  if ((int)tid < HD) {
    float o = 0.0f;
#pragma unroll 8
    for (uint32_t i = 0; i < nl; i++) o = fmaf(p[i * (HD + 2) + 2 + tid], wgt[i], o);
    a.O[(size_t)b * a.d + h * HD + tid] = o / den_s;
  }
}

hipError_t launch_attn_fast(const AttnArgs& a, hipStream_t st) {
  const uint32_t hd = a.d / a.heads;
  const uint32_t full = (a.ctx + kFastTS - 1) / kFastTS;
  const uint32_t ns = a.nsp ? min(a.nsp, full) : full;
  if (!a.part || hd % 4 || hd > 64 || full > 64) return hipErrorInvalidValue;
  // decode steps above kSmallB rows are off on this kernel; the partials
  // of every (row, head, split) must fit the buffer
  if (a.write_kv && a.B > kSmallB) return hipErrorInvalidValue;
  if ((size_t)a.B * a.heads * ns * (hd + 2) > a.part_cap) return hipErrorInvalidValue;
#define L_(H)                                                                                   \
  hipLaunchKernelGGL(k_attn_fast_part<H>, dim3(a.heads, ns, a.B), dim3(256), 0, st, a);        \
  hipLaunchKernelGGL(k_attn_fast_comb<H>, dim3(a.heads, a.B), dim3(64), 0, st, a, ns)
  switch (hd) {
    case 64: L_(64); break;
    case 32: L_(32); break;
    case 16: L_(16); break;
    default: return hipErrorInvalidValue;
  }
#undef L_
  return hipGetLastError();
}

// Decode attention of more than kSmallB rows in the fast modes: one
// workgroup per (head, row) over the row's live slots 0 .. npos. The row's
// k (qk-normed when on) and v go to its slot first; its own slot's score
// and product take them from LDS. A slot is L = HD / 4 lanes (a float4 of
// its K or V row each, so a slot's row is one 16 L-byte piece), the
// workgroup G = 256 / L slot groups, and a trip U slots a group, the next
// trip's loads in flight while one computes. Pass 1 keeps sc*s in LDS
// (ctx floats, dynamic); the max (with the sink) and the denominator come
// from wave and block reductions; pass 2 sums e*V per lane over its slots
// for its four columns, and the G slot groups meet in LDS. With a split
// grid (gridDim.z > 1) workgroup z takes slots z SL .. z SL + SL - 1 of the
// live ones (SL = kRowsSplit), and leaves its max m, its sum l = sum e and
// its o = sum e V (e = exp(sc s - m), no sink) in part for k_attn_rows_comb.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_rows(AttnArgs a) {
  constexpr int L = HD / 4, G = 256 / L, U = 4;
  extern __shared__ float ss[];   // [ctx] or [kRowsSplit]
  __shared__ __align__(16) float q[HD];
  __shared__ __align__(16) float kk[HD];
  __shared__ __align__(16) float vs[HD];
  __shared__ float red[4], red2[4], nrm[2];
  __shared__ float4 op[G][L];
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t d = a.d, ctx = a.ctx;
  const uint32_t pos = a.pos[b];
  const uint32_t slot = pos % ctx, npos = pos < ctx - 1 ? pos : ctx - 1;
  const uint32_t nsp = gridDim.z, sp = blockIdx.z;
  const uint32_t s0 = nsp > 1 ? sp * kRowsSplit : 0u;
  const uint32_t s1 = nsp > 1 ? min(npos + 1, s0 + kRowsSplit) : npos + 1;   // slots s0 .. s1 - 1
  float* part = nsp > 1 ? a.part + (((size_t)b * a.heads + h) * nsp + sp) * (HD + 2) : nullptr;
  if (s0 >= s1) {
    // no live slot in this split
    if (tid < HD) part[2 + tid] = 0.0f;
    if (tid == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    return;
  }
  float* Kr = a.KV.base + (size_t)a.seq[b] * a.KV.seq_stride + a.KV.layer_off;
  float* Vr = Kr + (size_t)ctx * d;
  const float* x = a.QKV + (size_t)b * 3 * d;
  if (tid < HD) {
    q[tid] = x[h * HD + tid];
    kk[tid] = x[d + h * HD + tid];
    vs[tid] = x[2 * d + h * HD + tid];
  }
  __syncthreads();
  if (a.gq) {
    // M.qkn (bend/Dense/Model.bend:39-42) on q (wave 0) and k (wave 1)
    if (wv < 2) {
      const float v = lane < (uint32_t)HD ? (wv == 0 ? q[lane] : kk[lane]) : 0.0f;
      const float t = wave_sum(v * v);
      if (lane == 0) nrm[wv] = 1.0f / sqrtf(t / (float)HD + 1.0e-5f);
    }
    __syncthreads();
    if (tid < HD) {
      q[tid] = (q[tid] * nrm[0]) * (1.0f + a.gq[tid]);
      kk[tid] = (kk[tid] * nrm[1]) * (1.0f + a.gk[tid]);
    }
    __syncthreads();
  }
  if (tid < HD && slot >= s0 && slot < s1) {
    Kr[(size_t)slot * d + h * HD + tid] = kk[tid];
    Vr[(size_t)slot * d + h * HD + tid] = vs[tid];
  }
  const uint32_t li = tid % L, g = tid / L;
  const float4 q4 = *reinterpret_cast<const float4*>(&q[4 * li]);
  float4 k4o = *reinterpret_cast<const float4*>(&kk[4 * li]);
  float4 v4o = *reinterpret_cast<const float4*>(&vs[4 * li]);
  // opaque register values from here: a select between them and a ring load
  // must stay a select (as a select of two loads it becomes one flat load
  // through a stack copy)
  asm volatile("" : "+v"(k4o.x), "+v"(k4o.y), "+v"(k4o.z), "+v"(k4o.w));
  asm volatile("" : "+v"(v4o.x), "+v"(v4o.y), "+v"(v4o.z), "+v"(v4o.w));
  const float sc = 1.0f / sqrtf((float)HD);
  // one trip's pieces of ring `base` (own slot from `own`), index clamped
  auto load = [&](const float* base, float4 own, uint32_t t0, float4* r) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t t = t0 + g + u * G;
      const float4 v = *reinterpret_cast<const float4*>(base + (size_t)(t < s1 ? t : s0) * d);
      r[u] = t == slot ? own : v;
    }
  };
  const float* kb = Kr + h * HD + 4 * li;
  const float* vb = Vr + h * HD + 4 * li;
  float4 cur[U], nxt[U];
  load(kb, k4o, s0, cur);
  for (uint32_t t0 = s0; t0 < s1; t0 += U * G) {
    const bool more = t0 + U * G < s1;
    if (more) load(kb, k4o, t0 + U * G, nxt);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t t = t0 + g + u * G;
      float sdot = (q4.x * cur[u].x + q4.y * cur[u].y) + (q4.z * cur[u].z + q4.w * cur[u].w);
#pragma unroll
      for (int mk = 1; mk < L; mk <<= 1) sdot += __shfl_xor(sdot, mk, 64);
      if (li == 0 && t < s1) ss[t - s0] = sc * sdot;
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < U; u++) cur[u] = nxt[u];
    }
  }
  // the first V trip flies through the reductions
  load(vb, v4o, s0, cur);
  __syncthreads();
  const uint32_t ns = s1 - s0;
  float r = -INFINITY;
  for (uint32_t t = tid; t < ns; t += 256) r = fmaxf(r, ss[t]);
#pragma unroll
  for (int mk = 32; mk >= 1; mk >>= 1) r = fmaxf(r, __shfl_xor(r, mk, 64));
  if (lane == 0) red[wv] = r;
  __syncthreads();
  float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sink = a.sink ? a.sink[h] : 0.0f;
  if (a.sink && nsp == 1) mx = fmaxf(mx, sink);
  float se = 0.0f;
  for (uint32_t t = tid; t < ns; t += 256) {
    const float e = expf(ss[t] - mx);
    ss[t] = e;
    se += e;
  }
  se = wave_sum(se);
  if (lane == 0) red2[wv] = se;
  __syncthreads();
  float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (uint32_t t0 = s0; t0 < s1; t0 += U * G) {
    const bool more = t0 + U * G < s1;
    if (more) load(vb, v4o, t0 + U * G, nxt);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t t = t0 + g + u * G;
      const float e = t < s1 ? ss[t - s0] : 0.0f;
      o.x = fmaf(e, cur[u].x, o.x);
      o.y = fmaf(e, cur[u].y, o.y);
      o.z = fmaf(e, cur[u].z, o.z);
      o.w = fmaf(e, cur[u].w, o.w);
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < U; u++) cur[u] = nxt[u];
    }
  }
  op[g][li] = o;
  __syncthreads();
  if (tid < HD) {
    const uint32_t c = tid / 4, e = tid % 4;
    float acc = 0.0f;
#pragma unroll 8
    for (int j = 0; j < G; j++) {
      const float4 p4 = op[j][c];
      acc += e == 0 ? p4.x : e == 1 ? p4.y : e == 2 ? p4.z : p4.w;
    }
    float den = ((red2[0] + red2[1]) + red2[2]) + red2[3];
    if (nsp > 1) {
      part[2 + tid] = acc;
      if (tid == 0) {
        part[0] = mx;
        part[1] = den;
      }
      return;
    }
    if (a.sink) den += expf(sink - mx);
    a.O[(size_t)b * d + h * HD + tid] = acc / den;
  }
}

// the splits of k_attn_rows for one (head, row), with the sink:
// M = max(m_i, sink), den = sum l_i e^(m_i - M) + e^(sink - M),
// o = sum o_i e^(m_i - M) / den
template <int HD>
__global__ __launch_bounds__(64) void k_attn_rows_comb(AttnArgs a, uint32_t nsp) {
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const float* part = a.part + ((size_t)b * a.heads + h) * nsp * (HD + 2);
  if (tid >= (uint32_t)HD) return;
  float M = a.sink ? a.sink[h] : -INFINITY;
  for (uint32_t i = 0; i < nsp; i++) M = fmaxf(M, part[i * (HD + 2)]);
  float den = a.sink ? expf(a.sink[h] - M) : 0.0f, acc = 0.0f;
  for (uint32_t i = 0; i < nsp; i++) {
    const float* p = part + i * (HD + 2);
    const float w = expf(p[0] - M);
    den = fmaf(p[1], w, den);
    acc = fmaf(p[2 + tid], w, acc);
  }
  a.O[(size_t)b * a.d + h * HD + tid] = acc / den;
}

hipError_t launch_attn_rows(const AttnArgs& a, bool split, hipStream_t st) {
  const uint32_t hd = a.heads ? a.d / a.heads : 0;
  if (!a.seq || !a.pos || !a.write_kv || a.ctx == 0 || hd * a.heads != a.d) return hipErrorInvalidValue;
  if (!split && a.ctx > kAttnRowsMaxCtx) return hipErrorInvalidValue;
  if (split && !a.part) return hipErrorInvalidValue;
  const uint32_t nsp = split ? (a.ctx + kRowsSplit - 1) / kRowsSplit : 1u;
  if (split && (size_t)a.B * a.heads * nsp * (hd + 2) > a.part_cap) return hipErrorInvalidValue;
  const size_t lds = (size_t)(split ? kRowsSplit : a.ctx) * 4;
#define L_(H)                                                                                       \
  hipLaunchKernelGGL(k_attn_rows<H>, dim3(a.heads, a.B, nsp), dim3(256), lds, st, a);              \
  if (split) hipLaunchKernelGGL(k_attn_rows_comb<H>, dim3(a.heads, a.B), dim3(64), 0, st, a, nsp)
  switch (hd) {
    case 64: L_(64); break;
    case 32: L_(32); break;
    case 16: L_(16); break;
    default: return hipErrorInvalidValue;
  }
#undef L_
  return hipGetLastError();
}

size_t attn_fast_part_floats(uint32_t B, uint32_t heads, uint32_t ctx, uint32_t hd) {
  return (size_t)B * heads * ((ctx + kFastTS - 1) / kFastTS) * (hd + 2);
}

// ------------------------------------------------------------------ prefill attention on the matrix cores

// Fresh prefill chunks (no slot past the ring's wrap): causal attention of a
// tile of up to kFlashQ query rows of one sequence over slots 0 .. the tile's
// last position, flash style. Per key tile of 64 slots: S = (sc q) K^T on
// v_mfma_f32_16x16x4f32, the running max m and sum l per row,
// O <- O e^(m_old - m_new) + P V; at the end the sink joins the max and the
// denominator as in the split kernels: o = O e^(m - m*) / (l e^(m - m*) +
// e^(sink - m*)). Wave w holds query rows 16 w .. 16 w + 15. Inside an MFMA
// the 4 k-lanes of lane group g take dims (or slots) [Q g, Q g + Q), so each
// lane reads its operands as contiguous 16-byte pieces.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_flash(AttnArgs a, const AttnTile* __restrict__ tab) {
  constexpr int KT = 64;                 // slots per key tile
  constexpr int DG = HD / 4;             // dims per lane group in S = Q K^T
  constexpr int NJ = HD / 16;            // 16-dim output tiles
  constexpr int KP = HD + 4, VP = KT + 4, PP = KT + 4;
  __shared__ __align__(16) float Ks[KT][KP];
  __shared__ __align__(16) float Vt[HD][VP];
  __shared__ __align__(16) float Ps[4][16][PP];
  const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t r16 = lane & 15, g = lane >> 4;
  const AttnTile tt = tab[blockIdx.y];
  const uint32_t d = a.d;
  const float* Kr = a.KV.base + (size_t)tt.seq * a.KV.seq_stride + a.KV.layer_off;
  const float* Vr = Kr + (size_t)a.ctx * d;
  const uint32_t last = tt.pos0 + tt.n - 1;          // the tile's last position (< ctx)
  // this lane's query row for the S operand, dims [DG g, DG g + DG), qk-normed
  // and scaled by 1 / sqrt(hd)
  float q[DG];
  {
    const uint32_t qr = 16 * w + r16;
    const float* x = a.QKV + (size_t)(tt.row0 + (qr < tt.n ? qr : 0)) * 3 * d + h * HD + DG * g;
#pragma unroll
    for (int i = 0; i < DG / 4; i++) {
      const float4 v = *reinterpret_cast<const float4*>(x + 4 * i);
      q[4 * i] = v.x;
      q[4 * i + 1] = v.y;
      q[4 * i + 2] = v.z;
      q[4 * i + 3] = v.w;
    }
    float s = 1.0f / sqrtf((float)HD);
    if (a.gq) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < DG; i++) ss = fmaf(q[i], q[i], ss);
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      const float rs = 1.0f / sqrtf(ss / (float)HD + 1.0e-5f);
#pragma unroll
      for (int i = 0; i < DG; i++) q[i] = (q[i] * rs) * (1.0f + a.gq[DG * g + i]);
    }
#pragma unroll
    for (int i = 0; i < DG; i++) q[i] *= s;
  }
  // rows of this lane in the result layout: 16 w + 4 g + r
  float m[4], l[4];
  f32x4_t o[NJ];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NJ; j++) o[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t nkt = last / KT + 1;
  for (uint32_t kt = 0; kt < nkt; kt++) {
    const uint32_t k0 = kt * KT;
    __syncthreads();   // the previous tile's K, V and P reads are done
    for (uint32_t e = tid; e < (uint32_t)KT * (HD / 4); e += 256) {
      const uint32_t s = e / (HD / 4), c4 = e % (HD / 4);
      const uint32_t slot = k0 + s <= last ? k0 + s : 0;
      const float4 kv = *reinterpret_cast<const float4*>(Kr + (size_t)slot * d + h * HD + 4 * c4);
      const float4 vv = *reinterpret_cast<const float4*>(Vr + (size_t)slot * d + h * HD + 4 * c4);
      *reinterpret_cast<float4*>(&Ks[s][4 * c4]) = kv;
      Vt[4 * c4][s] = vv.x;
      Vt[4 * c4 + 1][s] = vv.y;
      Vt[4 * c4 + 2][s] = vv.z;
      Vt[4 * c4 + 3][s] = vv.w;
    }
    __syncthreads();
    // scores of the wave's 16 rows against the tile's 4 x 16 slots
    f32x4_t sc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      sc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      const float* kr = &Ks[16 * j + r16][DG * g];
#pragma unroll
      for (int i = 0; i < DG / 4; i++) {
        const float4 kk = *reinterpret_cast<const float4*>(kr + 4 * i);
        sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * i], kk.x, sc[j], 0, 0, 0);
        sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * i + 1], kk.y, sc[j], 0, 0, 0);
        sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * i + 2], kk.z, sc[j], 0, 0, 0);
        sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * i + 3], kk.w, sc[j], 0, 0, 0);
      }
    }
    // causal mask, running max and sum per row (a row's slots lie across the
    // 16 lanes of its group)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t row = 16 * w + 4 * g + r;
      const uint32_t qpos = tt.pos0 + (row < tt.n ? row : tt.n - 1);
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t slot = k0 + 16 * j + r16;
        if (slot > qpos) sc[j][r] = -INFINITY;
        mx = fmaxf(mx, sc[j][r]);
      }
#pragma unroll
      for (int s2 = 1; s2 < 16; s2 <<= 1) mx = fmaxf(mx, __shfl_xor(mx, s2, 64));
      const float mn = fmaxf(m[r], mx);   // finite: slot k0 <= qpos always
      const float al = __expf(m[r] - mn);
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float p = __expf(sc[j][r] - mn);
        sum += p;
        Ps[w][4 * g + r][16 * j + r16] = p;
      }
#pragma unroll
      for (int s2 = 1; s2 < 16; s2 <<= 1) sum += __shfl_xor(sum, s2, 64);
      l[r] = l[r] * al + sum;
      m[r] = mn;
#pragma unroll
      for (int j = 0; j < NJ; j++) o[j][r] *= al;
    }
    __syncthreads();
    // O += P V: row r16 of the wave's P, slots [16 g, 16 g + 16)
    const float* pr = &Ps[w][r16][16 * g];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 p4 = *reinterpret_cast<const float4*>(pr + 4 * i);
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const float4 v4 = *reinterpret_cast<const float4*>(&Vt[16 * j + r16][16 * g + 4 * i]);
        o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.x, v4.x, o[j], 0, 0, 0);
        o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.y, v4.y, o[j], 0, 0, 0);
        o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.z, v4.z, o[j], 0, 0, 0);
        o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.w, v4.w, o[j], 0, 0, 0);
      }
    }
  }
  // the sink, then the rows out
  const float sink = a.sink ? a.sink[h] : -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t row = 16 * w + 4 * g + r;
    if (row >= tt.n) continue;
    const float ms = fmaxf(m[r], sink);
    const float e = __expf(m[r] - ms);
    const float den = l[r] * e + (a.sink ? __expf(sink - ms) : 0.0f);
    const float f = e / den;
    const size_t ob = (size_t)(tt.row0 + row) * d + h * HD;
    if (a.Oh) {
#pragma unroll
      for (int j = 0; j < NJ; j++) a.Oh[ob + 16 * j + r16] = (__bf16)(o[j][r] * f);
    } else {
#pragma unroll
      for (int j = 0; j < NJ; j++) a.O[ob + 16 * j + r16] = o[j][r] * f;
    }
  }
}

// k_attn_flash with its two products on the bf16 matrix cores (ANA_BF16,
// hd a multiple of 32): q (qk-normed and scaled), the K and V tiles and
// the probabilities rounded to bf16, S = q K^T and O += P V accumulated in
// fp32 on v_mfma_f32_16x16x32_bf16 (two instructions a 16 x 16 tile where
// the fp32 kernel takes sixteen); mask, online max and sum, sink and output
// as in k_attn_flash. Eight waves take a tile of up to kFlashQBf = 128
// query rows, so each staged K and V tile serves twice the rows of the
// fp32 kernel's 64 (each workgroup of a sequence restages every tile up to
// its last position). A lane's fragments: query row r16 of its wave's 16
// (or slot r16 of a 16-slot group, or output column r16), k elements
// 32 kk + 8 g4 .. + 7.
template <int HD>
__global__ __launch_bounds__(512) void k_attn_flash_bf(AttnArgs a, const AttnTile* __restrict__ tab) {
  constexpr int KT = 64;                 // slots per key tile
  constexpr int NK = HD / 32;            // 32-dim k steps of S = q K^T
  constexpr int NJ = HD / 16;            // 16-dim output tiles
  constexpr int KP = HD + 8, VP = KT + 8, PP = KT + 8;   // bf16 row pitches (16-byte multiples)
  static_assert(HD % 32 == 0, "hd a multiple of 32");
  __shared__ __align__(16) __bf16 Ks[KT][KP];
  __shared__ __align__(16) __bf16 Vt[HD][VP];
  __shared__ __align__(16) __bf16 Ps[8][16][PP];
  const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t r16 = lane & 15, g = lane >> 4;
  const AttnTile tt = tab[blockIdx.y];
  const uint32_t d = a.d;
  const float* Kr = a.KV.base + (size_t)tt.seq * a.KV.seq_stride + a.KV.layer_off;
  const float* Vr = Kr + (size_t)a.ctx * d;
  const uint32_t last = tt.pos0 + tt.n - 1;          // the tile's last position (< ctx)
  bf16x8_t qf[NK];
  {
    const uint32_t qr = 16 * w + r16;
    const float* x = a.QKV + (size_t)(tt.row0 + (qr < tt.n ? qr : 0)) * 3 * d + h * HD;
    float qv[NK][8];
#pragma unroll
    for (int kk = 0; kk < NK; kk++) {
      const float4 v0 = *reinterpret_cast<const float4*>(x + 32 * kk + 8 * g);
      const float4 v1 = *reinterpret_cast<const float4*>(x + 32 * kk + 8 * g + 4);
      qv[kk][0] = v0.x; qv[kk][1] = v0.y; qv[kk][2] = v0.z; qv[kk][3] = v0.w;
      qv[kk][4] = v1.x; qv[kk][5] = v1.y; qv[kk][6] = v1.z; qv[kk][7] = v1.w;
    }
    const float s = 1.0f / sqrtf((float)HD);
    if (a.gq) {
      float ss = 0.0f;
#pragma unroll
      for (int kk = 0; kk < NK; kk++)
#pragma unroll
        for (int e = 0; e < 8; e++) ss = fmaf(qv[kk][e], qv[kk][e], ss);
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      const float rs = 1.0f / sqrtf(ss / (float)HD + 1.0e-5f);
#pragma unroll
      for (int kk = 0; kk < NK; kk++)
#pragma unroll
        for (int e = 0; e < 8; e++) qv[kk][e] = (qv[kk][e] * rs) * (1.0f + a.gq[32 * kk + 8 * g + e]);
    }
#pragma unroll
    for (int kk = 0; kk < NK; kk++)
#pragma unroll
      for (int e = 0; e < 8; e++) qf[kk][e] = (__bf16)(qv[kk][e] * s);
  }
  // rows of this lane in the result layout: 16 w + 4 g + r
  float m[4], l[4];
  f32x4_t o[NJ];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NJ; j++) o[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t nkt = last / KT + 1;
  // this thread's float4s of a key tile's K and V rows (e = tid + 512 i:
  // slot e / (HD / 4), columns 4 (e % (HD / 4)) ..), loaded a tile ahead so
  // they are in flight through the tile before
  constexpr int NE = KT * (HD / 4) / 512;
  static_assert(NE >= 1 && NE * 512 == KT * (HD / 4), "whole float4s a thread");
  float4 kr[NE], vr[NE];
  auto load_tile = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < NE; i++) {
      const uint32_t e = tid + 512 * i, s = e / (HD / 4), c4 = e % (HD / 4);
      const uint32_t slot = k0 + s <= last ? k0 + s : 0;
      kr[i] = *reinterpret_cast<const float4*>(Kr + (size_t)slot * d + h * HD + 4 * c4);
      vr[i] = *reinterpret_cast<const float4*>(Vr + (size_t)slot * d + h * HD + 4 * c4);
    }
  };
  load_tile(0);
  for (uint32_t kt = 0; kt < nkt; kt++) {
    __syncthreads();   // the previous tile's K, V and P reads are done
#pragma unroll
    for (int i = 0; i < NE; i++) {
      const uint32_t e = tid + 512 * i, s = e / (HD / 4), c4 = e % (HD / 4);
      const float4 kv = kr[i], vv = vr[i];
      __bf16 kb[4] = {(__bf16)kv.x, (__bf16)kv.y, (__bf16)kv.z, (__bf16)kv.w};
      *reinterpret_cast<uint2*>(&Ks[s][4 * c4]) = *reinterpret_cast<const uint2*>(kb);
      Vt[4 * c4][s] = (__bf16)vv.x;
      Vt[4 * c4 + 1][s] = (__bf16)vv.y;
      Vt[4 * c4 + 2][s] = (__bf16)vv.z;
      Vt[4 * c4 + 3][s] = (__bf16)vv.w;
    }
    if (kt + 1 < nkt) load_tile((kt + 1) * KT);
    const uint32_t k0 = kt * KT;
    __syncthreads();
    // scores of the wave's 16 rows against the tile's 4 x 16 slots
    f32x4_t sc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      sc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < NK; kk++) {
        const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&Ks[16 * j + r16][32 * kk + 8 * g]);
        sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[kk], kf, sc[j], 0, 0, 0);
      }
    }
    // causal mask, running max and sum per row (a row's slots lie across the
    // 16 lanes of its group)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t row = 16 * w + 4 * g + r;
      const uint32_t qpos = tt.pos0 + (row < tt.n ? row : tt.n - 1);
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t slot = k0 + 16 * j + r16;
        if (slot > qpos) sc[j][r] = -INFINITY;
        mx = fmaxf(mx, sc[j][r]);
      }
      mx = row16_max(mx);
      const float mn = fmaxf(m[r], mx);   // finite: slot k0 <= qpos always
      const float al = __expf(m[r] - mn);
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float p = __expf(sc[j][r] - mn);
        sum += p;
        Ps[w][4 * g + r][16 * j + r16] = (__bf16)p;
      }
      sum = row16_sum(sum);
      l[r] = l[r] * al + sum;
      m[r] = mn;
#pragma unroll
      for (int j = 0; j < NJ; j++) o[j][r] *= al;
    }
    __syncthreads();
    // O += P V: row r16 of the wave's P, slots 32 kk + 8 g ..
#pragma unroll
    for (int kk = 0; kk < KT / 32; kk++) {
      const bf16x8_t pf = *reinterpret_cast<const bf16x8_t*>(&Ps[w][r16][32 * kk + 8 * g]);
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const bf16x8_t vf = *reinterpret_cast<const bf16x8_t*>(&Vt[16 * j + r16][32 * kk + 8 * g]);
        o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf, vf, o[j], 0, 0, 0);
      }
    }
  }
  // the sink, then the rows out
  const float sink = a.sink ? a.sink[h] : -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t row = 16 * w + 4 * g + r;
    if (row >= tt.n) continue;
    const float ms = fmaxf(m[r], sink);
    const float e = __expf(m[r] - ms);
    const float den = l[r] * e + (a.sink ? __expf(sink - ms) : 0.0f);
    const float f = e / den;
    const size_t ob = (size_t)(tt.row0 + row) * d + h * HD;
    if (a.Oh) {
#pragma unroll
      for (int j = 0; j < NJ; j++) a.Oh[ob + 16 * j + r16] = (__bf16)(o[j][r] * f);
    } else {
#pragma unroll
      for (int j = 0; j < NJ; j++) a.O[ob + 16 * j + r16] = o[j][r] * f;
    }
  }
}

uint32_t attn_flash_tile_rows(bool bf, uint32_t hd) { return bf && (hd == 64 || hd == 32) ? kFlashQBf : kFlashQ; }

hipError_t launch_attn_flash(const AttnArgs& a, const AttnTile* tab, uint32_t ntiles, bool bf, hipStream_t st) {
  const uint32_t hd = a.d / a.heads;
  if (ntiles == 0) return hipSuccess;
  if (attn_flash_tile_rows(bf, hd) == kFlashQBf) {
    if (hd == 64) hipLaunchKernelGGL(k_attn_flash_bf<64>, dim3(a.heads, ntiles), dim3(512), 0, st, a, tab);
    else hipLaunchKernelGGL(k_attn_flash_bf<32>, dim3(a.heads, ntiles), dim3(512), 0, st, a, tab);
    return hipGetLastError();
  }
#define L_(H) hipLaunchKernelGGL(k_attn_flash<H>, dim3(a.heads, ntiles), dim3(256), 0, st, a, tab)
  switch (hd) {
    case 64: L_(64); break;
    case 32: L_(32); break;
    case 16: L_(16); break;
    default: return hipErrorInvalidValue;
  }
#undef L_
  return hipGetLastError();
}

}  // namespace ana

namespace ana {

// ------------------------------------------------------------------ batched products on MFMA

// Larger batches (prefill chunks, batched decode) in the fast modes:
// Y[m][n] = sum_k X[m][k] W[n][k] on the matrix cores. A workgroup owns 16
// weight rows (n) and 64 batch rows (m); wave w computes the 16 x 16 tile
// of batch rows 16w.. with v_mfma_f32_16x16x32_bf16 (ANA_BF16: bf16
// weights and activations rounded to bf16) or v_mfma_f32_16x16x4f32
// (ANA_FAST_FP32). K goes in
// chunks of 64 through a ring of D register sets (D - 1 chunks in flight)
// and two LDS buffers. With `ng` the chunk is staged as x * g and each
// row's sum of squares is gathered on the way, so M.norm's scale
// 1/sqrt(ss/K + 1e-5) multiplies the row's results in the epilogue.
// Epilogues: plain, residual, SiLU (tile rows 0..7 gate j, 8..15 up j).
template <int WT, int D>
__global__ __launch_bounds__(256) void k_gemm_mfma(GemvArgs a) {
  constexpr int BK = 64, BM = 64, BN = 16;
  constexpr int XP = BK + 8;             // LDS row pitch (elements), bf16 or f32
  using E = typename std::conditional<WT == 1, __bf16, float>::type;
  __shared__ __align__(16) E Xs[2][BM][XP];
  __shared__ __align__(16) E Ws[2][BN][XP];
  __shared__ float ssp[4][BM];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t m0 = blockIdx.y * BM;
  const uint32_t nb = min((uint32_t)BM, a.B - m0);
  const uint32_t K = a.K, nch = (K + BK - 1) / BK;
  const Segs sgs(a);
  const bool norm = a.ng != nullptr;
  // this thread's share of a chunk: X rows xm (4 float4 of 16 k each), one
  // 16-byte piece of a weight row (bf16: 8 values; f32: 4 values, twice)
  const uint32_t xm = tid >> 2, xk = (tid & 3) * 16;
  const float* xsrc = a.X + (size_t)(m0 + (xm < nb ? xm : 0)) * a.ldx;
  const uint32_t wr = WT == 1 ? tid >> 3 : tid >> 4;          // weight row in tile
  const uint32_t wk = WT == 1 ? (tid & 7) * 8 : (tid & 15) * 4;
  const float* wf;
  uint32_t wsg, wlr;
  const bool wok = tid < (WT == 1 ? 128u : 256u) && sgs.row(BN, blockIdx.x, wr, &wf, &wsg, &wlr);
  const uint16_t* wh = (wsg ? a.Wh1 : a.Wh0) + (size_t)wlr * K;
  if (!wok) {
    wf = sgs.W0;
    wh = a.Wh0;
  }
  float4 xr[D][4];
  uint4 whr[D];
  float4 wfr[D];
  auto load = [&](int u, uint32_t c) {
    const uint32_t q0 = c * BK;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t q = q0 + xk + 4 * j;
      xr[u][j] = *reinterpret_cast<const float4*>(xsrc + (q < K ? q : 0));
    }
    const uint32_t q = q0 + wk;
    if constexpr (WT == 1) whr[u] = *reinterpret_cast<const uint4*>(wh + (q < K ? q : 0));
    else wfr[u] = *reinterpret_cast<const float4*>(wf + (q < K ? q : 0));
  };
  float ss = 0.0f;
  auto store = [&](int u, int buf, uint32_t c) {
    const uint32_t q0 = c * BK;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t q = q0 + xk + 4 * j;
      float4 x = xr[u][j];
      if (q >= K || xm >= nb) x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (norm) {
        ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
        const float4 g = *reinterpret_cast<const float4*>(a.ng + (q < K ? q : 0));
        x.x *= g.x;
        x.y *= g.y;
        x.z *= g.z;
        x.w *= g.w;
      }
      E* dst = &Xs[buf][xm][xk + 4 * j];
      dst[0] = (E)x.x;
      dst[1] = (E)x.y;
      dst[2] = (E)x.z;
      dst[3] = (E)x.w;
    }
    const uint32_t q = q0 + wk;
    if constexpr (WT == 1) {
      if (tid < 128) {
        uint4 w = whr[u];
        if (q >= K) w = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(&Ws[buf][wr][wk]) = w;
      }
    } else {
      float4 w = wfr[u];
      if (q >= K) w = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      *reinterpret_cast<float4*>(&Ws[buf][wr][wk]) = w;
    }
  };
#pragma unroll
  for (int u = 0; u < D; u++)
    if ((uint32_t)u < nch) load(u, u);
  store(0, 0, 0);
  __syncthreads();
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t am = wv * 16 + (lane & 15), g4 = lane >> 4;
  for (uint32_t c0 = 0; c0 < nch; c0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const uint32_t c = c0 + u;
      if (c < nch) {
        const int buf = c & 1;
        if constexpr (WT == 1) {
#pragma unroll
          for (int ks = 0; ks < BK; ks += 32) {
            const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(&Xs[buf][am][ks + 8 * g4]);
            const bf16x8_t bv = *reinterpret_cast<const bf16x8_t*>(&Ws[buf][lane & 15][ks + 8 * g4]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int ks = 0; ks < BK; ks += 16) {
            const float4 av = *reinterpret_cast<const float4*>(&Xs[buf][am][ks + 4 * g4]);
            const float4 bv = *reinterpret_cast<const float4*>(&Ws[buf][lane & 15][ks + 4 * g4]);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc, 0, 0, 0);
          }
        }
        if (c + 1 < nch) store((u + 1) % D, buf ^ 1, c + 1);
        if (c + D < nch) load(u, c + D);
        __syncthreads();
      }
    }
  }
  // the rows' sums of squares: 4 threads a row, then the scale
  if (norm) {
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    if ((tid & 3) == 0) ssp[0][xm] = 1.0f / sqrtf(ss / (float)K + 1.0e-5f);
    __syncthreads();
  }
  // result tile: lane holds rows 4*g4 + r of the wave's block, column lane & 15
  const uint32_t n = lane & 15;
  const float* w_;
  uint32_t sg, lr;
  const bool nok = sgs.row(BN, blockIdx.x, n, &w_, &sg, &lr);
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t m = wv * 16 + 4 * g4 + r;
    float y = acc[r];
    if (norm) y *= ssp[0][m < BM ? m : 0];
    if (a.mode == GM_SILU) {
      const float up = __shfl_xor(y, 8, 64);
      if (n < 8 && nok && m < nb) a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = fast_silu(y) * up;
    } else if (nok && m < nb) {
      if (a.mode == GM_RESID) y = a.R[(size_t)(m0 + m) * a.ldr + lr] + y;
      if (sg) a.seg[1].Y[(size_t)(m0 + m) * a.seg[1].ldy + lr] = y;
      else a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = y;
    }
  }
}

// ------------------------------------------------------------------ packed weights

// A product's weights re-laid for the decode-batch GEMM (k_gemm_pw): tile t
// (16 weight rows in Segs order, 8 gate + 8 up rows with SiLU) and step s
// (32 k) form one block, blocks ordered (t, s), so a wave streams its k range
// of a tile as consecutive 1 KB pieces. In a block, lane l of a wave owns
// weight row l % 16 at k = 32 s + 8 (l / 16) .. + 7: fp32 (2 KB) as two 1 KB
// halves, half h holding k + 4 h .. + 3 of every lane at 16 l; bf16 (1 KB)
// the lane's eight values at 16 l. Rows past the segments are zero. With
// `ng` (the product's RMSNorm gains) each weight is stored as g[k] * W[n][k]
// (then rounded to bf16, nearest even, in the bf16 form), so the product
// needs only the raw x and its rows' norm scales.
__global__ void k_pack(GemvArgs a, uint32_t tiles, uint4* __restrict__ dst, int bf) {
  const Segs sgs(a);
  const uint32_t K = a.K, nsa = K >> 5;
  const uint64_t n = (uint64_t)tiles * nsa * (bf ? 64 : 128);
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t lane = (uint32_t)(i & 63);
    const uint32_t h = bf ? 0u : (uint32_t)((i >> 6) & 1);
    const uint64_t ts = bf ? i >> 6 : i >> 7;
    const uint32_t s = (uint32_t)(ts % nsa), t = (uint32_t)(ts / nsa);
    const float* w;
    uint32_t sg, lr;
    const bool ok = sgs.row(16, t, lane & 15, &w, &sg, &lr);
    const uint32_t k = 32 * s + 8 * (lane >> 4) + 4 * h;
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t ke = k + (bf || e < 4 ? e : 0);
      x[e] = ok ? w[ke] * (a.ng ? a.ng[ke] : 1.0f) : 0.0f;
    }
    uint4 v;
    if (bf) {
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const uint32_t u = __float_as_uint(x[e]);
        b[e] = (u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x40u) : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
      }
      v = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
    } else {
      v = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
    }
    dst[i] = v;
  }
}

static uint32_t pk_tiles(const GemvArgs& a) {
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  return (rows + 15) / 16;
}

uint64_t pack_bytes(const GemvArgs& a, int bf) {
  return (uint64_t)pk_tiles(a) * (a.K / 32) * (bf ? 1024 : 2048);
}

hipError_t launch_pack(const GemvArgs& a, void* dst, int bf, hipStream_t st) {
  if (a.K % 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pack, dim3(2048), dim3(256), 0, st, a, pk_tiles(a), static_cast<uint4*>(dst), bf);
  return hipGetLastError();
}

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>), in order
template <typename F, int... I>
__device__ __forceinline__ void static_for_(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_(f, std::make_integer_sequence<int, N>{});
}

// Decode batches and prefill steps of 5..127 rows in the fast modes:
// Y[m][n] = sum_k X[m][k] W[n][k] over packed weights (the norm gains folded
// in when `ng` is set). A workgroup owns NT 16-row weight tiles and 16 batch
// rows (each x fragment serves the NT tiles); K = 128 NS, and its four
// waves take a quarter of K each (NS steps of 32 k), every wave on its own. Per step a wave issues its weight pieces
// (coalesced 1 KB loads into a ring of D register sets) and two
// global_load_lds_dwordx4 of the 16 rows' x for that step (each 1 KB: 8 rows
// x 128 bytes, a row's 16-byte units at unit ^ (row & 7), so the fragment
// reads of 16 rows at one k fall in distinct bank groups) into an LDS block
// of its own. Its loads retire in issue order: before step s it waits until
// only the ops of steps s + 1 .. s + D - 1 are outstanding (a count fixed at
// compile time) and reads the step's x with no barrier. MFMA operands: lane
// l holds row l % 16 of x and of the tile at k = 8 (l / 16) + e of the step;
// fp32 (WT 0) takes v_mfma_f32_16x16x4f32 once per e, bf16 (WT 1) one
// v_mfma_f32_16x16x32_bf16 on x rounded to bf16. With `ng`
// each wave also sums its rows' x^2 from the same fragments. Waves 1..3 hand
// their partial tiles and sums to wave 0, which adds them in wave order and
// applies the norm scale 1/sqrt(ss/K + 1e-5) and the epilogue (plain,
// residual, SiLU with tile rows 0..7 gate j and 8..15 up j). The result
// tile: lane l holds batch rows 4 (l / 16) + r, weight row l % 16.
template <int WT, int NS, int D, int NT>
__global__ __launch_bounds__(256) void k_gemm_pw(GemvArgs a, const uint4* __restrict__ pk, uint32_t tiles) {
  constexpr int WP = WT == 1 ? 1 : 2, OPS = NT * WP + 2;
  __shared__ __align__(1024) float xs[4][NS][512];
  __shared__ f32x4_t red[3][NT][64];
  __shared__ float ssr[4][16];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  const uint32_t K = 128 * NS, nsa = 4 * NS;
  const uint32_t m0 = blockIdx.y * 16;
  const bool norm = a.ng != nullptr;
  // the workgroup's tiles NT x .. NT x + NT - 1; one past the last reads the
  // last tile again and stores nothing
  const uint4* wsrc[NT];
#pragma unroll
  for (int j = 0; j < NT; j++)
    wsrc[j] = pk + ((size_t)min(NT * blockIdx.x + j, tiles - 1) * nsa + wv * NS) * (64 * WP) + lane;
  // this lane's x piece in each half of a step: row 8 h + (lane >> 3), its
  // unit (lane & 7) ^ row
  const uint32_t dr = lane >> 3, sl = (lane & 7) ^ dr;
  uint32_t xo[2];
#pragma unroll
  for (int h = 0; h < 2; h++) xo[h] = min(m0 + 8 * h + dr, a.B - 1) * a.ldx + wv * (K / 4) + 4 * sl;
  // wave 0's residuals (its epilogue's) first: they depend on nothing, and
  // loaded after its stores each would wait on the one before
  float res[NT][4];
#pragma unroll
  for (int j = 0; j < NT; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) res[j][r] = 0.0f;
  if (a.mode == GM_RESID && wv == 0) {
    const Segs sg0(a);
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint32_t t = NT * blockIdx.x + j;
      const float* w_;
      uint32_t sg, lr;
      const bool ok = t < tiles && sg0.row(16, t, r16, &w_, &sg, &lr);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = m0 + 4 * g4 + r;
        if (ok && m < a.B) res[j][r] = a.R[(size_t)m * a.ldr + lr];
      }
    }
  }
  uint4 wr[D][NT][WP];
  auto issue = [&](auto S) {
    constexpr int s = decltype(S)::value;
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int p = 0; p < WP; p++) wr[s % D][j][p] = wsrc[j][s * 64 * WP + 64 * p];
#pragma unroll
    for (int h = 0; h < 2; h++)
      __builtin_amdgcn_global_load_lds((const void*)(a.X + xo[h] + 32 * s), (lds_void*)&xs[wv][s][256 * h], 16, 0, 0);
  };
  static_for<(D < NS ? D : NS)>(issue);
  f32x4_t acc[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) acc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float ss = 0.0f;
  const uint32_t fo0 = (r16 >> 3) * 256 + (r16 & 7) * 32 + 4 * ((2 * g4) ^ (r16 & 7));
  const uint32_t fo1 = (r16 >> 3) * 256 + (r16 & 7) * 32 + 4 * ((2 * g4 + 1) ^ (r16 & 7));
  static_for<NS>([&](auto S) {
    constexpr int s = decltype(S)::value;
    constexpr int last = s + D - 1 < NS - 1 ? s + D - 1 : NS - 1;
    ANA_VMCNT(OPS * (last - s));
    const float4 x0 = *reinterpret_cast<const float4*>(&xs[wv][s][fo0]);
    const float4 x1 = *reinterpret_cast<const float4*>(&xs[wv][s][fo1]);
    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    if (norm) {
#pragma unroll
      for (int e = 0; e < 8; e++) ss += x[e] * x[e];
    }
    if constexpr (WT == 0) {
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const uint4 w0 = wr[s % D][j][0], w1 = wr[s % D][j][WP - 1];
        const float w[8] = {__uint_as_float(w0.x), __uint_as_float(w0.y), __uint_as_float(w0.z),
                            __uint_as_float(w0.w), __uint_as_float(w1.x), __uint_as_float(w1.y),
                            __uint_as_float(w1.z), __uint_as_float(w1.w)};
#pragma unroll
        for (int e = 0; e < 8; e++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[e], w[e], acc[j], 0, 0, 0);
      }
    } else {
      bf16x8_t hi;
#pragma unroll
      for (int e = 0; e < 8; e++) hi[e] = (__bf16)x[e];
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const bf16x8_t wb8 = __builtin_bit_cast(bf16x8_t, wr[s % D][j][0]);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, wb8, acc[j], 0, 0, 0);
      }
    }
    if constexpr (s + D < NS) issue(std::integral_constant<int, s + D>{});
  });
  if (wv > 0) {
#pragma unroll
    for (int j = 0; j < NT; j++) red[wv - 1][j][lane] = acc[j];
  }
  if (norm) {
    float v = ss;
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (g4 == 0) ssr[wv][r16] = v;
  }
  __syncthreads();
  if (wv > 0) return;
  const Segs sgs(a);
  float rs[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t mi = 4 * g4 + r;
    rs[r] = norm ? 1.0f / sqrtf((((ssr[0][mi] + ssr[1][mi]) + ssr[2][mi]) + ssr[3][mi]) / (float)K + 1.0e-5f) : 1.0f;
  }
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const uint32_t t = NT * blockIdx.x + j;
    const float* w_;
    uint32_t sg, lr;
    const bool nok = t < tiles && sgs.row(16, t, r16, &w_, &sg, &lr);
    f32x4_t y4 = acc[j];
#pragma unroll
    for (int p = 0; p < 3; p++) {
      const f32x4_t o = red[p][j][lane];
      y4[0] += o[0]; y4[1] += o[1]; y4[2] += o[2]; y4[3] += o[3];
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t m = m0 + 4 * g4 + r;
      float y = y4[r];
      if (norm) y *= rs[r];
      if (a.mode == GM_SILU) {
        const float up = __shfl_xor(y, 8, 64);
        if (r16 < 8 && nok && m < a.B) a.seg[0].Y[(size_t)m * a.seg[0].ldy + lr] = fast_silu(y) * up;
      } else if (nok && m < a.B) {
        if (a.mode == GM_RESID) y = res[j][r] + y;
        if (sg) a.seg[1].Y[(size_t)m * a.seg[1].ldy + lr] = y;
        else a.seg[0].Y[(size_t)m * a.seg[0].ldy + lr] = y;
      }
    }
  }
}

// Wide products over packed weights at 5..127 rows (the LM head): a
// workgroup of NW waves owns 32 batch rows and TPW consecutive 16-row weight
// tiles (with `amax` also the rows' greedy argmax keys: per tile the best of
// its 16 columns, one atomicMax into the row's slot t % kAmaxSlots). The 32
// rows' x go to LDS once (global_load_lds_dwordx4, a row's
// 16-byte units at unit ^ (row & 7)); with `ng` the waves then share the
// rows for their norm scales. Wave w takes tiles w, w + NW, .. of the TPW,
// each over the whole K, its (tile, 32-k step) pieces as one stream in
// blocks of D steps (D divides a tile's K / 32 steps, so a block never spans
// two tiles), double-buffered in registers with every load unconditional
// and the index clamped: the next block's weights, the next tile's too, are
// in flight while a block computes. After a tile's last block the wave
// scales, stores and clears its two accumulators (batch rows 0..15 and
// 16..31). The x tile is read once per TPW weight tiles instead of once per
// tile.
// With PICK = LPT (the sampler's leaves a thread), the fused form of the
// head and the sampler: the logits are stored with agent-scope stores
// (written through to the level every XCD reads), and once its stores are
// complete the workgroup counts itself in on its row block's counter (a
// running total, so no reset between launches); the last `rows` arrivals
// wait (bounded) until every workgroup of the block has counted in, then
// each copies one of the block's rows into LDS with agent-scope loads and
// runs pick_row on it. The host launches it only when the whole grid is resident at
// once (so no waiting workgroup holds a slot another needs) and a block has
// at least as many workgroups as rows.
template <int WT, int TPW, int D, int NW, int PICK>
__global__ __launch_bounds__(64 * NW) void k_head_pw(GemvArgs a, const uint4* __restrict__ pk, uint32_t tiles,
                                                     HeadPick hp) {
  constexpr int WP = WT == 1 ? 1 : 2;
  constexpr uint32_t BM = 32;
  __shared__ __align__(1024) float xs[BM * kHeadMaxK];
  __shared__ float rsc[BM];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  const uint32_t K = a.K, U = K >> 2, nsa = K >> 5;
  const uint32_t m0 = blockIdx.y * BM, t0 = blockIdx.x * TPW;
  const bool norm = a.ng != nullptr;
  // this wave's blocks: tiles t0 + wv + NW i (i < TPW / NW), nsa / D blocks each
  const uint32_t bpt = nsa / D, nb = (TPW / NW) * bpt;
  auto block_base = [&](uint32_t k) {   // first piece of block k (clamped)
    k = min(k, nb - 1);
    const uint32_t i = k / bpt, s0 = (k - i * bpt) * D;
    const uint32_t t = min(t0 + wv + NW * i, tiles - 1);
    return pk + ((size_t)t * nsa + s0) * (64 * WP) + lane;
  };
  uint4 wr[D][WP];
  auto wload = [&](const uint4* p) {
#pragma unroll
    for (int u = 0; u < D; u++)
#pragma unroll
      for (int j = 0; j < WP; j++) wr[u][j] = p[(u * WP + j) * 64];
  };
  wload(block_base(0));
  for (uint32_t q0 = wv * 64; q0 < BM * U; q0 += 64 * NW) {
    const uint32_t q = q0 + lane, r = q / U, u = q - r * U;
    const uint32_t m = min(m0 + r, a.B - 1);
    __builtin_amdgcn_global_load_lds((const void*)(a.X + (size_t)m * a.ldx + 4 * (u ^ (r & 7))),
                                     (lds_void*)(xs + 4 * q0), 16, 0, 0);
  }
  ANA_VMCNT(0);
  __syncthreads();
  if (norm) {
    for (uint32_t r = wv; r < BM; r += NW) {
      float ss = 0.0f;
      for (uint32_t v = lane; v < U; v += 64) {
        const float4 x = *reinterpret_cast<const float4*>(xs + 4 * (r * U + (v ^ (r & 7))));
        ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
      }
      ss = wave_sum(ss);
      if (lane == 0) rsc[r] = 1.0f / sqrtf(ss / (float)K + 1.0e-5f);
    }
    __syncthreads();
  }
  f32x4_t acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  const Segs sgs(a);
  for (uint32_t k = 0; k < nb; k++) {
    const uint32_t i = k / bpt, s0 = (k - i * bpt) * D;
    // this block's weights out of the ring, the next block's in
    uint4 cw[D][WP];
#pragma unroll
    for (int u = 0; u < D; u++)
#pragma unroll
      for (int j = 0; j < WP; j++) cw[u][j] = wr[u][j];
    wload(block_base(k + 1));
#pragma unroll
    for (int u = 0; u < D; u++) {
      const uint32_t v0 = 8 * (s0 + u) + 2 * g4;
      float w[8];
      if constexpr (WT == 0) {
        w[0] = __uint_as_float(cw[u][0].x); w[1] = __uint_as_float(cw[u][0].y);
        w[2] = __uint_as_float(cw[u][0].z); w[3] = __uint_as_float(cw[u][0].w);
        w[4] = __uint_as_float(cw[u][WP - 1].x); w[5] = __uint_as_float(cw[u][WP - 1].y);
        w[6] = __uint_as_float(cw[u][WP - 1].z); w[7] = __uint_as_float(cw[u][WP - 1].w);
      }
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        const uint32_t r = 16 * tt + r16, base = r * U, sw = r & 7;
        const float4 x0 = *reinterpret_cast<const float4*>(xs + 4 * (base + (v0 ^ sw)));
        const float4 x1 = *reinterpret_cast<const float4*>(xs + 4 * (base + ((v0 + 1) ^ sw)));
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        if constexpr (WT == 0) {
#pragma unroll
          for (int e = 0; e < 8; e++) acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[e], w[e], acc[tt], 0, 0, 0);
        } else {
          bf16x8_t hi;
#pragma unroll
          for (int e = 0; e < 8; e++) hi[e] = (__bf16)x[e];
          const bf16x8_t wb8 = __builtin_bit_cast(bf16x8_t, cw[u][0]);
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, wb8, acc[tt], 0, 0, 0);
        }
      }
    }
    if (s0 + D == nsa) {
      // the tile is done: scale, store, clear
      const uint32_t t = t0 + wv + NW * i;
      const float* w_;
      uint32_t sg, lr;
      const bool nok = t < tiles && sgs.row(16, t, r16, &w_, &sg, &lr);
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t mi = 16 * tt + 4 * g4 + r, m = m0 + mi;
          float y = acc[tt][r];
          if (norm) y *= rsc[mi];
          if (nok && m < a.B) {
            float* yp = sg ? a.seg[1].Y + (size_t)m * a.seg[1].ldy + lr : a.seg[0].Y + (size_t)m * a.seg[0].ldy + lr;
            if constexpr (PICK != 0) __hip_atomic_store(yp, y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else *yp = y;
          }
          if (a.amax) {
            // the row's best key over the tile's 16 columns, one atomic
            unsigned long long key = nok && m < a.B && sg == 0 ? argmax_key(y, lr) : 0ull;
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) {
              const unsigned long long o = __shfl_xor(key, sh, 64);
              key = o > key ? o : key;
            }
            if (r16 == 0 && key) atomicMax(&a.amax[amax_at(m, t % kAmaxSlots)], key);
          }
        }
        acc[tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
  }
  if constexpr (PICK != 0) {
    __shared__ uint32_t samp_s;
    ANA_VMCNT(0);   // this wave's stores are complete, then every wave's
    __syncthreads();
    if (tid == 0) {
      // (the host launches this form with at least as many workgroups a
      // block as rows in it: one row a sampler)
      const uint32_t per = gridDim.x, ns = min(BM, a.B - m0);
      const unsigned long long old =
          __hip_atomic_fetch_add(hp.cnt + blockIdx.y, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t ai = (uint32_t)(old % per);
      uint32_t j = ~0u;
      if (ai >= per - ns) {
        j = ai - (per - ns);
        const unsigned long long target = old - ai + per;
        for (uint32_t polls = 0;
             __hip_atomic_load(hp.cnt + blockIdx.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target; polls++) {
          if (polls >= kPickPollMax) {
            __hip_atomic_store(hp.ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            j = ~0u;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
      }
      samp_s = j;
    }
    __syncthreads();
    const uint32_t j = samp_s;
    if (j == ~0u) return;
    static_assert(BM * kHeadMaxK >= 32768, "the x tile holds a row of the fused forms' vocabularies");
    // the row into the x tile's LDS (dead now, and as large as the
    // vocabulary the fused forms take): agent-scope loads, lane t of
    // consecutive floats so each load of a wave is one 256-byte piece
    const uint32_t v = hp.pa.vocab;
    const float* lg = hp.pa.logits + (size_t)(m0 + j) * v;
    for (uint32_t i = tid; i < v; i += 64 * NW)
      xs[i] = __hip_atomic_load(const_cast<float*>(lg) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    uint32_t dv = 0;
    while ((1u << dv) < v) dv++;
    pick_row<PICK>(hp.pa, m0 + j, (1u << dv) / PICK, dv, xs);
  }
}

bool head_pw_fits(const GemvArgs& a) {
  return a.mode == GM_PLAIN && a.B > 0 && a.K % 256 == 0 && a.K <= kHeadMaxK && (a.ldx & 3) == 0 &&
         (reinterpret_cast<uintptr_t>(a.X) & 15) == 0;
}

hipError_t launch_head_pw(const GemvArgs& a, const void* pk, int bf, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  if (!head_pw_fits(a) || !pk) return hipErrorInvalidValue;
  constexpr int TPW = 16;
  const uint32_t tiles = pk_tiles(a);
  const dim3 grid((tiles + TPW - 1) / TPW, (a.B + 31) / 32);
  const uint4* p = static_cast<const uint4*>(pk);
  // the x tile fills LDS (one workgroup a CU): sixteen waves, four a SIMD,
  // one tile each (measured at B = 64: 55 -> 41 us fp32, 37 -> 26 us bf16
  // from four waves to sixteen); fp32 blocks of two steps (114 -> 100 VGPRs,
  // 43 -> 41 us at B = 64), bf16 of four
  const HeadPick none{};
  if (bf) ANA_LAUNCH_F((k_head_pw<1, TPW, 4, 16, 0>), grid, dim3(1024), 0, st, e0, e1, a, p, tiles, none);
  else ANA_LAUNCH_F((k_head_pw<0, TPW, 2, 16, 0>), grid, dim3(1024), 0, st, e0, e1, a, p, tiles, none);
  return hipGetLastError();
}

// workgroups of kernel k the GPU holds at once (1024 threads each)
template <class Kern>
static uint64_t resident_wgs(Kern k) {
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, 1024, 0) != hipSuccess)
    return 0;
  return (uint64_t)cus * (uint64_t)per;
}

template <int WT, int D, int L>
static hipError_t head_pick_go(const GemvArgs& a, const uint4* p, uint32_t tiles, const dim3& grid,
                               const HeadPick& hp, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  static const uint64_t cap = resident_wgs(k_head_pw<WT, 16, D, 16, L>);
  if ((uint64_t)grid.x * grid.y > cap) return hipErrorNotSupported;
  ANA_LAUNCH_F((k_head_pw<WT, 16, D, 16, L>), grid, dim3(1024), 0, st, e0, e1, a, p, tiles, hp);
  return hipGetLastError();
}

hipError_t launch_head_pick(const GemvArgs& a, const void* pk, int bf, const HeadPick& hp, hipStream_t st,
                            hipEvent_t e0, hipEvent_t e1) {
  if (!head_pw_fits(a) || !pk || !hp.cnt || !hp.ctl || hp.pa.logits != a.seg[0].Y || a.nseg != 1 ||
      hp.pa.B != a.B || hp.pa.vocab != a.seg[0].rows)
    return hipErrorInvalidValue;
  // the sampler's geometry (as launch_pick's): 1024 threads of LPT leaves
  // over the vocabulary padded to a power of two; fused forms for LPT 1
  // (up to 1024 entries) and 32 (16385 .. 32768)
  uint32_t dv = 0;
  while ((1ull << dv) < a.seg[0].rows) dv++;
  const uint64_t vpad = 1ull << dv;
  const uint32_t lpt = vpad > 1024 ? (uint32_t)(vpad / 1024) : 1u;
  constexpr int TPW = 16;
  const uint32_t tiles = pk_tiles(a);
  const dim3 grid((tiles + TPW - 1) / TPW, (a.B + 31) / 32);
  if (grid.x < std::min(a.B, 32u)) return hipErrorNotSupported;   // one row a sampler
  const uint4* p = static_cast<const uint4*>(pk);
  if (lpt == 1) return bf ? head_pick_go<1, 4, 1>(a, p, tiles, grid, hp, st, e0, e1)
                          : head_pick_go<0, 2, 1>(a, p, tiles, grid, hp, st, e0, e1);
  if (lpt == 32) return bf ? head_pick_go<1, 4, 32>(a, p, tiles, grid, hp, st, e0, e1)
                           : head_pick_go<0, 2, 32>(a, p, tiles, grid, hp, st, e0, e1);
  return hipErrorNotSupported;
}

bool gemm_pk_fits(const GemvArgs& a) {
  return !a.amax && a.B > 0 && a.K % 128 == 0 && a.K <= 2048 && (a.ldx & 3) == 0 &&
         (reinterpret_cast<uintptr_t>(a.X) & 15) == 0;
}

// two weight tiles a workgroup when the one-tile grid has 4 to 16
// workgroups a CU (measured at B = 64: gate|up 10.3 -> 8.9 us fp32, 7.9 ->
// 6.4 us bf16; with fewer, q|k|v|z and Wo lose the spread over the CUs,
// with more, the head gains nothing), and K <= 1024 (the register ring of
// two tiles' weights)
constexpr uint32_t kPwTwoTileMin = 1024, kPwTwoTileMax = 4096;

// The register ring holds D steps: three for K <= 1024, four above (a sweep
// at B = 16 and 64 with the weights evicted between launches: one step
// ahead starves the loads; six or eight ahead, every load issued at once,
// cost 0.3-1.1 us more a product than three)
template <int NS>
static hipError_t pw_go(const GemvArgs& a, const uint4* p, int bf, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  constexpr int D = NS < 3 ? NS : NS <= 8 ? 3 : 4;
  const uint32_t tiles = pk_tiles(a), mt = (a.B + 15) / 16;
  if constexpr (NS <= 8) {
    if (tiles * mt >= kPwTwoTileMin && tiles * mt <= kPwTwoTileMax) {
      const dim3 grid((tiles + 1) / 2, mt);
      if (bf) ANA_LAUNCH_F((k_gemm_pw<1, NS, D, 2>), grid, dim3(256), 0, st, e0, e1, a, p, tiles);
      else ANA_LAUNCH_F((k_gemm_pw<0, NS, D, 2>), grid, dim3(256), 0, st, e0, e1, a, p, tiles);
      return hipGetLastError();
    }
  }
  const dim3 grid(tiles, mt);
  if (bf) ANA_LAUNCH_F((k_gemm_pw<1, NS, D, 1>), grid, dim3(256), 0, st, e0, e1, a, p, tiles);
  else ANA_LAUNCH_F((k_gemm_pw<0, NS, D, 1>), grid, dim3(256), 0, st, e0, e1, a, p, tiles);
  return hipGetLastError();
}

template <int... I>
static hipError_t pw_dispatch(const GemvArgs& a, const uint4* p, int bf, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                              std::integer_sequence<int, I...>) {
  hipError_t e = hipErrorInvalidValue;
  ((a.K == 128u * (I + 1) ? (void)(e = pw_go<I + 1>(a, p, bf, st, e0, e1)) : (void)0), ...);
  return e;
}

hipError_t launch_gemm_pk(const GemvArgs& a, const void* pk, int bf, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  if (!gemm_pk_fits(a) || !pk) return hipErrorInvalidValue;
  return pw_dispatch(a, static_cast<const uint4*>(pk), bf, st, e0, e1, std::make_integer_sequence<int, 16>{});
}

hipError_t launch_gemm_mfma(const GemvArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  if (a.amax || (a.K & 7) || a.B == 0) return hipErrorInvalidValue;
  const bool bf = a.Wh0 != nullptr;
  if (bf && a.nseg > 1 && !a.Wh1) return hipErrorInvalidValue;
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  const uint32_t per = a.mode == GM_SILU ? 8 : 16;
  const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
  dim3 grid(tiles, (a.B + 63) / 64);
  if (bf) ANA_LAUNCH_F((k_gemm_mfma<1, 4>), grid, dim3(256), 0, st, e0, e1, a);
  else ANA_LAUNCH_F((k_gemm_mfma<0, 4>), grid, dim3(256), 0, st, e0, e1, a);
  return hipGetLastError();
}

}  // namespace ana

namespace ana {

// ------------------------------------------------------------------ GLA over prefill chunks

// The pair weights of a kGlaSub-token sub-chunk: P[t][s] =
// sum_a qh_t[a] kh_s[a] e^(c_t[a] - c_s[a]) for s <= t < n, zero elsewhere
// (c the running sum of log a inside the sub-chunk, non-increasing). A pair
// s < t goes by the highest bit in which t and s differ: at level l they sit
// in one 2^(l+1)-token block, t in its upper half, s in its lower one, and
// with r the first token of the upper half
//   e^(c_t - c_s) = e^(c_t - c_r) e^(c_r - c_s), both exponents <= 0,
// so the pairs of a level are the in-block entries of one 16 x 16 product of
// the 16 upper-half rows qh_t e^(c_t - c_r) by the 16 lower-half columns
// kh_s e^(c_r - c_s) (v_mfma_f32_16x16x4f32; lane l: row l % 16 and column
// l % 16 at k = l / 16 of each step of 4; result rows 4 (l / 16) + r).
// Levels 1-4 take one wave each; the diagonal (exponent 0) and level 0's 16
// neighbour pairs are sums over a on lane groups. Reads qh, kh, cl; writes
// every entry of P once; the caller synchronises after.
template <int HD, typename TQ, typename TK, typename TC, typename TP>
__device__ __forceinline__ void gla_pairs(const TQ* qh, const TK* kh, const TC* cl, TP* P, uint32_t n,
                                          uint32_t tid) {
  constexpr int L = kGlaSub;
  static_assert(L == 32 && HD % 16 == 0, "five levels of 16 x 16 tiles");
  // above the diagonal and past the last token: zero
  for (uint32_t e = tid; e < (uint32_t)L * L; e += 256) {
    const uint32_t t = e / L, s = e % L;
    if (s > t || t >= n) P[t][s] = 0.0f;
  }
  {  // the diagonal, 8 lanes a token
    const uint32_t t = tid >> 3, l = tid & 7;
    float p = 0.0f;
    for (uint32_t a = l; a < (uint32_t)HD; a += 8) p = fmaf(qh[t][a], kh[t][a], p);
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1) p += __shfl_xor(p, m, 64);
    if (l == 0 && t < n) P[t][t] = p;
  }
  {  // level 0: (2i + 1, 2i), 16 lanes a pair
    const uint32_t i = tid >> 4, l = tid & 15, t = 2 * i + 1, s2 = 2 * i;
    float p = 0.0f;
    for (uint32_t a = l; a < (uint32_t)HD; a += 16)
      p = fmaf(qh[t][a] * kh[s2][a], __expf(cl[t][a] - cl[s2][a]), p);
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) p += __shfl_xor(p, m, 64);
    if (l == 0 && t < n) P[t][s2] = p;
  }
  // levels 1-4 on the matrix cores
  const uint32_t lane = tid & 63, lv = (tid >> 6) + 1, r16 = lane & 15, g4 = lane >> 4;
  const uint32_t lo = (1u << lv) - 1;
  const uint32_t ti = ((r16 >> lv) << (lv + 1)) | (1u << lv) | (r16 & lo), rt = ti & ~lo;
  const uint32_t si = ((r16 >> lv) << (lv + 1)) | (r16 & lo), rs = (si & ~lo) | (1u << lv);
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k0 = 0; k0 < HD; k0 += 4) {
    const uint32_t a = k0 + g4;
    const float x = qh[ti][a] * __expf(cl[ti][a] - cl[rt][a]);
    const float y = kh[si][a] * __expf(cl[rs][a] - cl[si][a]);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t i = 4 * g4 + r;
    const uint32_t t = ((i >> lv) << (lv + 1)) | (1u << lv) | (i & lo);
    if ((i >> lv) == (r16 >> lv) && t < n) P[t][si] = acc[r];
  }
}

// T tokens of one sequence through one head's GLA (bend/Dense/Decode.bend
// dd.gla over a chunk): the recurrence S_t = diag(a_t) S_(t-1) + kh_t v_t^T,
// o_t = qh_t^T S_t, taken kGlaSub tokens at a time in closed form. With c_t
// the running sum of log a inside a sub-chunk,
//   S_t = e^(c_t) S_prev + sum_(s<=t) e^(c_t - c_s) kh_s v_s^T, so
//   o_t = (qh_t e^(c_t))^T S_prev + sum_(s<=t) P_ts v_s,
//   P_ts = sum_a qh_t[a] kh_s[a] e^(c_t[a] - c_s[a]),
// and every exponent is <= 0 (nothing overflows however small the gates).
// Every sub-chunk of every chunk in a prefill step runs in parallel (a
// chunked scan over a table of sub-chunks; those of one chunk consecutive).
// Pass 1, per (head, sub-chunk): the gates, the intra terms
// o_t = sum_(s<=t) P_ts v_s, the sub-chunk's decay D = e^(c_last), its state
// contribution U = sum_s e^(c_last - c_s) kh_s v_s^T and qt_t = qh_t e^(c_t);
// a chunk's first sub-chunk also copies the state entering the chunk (pass 2
// rewrites the state). Pass 2, per (head, column block, sub-chunk j): the
// state entering j, S_(j-1) = D_(j-1) (... (D_0 S_0 + U_0) ...) + U_(j-1),
// then o_t += qt_t^T S_(j-1); the chunk's last sub-chunk writes its final
// state. The matrix products run on v_mfma_f32_16x16x4f32 (lane l: row
// l % 16 of the left operand and column l % 16 of the right at k = l / 16 of
// each step of 4; result rows 4 (l / 16) + r): o_intra = P V, U = Kd^T V,
// and pass 2's qt S; P itself by gla_pairs.
template <int HD>
__global__ __launch_bounds__(256) void k_gla_sub(const float* __restrict__ QKV,
                                                  const float* __restrict__ Z,
                                                  const float* __restrict__ lam, float* __restrict__ O,
                                                  GlaScratch g, StateRef S,
                                                  const GlaSub* __restrict__ tab, uint32_t d,
                                                  uint32_t rglru) {
  constexpr int L = kGlaSub;
  __shared__ float qh[L][HD + 1], kh[L][HD + 1], cl[L][HD + 1], vv[L][HD + 1];
  __shared__ float P[L][L + 1], nr[L][2];
  const uint32_t h = blockIdx.x, J = blockIdx.y, tid = threadIdx.x, heads = gridDim.x;
  const GlaSub u = tab[J];
  const uint32_t s0 = u.row, n = u.n;
  if (u.j == 0) {
    const float4* src = reinterpret_cast<const float4*>(S.base + (size_t)u.seq * S.seq_stride + S.layer_off +
                                                        (size_t)h * HD * HD);
    float4* dst = reinterpret_cast<float4*>(g.S0 + ((size_t)u.seg * heads + h) * HD * HD);
    for (uint32_t e = tid; e < (uint32_t)HD * HD / 4; e += 256) dst[e] = src[e];
  }
  // q, k, v, z of the sub-chunk's tokens (zeros past its end)
  for (uint32_t e = tid; e < (uint32_t)L * HD; e += 256) {
    const uint32_t t = e / HD, a = e % HD;
    float q = 0.0f, k = 0.0f, v = 0.0f, z = 0.0f;
    if (t < n) {
      const float* x = QKV + (size_t)(s0 + t) * 3 * d + h * HD;
      q = x[a];
      k = x[d + a];
      v = x[2 * d + a];
      z = Z[(size_t)(s0 + t) * d + h * HD + a];
    }
    qh[t][a] = q;
    kh[t][a] = k;
    vv[t][a] = v;
    cl[t][a] = z;
  }
  __syncthreads();
  // L2 norms: 8 lanes a token
  {
    const uint32_t t = tid / 8, l = tid % 8;
    float sq = 0.0f, sk = 0.0f;
    for (uint32_t a = l; a < (uint32_t)HD; a += 8) {
      sq = fmaf(qh[t][a], qh[t][a], sq);
      sk = fmaf(kh[t][a], kh[t][a], sk);
    }
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1) {
      sq += __shfl_xor(sq, m, 64);
      sk += __shfl_xor(sk, m, 64);
    }
    if (l == 0) {
      nr[t][0] = 1.0f / sqrtf(1.0e-6f + sq);
      nr[t][1] = 1.0f / sqrtf(1.0e-6f + sk);
    }
  }
  __syncthreads();
  // gates: log a and kh (dd.gate), qh
  for (uint32_t e = tid; e < (uint32_t)L * HD; e += 256) {
    const uint32_t t = e / HD, a = e % HD;
    float lq = 0.0f, lk = 0.0f, la = 0.0f;
    if (t < n) {
      const float z = cl[t][a];
      lq = qh[t][a] * nr[t][0];
      const float kn = kh[t][a] * nr[t][1];
      if (rglru) {
        la = fminf(ANA_CAP, (8.0f * f_sigmoid(z)) * f_log_sigmoid(lam[h * HD + a]));
        lk = kn * sqrtf(1.0f - expf(2.0f * la));
      } else {
        la = f_log_sigmoid(z);
        lk = kn;
      }
    }
    qh[t][a] = lq;
    kh[t][a] = lk;
    cl[t][a] = la;
  }
  __syncthreads();
  if (tid < (uint32_t)HD) {
    float c = 0.0f;
    for (int t = 0; t < L; t++) {
      c += cl[t][tid];
      cl[t][tid] = c;
    }
  }
  __syncthreads();
  for (uint32_t e = tid; e < n * HD; e += 256) {
    const uint32_t t = e / HD, a = e % HD;
    g.Qt[(size_t)(s0 + t) * d + h * HD + a] = qh[t][a] * __expf(cl[t][a]);
  }
  if (tid < (uint32_t)HD) g.Dj[((size_t)J * heads + h) * HD + tid] = __expf(cl[n - 1][tid]);
  gla_pairs<HD>(qh, kh, cl, P, n, tid);
  __syncthreads();
  const uint32_t lane = tid & 63, wv = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  // kh_s e^(c_last - c_s) in place (P holds what needed kh); the intra terms
  // o = P V, 16 x 16 tiles (t half, column block)
  for (uint32_t e = tid; e < (uint32_t)L * HD; e += 256) {
    const uint32_t t = e / HD, a = e % HD;
    kh[t][a] = t < n ? kh[t][a] * __expf(cl[n - 1][a] - cl[t][a]) : 0.0f;
  }
  constexpr uint32_t CBS = HD / 16;
  for (uint32_t tile = wv; tile < 2 * CBS; tile += 4) {
    const uint32_t tb = tile / CBS, bb = tile % CBS;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k0 = 0; k0 < L; k0 += 4) {
      const uint32_t sk = k0 + g4;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(P[16 * tb + r16][sk], vv[sk][16 * bb + r16], acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t t = 16 * tb + 4 * g4 + r;
      if (t < n) O[(size_t)(s0 + t) * d + h * HD + 16 * bb + r16] = acc[r];
    }
  }
  __syncthreads();
  // U = Kd^T V, 16 x 16 tiles (row block of a, column block of b)
  float* U = g.Uj + ((size_t)J * heads + h) * HD * HD;
  for (uint32_t tile = wv; tile < CBS * CBS; tile += 4) {
    const uint32_t ab = tile / CBS, bb = tile % CBS;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k0 = 0; k0 < L; k0 += 4) {
      const uint32_t sk = k0 + g4;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kh[sk][16 * ab + r16], vv[sk][16 * bb + r16], acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) U[(size_t)(16 * ab + 4 * g4 + r) * HD + 16 * bb + r16] = acc[r];
  }
}

template <int HD>
__global__ __launch_bounds__(256) void k_gla_carry(GlaScratch g, StateRef S, float* __restrict__ O,
                                                    const GlaSub* __restrict__ tab, uint32_t d) {
  constexpr int CB = 16, L = kGlaSub;
  __shared__ float Sb[HD][CB + 1], qs[L][HD + 1];
  const uint32_t h = blockIdx.x, cb = blockIdx.y, J = blockIdx.z, tid = threadIdx.x, heads = gridDim.x;
  const GlaSub u = tab[J];
  const uint32_t s0 = u.row, n = u.n;
  for (uint32_t e = tid; e < (uint32_t)L * HD; e += 256) {
    const uint32_t t = e / HD, a = e % HD;
    qs[t][a] = t < n ? g.Qt[(size_t)(s0 + t) * d + h * HD + a] : 0.0f;
  }
  // S_(j-1): the chunk's entering state through its earlier sub-chunks
  // (table entries J - j .. J - 1), HD * CB / 256 elements a thread
  const float* S0g = g.S0 + ((size_t)u.seg * heads + h) * HD * HD + cb * CB;
  constexpr int NE = HD * CB / 256;
  float sv[NE];
#pragma unroll
  for (int i = 0; i < NE; i++) {
    const uint32_t e = tid + 256 * i, a = e / CB, b = e % CB;
    sv[i] = S0g[(size_t)a * HD + b];
  }
  for (uint32_t I = J - u.j; I < J; I++) {
    const float* D = g.Dj + ((size_t)I * heads + h) * HD;
    const float* U = g.Uj + ((size_t)I * heads + h) * HD * HD + cb * CB;
#pragma unroll
    for (int q = 0; q < NE; q++) {
      const uint32_t e = tid + 256 * q, a = e / CB, b = e % CB;
      sv[q] = fmaf(D[a], sv[q], U[(size_t)a * HD + b]);
    }
  }
#pragma unroll
  for (int i = 0; i < NE; i++) {
    const uint32_t e = tid + 256 * i;
    Sb[e / CB][e % CB] = sv[i];
  }
  if (u.j == u.nsub - 1) {
    float* Sg = S.base + (size_t)u.seq * S.seq_stride + S.layer_off + (size_t)h * HD * HD + cb * CB;
    const float* D = g.Dj + ((size_t)J * heads + h) * HD;
    const float* U = g.Uj + ((size_t)J * heads + h) * HD * HD + cb * CB;
#pragma unroll
    for (int q = 0; q < NE; q++) {
      const uint32_t e = tid + 256 * q, a = e / CB, b = e % CB;
      Sg[(size_t)a * HD + b] = fmaf(D[a], sv[q], U[(size_t)a * HD + b]);
    }
  }
  __syncthreads();
  // o_t += qt_t^T S_(j-1) on the column block: one 16 x 16 tile per half
  const uint32_t lane = tid & 63, wv = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  if (wv < 2) {
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k0 = 0; k0 < HD; k0 += 4) {
      const uint32_t a = k0 + g4;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[16 * wv + r16][a], Sb[a][r16], acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t t = 16 * wv + 4 * g4 + r;
      if (t < n) O[(size_t)(s0 + t) * d + h * HD + cb * CB + r16] += acc[r];
    }
  }
}

// Every chunk of a prefill step through one head's GLA in one workgroup:
// its kGlaSub-token sub-chunks in order (the host gives it chunks of at most
// kGlaRunMaxT tokens; longer ones take the scan, whose sub-chunks run in
// parallel). Per sub-chunk, with c, P, qt and Kd as in k_gla_sub,
//   o_t = sum_(s<=t) P_ts v_s + qt_t^T S,   S <- diag(e^(c_last)) S + Kd^T V.
// The state lives in the waves' MFMA accumulators: wave w holds column block
// w % (HD / 16) of S, every row block, as the 16 x 16 result tiles of
// Kd^T V (lane l: rows 16 ab + 4 (l / 16) + y, column l % 16), and the qt S
// product takes its k steps in that same order (step (ab, y): k = 16 ab +
// 4 (l / 16) + y), so the accumulators are its right operand as they stand.
// S is read and written once per chunk and never passes through LDS; with
// HD < 64 the waves past the column blocks hold copies. The gate pass is
// token-major: eight lanes a token, HD / 8 columns a lane, loaded as
// float4s a sub-chunk ahead, so a token's L2 norms are a lane's own sum
// and three DPP adds; the running sums of log a then go down each column
// (thread (a, token block): TPT tokens in registers, the block totals
// through LDS).
// CPT consecutive columns c0 .. c0 + CPT - 1 of q, k, v (QKV) and z (Z) for
// token row + t (t clamped to T - 1: a token past T reads the last one, and
// its values are discarded where used), as 16- or 8-byte loads; branch-free,
// so the loads stay in flight while the caller works on
template <int CPT>
__device__ __forceinline__ void gla_run_load(const float* __restrict__ QKV, const float* __restrict__ Z,
                                             uint32_t row, uint32_t t, uint32_t T, uint32_t c0, uint32_t d,
                                             float (&q)[CPT], float (&k)[CPT], float (&v)[CPT],
                                             float (&z)[CPT]) {
  static_assert(CPT % 4 == 0 || CPT == 2, "whole float4s or one float2");
  const uint32_t tt = min(t, T - 1);
  const float* x = QKV + (size_t)(row + tt) * 3 * d + c0;
  const float* zz = Z + (size_t)(row + tt) * d + c0;
  if constexpr (CPT == 2) {
    const float2 a = *reinterpret_cast<const float2*>(x), b = *reinterpret_cast<const float2*>(x + d),
                 c = *reinterpret_cast<const float2*>(x + 2 * d), e = *reinterpret_cast<const float2*>(zz);
    q[0] = a.x; q[1] = a.y; k[0] = b.x; k[1] = b.y; v[0] = c.x; v[1] = c.y; z[0] = e.x; z[1] = e.y;
  } else {
#pragma unroll
    for (int u = 0; u < CPT; u += 4) {
      const float4 a = *reinterpret_cast<const float4*>(x + u), b = *reinterpret_cast<const float4*>(x + d + u),
                   c = *reinterpret_cast<const float4*>(x + 2 * d + u),
                   e = *reinterpret_cast<const float4*>(zz + u);
      q[u] = a.x; q[u + 1] = a.y; q[u + 2] = a.z; q[u + 3] = a.w;
      k[u] = b.x; k[u + 1] = b.y; k[u + 2] = b.z; k[u + 3] = b.w;
      v[u] = c.x; v[u + 1] = c.y; v[u + 2] = c.z; v[u + 3] = c.w;
      z[u] = e.x; z[u + 1] = e.y; z[u + 2] = e.z; z[u + 3] = e.w;
    }
  }
}

// the sum over each group of 8 consecutive lanes (a quad, then the
// mirrored quad), in every lane of the group
__device__ __forceinline__ float sum8(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v;
}

// 1 - e^x for x <= 0 without cancellation near 0: the series to x^7 where
// x > -1/2 (truncation below 2e-7 of the result), the hardware exp elsewhere
__device__ __forceinline__ float one_minus_exp(float x) {
  float p = fmaf(x, 1.0f / 5040.0f, 1.0f / 720.0f);
  p = fmaf(x, p, 1.0f / 120.0f);
  p = fmaf(x, p, 1.0f / 24.0f);
  p = fmaf(x, p, 1.0f / 6.0f);
  p = fmaf(x, p, 0.5f);
  p = fmaf(x, p, 1.0f);
  return x > -0.5f ? -x * p : 1.0f - __expf(x);
}

template <int HD>
__global__ __launch_bounds__(256, 3) void k_gla_run(const float* __restrict__ QKV,
                                                     const float* __restrict__ Z,
                                                     const float* __restrict__ lam, float* __restrict__ O,
                                                     __bf16* __restrict__ Oh, StateRef S,
                                                     const GlaRun* __restrict__ runs, uint32_t d, uint32_t rglru) {
  constexpr int L = kGlaSub, TPA = 256 / HD, TPT = L / TPA, CBS = HD / 16, R = 4 / CBS;
  static_assert(TPT >= 1 && TPA * TPT == L && CBS * R == 4, "whole tokens a thread, a column block a wave");
  // the gate pass: TPK threads a token, CPT columns a thread
  constexpr int TPK = 256 / L, CPT = HD / TPK;
  static_assert(TPK == 8 && CPT * TPK == HD, "a token's columns over 8 lanes");
  // row strides (floats) picked by a model of the 64 lanes' bank use for
  // each read pattern at HD = 64: the pair levels' 16 rows x 4 k and the
  // diagonal's 8 x 8 on qh, kh and cl; qt S's 16 rows x 4 columns 4 apart
  // on qh; Kd^T V's and P V's 4 rows x 16 columns on kh and vv (stride 16
  // mod 64 spreads those over all 64 banks); P V's 16 rows x 4 k on P
  constexpr int SQ = HD + 5, SK = HD + 10, SC = HD + 6, SV = HD + 16, SP = L + 4;
  __shared__ float qh[L][SQ], kh[L][SK], cl[L][SC], vv[L][SV];
  __shared__ float P[L][SP], tot[TPA][HD];
  const uint32_t h = blockIdx.x, tid = threadIdx.x;
  const GlaRun r = runs[blockIdx.y];
  const uint32_t a = tid % HD, tb = tid / HD;
  const uint32_t tk = tid / TPK, c0 = h * HD + (tid % TPK) * CPT, e0 = (tid % TPK) * CPT;
  const uint32_t lane = tid & 63, wv = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  const uint32_t bw = wv % CBS, rep = wv / CBS;
  float* Sg = S.base + (size_t)r.seq * S.seq_stride + S.layer_off + (size_t)h * HD * HD;
  f32x4_t Sr[CBS];
#pragma unroll
  for (int ab = 0; ab < CBS; ab++)
#pragma unroll
    for (int y = 0; y < 4; y++) Sr[ab][y] = Sg[(16 * ab + 4 * g4 + y) * HD + 16 * bw + r16];
  float lv[CPT];
#pragma unroll
  for (int e = 0; e < CPT; e++) lv[e] = rglru ? f_log_sigmoid(lam[c0 + e]) : 0.0f;
  float q[CPT], k[CPT], v[CPT], z[CPT];
  gla_run_load<CPT>(QKV, Z, r.row, tk, r.T, c0, d, q, k, v, z);
  for (uint32_t j0 = 0; j0 < r.T; j0 += L) {
    const uint32_t n = min((uint32_t)L, r.T - j0);
    // token tk's norms (sums over its 8 lanes) and gates (dd.gate), token
    // by token: the hardware's reciprocal square root, exp, log and square
    // root (~1 ulp), and 1 - e^(2 la) by one_minus_exp, as la ends near the
    // cap of -1e-4 there
    float lqr[CPT], lkr[CPT], lar[CPT], vr[CPT];
    {
      const bool ok = tk < n;
      float sq = 0.0f, sk = 0.0f;
#pragma unroll
      for (int e = 0; e < CPT; e++) {
        sq = fmaf(q[e], q[e], sq);
        sk = fmaf(k[e], k[e], sk);
      }
      const float rq = __builtin_amdgcn_rsqf(1.0e-6f + sum8(sq)), rk = __builtin_amdgcn_rsqf(1.0e-6f + sum8(sk));
#pragma unroll
      for (int e = 0; e < CPT; e++) {
        float la, lk;
        if (rglru) {
          la = fminf(ANA_CAP, (8.0f * __builtin_amdgcn_rcpf(1.0f + __expf(-z[e]))) * lv[e]);
          lk = (k[e] * rk) * __builtin_amdgcn_sqrtf(one_minus_exp(2.0f * la));
        } else {
          la = -(fmaxf(-z[e], 0.0f) + __logf(1.0f + __expf(-fabsf(z[e]))));
          lk = k[e] * rk;
        }
        lqr[e] = ok ? q[e] * rq : 0.0f;
        lkr[e] = ok ? lk : 0.0f;
        lar[e] = ok ? la : 0.0f;
        vr[e] = ok ? v[e] : 0.0f;
      }
    }
    // the next sub-chunk's inputs, in flight through this one's work
    if (j0 + L < r.T) gla_run_load<CPT>(QKV, Z, r.row, j0 + L + tk, r.T, c0, d, q, k, v, z);
    __syncthreads();   // (the previous sub-chunk's reads of the arrays are done)
#pragma unroll
    for (int e = 0; e < CPT; e++) {
      qh[tk][e0 + e] = lqr[e];
      kh[tk][e0 + e] = lkr[e];
      cl[tk][e0 + e] = lar[e];
      vv[tk][e0 + e] = vr[e];
    }
    __syncthreads();
    // the running sums of log a down each column: thread (a, tb) over its
    // TPT tokens, then the earlier blocks' totals
    {
      float c[TPT];
#pragma unroll
      for (int i = 0; i < TPT; i++) c[i] = (i ? c[i - 1] : 0.0f) + cl[tb * TPT + i][a];
      tot[tb][a] = c[TPT - 1];
      __syncthreads();
      float off = 0.0f;
      for (uint32_t b = 0; b < tb; b++) off += tot[b][a];
#pragma unroll
      for (int i = 0; i < TPT; i++) cl[tb * TPT + i][a] = c[i] + off;
    }
    __syncthreads();
    gla_pairs<HD>(qh, kh, cl, P, n, tid);
    __syncthreads();
    // qt = qh e^(c) and Kd = kh e^(c_last - c) in place (zero past n: the
    // gates there are zero)
    const float clast = cl[n - 1][a];
#pragma unroll
    for (int i = 0; i < TPT; i++) {
      const uint32_t t = tb * TPT + i;
      const float ct = cl[t][a];
      qh[t][a] *= __expf(ct);
      kh[t][a] *= __expf(clast - ct);
    }
    __syncthreads();
    // o = P V + qt S on column block bw, token halves th (split over the
    // copies)
    for (uint32_t th = rep; th < 2; th += R) {
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k0 = 0; k0 < L; k0 += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(P[16 * th + r16][k0 + g4], vv[k0 + g4][16 * bw + r16], acc,
                                                   0, 0, 0);
#pragma unroll
      for (int ab = 0; ab < CBS; ab++)
#pragma unroll
        for (int y = 0; y < 4; y++)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qh[16 * th + r16][16 * ab + 4 * g4 + y], Sr[ab][y], acc,
                                                     0, 0, 0);
#pragma unroll
      for (int x = 0; x < 4; x++) {
        const uint32_t t = 16 * th + 4 * g4 + x;
        if (t < n) {
          const size_t o = (size_t)(r.row + j0 + t) * d + h * HD + 16 * bw + r16;
          if (Oh) Oh[o] = (__bf16)acc[x];
          else O[o] = acc[x];
        }
      }
    }
    // S' = D S + Kd^T V on the wave's own tiles (the next sub-chunk writes
    // LDS only after its first barrier)
#pragma unroll
    for (int ab = 0; ab < CBS; ab++) {
#pragma unroll
      for (int y = 0; y < 4; y++) Sr[ab][y] *= __expf(cl[n - 1][16 * ab + 4 * g4 + y]);
#pragma unroll
      for (int k0 = 0; k0 < L; k0 += 4)
        Sr[ab] = __builtin_amdgcn_mfma_f32_16x16x4f32(kh[k0 + g4][16 * ab + r16], vv[k0 + g4][16 * bw + r16],
                                                      Sr[ab], 0, 0, 0);
    }
  }
  if (rep == 0)
#pragma unroll
    for (int ab = 0; ab < CBS; ab++)
#pragma unroll
      for (int y = 0; y < 4; y++) Sg[(16 * ab + 4 * g4 + y) * HD + 16 * bw + r16] = Sr[ab][y];
}

hipError_t launch_gla_run(const float* QKV, const float* Z, const float* lam, StateRef S, float* O, __bf16* Oh,
                          const GlaRun* runs, uint32_t nrun, uint32_t rows, uint32_t d, uint32_t heads,
                          uint32_t rglru, hipStream_t st) {
  const uint32_t hd = d / heads;
  if (nrun == 0 || hd * heads != d || (uint64_t)rows * 3 * d >= (1ull << 32)) return hipErrorInvalidValue;
  switch (hd) {
    case 64: hipLaunchKernelGGL(k_gla_run<64>, dim3(heads, nrun), dim3(256), 0, st, QKV, Z, lam, O, Oh, S, runs, d, rglru); break;
    case 32: hipLaunchKernelGGL(k_gla_run<32>, dim3(heads, nrun), dim3(256), 0, st, QKV, Z, lam, O, Oh, S, runs, d, rglru); break;
    case 16: hipLaunchKernelGGL(k_gla_run<16>, dim3(heads, nrun), dim3(256), 0, st, QKV, Z, lam, O, Oh, S, runs, d, rglru); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// A fast-mode prefill step's K and V rows into the rings (dd.sm.write over
// every row): wave w of workgroup x takes row 4 x + w, lane l its float4
// columns 4 (l + 64 j), so a head's HD columns are HD / 4 consecutive lanes;
// the qk-norm's sum of squares is their group sum (reassociated),
// k = (k * s) * (1 + gk), and K and V go to slot pos mod ctx. The exact
// kernel takes one workgroup a (head, row) with an in-order chain instead.
template <int HD>
__global__ __launch_bounds__(256) void k_kv_write_fast(AttnArgs a) {
  // a wave a row, four columns a lane (float4), so each lane's loads and
  // stores are 16 bytes and a workgroup moves four whole rows; a head's
  // HD / 4 lanes sum its squares by DPP within their 16-lane row
  constexpr int G = HD / 4;
  static_assert(G == 4 || G == 8 || G == 16, "a head's lanes inside one DPP row");
  const uint32_t lane = threadIdx.x & 63, b = blockIdx.x * 4 + (threadIdx.x >> 6), d = a.d, d4 = d >> 2;
  if (b >= a.B) return;
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t slot = pos % a.ctx;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  const float4* x = reinterpret_cast<const float4*>(a.QKV + (size_t)b * 3 * d);
  float4* Kr = reinterpret_cast<float4*>(a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off +
                                         (size_t)slot * d);
  float4* Vr = Kr + (size_t)a.ctx * d4;
  // (d4 is a multiple of 64 lanes' worth or the tail lanes sit out whole
  // groups: d is heads x HD, so a group never straddles the end)
  for (uint32_t q = lane; q < ((d4 + 63) & ~63u); q += 64) {
    const bool in = q < d4;
    float4 k = in ? x[d4 + q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 v = in ? x[2 * d4 + q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (a.gk) {
      float ss = k.x * k.x + k.y * k.y + k.z * k.z + k.w * k.w;
      ss += dpp<0xB1>(ss);
      ss += dpp<0x4E>(ss);
      if constexpr (G >= 8) ss += dpp<0x141>(ss);
      if constexpr (G >= 16) ss += dpp<0x140>(ss);
      const float r = 1.0f / sqrtf(ss / (float)HD + 1.0e-5f);
      // (the gains one float at a time: their offset in the parameters need
      // not be a multiple of four)
      const float* g = a.gk + (4 * q) % HD;
      k = make_float4((k.x * r) * (1.0f + g[0]), (k.y * r) * (1.0f + g[1]), (k.z * r) * (1.0f + g[2]),
                      (k.w * r) * (1.0f + g[3]));
    }
    if (in) {
      Kr[q] = k;
      Vr[q] = v;
    }
  }
}

hipError_t launch_kv_write_fast(const AttnArgs& a, hipStream_t st) {
  const uint32_t hd = a.d / a.heads;
  if (a.B == 0 || hd * a.heads != a.d) return hipErrorInvalidValue;
  const dim3 grid((a.B + 3) / 4);
  switch (hd) {
    case 64: hipLaunchKernelGGL(k_kv_write_fast<64>, grid, dim3(256), 0, st, a); break;
    case 32: hipLaunchKernelGGL(k_kv_write_fast<32>, grid, dim3(256), 0, st, a); break;
    case 16: hipLaunchKernelGGL(k_kv_write_fast<16>, grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static size_t round64(size_t n) { return (n + 63) & ~(size_t)63; }

size_t gla_scan_floats(uint32_t rows, uint32_t nsub, uint32_t nseg, uint32_t d, uint32_t heads) {
  const size_t hd = d / heads;
  return round64((size_t)rows * d) + round64((size_t)nsub * heads * hd) +
         round64((size_t)nsub * heads * hd * hd) + round64((size_t)nseg * heads * hd * hd);
}

GlaScratch gla_scan_carve(float* p, uint32_t rows, uint32_t nsub, uint32_t nseg, uint32_t d,
                          uint32_t heads) {
  const size_t hd = d / heads;
  GlaScratch g;
  g.Qt = p;
  g.Dj = g.Qt + round64((size_t)rows * d);
  g.Uj = g.Dj + round64((size_t)nsub * heads * hd);
  g.S0 = g.Uj + round64((size_t)nsub * heads * hd * hd);
  g.rows_cap = rows;
  g.nsub_cap = nsub;
  g.nseg_cap = nseg;
  return g;
}

hipError_t launch_gla_scan(const float* QKV, const float* Z, const float* lam, StateRef S, float* O,
                           const GlaScratch& g, const GlaSub* tab, uint32_t nsub, uint32_t d,
                           uint32_t heads, uint32_t rglru, hipStream_t st) {
  const uint32_t hd = d / heads;
  if (hd % 16 || hd * 16 < 256 || nsub == 0) return hipErrorInvalidValue;
  if (nsub > g.nsub_cap) return hipErrorInvalidValue;
#define L_(H)                                                                                        \
  hipLaunchKernelGGL(k_gla_sub<H>, dim3(heads, nsub), dim3(256), 0, st, QKV, Z, lam, O, g, S, tab, d, \
                     rglru);                                                                         \
  hipLaunchKernelGGL(k_gla_carry<H>, dim3(heads, H / 16, nsub), dim3(256), 0, st, g, S, O, tab, d)
  switch (hd) {
    case 64: L_(64); break;
    case 32: L_(32); break;
    case 16: L_(16); break;
    default: return hipErrorInvalidValue;
  }
#undef L_
  return hipGetLastError();
}

}  // namespace ana

namespace ana {

// ------------------------------------------------------------------ large-M products on MFMA

// Y[m][n] = sum_k X[m][k] W[n][k] for M >= 128 (prefill batches): a 128 x
// 128 tile per workgroup, four waves in 2 x 2 each computing 64 x 64 as
// 4 x 4 MFMA 16 x 16 tiles. K goes in stages of BK through two LDS buffers,
// the next stage's global loads in registers while the current one is
// multiplied. ANA_BF16: v_mfma_f32_16x16x32_bf16 on the bf16 weights and
// the activations rounded to bf16;
// ANA_FAST_FP32: v_mfma_f32_16x16x4f32. Norm, residual and SiLU as in
// k_gemm_mfma (SiLU: tile rows 0..63 gate j, 64..127 up j).
template <int WT>
__global__ __launch_bounds__(256) void k_gemm_big(GemvArgs a) {
  constexpr int BM = 128, BN = 128, BK = WT == 1 ? 32 : 16;
  constexpr int AP = BK + 8;                      // LDS row pitch (elements)
  using E = typename std::conditional<WT == 1, __bf16, float>::type;
  __shared__ __align__(16) E As[2][BM][AP];
  __shared__ __align__(16) E Bs[2][BN][AP];
  __shared__ float rsc[BM];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t wm = wv >> 1, wn = wv & 1;       // the wave's 64 x 64 block
  const uint32_t m0 = blockIdx.y * BM;
  const uint32_t nb = min((uint32_t)BM, a.B - m0);
  const uint32_t K = a.K, nst = (K + BK - 1) / BK;
  const Segs sgs(a);
  const bool norm = a.ng != nullptr;
  // staging: A (fp32 activations) BM x BK, B (weights) BN x BK
  constexpr int AF4 = BM * BK / 4 / 256;          // float4 of A a thread (bf16: 4, f32: 2)
  constexpr int BV = WT == 1 ? BN * BK / 8 / 256 : BN * BK / 4 / 256;  // 16-byte pieces of B
  const float* asrc[AF4];
  uint32_t am_[AF4], ak_[AF4];
#pragma unroll
  for (int j = 0; j < AF4; j++) {
    const uint32_t i = tid + 256 * j, m = i / (BK / 4), k4 = i % (BK / 4);
    am_[j] = m;
    ak_[j] = 4 * k4;
    asrc[j] = a.X + (size_t)(m0 + (m < nb ? m : 0)) * a.ldx;
  }
  const float* bsrcf[BV];
  const uint16_t* bsrch[BV];
  uint32_t bn_[BV], bk_[BV];
#pragma unroll
  for (int j = 0; j < BV; j++) {
    const uint32_t i = tid + 256 * j;
    const uint32_t n = WT == 1 ? i / (BK / 8) : i / (BK / 4);
    const uint32_t k = WT == 1 ? 8 * (i % (BK / 8)) : 4 * (i % (BK / 4));
    bn_[j] = n;
    bk_[j] = k;
    const float* w;
    uint32_t sg, lr;
    const bool ok = sgs.row(BN, blockIdx.x, n, &w, &sg, &lr);
    bsrcf[j] = ok ? w : sgs.W0;
    bsrch[j] = ok ? (sg ? a.Wh1 : a.Wh0) + (size_t)lr * K : a.Wh0;
  }
  float4 ar[AF4];
  uint4 brh[BV];
  float4 brf[BV];
  auto load = [&](uint32_t s) {
    const uint32_t q0 = s * BK;
#pragma unroll
    for (int j = 0; j < AF4; j++) {
      const uint32_t q = q0 + ak_[j];
      ar[j] = *reinterpret_cast<const float4*>(asrc[j] + (q < K ? q : 0));
    }
#pragma unroll
    for (int j = 0; j < BV; j++) {
      const uint32_t q = q0 + bk_[j];
      if constexpr (WT == 1) brh[j] = *reinterpret_cast<const uint4*>(bsrch[j] + (q < K ? q : 0));
      else brf[j] = *reinterpret_cast<const float4*>(bsrcf[j] + (q < K ? q : 0));
    }
  };
  float ss[AF4];
#pragma unroll
  for (int j = 0; j < AF4; j++) ss[j] = 0.0f;
  auto store = [&](int buf, uint32_t s) {
    const uint32_t q0 = s * BK;
#pragma unroll
    for (int j = 0; j < AF4; j++) {
      const uint32_t q = q0 + ak_[j];
      float4 x = ar[j];
      if (q >= K || am_[j] >= nb) x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (norm) {
        ss[j] += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
        const float4 g = *reinterpret_cast<const float4*>(a.ng + (q < K ? q : 0));
        x.x *= g.x;
        x.y *= g.y;
        x.z *= g.z;
        x.w *= g.w;
      }
      E* dst = &As[buf][am_[j]][ak_[j]];
      dst[0] = (E)x.x;
      dst[1] = (E)x.y;
      dst[2] = (E)x.z;
      dst[3] = (E)x.w;
    }
#pragma unroll
    for (int j = 0; j < BV; j++) {
      const uint32_t q = q0 + bk_[j];
      if constexpr (WT == 1) {
        uint4 w = brh[j];
        if (q >= K) w = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(&Bs[buf][bn_[j]][bk_[j]]) = w;
      } else {
        float4 w = brf[j];
        if (q >= K) w = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *reinterpret_cast<float4*>(&Bs[buf][bn_[j]][bk_[j]]) = w;
      }
    }
  };
  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t r16 = lane & 15, g4 = lane >> 4;
  load(0);
  store(0, 0);
  __syncthreads();
  for (uint32_t s = 0; s < nst; s++) {
    const int buf = s & 1;
    if (s + 1 < nst) load(s + 1);
    if constexpr (WT == 1) {
      bf16x8_t bfr[4], ah[4];
#pragma unroll
      for (int j = 0; j < 4; j++) bfr[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[buf][wn * 64 + 16 * j + r16][8 * g4]);
#pragma unroll
      for (int i = 0; i < 4; i++) ah[i] = *reinterpret_cast<const bf16x8_t*>(&As[buf][wm * 64 + 16 * i + r16][8 * g4]);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bfr[j], acc[i][j], 0, 0, 0);
    } else {
      float4 bfr[4], afr[4];
#pragma unroll
      for (int j = 0; j < 4; j++) bfr[j] = *reinterpret_cast<const float4*>(&Bs[buf][wn * 64 + 16 * j + r16][4 * g4]);
#pragma unroll
      for (int i = 0; i < 4; i++) afr[i] = *reinterpret_cast<const float4*>(&As[buf][wm * 64 + 16 * i + r16][4 * g4]);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(afr[i].x, bfr[j].x, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(afr[i].y, bfr[j].y, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(afr[i].z, bfr[j].z, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(afr[i].w, bfr[j].w, acc[i][j], 0, 0, 0);
        }
    }
    if (s + 1 < nst) store(buf ^ 1, s + 1);
    __syncthreads();
  }
  // rows' norm scales: the threads of a row (BK / 4 / AF4... all threads
  // staging row m) add their sums of squares in LDS
  if (norm) {
    if (tid < BM) rsc[tid] = 0.0f;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < AF4; j++) atomicAdd(&rsc[am_[j]], ss[j]);
    __syncthreads();
    if (tid < BM) rsc[tid] = 1.0f / sqrtf(rsc[tid] / (float)K + 1.0e-5f);
    __syncthreads();
  }
  // results: tile (i, j) of the wave holds rows wm*64 + 16i + 4*g4 + r,
  // column wn*64 + 16j + r16
  if (a.mode == GM_SILU) {
    // up columns (wn = 1) through LDS to the gate columns (wn = 0), one
    // 64-row half at a time (64 x 64 floats fit in Bs in both modes)
    float* up = reinterpret_cast<float*>(&Bs[0][0][0]);
    static_assert(sizeof(Bs) >= 64 * 64 * sizeof(float), "exchange buffer");
    for (uint32_t half = 0; half < 2; half++) {
      if (wn == 1 && wm == half) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const uint32_t ml = 16 * i + 4 * g4 + r, n = 16 * j + r16;
              float y = acc[i][j][r];
              if (norm) y *= rsc[wm * 64 + ml];
              up[ml * 64 + n] = y;
            }
      }
      __syncthreads();
      if (wn == 0 && wm == half) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t n = 16 * j + r16;
          const float* w_;
          uint32_t sg, lr;
          if (!sgs.row(BN, blockIdx.x, n, &w_, &sg, &lr)) continue;
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const uint32_t ml = 16 * i + 4 * g4 + r, m = wm * 64 + ml;
              if (m >= nb) continue;
              float y = acc[i][j][r];
              if (norm) y *= rsc[m];
              a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = fast_silu(y) * up[ml * 64 + n];
            }
        }
      }
      __syncthreads();
    }
    return;
  }
  // per column block: its residuals loaded together before any store (a
  // load after a store through another pointer would wait on it, one round
  // trip per element)
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t n = wn * 64 + 16 * j + r16;
    const float* w_;
    uint32_t sg, lr;
    if (!sgs.row(BN, blockIdx.x, n, &w_, &sg, &lr)) continue;
    float res[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = wm * 64 + 16 * i + 4 * g4 + r;
        res[i][r] = a.mode == GM_RESID && m < nb ? a.R[(size_t)(m0 + m) * a.ldr + lr] : 0.0f;
      }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = wm * 64 + 16 * i + 4 * g4 + r;
        if (m >= nb) continue;
        float y = acc[i][j][r];
        if (norm) y *= rsc[m];
        if (a.mode == GM_RESID) y = res[i][r] + y;
        if (sg) a.seg[1].Y[(size_t)(m0 + m) * a.seg[1].ldy + lr] = y;
        else a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = y;
      }
  }
}

hipError_t launch_gemm_big(const GemvArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  if (a.amax || (a.K & 7) || a.B == 0) return hipErrorInvalidValue;
  const bool bf = a.Wh0 != nullptr;
  if (bf && a.nseg > 1 && !a.Wh1) return hipErrorInvalidValue;
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  const uint32_t per = a.mode == GM_SILU ? 64 : 128;
  const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
  dim3 grid(tiles, (a.B + 127) / 128);
  if (bf) ANA_LAUNCH_F((k_gemm_big<1>), grid, dim3(256), 0, st, e0, e1, a);
  else ANA_LAUNCH_F((k_gemm_big<0>), grid, dim3(256), 0, st, e0, e1, a);
  return hipGetLastError();
}

}  // namespace ana

namespace ana {

// ------------------------------------------------------------------ bf16 prefill products, direct to LDS

// The activations of an ANA_BF16 prefill product as bf16: each value
// (times the norm's gain) rounded to nearest even; with a gain, also each
// row's norm scale 1 / sqrt(ss / K + 1e-5) over the unscaled row. One wave
// a row.
__global__ __launch_bounds__(256) void k_split(const float* __restrict__ X, uint32_t ldx, uint32_t K,
                                                const float* __restrict__ g, uint32_t M,
                                                __bf16* __restrict__ Ah, float* __restrict__ rsc) {
  const uint32_t m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (m >= M) return;
  const float* x = X + (size_t)m * ldx;
  float ss = 0.0f;
  for (uint32_t k = 4 * lane; k < K; k += 256) {
    float4 v = *reinterpret_cast<const float4*>(x + k);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    if (g) {
      const float4 gg = *reinterpret_cast<const float4*>(g + k);
      v.x *= gg.x;
      v.y *= gg.y;
      v.z *= gg.z;
      v.w *= gg.w;
    }
    __bf16 h[4] = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
    *reinterpret_cast<uint2*>(Ah + (size_t)m * K + k) = *reinterpret_cast<const uint2*>(h);
  }
  if (g) {
    ss = wave_sum(ss);
    if (lane == 0) rsc[m] = 1.0f / sqrtf(ss / (float)K + 1.0e-5f);
  }
}

// Y[m][n] = sum_k A[m][k] W[n][k] for ANA_BF16 prefill steps of >= 128 rows,
// A given as bf16 (k_split): a 128 x 128 tile per workgroup, four waves of
// 64 x 64 (4 x 4 v_mfma_f32_16x16x32_bf16 tiles). K goes in stages of 64
// through a ring of NS LDS stages filled by global_load_lds_dwordx4 (no
// registers between global memory and LDS): each stage holds the A and
// weight tiles as 1 KB chunks of 8 rows, each row's whole 128-byte line, its
// eight 16-byte k pieces at slot piece ^ (row & 7), so a fragment read
// touches eight distinct 16-byte bank groups at a time (loads of half
// lines, 16 rows x 64 bytes, moved the same bytes at two thirds the rate).
// A wave waits on its own loads of the stage it is about to read, then a
// barrier (no fence, which would wait on every load in flight) makes the
// other waves' loads visible; loads of the next stage go out right after
// it (the barrier also says every wave is done with the stage they
// overwrite). Norm scale, residual and SiLU as in k_gemm_big.
template <int NS, bool SILU, int BN>
__global__ __launch_bounds__(256, 2) void k_gemm_dl(GemvArgs a, const __bf16* __restrict__ Ahg,
                                                  const float* __restrict__ rscg) {
  constexpr int BM = 128, BK = 64, NJ = BN / 32, HN = BN / 2;   // (NJ 16-column MFMA tiles a wave, HN its columns)
  static_assert(BN == 128 || (BN == 96 && !SILU), "tile width");
  constexpr int OPE = BM * BK;   // bf16 elements of one operand's stage (16 KB, 16 chunks)
  static_assert(NS == 2, "two stage objects");
  // one LDS object per stage: a stage's fragment reads then provably miss
  // the loads in flight into the other, and the compiler does not wait for
  // them (one array indexed by stage made it drain every load before each
  // stage's reads, and the loads never overlapped the MFMAs)
  __shared__ __align__(1024) __bf16 st0[2][OPE], st1[2][OPE];
  __shared__ float rsl[BM];
  auto stage = [&](auto B) -> __bf16(*)[OPE] {
    if constexpr (decltype(B)::value == 0) return st0;
    else return st1;
  };
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t wm = wv >> 1, wn = wv & 1;
  uint32_t ntile, mtile;
  xcd_tile(&ntile, &mtile);
  const uint32_t m0 = mtile * BM;
  const uint32_t nb = min((uint32_t)BM, a.B - m0);
  const uint32_t K = a.K, nst = K / BK;
  const Segs sgs(a);
  // this lane's piece of the wave's four 1 KB chunks per operand (chunk
  // c = 4 wv + h: tile rows 8 c .. 8 c + 7): row lane / 8 of the chunk,
  // slot lane % 8 holding k piece (lane % 8) ^ row
  const uint32_t pr = lane >> 3, pq = (lane & 7) ^ pr;
  uint32_t aoff[4];
  const uint16_t* bptr[NJ];
#pragma unroll
  for (int h = 0; h < 4; h++) {
    const uint32_t r = 8 * (4 * wv + h) + pr;
    aoff[h] = (m0 + (r < nb ? r : 0)) * K + 8 * pq;
  }
  // the weight tile's BN / 8 chunks: NJ a wave (chunk NJ wv + h)
#pragma unroll
  for (int h = 0; h < NJ; h++) {
    const uint32_t r = 8 * (NJ * wv + h) + pr;
    const float* w;
    uint32_t sg, lr;
    const bool ok = sgs.row(BN, ntile, r, &w, &sg, &lr);
    bptr[h] = ok ? (sg ? a.Wh1 : a.Wh0) + (size_t)lr * K + 8 * pq : a.Wh0 + 8 * pq;
  }
  auto issue = [&](uint32_t s, auto B) {
    const uint32_t k0 = s * BK;
#pragma unroll
    for (int h = 0; h < 4; h++) {
      __builtin_amdgcn_global_load_lds((const void*)(Ahg + aoff[h] + k0), (lds_void*)&stage(B)[0][(4 * wv + h) * 512], 16, 0, 0);
      if (h < NJ)
        __builtin_amdgcn_global_load_lds((const void*)(bptr[h] + k0), (lds_void*)&stage(B)[1][(NJ * wv + h) * 512], 16, 0, 0);
    }
  };
  f32x4_t acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t r16 = lane & 15, g4 = lane >> 4;
  // fragment read offsets (elements) in a 16-row MFMA tile (two chunks):
  // row r16, k piece 4 kh + g4
  const uint32_t fbase = (r16 >> 3) * 512 + (r16 & 7) * 64;
  const uint32_t foff[2] = {fbase + 8 * (g4 ^ (r16 & 7)), fbase + 8 * ((4 + g4) ^ (r16 & 7))};
  auto compute = [&](auto B) {
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
      const __bf16* A0 = &stage(B)[0][0];
      const __bf16* B0 = &stage(B)[1][0];
      bf16x8_t bfr[NJ], ah[4];
#pragma unroll
      for (int j = 0; j < NJ; j++) bfr[j] = *reinterpret_cast<const bf16x8_t*>(B0 + (wn * NJ + j) * 1024 + foff[kh]);
#pragma unroll
      for (int i = 0; i < 4; i++) ah[i] = *reinterpret_cast<const bf16x8_t*>(A0 + (wm * 4 + i) * 1024 + foff[kh]);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  };
  // the wait and the barrier, with no LDS access moved across them (the
  // barrier builtin alone orders no memory)
  auto step_barrier = [&]() {
    asm volatile("" ::: "memory");
    ANA_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  constexpr std::integral_constant<int, 0> S0{};
  constexpr std::integral_constant<int, 1> S1{};
  // full tiles (every row and column valid) of plain and residual products
  // take the epilogue without checks; their residuals are loaded here,
  // before the k loop, so those loads overlap the MFMAs instead of waiting
  // in the epilogue with every other workgroup's
  const uint32_t wrows = a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  const bool full = !SILU && nb == (uint32_t)BM && (ntile + 1) * BN <= wrows;
  uint32_t col[NJ];
  bool s1[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const uint32_t v = ntile * BN + wn * HN + 16 * j + r16;
    s1[j] = v >= a.seg[0].rows;
    col[j] = s1[j] ? v - a.seg[0].rows : v;
  }
  const size_t mrow = m0 + wm * 64 + 4 * g4;   // this lane's first row
  float res[NJ][4][4];
  if (full && a.mode == GM_RESID) {
    const float* rb = a.R + mrow * a.ldr;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) res[j][i][r] = rb[(size_t)(16 * i + r) * a.ldr + col[j]];
  } else {
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) res[j][i][r] = 0.0f;
  }
  issue(0, S0);
  // stage s: this wave's loads of it are done (the only ones in flight),
  // then every wave's (the barrier, which also says every wave is done with
  // the other stage object); the next stage's loads go out, then s's MFMAs
  for (uint32_t s = 0; s < nst; s += 2) {
    step_barrier();
    if (s + 1 < nst) issue(s + 1, S1);
    compute(S0);
    if (s + 1 < nst) {
      step_barrier();
      if (s + 2 < nst) issue(s + 2, S0);
      compute(S1);
    }
  }
  const bool norm = a.ng != nullptr;
  // results: tile (i, j) of the wave holds rows wm*64 + 16i + 4*g4 + r,
  // column wn*HN + 16j + r16. The tile's row norm scales go to LDS before
  // any store (a global load after a store through another pointer would
  // wait on it, one round trip per element)
  if (norm) {
    if (tid < (uint32_t)BM) {
      const uint32_t m = m0 + (tid < nb ? tid : 0);
      rsl[tid] = a.sspi ? norm_from_partials(a.sspi + (size_t)m * a.nspi, a.nspi, K) : rscg[m];
    }
    __syncthreads();
  }
  auto rs = [&](int i, int r) { return norm ? rsl[wm * 64 + 16 * i + 4 * g4 + r] : 1.0f; };
  // full tiles store without a check among the stores (the residuals came
  // in before the k loop): with per-element checks and each column block's
  // residual loads after the previous block's stores, the compiler drained
  // the stores (vmcnt(0)) before every block
  if (full) {
    float sc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) sc[i][r] = norm ? rsl[wm * 64 + 16 * i + 4 * g4 + r] : 1.0f;
    // with Yn (one segment): the outputs times the next norm's gain in bf16
    // too, and each row's sum of squares over the wave's HN columns (the
    // 16 lanes of a row group by DPP, then one partial a row)
    float ss[4][4], gn[NJ];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) ss[i][r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) gn[j] = a.Yn ? a.gn[col[j]] : 0.0f;   // (loaded before any store)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      float* const Yb = s1[j] ? a.seg[1].Y : a.seg[0].Y;
      const uint32_t ld = s1[j] ? a.seg[1].ldy : a.seg[0].ldy;
      float* yb = Yb + mrow * ld + col[j];
      const float gj = gn[j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          float y = acc[i][j][r] * sc[i][r];
          if (a.mode == GM_RESID) y = res[j][i][r] + y;
          yb[(size_t)(16 * i + r) * ld] = y;
          if (a.Yn) {
            a.Yn[(mrow + 16 * i + r) * a.seg[0].rows + col[j]] = (__bf16)(y * gj);
            ss[i][r] = fmaf(y, y, ss[i][r]);
          }
        }
    }
    if (a.Yn) {
      const uint32_t nsp = a.seg[0].rows / HN;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float t = row16_sum(ss[i][r]);
          if (r16 == 0) a.ssp[(mrow + 16 * i + r) * nsp + 2 * ntile + wn] = t;
        }
    }
    return;
  }
  if constexpr (SILU && BN == 128) {
    // up columns (wn = 1) through LDS to the gate columns (wn = 0), one
    // 64-row half at a time
    ANA_VMCNT(0);
    __syncthreads();
    float* up = reinterpret_cast<float*>(&st0[0][0]);
    static_assert(sizeof(st0) >= 64 * 64 * sizeof(float), "exchange buffer");
    for (uint32_t half = 0; half < 2; half++) {
      if (wn == 1 && wm == half) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const uint32_t ml = 16 * i + 4 * g4 + r, n = 16 * j + r16;
              up[ml * 64 + n] = acc[i][j][r] * rs(i, r);
            }
      }
      __syncthreads();
      if (wn == 0 && wm == half) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t n = 16 * j + r16;
          const float* w_;
          uint32_t sg, lr;
          if (!sgs.row(BN, ntile, n, &w_, &sg, &lr)) continue;
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const uint32_t ml = 16 * i + 4 * g4 + r, m = wm * 64 + ml;
              if (m >= nb) continue;
              const float y = acc[i][j][r] * rs(i, r);
              a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = fast_silu(y) * up[ml * 64 + n];
            }
        }
      }
      __syncthreads();
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    // one column block's residuals live at a time: the compiler barrier
    // keeps the next block's loads below this one's stores
    asm volatile("" ::: "memory");
    const uint32_t n = wn * HN + 16 * j + r16;
    const float* w_;
    uint32_t sg, lr;
    if (!sgs.row(BN, ntile, n, &w_, &sg, &lr)) continue;
    // the column block's residuals together, before its stores
    float res[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = wm * 64 + 16 * i + 4 * g4 + r;
        res[i][r] = a.mode == GM_RESID && m < nb ? a.R[(size_t)(m0 + m) * a.ldr + lr] : 0.0f;
      }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = wm * 64 + 16 * i + 4 * g4 + r;
        if (m >= nb) continue;
        float y = acc[i][j][r] * rs(i, r);
        if (a.mode == GM_RESID) y = res[i][r] + y;
        if (sg) a.seg[1].Y[(size_t)(m0 + m) * a.seg[1].ldy + lr] = y;
        else a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = y;
      }
  }
}

// k_gemm_dl's tile width: 96 where its tiles fill the workgroup slots (two
// a CU) at less tile width a CU than 128-wide ones do. At N = 768 and 8192
// rows, 128-wide tiles are 384 workgroups on 512 slots, so half the CUs
// take two and set the time while the rest take one; 96-wide tiles are
// 512, two on every CU, each CU a quarter fewer columns.
uint32_t gemm_dl_cols(const GemvArgs& a) {
  if (a.mode == GM_SILU) return 128;
  static uint32_t slots = 0;
  if (slots == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    slots = 2 * (uint32_t)n;
  }
  const uint32_t rows = a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0), mt = (a.B + 127) / 128;
  auto cost = [&](uint32_t bn) { return ((rows + bn - 1) / bn * mt + slots - 1) / slots * bn; };
  return cost(96) < cost(128) ? 96 : 128;
}

hipError_t launch_gemm_dl(const GemvArgs& a, __bf16* Ah, float* rsc, uint32_t cap_rows,
                          hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  if (a.amax || (a.K % 64) || a.B == 0 || !a.Wh0 || (a.nseg > 1 && !a.Wh1)) return hipErrorInvalidValue;
  if (a.B > cap_rows) return hipErrorInvalidValue;
  if (a.Xh && a.ng && !a.sspi) return hipErrorInvalidValue;   // (bf16 input with a norm: its partials)
  const uint32_t BN = gemm_dl_cols(a);
  // Yn: k_gemm_dl's full tiles only (its epilogue writes it), one segment;
  // its partial sums of squares go a row per BN / 2 columns
  if (a.Yn && (a.nseg != 1 || a.mode == GM_SILU || a.B % 128 || a.seg[0].rows % BN || !a.gn || !a.ssp ||
               gemm_wide_takes(a)))
    return hipErrorInvalidValue;
  // the split first (its time is inside the events), unless X came in bf16
  if (e0) (void)hipEventRecord(e0, st);
  if (a.Xh) Ah = const_cast<__bf16*>(a.Xh);
  else hipLaunchKernelGGL(k_split, dim3((a.B + 3) / 4), dim3(256), 0, st, a.X, a.ldx, a.K, a.ng, a.B, Ah, rsc);
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  // the 256 x 256 wide-wave tiles (gemm_wide.hip) where they still give
  // every CU a workgroup
  if (gemm_wide_takes(a)) {
    const hipError_t e = launch_gemm_wide(a, Ah, rsc, st);
    if (e1) (void)hipEventRecord(e1, st);
    return e;
  }
  if (a.Yh) return hipErrorInvalidValue;   // (only the large tiles write bf16 outputs)
  const uint32_t per = a.mode == GM_SILU ? 64 : BN;
  const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
  dim3 grid(tiles, (a.B + 127) / 128);
  // two LDS stages (48 KB) ran 5-12% faster than three (72 KB) at the
  // 8192-row prefill shapes with random operands (two workgroups a CU
  // either way, by registers)
  // (SiLU a compile-time choice: its code in the other products' kernel
  // changes how the compiler schedules their k loop)
  if (a.mode == GM_SILU) hipLaunchKernelGGL((k_gemm_dl<2, true, 128>), grid, dim3(256), 0, st, a, Ah, rsc);
  else if (BN == 96) hipLaunchKernelGGL((k_gemm_dl<2, false, 96>), grid, dim3(256), 0, st, a, Ah, rsc);
  else hipLaunchKernelGGL((k_gemm_dl<2, false, 128>), grid, dim3(256), 0, st, a, Ah, rsc);
  if (e1) (void)hipEventRecord(e1, st);
  return hipGetLastError();
}

}  // namespace ana

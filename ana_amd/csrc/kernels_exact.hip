// Exact-fp32 decode kernels for gfx950.
//
// Every output takes the F32 steps the reference's CPU kernels take
// (bend/effs/bulk.c:49-71 for products, 979-1088 for einsums): sums run in
// index order from 0.0f, a product and the sum it joins are two roundings
// (this file is compiled with -ffp-contract=off and the pragma below),
// exp/log go through double and are rounded to float, sqrt and division are
// the correctly rounded IEEE operations. Parallelism is only ever across
// outputs (rows, heads, sequences); each reduction chain stays in one lane,
// and the wide, parallel part of the work (loading weights, forming
// products) is spread over the whole workgroup and staged in LDS so that
// the in-order chains only add.
#include <hip/hip_ext.h>
#include <stdlib.h>

#include "ana_internal.h"
#include "numerics.h"

#pragma clang fp contract(off)

namespace ana {

// a zero float4 in registers (a namespace-scope constant would be loaded
// from memory through a flat pointer select)
#define kZero4 make_float4(0.0f, 0.0f, 0.0f, 0.0f)

// ------------------------------------------------------------------ products

// the result of chain (b, row lr of segment sg): plain or plus the residual
__device__ __forceinline__ void gemv_store(const GemvArgs& a, uint32_t sg, uint32_t lr, uint32_t b,
                                           float s) {
  float y = s;
  if (a.mode == GM_RESID) y = a.R[(size_t)b * a.ldr + lr] + s;
  if (sg) a.seg[1].Y[(size_t)b * a.seg[1].ldy + lr] = y;
  else a.seg[0].Y[(size_t)b * a.seg[0].ldy + lr] = y;
}

// Small batches (B <= 4 rows per workgroup): R x BT chain lanes (<= 64, one
// wave). The weights of a K chunk are loaded into registers, up to 16 float4
// a thread, all in flight at once (the next chunk's while the current one
// is being summed); the activations sit in LDS. With `ng` the workgroup
// first normalises its activation rows (M.norm, bend/Dense/Model.bend:27-30:
// ss = sum x*x in order, x * (1/sqrt(ss/K + 1e-5)) * g) while the first
// weights are still arriving. Every thread multiplies its weights by the
// activations and writes the products; lane c = b*R + r then adds its row's
// products in q order: bulk.c's ft_gemm_loop, one lane per output. With
// `amax` the outputs of segment 0 also compete for dd.pick's argmax.
template <int BT>
__global__ __launch_bounds__(256) void k_gemv_small(GemvArgs a, uint32_t R, uint32_t QC) {
  extern __shared__ float4 lds4[];
  const uint32_t Q4 = QC >> 2, PS4 = Q4 + 1;
  const uint32_t tid = threadIdx.x;
  const uint32_t b0 = blockIdx.y * BT;
  const uint32_t nb = min((uint32_t)BT, a.B - b0);
  const uint32_t Lc = R * BT;
  const uint32_t K = a.K;
  float4* Xs = lds4;                                      // [BT][Q4]
  float4* P = Xs + BT * Q4;                               // [Lc][PS4]
  float* outs = reinterpret_cast<float*>(P + Lc * PS4);  // [Lc, rounded up to 4]
  float* rs = outs + ((Lc + 3) & ~3u);                    // [4]
  float4* Xf = reinterpret_cast<float4*>(rs + 4);         // [BT][K/4] when ng

  const Segs sgs(a);
  // the residual a chain lane's output adds, loaded now rather than after
  // the chain (which would add a dependent memory round trip at the end)
  float res = 0.0f;
  if (a.mode == GM_RESID && tid < Lc) {
    const uint32_t b = tid / R, r = tid - b * R;
    const float* wp;
    uint32_t sg, lr;
    if (b < nb && sgs.row(R, blockIdx.x, r, &wp, &sg, &lr)) res = a.R[(size_t)(b0 + b) * a.ldr + lr];
  }
  float4 w[16];
  // weights of the chunk at q0 into w[]; item i = tid + 256 j is (row r, float4 q4)
  auto load_w = [&](uint32_t q0) {
    // branch-free, so the compiler keeps all 16 loads in flight (a load
    // inside a branch gets a full wait at the branch's end)
    const uint32_t qc4 = min(QC, K - q0) >> 2;
    const uint32_t dr = 256 / qc4, dq = 256 - dr * qc4;
    uint32_t r = tid / qc4, q4 = tid - r * qc4;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const float* wp;
      uint32_t sg, lr;
      const bool okr = sgs.row(R, blockIdx.x, r, &wp, &sg, &lr);
      const bool ok = (r < R) & okr;
      // an item outside the tile loads W0's first float4 instead: its
      // products belong to no stored output, so its value never matters
      const size_t off = ok ? (size_t)(wp - sgs.W0) + q0 + 4 * q4 : 0;
      w[j] = *reinterpret_cast<const float4*>(sgs.W0 + off);
      r += dr;
      q4 += dq;
      const uint32_t wrap = q4 >= qc4 ? 1u : 0u;
      q4 -= wrap * qc4;
      r += wrap;
    }
  };
  if (a.ng) {
    // the activation rows into LDS first, then the weights are issued and
    // the norm's chain runs while they arrive
    const uint32_t K4 = K >> 2, n4 = BT * K4;
    for (uint32_t i = tid; i < n4; i += 256) {
      const uint32_t b = i / K4, k4 = i - b * K4;
      float4 x = kZero4;
      if (b < nb) x = *reinterpret_cast<const float4*>(a.X + (size_t)(b0 + b) * a.ldx + 4 * k4);
      Xf[i] = x;
    }
    __syncthreads();
    load_w(0);
    if (tid < nb) rs[tid] = ex_rms_scale(chain_sumsq_lds(0.0f, reinterpret_cast<const float*>(Xf + tid * K4), K), (float)K);
    __syncthreads();
  } else {
    load_w(0);
  }
  float s = 0.0f;
  for (uint32_t q0 = 0; q0 < K; q0 += QC) {
    const uint32_t qc4 = min(QC, K - q0) >> 2;
    for (uint32_t i = tid; i < BT * qc4; i += 256) {
      const uint32_t b = i / qc4, q4 = i - b * qc4;
      float4 x = kZero4;
      if (b < nb) {
        if (a.ng) {
          const float4 v = Xf[b * (K >> 2) + (q0 >> 2) + q4];
          const float4 g = *reinterpret_cast<const float4*>(a.ng + q0 + 4 * q4);
          const float sc = rs[b];
          x = make_float4((v.x * sc) * g.x, (v.y * sc) * g.y, (v.z * sc) * g.z, (v.w * sc) * g.w);
        } else {
          x = *reinterpret_cast<const float4*>(a.X + (size_t)(b0 + b) * a.ldx + q0 + 4 * q4);
        }
      }
      Xs[b * Q4 + q4] = x;
    }
    __syncthreads();
    {
      const uint32_t dr = 256 / qc4, dq = 256 - dr * qc4;
      uint32_t r = tid / qc4, q4 = tid - r * qc4;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        if (r < R) {
#pragma unroll
          for (int b = 0; b < BT; b++) {
            const float4 x = Xs[b * Q4 + q4];
            P[(b * R + r) * PS4 + q4] = make_float4(x.x * w[j].x, x.y * w[j].y, x.z * w[j].z, x.w * w[j].w);
          }
        }
        r += dr;
        q4 += dq;
        if (q4 >= qc4) { q4 -= qc4; r++; }
      }
    }
    if (q0 + QC < K) load_w(q0 + QC);
    __syncthreads();
    if (tid < Lc) s = chain_sum_lds(s, reinterpret_cast<const float*>(P + tid * PS4), qc4 * 4);
    __syncthreads();
  }
  const uint32_t b = tid / R, r = tid - b * R;
  if (a.mode == GM_SILU) {
    if (tid < Lc) outs[tid] = s;
    __syncthreads();
    const uint32_t half = R >> 1;
    if (tid < Lc && r < half && b < nb) {
      const uint32_t j = blockIdx.x * half + r;
      // hh = silu(g) * u (bend/Dense/Model.bend:58-59)
      if (j < a.seg[0].rows)
        a.seg[0].Y[(size_t)(b0 + b) * a.seg[0].ldy + j] = ex_silu(s) * outs[b * R + r + half];
    }
    return;
  }
  if (tid < Lc && b < nb) {
    const float* wp;
    uint32_t sg, lr;
    if (sgs.row(R, blockIdx.x, r, &wp, &sg, &lr)) {
      // plain or plus the residual (add2 of bend/Dense/Model.bend:44-45)
      const float y = a.mode == GM_RESID ? res + s : s;
      if (sg) a.seg[1].Y[(size_t)(b0 + b) * a.seg[1].ldy + lr] = y;
      else a.seg[0].Y[(size_t)(b0 + b) * a.seg[0].ldy + lr] = y;
    }
  }
  if (a.amax && tid < 64) {
    // the workgroup's best key per batch row, then one atomic each
    unsigned long long key = 0;
    if (tid < Lc && b < nb) {
      const uint32_t vr = blockIdx.x * R + r;
      if (vr < a.seg[0].rows) key = argmax_key(s, vr);
    }
#pragma unroll
    for (int bb = 0; bb < BT; bb++) {
      unsigned long long k = (tid < Lc && b == (uint32_t)bb) ? key : 0ull;
      for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(k, m, 64);
        k = o > k ? o : k;
      }
      if (tid == 0 && (uint32_t)bb < nb && k) atomicMax(&a.amax[amax_at(b0 + bb, blockIdx.x % kAmaxSlots)], k);
    }
  }
}

// Larger batches (prefill chunks, batched decode): a tile of TR weight rows
// x TB batch rows per workgroup; thread (ti, tj) owns RI x BJ chains (rows
// ti*RI.., batch rows tj*BJ..). The K axis goes in chunks of KC. Every
// thread moves NL float4 of each chunk (weights and activations, coalesced
// along k) through a ring of D register sets, so D-1 chunks are in flight
// from HBM while one is added; a chunk is stored k-major into one of two
// LDS buffers, and each chain multiplies and adds in q order out of LDS:
// bulk.c's ft_gemm_loop, one lane per output. With `ng` the workgroup first
// runs M.norm's sum of squares for its TB rows (one in-order chain per row,
// while the first chunks are in flight) and stages (x * rs) * g.
template <int TR, int TB, int RI, int BJ, int KC, int D, int G>
__global__ __launch_bounds__(256) void k_gemm_exact(GemvArgs a) {
  constexpr int NJ = TB / BJ, NI = TR / RI;
  static_assert(NI * NJ == 256, "one chain block per thread");
  constexpr int K4 = KC / 4;
  constexpr int LW = TR * K4, LX = TB * K4, NL = (LW + LX + 255) / 256;
  static_assert(K4 % (2 * G) == 0, "whole read groups per chunk");
  __shared__ float4 Ws[2][K4][TR + 1];
  __shared__ float4 Xs[2][K4][TB + 1];
  __shared__ float rs[TB];
  __shared__ float outs[TB][TR + 1];
  const uint32_t tid = threadIdx.x;
  const uint32_t tj = tid % NJ, ti = tid / NJ;
  const uint32_t b0 = blockIdx.y * TB;
  const uint32_t nb = min((uint32_t)TB, a.B - b0);
  const Segs sgs(a);
  const bool norm = a.ng != nullptr;
  const uint32_t nch = (a.K + KC - 1) / KC;

  // the NL float4 this thread moves per chunk: item i = tid + 256 j;
  // i < LW: weight row i / K4, k4 = i % K4; else batch row (i-LW) / K4
  const float* src[NL];
  uint32_t dk4[NL], drow[NL];
  bool ok[NL];
#pragma unroll
  for (int j = 0; j < NL; j++) {
    const uint32_t i = tid + 256 * j;
    if (i < (uint32_t)LW) {
      const uint32_t r = i / K4;
      const float* w;
      uint32_t sg, lr;
      ok[j] = sgs.row(TR, blockIdx.x, r, &w, &sg, &lr);
      src[j] = ok[j] ? w : sgs.W0;
      dk4[j] = i % K4;
      drow[j] = r;
    } else {
      const uint32_t b = (i - LW) / K4;
      ok[j] = b < nb && i < (uint32_t)(LW + LX);
      src[j] = a.X + (size_t)(b0 + (ok[j] ? b : 0)) * a.ldx;
      dk4[j] = (i - LW) % K4;
      drow[j] = b;
    }
  }
  float4 v[D][NL];
  auto load = [&](float4 (&r)[NL], uint32_t c) {
#pragma unroll
    for (int j = 0; j < NL; j++) {
      const uint32_t q = c * KC + 4 * dk4[j];
      const bool in = ok[j] && q < a.K;
      // an unconditional load from a clamped address, so that it stays in
      // flight; items out of range are never added or stored, so they are
      // not zeroed (writing the destination would wait for the load)
      r[j] = *reinterpret_cast<const float4*>(src[j] + (in ? q : 0));
    }
  };
  auto store = [&](const float4 (&r)[NL], int buf, uint32_t c) {
#pragma unroll
    for (int j = 0; j < NL; j++) {
      const uint32_t i = tid + 256 * j;
      if (i < (uint32_t)LW) {
        Ws[buf][dk4[j]][drow[j]] = r[j];
      } else if (i < (uint32_t)(LW + LX)) {
        float4 x = r[j];
        if (norm) {
          const uint32_t q = c * KC + 4 * dk4[j];
          const float sc = rs[drow[j]];
          const float4 g = *reinterpret_cast<const float4*>(a.ng + (q < a.K ? q : 0));
          x.x = (x.x * sc) * g.x;
          x.y = (x.y * sc) * g.y;
          x.z = (x.z * sc) * g.z;
          x.w = (x.w * sc) * g.w;
        }
        Xs[buf][dk4[j]][drow[j]] = x;
      }
    }
  };

#pragma unroll
  for (int u = 0; u < D; u++)
    if ((uint32_t)u < nch) load(v[u], u);
  if (norm) {
    // M.norm (bend/Dense/Model.bend:27-30): ss = sum_q x_q * x_q in order,
    // one chain per batch row over the activations staged chunk by chunk
    // through the X buffers (the weights of the first chunks keep arriving)
    constexpr int PX = (LX + 255) / 256;
    float4 xr[2][PX];
    auto xload = [&](float4 (&r)[PX], uint32_t c) {
#pragma unroll
      for (int j = 0; j < PX; j++) {
        const uint32_t i = tid + 256 * j, b = i / K4, q = c * KC + 4 * (i % K4);
        const bool in = i < (uint32_t)LX && b < nb && q < a.K;
        r[j] = *reinterpret_cast<const float4*>(a.X + (size_t)(b0 + (in ? b : 0)) * a.ldx + (in ? q : 0));
      }
    };
    auto xstore = [&](const float4 (&r)[PX], int buf) {
#pragma unroll
      for (int j = 0; j < PX; j++) {
        const uint32_t i = tid + 256 * j;
        if (i < (uint32_t)LX) Xs[buf][i % K4][i / K4] = r[j];
      }
    };
    float ss = 0.0f;
    xload(xr[0], 0);
    xstore(xr[0], 0);
    __syncthreads();
    for (uint32_t c = 0; c < nch; c++) {
      const int bf = c & 1;
      if (c + 1 < nch) xload(xr[1], c + 1);
      if (tid < (uint32_t)TB) {
        const uint32_t n4 = min((uint32_t)K4, (a.K - c * KC) >> 2);
#pragma unroll 8
        for (uint32_t k4 = 0; k4 < n4; k4++) {
          const float4 x = Xs[bf][k4][tid];
          ss = ss + x.x * x.x;
          ss = ss + x.y * x.y;
          ss = ss + x.z * x.z;
          ss = ss + x.w * x.w;
        }
      }
      if (c + 1 < nch) xstore(xr[1], bf ^ 1);
      __syncthreads();
    }
    if (tid < (uint32_t)TB) rs[tid] = ex_rms_scale(ss, (float)a.K);
    __syncthreads();
  }
  store(v[0], 0, 0);
  __syncthreads();

  float s[RI][BJ];
#pragma unroll
  for (int i = 0; i < RI; i++)
#pragma unroll
    for (int j = 0; j < BJ; j++) s[i][j] = 0.0f;

  auto step = [&](const float4 (&w)[RI], const float4 (&x)[BJ]) {
#pragma unroll
    for (int i = 0; i < RI; i++)
#pragma unroll
      for (int j = 0; j < BJ; j++) s[i][j] = s[i][j] + x[j].x * w[i].x;
#pragma unroll
    for (int i = 0; i < RI; i++)
#pragma unroll
      for (int j = 0; j < BJ; j++) s[i][j] = s[i][j] + x[j].y * w[i].y;
#pragma unroll
    for (int i = 0; i < RI; i++)
#pragma unroll
      for (int j = 0; j < BJ; j++) s[i][j] = s[i][j] + x[j].z * w[i].z;
#pragma unroll
    for (int i = 0; i < RI; i++)
#pragma unroll
      for (int j = 0; j < BJ; j++) s[i][j] = s[i][j] + x[j].w * w[i].w;
  };
  // one chunk out of LDS buffer buf: groups of G k4 steps in two register
  // sets, the next group's reads issued before the current group adds
  auto chunk = [&](int buf, uint32_t n4) {
    float4 wa[G][RI], xa[G][BJ], wb[G][RI], xb[G][BJ];
    auto rd = [&](float4 (&w)[G][RI], float4 (&x)[G][BJ], uint32_t kb) {
#pragma unroll
      for (int u = 0; u < G; u++) {
#pragma unroll
        for (int i = 0; i < RI; i++) w[u][i] = Ws[buf][kb + u][ti * RI + i];
#pragma unroll
        for (int j = 0; j < BJ; j++) x[u][j] = Xs[buf][kb + u][tj * BJ + j];
      }
    };
    uint32_t k4 = 0;
    if (n4 >= 2 * G) {
      rd(wa, xa, 0);
      for (; k4 + 2 * G <= n4; k4 += 2 * G) {
        rd(wb, xb, k4 + G);
#pragma unroll
        for (int u = 0; u < G; u++) step(wa[u], xa[u]);
        const uint32_t kn = k4 + 2 * G <= (uint32_t)K4 - G ? k4 + 2 * G : 0;
        rd(wa, xa, kn);
#pragma unroll
        for (int u = 0; u < G; u++) step(wb[u], xb[u]);
      }
    }
    for (; k4 < n4; k4++) {
      float4 w[RI], x[BJ];
#pragma unroll
      for (int i = 0; i < RI; i++) w[i] = Ws[buf][k4][ti * RI + i];
#pragma unroll
      for (int j = 0; j < BJ; j++) x[j] = Xs[buf][k4][tj * BJ + j];
      step(w, x);
    }
  };

  // chunk c sits in LDS buffer c & 1 and (before that) in register set c % D
  for (uint32_t c0 = 0; c0 < nch; c0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const uint32_t c = c0 + u;
      if (c < nch) {
        chunk(c & 1, min((uint32_t)K4, (a.K - c * KC) >> 2));
        if (c + 1 < nch) store(v[(u + 1) % D], (c + 1) & 1, c + 1);
        if (c + D < nch) load(v[u], c + D);
        __syncthreads();
      }
    }
  }

  if (a.mode == GM_SILU) {
    // gate rows are tile rows [0, TR/2), their up rows TR/2 further
#pragma unroll
    for (int i = 0; i < RI; i++)
#pragma unroll
      for (int j = 0; j < BJ; j++) outs[tj * BJ + j][ti * RI + i] = s[i][j];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RI; i++) {
      const uint32_t r = ti * RI + i;
      const float* w;
      uint32_t sg, lr;
      if (r < (uint32_t)TR / 2 && sgs.row(TR, blockIdx.x, r, &w, &sg, &lr)) {
#pragma unroll
        for (int j = 0; j < BJ; j++) {
          const uint32_t b = tj * BJ + j;
          if (b < nb)
            a.seg[0].Y[(size_t)(b0 + b) * a.seg[0].ldy + lr] = ex_silu(s[i][j]) * outs[b][r + TR / 2];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < RI; i++) {
    const float* w;
    uint32_t sg, lr;
    if (sgs.row(TR, blockIdx.x, ti * RI + i, &w, &sg, &lr)) {
#pragma unroll
      for (int j = 0; j < BJ; j++) {
        const uint32_t b = tj * BJ + j;
        if (b < nb) gemv_store(a, sg, lr, b0 + b, s[i][j]);
      }
    }
  }
}

static size_t small_lds(uint32_t R, uint32_t BT, uint32_t QC, uint32_t K, bool norm) {
  const uint32_t Lc = R * BT, Lc4 = (Lc + 3) & ~3u;
  return (size_t)BT * (QC / 4) * 16 + (size_t)Lc * (QC / 4 + 1) * 16 + (size_t)Lc4 * 4 + 16 +
         (norm ? (size_t)BT * K * 4 + 16 : 0);
}

// tile sizing knobs (environment, read once): workgroups a small-batch
// product aims for, and its most rows per workgroup
static uint32_t env_u32(const char* name, uint32_t dflt) {
  const char* v = getenv(name);
  if (!v || !*v) return dflt;
  const unsigned long x = strtoul(v, nullptr, 10);
  return x ? (uint32_t)x : dflt;
}
static const uint32_t kTargetWgs = env_u32("ANA_GEMV_WGS", 256);
static const uint32_t kRmax = env_u32("ANA_GEMV_RMAX", 64);

// a launch, through hipExtLaunchKernelGGL when timing events are given
#define ANA_LAUNCH(K, GRID, BLOCK, LDS, ST, E0, E1, ...)                                 \
  do {                                                                                  \
    if (E0) hipExtLaunchKernelGGL(K, GRID, BLOCK, LDS, ST, E0, E1, 0, __VA_ARGS__);      \
    else hipLaunchKernelGGL(K, GRID, BLOCK, LDS, ST, __VA_ARGS__);                      \
  } while (0)

hipError_t launch_gemv(const GemvArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  if (a.B <= kSmallB) {
    const uint32_t BT = a.B <= 1 ? 1 : a.B <= 2 ? 2 : 4;
    // rows per workgroup: chain lanes fill (at most) one wave, and a wave
    // of chains costs the SIMD the same issue slots however few lanes it
    // has, so fewer, fuller workgroups win
    uint32_t R = rows / kTargetWgs;
    R = R < 1 ? 1 : R;
    uint32_t rmax = 64 / BT;
    rmax = rmax > kRmax ? kRmax : rmax;
    R = R > rmax ? rmax : R;
    if (a.mode == GM_SILU) R = R < 2 ? 2 : (R & ~1u);
    const uint32_t Lc = R * BT;
    uint32_t QC = a.K;
    const uint32_t fixed = 16 * Lc + 4 * ((Lc + 3) & ~3u) + 16 + (a.ng ? BT * a.K * 4 + 16 : 0);
    const uint32_t by_lds = (65536 - fixed) / (4 * (BT + Lc));
    const uint32_t by_regs = 16384 / R;
    QC = QC < by_lds ? QC : by_lds;
    QC = QC < by_regs ? QC : by_regs;
    QC &= ~3u;
    const uint32_t per = a.mode == GM_SILU ? R / 2 : R;
    const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
    dim3 grid(tiles, (a.B + BT - 1) / BT);
    const size_t lds = small_lds(R, BT, QC, a.K, a.ng != nullptr);
    if (QC < 4 || lds > 65536 || R * (QC / 4) > 16 * 256 || (a.ng && BT * a.K > 8192))
      return hipErrorInvalidValue;
    switch (BT) {
      case 1: ANA_LAUNCH(k_gemv_small<1>, grid, dim3(256), lds, st, e0, e1, a, R, QC); break;
      case 2: ANA_LAUNCH(k_gemv_small<2>, grid, dim3(256), lds, st, e0, e1, a, R, QC); break;
      default: ANA_LAUNCH(k_gemv_small<4>, grid, dim3(256), lds, st, e0, e1, a, R, QC); break;
    }
    return hipGetLastError();
  }
  if (a.amax) return hipErrorInvalidValue;  // batched products store logits instead
  if (a.ng && (a.K & 3)) return hipErrorInvalidValue;
  // one chain per thread over 16 x 16 tiles while that still leaves a few
  // workgroups per CU; 2 x 2 chains per thread over 32 x 32 tiles beyond
  const bool big = (uint64_t)rows * a.B >= 256ull * 1024;
  const uint32_t TR = big ? 32 : 16, TB = TR;
  const uint32_t per = a.mode == GM_SILU ? TR / 2 : TR;
  const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
  dim3 grid(tiles, (a.B + TB - 1) / TB);
  if (big) ANA_LAUNCH((k_gemm_exact<32, 32, 2, 2, 64, 3, 1>), grid, dim3(256), 0, st, e0, e1, a);
  else ANA_LAUNCH((k_gemm_exact<16, 16, 1, 1, 128, 4, 4>), grid, dim3(256), 0, st, e0, e1, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ norm

__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ X,
                                                 const float* __restrict__ g, uint32_t d,
                                                 float* __restrict__ Y) {
  extern __shared__ float4 xs4[];
  __shared__ float scale;
  const uint32_t tid = threadIdx.x, d4 = d >> 2;
  const float4* x = reinterpret_cast<const float4*>(X + (size_t)blockIdx.x * d);
  for (uint32_t i = tid; i < d4; i += 256) xs4[i] = x[i];
  __syncthreads();
  if (tid == 0) scale = ex_rms_scale(chain_sumsq_lds(0.0f, reinterpret_cast<const float*>(xs4), d), (float)d);
  __syncthreads();
  const float sc = scale;
  const float4* g4 = reinterpret_cast<const float4*>(g);
  float4* y = reinterpret_cast<float4*>(Y + (size_t)blockIdx.x * d);
  for (uint32_t i = tid; i < d4; i += 256) {
    const float4 v = xs4[i], gg = g4[i];
    y[i] = make_float4((v.x * sc) * gg.x, (v.y * sc) * gg.y, (v.z * sc) * gg.z, (v.w * sc) * gg.w);
  }
}

hipError_t launch_rmsnorm(const float* X, const float* g, uint32_t d, uint32_t B, float* Y,
                          hipStream_t st) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(B), dim3(256), (size_t)d * 4, st, X, g, d, Y);
  return hipGetLastError();
}

// ------------------------------------------------------------------ embed

__global__ void k_embed(const float* __restrict__ E, const uint32_t* __restrict__ tok, uint32_t d,
                        float* __restrict__ X, unsigned long long* amax) {
  const uint32_t b = blockIdx.x;
  if (amax && threadIdx.x < kAmaxSlots) amax[amax_at(b, threadIdx.x)] = 0ull;
  const float* src = E + (size_t)tok[b] * d;
  for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) X[(size_t)b * d + j] = src[j];
}

hipError_t launch_embed(const float* E, const uint32_t* tok, uint32_t d, uint32_t B, float* X,
                        unsigned long long* amax, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(B), dim3(256), 0, st, E, tok, d, X, amax);
  return hipGetLastError();
}

__global__ void k_bswap(uint32_t* w, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    w[i] = __builtin_bswap32(w[i]);
}

hipError_t launch_bswap(uint32_t* w, uint64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_bswap, dim3(4096), dim3(256), 0, st, w, n);
  return hipGetLastError();
}

// ------------------------------------------------------------------ GLA

// dd.gla's per-token part (bend/Dense/Decode.bend:252-266, 275-290) for one
// head: L2 norms (M.l2), the gate (dd.gate: RG-LRU or sigmoid), the state
// update S' = al*S + kh*v and the readout o = qh^T S' (no 1/sqrt(hd)).
// nT tokens run in order, S staying in LDS between them.
template <int HD>
__global__ __launch_bounds__(256) void k_gla(const float* __restrict__ QKV,
                                              const float* __restrict__ Z,
                                              const float* __restrict__ lam, StateRef S,
                                              const uint32_t* __restrict__ seq, uint32_t seq0,
                                              float* __restrict__ O, uint32_t d, uint32_t rglru,
                                              uint32_t nT) {
  constexpr int SP = HD + 1;
  constexpr int NE = (HD * HD + 255) / 256;
  __shared__ float q[HD], k[HD], v[HD], z[HD], al[HD], kh[HD], qh[HD], sq[2];
  __shared__ float Sl[HD * SP];
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const uint32_t sl = seq ? seq[b] : seq0;
  float* Sg = S.base + (size_t)sl * S.seq_stride + S.layer_off + (size_t)h * HD * HD;
#pragma unroll
  for (int j = 0; j < NE; j++) {
    const uint32_t e = tid + 256 * j;
    if (e < HD * HD) Sl[(e / HD) * SP + (e % HD)] = Sg[e];
  }
  for (uint32_t t = 0; t < nT; t++) {
    const uint32_t row = seq ? b : t;   // batch row (step) or token row (chunk)
    const float* x = QKV + (size_t)row * 3 * d;
    __syncthreads();
    if (tid < HD) {
      q[tid] = x[h * HD + tid];
      k[tid] = x[d + h * HD + tid];
      v[tid] = x[2 * d + h * HD + tid];
      z[tid] = Z[(size_t)row * d + h * HD + tid];
    }
    __syncthreads();
    if (tid == 0) sq[0] = chain_sumsq_lds(0.0f, q, HD);
    else if (tid == 64) sq[1] = chain_sumsq_lds(0.0f, k, HD);
    __syncthreads();
    if (tid < HD) {
      qh[tid] = q[tid] / csqrt(1.0e-6f + sq[0]);
      const float kn = k[tid] / csqrt(1.0e-6f + sq[1]);
      if (rglru) {
        const float la = ex_rglru_log_gate(z[tid], lam[h * HD + tid]);
        kh[tid] = kn * ex_rglru_write_scale(la);
        al[tid] = dexp(la);
      } else {
        al[tid] = ex_sigmoid(z[tid]);
        kh[tid] = kn;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NE; j++) {
      const uint32_t e = tid + 256 * j;
      if (e < HD * HD) {
        const uint32_t ia = e / HD, ib = e % HD;
        float* p = &Sl[ia * SP + ib];
        *p = (al[ia] * *p) + (kh[ia] * v[ib]);
      }
    }
    __syncthreads();
    if (tid < HD) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < HD; i++) acc = acc + qh[i] * Sl[i * SP + tid];
      O[(size_t)row * d + h * HD + tid] = acc;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NE; j++) {
    const uint32_t e = tid + 256 * j;
    if (e < HD * HD) Sg[e] = Sl[(e / HD) * SP + (e % HD)];
  }
}

// The same token step for one (head, sequence) of a decode step with
// hd = 64, on one wave: lane b keeps column b of the head's state in
// registers (loaded and stored one row of 64 consecutive floats at a time),
// so nothing of S goes through LDS and the only barriers are the two that
// publish q, k and the per-row gate values. Every value takes k_gla's
// operations in k_gla's order: the norms' chains over q and k (each lane
// runs them, from broadcast LDS reads), S' = (al_a * S) + (kh_a * v_b), and
// o_b = ((0 + qh_0 S'_0b) + qh_1 S'_1b) + ..., a ascending.
__global__ __launch_bounds__(64) void k_gla_w(const float* __restrict__ QKV, const float* __restrict__ Z,
                                              const float* __restrict__ lam, StateRef S,
                                              const uint32_t* __restrict__ seq, float* __restrict__ O,
                                              uint32_t d, uint32_t rglru) {
  constexpr int HD = 64;
  __shared__ __align__(16) float q[HD];
  __shared__ __align__(16) float k[HD];
  __shared__ float al[HD], kh[HD], qh[HD];
  const uint32_t h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  float* Sg = S.base + (size_t)seq[b] * S.seq_stride + S.layer_off + (size_t)h * HD * HD;
  const float* x = QKV + (size_t)b * 3 * d;
  const float qv = x[h * HD + lane], kv = x[d + h * HD + lane], vv = x[2 * d + h * HD + lane];
  const float zv = Z[(size_t)b * d + h * HD + lane];
  const float lv = rglru ? lam[h * HD + lane] : 0.0f;
  float s[HD];
#pragma unroll
  for (int a = 0; a < HD; a++) s[a] = Sg[a * HD + lane];
  q[lane] = qv;
  k[lane] = kv;
  __syncthreads();
  const float s0 = chain_sumsq_lds(0.0f, q, HD), s1 = chain_sumsq_lds(0.0f, k, HD);
  const float kn = kv / csqrt(1.0e-6f + s1);
  float alv, khv;
  if (rglru) {
    const float la = ex_rglru_log_gate(zv, lv);
    khv = kn * ex_rglru_write_scale(la);
    alv = dexp(la);
  } else {
    alv = ex_sigmoid(zv);
    khv = kn;
  }
  qh[lane] = qv / csqrt(1.0e-6f + s0);
  al[lane] = alv;
  kh[lane] = khv;
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int a = 0; a < HD; a++) {
    const float sa = (al[a] * s[a]) + (kh[a] * vv);
    Sg[a * HD + lane] = sa;
    acc = acc + qh[a] * sa;
  }
  O[(size_t)b * d + h * HD + lane] = acc;
}

#define ANA_HD_DISPATCH(HDV, LAUNCH) \
  switch (HDV) {                     \
    case 64: LAUNCH(64); break;      \
    case 32: LAUNCH(32); break;      \
    case 16: LAUNCH(16); break;      \
    default: return hipErrorInvalidValue; \
  }

hipError_t launch_gla_step(const float* QKV, const float* Z, const float* lam, StateRef S,
                           const uint32_t* seq, float* O, uint32_t d, uint32_t heads,
                           uint32_t rglru, uint32_t B, hipStream_t st) {
  if (d / heads == 64) {
    hipLaunchKernelGGL(k_gla_w, dim3(heads, B), dim3(64), 0, st, QKV, Z, lam, S, seq, O, d, rglru);
    return hipGetLastError();
  }
#define L_(H) hipLaunchKernelGGL(k_gla<H>, dim3(heads, B), dim3(256), 0, st, QKV, Z, lam, S, seq, 0u, O, d, rglru, 1u)
  ANA_HD_DISPATCH(d / heads, L_)
#undef L_
  return hipGetLastError();
}

hipError_t launch_gla_chunk(const float* QKV, const float* Z, const float* lam, float* Sbase,
                            float* O, uint32_t d, uint32_t heads, uint32_t rglru, uint32_t T,
                            hipStream_t st) {
  StateRef S{Sbase, 0, 0};
#define L_(H) hipLaunchKernelGGL(k_gla<H>, dim3(heads, 1), dim3(256), 0, st, QKV, Z, lam, S, (const uint32_t*)nullptr, 0u, O, d, rglru, T)
  ANA_HD_DISPATCH(d / heads, L_)
#undef L_
  return hipGetLastError();
}

// ------------------------------------------------------------------ softmax

__device__ __forceinline__ float wave_max_gt(float r) {
  // combine r = t > r ? t : r; partials are never NaN (a NaN never wins)
  for (int m = 32; m >= 1; m >>= 1) {
    const float t = __shfl_xor(r, m, 64);
    r = t > r ? t : r;
  }
  return r;
}

#define ATTN_TC 128

// dd.sm.attend (bend/Dense/Decode.bend:321-353) for one (row, head). With
// write_kv the row's k (qk-normed) and v go into slot pos mod ctx first
// (dd.sm.write) and the row reads its own slot from LDS; else every slot was
// written before. Scores over the live slots t' <= npos (each a chain over
// c), the masked max (with the sink), e = exp(sc*s - m), se = sum e in slot
// order, den (+ exp(sink - m)), oi = sum_t' e*V in slot order,
// o = (1/den) * oi. Masked slots are skipped: the reference adds exactly +0
// to each sum there (e = 0 and, with finite V, 0*V = +-0 to a sum that is
// never -0) and -inf to the max.
template <int HD>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
  extern __shared__ float dyn[];
  __shared__ float q[HD], kk[HD], vs[HD], red[4], nrm[2];
  constexpr int PS = ATTN_TC + 4;
  constexpr int NV = (ATTN_TC * HD / 4 + 255) / 256;
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const uint32_t d = a.d, ctx = a.ctx;
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t slot = pos % ctx, npos = pos < ctx - 1 ? pos : ctx - 1;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  float* Kr = a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off;
  float* Vr = Kr + (size_t)ctx * d;
  float* ss = dyn;                          // [ctx]: sc*s, then e
  float* P = dyn + ctx;                     // [HD][PS]
  const float* x = a.QKV + (size_t)b * 3 * d;
  const bool wkv = a.write_kv != 0;
  if (tid < HD) {
    q[tid] = x[h * HD + tid];
    if (wkv) {
      kk[tid] = x[d + h * HD + tid];
      vs[tid] = x[2 * d + h * HD + tid];
    }
  }
  __syncthreads();
  if (a.gq) {
    // M.qkn on q and k (bend/Dense/Model.bend:39-42), two chains at once
    if (tid == 0) nrm[0] = ex_rms_scale(chain_sumsq_lds(0.0f, q, HD), (float)HD);
    else if (tid == 64 && wkv) nrm[1] = ex_rms_scale(chain_sumsq_lds(0.0f, kk, HD), (float)HD);
    __syncthreads();
    if (tid < HD) {
      q[tid] = (q[tid] * nrm[0]) * (1.0f + a.gq[tid]);
      if (wkv) kk[tid] = (kk[tid] * nrm[1]) * (1.0f + a.gk[tid]);
    }
    __syncthreads();
  }
  if (wkv && tid < HD) {
    Kr[(size_t)slot * d + h * HD + tid] = kk[tid];
    Vr[(size_t)slot * d + h * HD + tid] = vs[tid];
  }
  float qr[HD];
#pragma unroll
  for (int c = 0; c < HD; c++) qr[c] = q[c];
  const float sc = 1.0f / csqrt((float)HD);
  // scores: s = sum_c q_c K[t'][c] (a gemm chain over c), kept as sc*s
  for (uint32_t t = tid; t <= npos; t += 256) {
    float acc = 0.0f;
    if (wkv && t == slot) {
#pragma unroll
      for (int c = 0; c < HD; c++) acc = acc + qr[c] * kk[c];
    } else {
      const float4* k4 = reinterpret_cast<const float4*>(Kr + (size_t)t * d + h * HD);
      float4 kv[HD / 4];
#pragma unroll
      for (int u = 0; u < HD / 4; u++) kv[u] = k4[u];
#pragma unroll
      for (int u = 0; u < HD / 4; u++) {
        acc = acc + qr[4 * u + 0] * kv[u].x;
        acc = acc + qr[4 * u + 1] * kv[u].y;
        acc = acc + qr[4 * u + 2] * kv[u].z;
        acc = acc + qr[4 * u + 3] * kv[u].w;
      }
    }
    ss[t] = sc * acc;
  }
  __syncthreads();
  float r = -INFINITY;
  for (uint32_t t = tid; t <= npos; t += 256) {
    const float y = ss[t];
    r = y > r ? y : r;
  }
  r = wave_max_gt(r);
  if ((tid & 63) == 0) red[tid >> 6] = r;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < 4; w++) m = red[w] > m ? red[w] : m;
  float sink = 0.0f;
  if (a.sink) {
    sink = a.sink[h];
    m = ex_max(m, sink);    // dd.sm.max: m1 < sink ? sink : m1
  }
  for (uint32_t t = tid; t <= npos; t += 256) ss[t] = dexp(ss[t] - m);
  __syncthreads();
  float oi = 0.0f, se = 0.0f;
  float4 vv[NV];
  auto load_v = [&](uint32_t t0) {
    const uint32_t tc = min((uint32_t)ATTN_TC, npos + 1 - t0);
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const uint32_t i = tid + 256 * j, t = i / (HD / 4), c4 = i % (HD / 4);
      vv[j] = kZero4;
      if (t < tc) {
        if (wkv && t0 + t == slot) vv[j] = *reinterpret_cast<const float4*>(&vs[4 * c4]);
        else vv[j] = *reinterpret_cast<const float4*>(Vr + (size_t)(t0 + t) * d + h * HD + 4 * c4);
      }
    }
  };
  load_v(0);
  for (uint32_t t0 = 0; t0 <= npos; t0 += ATTN_TC) {
    const uint32_t tc = min((uint32_t)ATTN_TC, npos + 1 - t0);
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const uint32_t i = tid + 256 * j, t = i / (HD / 4), c4 = i % (HD / 4);
      if (t < tc) {
        const float e = ss[t0 + t];
        P[(4 * c4 + 0) * PS + t] = e * vv[j].x;
        P[(4 * c4 + 1) * PS + t] = e * vv[j].y;
        P[(4 * c4 + 2) * PS + t] = e * vv[j].z;
        P[(4 * c4 + 3) * PS + t] = e * vv[j].w;
      }
    }
    if (t0 + ATTN_TC <= npos) load_v(t0 + ATTN_TC);
    __syncthreads();
    if (tid < HD) oi = chain_sum_lds(oi, P + tid * PS, tc);
    else if (tid == 64) se = chain_sum_lds(se, ss + t0, tc);
    __syncthreads();
  }
  if (tid == 64) red[0] = a.sink ? se + dexp(sink - m) : se;
  __syncthreads();
  if (tid < HD) a.O[(size_t)b * d + h * HD + tid] = (1.0f / red[0]) * oi;
}

// The same attention split over workgroups, for few rows at long context.
// Pass 1, per (head, block of kAttnTS slots, row): the row's write (by the
// block holding its slot), its scores sc*s into `ss` and the block's max
// into `pm`. Pass 2, per (head, 16 columns, row): m from the blocks' maxima
// (a max is exact in any order), then e = exp(sc*s - m), the products e*V
// and the in-order chains se and oi, slot block after slot block.
template <int HD>
__global__ __launch_bounds__(kAttnTS) void k_attn_scores(AttnArgs a) {
  __shared__ float q[HD], kk[HD], vs[HD], red[2], nrm[2];
  const uint32_t h = blockIdx.x, sb = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const uint32_t d = a.d, ctx = a.ctx, ns = (ctx + kAttnTS - 1) / kAttnTS;
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t slot = pos % ctx, npos = pos < ctx - 1 ? pos : ctx - 1;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  float* Kr = a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off;
  float* Vr = Kr + (size_t)ctx * d;
  const uint32_t t0 = sb * kAttnTS;
  float* pm = a.pm + ((size_t)b * a.heads + h) * ns;
  if (t0 > npos) {
    if (tid == 0) pm[sb] = -INFINITY;
    return;
  }
  const bool mine = a.write_kv && slot >= t0 && slot < t0 + kAttnTS;
  const float* x = a.QKV + (size_t)b * 3 * d;
  if (tid < HD) {
    q[tid] = x[h * HD + tid];
    if (mine) {
      kk[tid] = x[d + h * HD + tid];
      vs[tid] = x[2 * d + h * HD + tid];
    }
  }
  __syncthreads();
  if (a.gq) {
    if (tid == 0) nrm[0] = ex_rms_scale(chain_sumsq_lds(0.0f, q, HD), (float)HD);
    else if (tid == 64 && mine) nrm[1] = ex_rms_scale(chain_sumsq_lds(0.0f, kk, HD), (float)HD);
    __syncthreads();
    if (tid < HD) {
      q[tid] = (q[tid] * nrm[0]) * (1.0f + a.gq[tid]);
      if (mine) kk[tid] = (kk[tid] * nrm[1]) * (1.0f + a.gk[tid]);
    }
    __syncthreads();
  }
  if (mine && tid < HD) {
    Kr[(size_t)slot * d + h * HD + tid] = kk[tid];
    Vr[(size_t)slot * d + h * HD + tid] = vs[tid];
  }
  const float sc = 1.0f / csqrt((float)HD);
  const uint32_t t = t0 + tid;
  float y = -INFINITY;
  if (t <= npos) {
    float acc = 0.0f;
    if (mine && t == slot) {
#pragma unroll
      for (int c = 0; c < HD; c++) acc = acc + q[c] * kk[c];
    } else {
      const float4* k4 = reinterpret_cast<const float4*>(Kr + (size_t)t * d + h * HD);
      float4 kv[HD / 4];
#pragma unroll
      for (int u = 0; u < HD / 4; u++) kv[u] = k4[u];
#pragma unroll
      for (int u = 0; u < HD / 4; u++) {
        acc = acc + q[4 * u + 0] * kv[u].x;
        acc = acc + q[4 * u + 1] * kv[u].y;
        acc = acc + q[4 * u + 2] * kv[u].z;
        acc = acc + q[4 * u + 3] * kv[u].w;
      }
    }
    y = sc * acc;
    a.ss[((size_t)b * a.heads + h) * ctx + t] = y;
  }
  const float r = wave_max_gt(y);
  if ((tid & 63) == 0) red[tid >> 6] = r;
  __syncthreads();
  if (tid == 0) pm[sb] = red[1] > red[0] ? red[1] : red[0];
}

#define ATTN_CG 16
#define ATTN_TC2 256

template <int HD>
__global__ __launch_bounds__(256) void k_attn_out(AttnArgs a) {
  constexpr int PS = ATTN_TC2 + 4;
  __shared__ __align__(16) float es[ATTN_TC2];
  __shared__ __align__(16) float P[ATTN_CG * PS];
  __shared__ float red[1];
  const uint32_t h = blockIdx.x, cg = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const uint32_t d = a.d, ctx = a.ctx, ns = (ctx + kAttnTS - 1) / kAttnTS;
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t npos = pos < ctx - 1 ? pos : ctx - 1;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  const float* Vr = a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off + (size_t)ctx * d;
  const float* ssr = a.ss + ((size_t)b * a.heads + h) * ctx;
  const float* pm = a.pm + ((size_t)b * a.heads + h) * ns;
  float m = -INFINITY;
  for (uint32_t i = 0; i <= npos / kAttnTS; i++) m = pm[i] > m ? pm[i] : m;
  float sink = 0.0f;
  if (a.sink) {
    sink = a.sink[h];
    m = ex_max(m, sink);    // dd.sm.max: m1 < sink ? sink : m1
  }
  const uint32_t c0 = cg * ATTN_CG;
  float oi = 0.0f, se = 0.0f;
  // V for a chunk: items (t, float4 c4) of this column group, 4 a thread
  constexpr int NV = ATTN_TC2 * (ATTN_CG / 4) / 256;
  float4 vv[NV];
  float sv = 0.0f;
  auto load = [&](uint32_t t0) {
    const uint32_t tc = min((uint32_t)ATTN_TC2, npos + 1 - t0);
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const uint32_t i = tid + 256 * j, t = i / (ATTN_CG / 4), c4 = i % (ATTN_CG / 4);
      const uint32_t tt = t < tc ? t0 + t : t0;
      vv[j] = *reinterpret_cast<const float4*>(Vr + (size_t)tt * d + h * HD + c0 + 4 * c4);
    }
    sv = tid < tc ? ssr[t0 + tid] : 0.0f;
  };
  load(0);
  for (uint32_t t0 = 0; t0 <= npos; t0 += ATTN_TC2) {
    const uint32_t tc = min((uint32_t)ATTN_TC2, npos + 1 - t0);
    if (tid < tc) es[tid] = dexp(sv - m);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const uint32_t i = tid + 256 * j, t = i / (ATTN_CG / 4), c4 = i % (ATTN_CG / 4);
      if (t < tc) {
        const float e = es[t];
        P[(4 * c4 + 0) * PS + t] = e * vv[j].x;
        P[(4 * c4 + 1) * PS + t] = e * vv[j].y;
        P[(4 * c4 + 2) * PS + t] = e * vv[j].z;
        P[(4 * c4 + 3) * PS + t] = e * vv[j].w;
      }
    }
    if (t0 + ATTN_TC2 <= npos) load(t0 + ATTN_TC2);
    __syncthreads();
    if (tid < ATTN_CG) oi = chain_sum_lds(oi, P + tid * PS, tc);
    else if (tid == 64) se = chain_sum_lds(se, es, tc);
    __syncthreads();
  }
  if (tid == 64) red[0] = a.sink ? se + dexp(sink - m) : se;
  __syncthreads();
  if (tid < ATTN_CG) a.O[(size_t)b * d + h * HD + c0 + tid] = (1.0f / red[0]) * oi;
}

// From kAttnWideB rows on, one workgroup per (head, row) (k_attn) keeps
// every CU busy, and the split kernels would dispatch ctx / kAttnTS score
// blocks per (head, row) whatever the row's position.
constexpr uint32_t kAttnWideB = 8;

hipError_t launch_attn(const AttnArgs& a, hipStream_t st) {
  const uint32_t hd = a.d / a.heads;
  if (a.ss && a.pm && hd % ATTN_CG == 0 && a.B < kAttnWideB) {
    if (a.B > a.ss_rows) return hipErrorInvalidValue;
    const uint32_t ns = (a.ctx + kAttnTS - 1) / kAttnTS;
#define L_(H)                                                                                   \
  hipLaunchKernelGGL(k_attn_scores<H>, dim3(a.heads, ns, a.B), dim3(kAttnTS), 0, st, a);      \
  hipLaunchKernelGGL(k_attn_out<H>, dim3(a.heads, H / ATTN_CG, a.B), dim3(256), 0, st, a)
    ANA_HD_DISPATCH(hd, L_)
#undef L_
    return hipGetLastError();
  }
  const size_t lds = ((size_t)a.ctx + (size_t)hd * (ATTN_TC + 4)) * 4;
#define L_(H) hipLaunchKernelGGL(k_attn<H>, dim3(a.heads, a.B), dim3(256), lds, st, a)
  ANA_HD_DISPATCH(hd, L_)
#undef L_
  return hipGetLastError();
}

// dd.sm.write (bend/Dense/Decode.bend:295-304): row b's k (after qk-norm
// when on) and v into slot pos mod ctx of its sequence's rings
template <int HD>
__global__ __launch_bounds__(64) void k_kv_write(AttnArgs a) {
  __shared__ float k[HD], nrm;
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const uint32_t d = a.d;
  const float* x = a.QKV + (size_t)b * 3 * d;
  if (tid < HD) k[tid] = x[d + h * HD + tid];
  __syncthreads();
  if (a.gk) {
    if (tid == 0) nrm = ex_rms_scale(chain_sumsq_lds(0.0f, k, HD), (float)HD);
    __syncthreads();
    if (tid < HD) k[tid] = (k[tid] * nrm) * (1.0f + a.gk[tid]);
  }
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t slot = pos % a.ctx;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  float* Kr = a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off;
  if (tid < HD) {
    Kr[(size_t)slot * d + h * HD + tid] = k[tid];
    Kr[(size_t)a.ctx * d + (size_t)slot * d + h * HD + tid] = x[2 * d + h * HD + tid];
  }
}

hipError_t launch_kv_write(const AttnArgs& a, hipStream_t st) {
#define L_(H) hipLaunchKernelGGL(k_kv_write<H>, dim3(a.heads, a.B), dim3(64), 0, st, a)
  ANA_HD_DISPATCH(a.d / a.heads, L_)
#undef L_
  return hipGetLastError();
}

// ------------------------------------------------------------------ pick

// dd.pick (bend/Dense/Decode.bend:481-484): top = max l_i (t > r ? t : r
// from -inf), then the least i with top <= l_i; vocab when there is none.
__global__ __launch_bounds__(1024) void k_top(const float* __restrict__ lg, uint32_t v,
                                              uint32_t* __restrict__ tok) {
  __shared__ float redf[16];
  __shared__ uint32_t redu[16];
  const uint32_t b = blockIdx.x, tid = threadIdx.x;
  const float* x = lg + (size_t)b * v;
  float r = -INFINITY;
  for (uint32_t i = tid; i < v; i += 1024) r = x[i] > r ? x[i] : r;
  r = wave_max_gt(r);
  if ((tid & 63) == 0) redf[tid >> 6] = r;
  __syncthreads();
  float top = redf[0];
  for (int w = 1; w < 16; w++) top = redf[w] > top ? redf[w] : top;
  uint32_t best = v;
  for (uint32_t i = tid; i < v; i += 1024)
    if (top <= x[i]) { best = i; break; }
  for (int m = 32; m >= 1; m >>= 1) {
    const uint32_t o = __shfl_xor(best, m, 64);
    best = o < best ? o : best;
  }
  if ((tid & 63) == 0) redu[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    uint32_t bb = redu[0];
    for (int w = 1; w < 16; w++) bb = redu[w] < bb ? redu[w] : bb;
    tok[b] = bb;
  }
}

hipError_t launch_top(const float* logits, uint32_t vocab, uint32_t B, uint32_t* tok,
                      hipStream_t st) {
  hipLaunchKernelGGL(k_top, dim3(B), dim3(1024), 0, st, logits, vocab, tok);
  return hipGetLastError();
}

// ------------------------------------------------------------------ helpers

__global__ void k_rows(const float* __restrict__ src, const uint32_t* __restrict__ idx, uint32_t d,
                       float* __restrict__ dst, int gather) {
  const uint32_t b = blockIdx.x;
  const float* s = src + (size_t)(gather ? idx[b] : b) * d;
  float* t = dst + (size_t)(gather ? b : idx[b]) * d;
  for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) t[j] = s[j];
}

hipError_t launch_gather_rows(const float* src, const uint32_t* idx, uint32_t n, uint32_t d,
                              float* dst, hipStream_t st) {
  hipLaunchKernelGGL(k_rows, dim3(n), dim3(256), 0, st, src, idx, d, dst, 1);
  return hipGetLastError();
}

hipError_t launch_scatter_rows(const float* src, const uint32_t* idx, uint32_t n, uint32_t d,
                               float* dst, hipStream_t st) {
  hipLaunchKernelGGL(k_rows, dim3(n), dim3(256), 0, st, src, idx, d, dst, 0);
  return hipGetLastError();
}

// dst row pairs[2 b + 1] = src row pairs[2 b], for every b < n
__global__ void k_copy_rows(const float* __restrict__ src, const uint32_t* __restrict__ pairs, uint32_t d,
                            float* __restrict__ dst) {
  const uint32_t b = blockIdx.x;
  const float* s = src + (size_t)pairs[2 * b] * d;
  float* t = dst + (size_t)pairs[2 * b + 1] * d;
  for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) t[j] = s[j];
}

hipError_t launch_copy_rows(const float* src, const uint32_t* pairs, uint32_t n, uint32_t d, float* dst,
                            hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_copy_rows, dim3(n), dim3(256), 0, st, src, pairs, d, dst);
  return hipGetLastError();
}

__global__ void k_zero(float* p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

hipError_t launch_zero(float* p, uint64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_zero, dim3(2048), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

__global__ void k_zero_u32(uint32_t* p, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

hipError_t launch_zero_u32(uint32_t* p, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_zero_u32, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

__global__ void k_zero_u64(unsigned long long* p, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0ull;
}

hipError_t launch_zero_u64(unsigned long long* p, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_zero_u64, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

__global__ void k_keys_to_tok(const unsigned long long* amax, uint32_t vocab, uint32_t B, uint32_t* tok) {
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  unsigned long long k = 0;
  for (uint32_t s = 0; s < kAmaxSlots; s++) k = amax[amax_at(b, s)] > k ? amax[amax_at(b, s)] : k;
  tok[b] = k ? 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull) : vocab;
}

hipError_t launch_keys_to_tok(const unsigned long long* amax, uint32_t vocab, uint32_t B,
                              uint32_t* tok, hipStream_t st) {
  hipLaunchKernelGGL(k_keys_to_tok, dim3((B + 255) / 256), dim3(256), 0, st, amax, vocab, B, tok);
  return hipGetLastError();
}

}  // namespace ana

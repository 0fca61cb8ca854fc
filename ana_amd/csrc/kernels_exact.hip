// Exact-fp32 decode kernels for gfx950.
//
// Every output takes the F32 steps the reference's CPU kernels take
// (bend/effs/bulk.c:49-71 for products, 979-1088 for einsums): sums run in
// index order from 0.0f, a product and the sum it joins are two roundings
// (this file is compiled with -ffp-contract=off and the pragma below),
// exp/log go through double and are rounded to float, sqrt and division are
// the correctly rounded IEEE operations. Parallelism is only ever across
// outputs (rows, heads, sequences); each reduction chain stays in one lane.
#include "ana_internal.h"
#include "numerics.h"

#pragma clang fp contract(off)

namespace ana {

// ------------------------------------------------------------------ products

// Row pointer and output slot for tile row r of workgroup tile t.
__device__ __forceinline__ bool gemv_row(const GemvArgs& a, uint32_t t, uint32_t r,
                                         const float** w, uint32_t* seg, uint32_t* lr) {
  if (a.mode == GM_SILU) {
    const uint32_t half = a.rows_wg >> 1;
    const uint32_t s = r < half ? 0u : 1u;
    const uint32_t j = t * half + (s ? r - half : r);
    if (j >= a.seg[s].rows) return false;
    *w = a.seg[s].W + (size_t)j * a.K;
    *seg = s;
    *lr = j;
    return true;
  }
  const uint32_t vr = t * a.rows_wg + r;
  uint32_t s = 0, j = vr;
  if (j >= a.seg[0].rows) {
    j -= a.seg[0].rows;
    s = 1;
    if (a.nseg < 2 || j >= a.seg[1].rows) return false;
  }
  *w = a.seg[s].W + (size_t)j * a.K;
  *seg = s;
  *lr = j;
  return true;
}

// One workgroup: rows_wg output rows x bt batch rows. Per K chunk the
// weights and the (normalised) activations are staged in LDS, every thread
// forms products x*w, and lane c = b*rows_wg + r adds its row's products in
// q order: the chain of bulk.c's ft_gemm_loop, one lane per output.
__global__ __launch_bounds__(256) void k_gemv_exact(GemvArgs a) {
  extern __shared__ float4 lds4[];
  const uint32_t R = a.rows_wg, BT = a.bt, QC = a.qc, K = a.K;
  const uint32_t Q4 = QC >> 2;
  const uint32_t tid = threadIdx.x;
  const uint32_t b0 = blockIdx.y * BT;
  const uint32_t nb = min(BT, a.B - b0);
  const uint32_t Lc = R * BT;
  float4* Ws = lds4;                          // [R][Q4]
  float4* Xs = Ws + R * Q4;                   // [BT][Q4]
  float4* P = Xs + BT * Q4;                   // [Lc][Q4 + 1]
  float* rs = reinterpret_cast<float*>(P + Lc * (Q4 + 1));  // [BT]
  float* outs = rs + BT;                      // [Lc]

  // RMSNorm prologue (M.norm, bend/Dense/Model.bend:27-30): ss = sum x*x in
  // j order, scale = 1 / sqrt(ss / K + 1e-5)
  if (a.ng) {
    if (tid < nb) {
      const float4* x = reinterpret_cast<const float4*>(a.X + (size_t)(b0 + tid) * a.ldx);
      float ss = 0.0f;
      for (uint32_t j = 0; j < (K >> 2); j++) {
        const float4 v = x[j];
        ss = ss + v.x * v.x;
        ss = ss + v.y * v.y;
        ss = ss + v.z * v.z;
        ss = ss + v.w * v.w;
      }
      rs[tid] = ex_rms_scale(ss, (float)K);
    }
    __syncthreads();
  }

  float s = 0.0f;
  for (uint32_t q0 = 0; q0 < K; q0 += QC) {
    const uint32_t qc4 = (min(QC, K - q0)) >> 2;
    for (uint32_t i = tid; i < R * qc4; i += 256) {
      const uint32_t r = i / qc4, q4 = i - r * qc4;
      const float* wp;
      uint32_t sg, lr;
      float4 w = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (gemv_row(a, blockIdx.x, r, &wp, &sg, &lr))
        w = *reinterpret_cast<const float4*>(wp + q0 + 4 * q4);
      Ws[r * Q4 + q4] = w;
    }
    for (uint32_t i = tid; i < BT * qc4; i += 256) {
      const uint32_t b = i / qc4, q4 = i - b * qc4;
      float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (b < nb) {
        x = *reinterpret_cast<const float4*>(a.X + (size_t)(b0 + b) * a.ldx + q0 + 4 * q4);
        if (a.ng) {
          const float sc = rs[b];
          const float4 g = *reinterpret_cast<const float4*>(a.ng + q0 + 4 * q4);
          x.x = (x.x * sc) * g.x;
          x.y = (x.y * sc) * g.y;
          x.z = (x.z * sc) * g.z;
          x.w = (x.w * sc) * g.w;
        }
      }
      Xs[b * Q4 + q4] = x;
    }
    __syncthreads();
    for (uint32_t i = tid; i < Lc * qc4; i += 256) {
      const uint32_t c = i / qc4, q4 = i - c * qc4;
      const uint32_t b = c / R, r = c - b * R;
      const float4 x = Xs[b * Q4 + q4], w = Ws[r * Q4 + q4];
      P[c * (Q4 + 1) + q4] = make_float4(x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w);
    }
    __syncthreads();
    if (tid < Lc) {
      const float4* p = P + tid * (Q4 + 1);
      for (uint32_t q4 = 0; q4 < qc4; q4++) {
        const float4 v = p[q4];
        s = s + v.x;
        s = s + v.y;
        s = s + v.z;
        s = s + v.w;
      }
    }
    __syncthreads();
  }

  if (a.mode == GM_SILU) {
    if (tid < Lc) outs[tid] = s;
    __syncthreads();
    const uint32_t half = R >> 1;
    if (tid < Lc) {
      const uint32_t b = tid / R, r = tid - b * R;
      if (r < half && b < nb) {
        const uint32_t j = blockIdx.x * half + r;
        if (j < a.seg[0].rows) {
          // hh = silu(g) * u (bend/Dense/Model.bend:58-59)
          const float u = outs[b * R + r + half];
          a.seg[0].Y[(size_t)(b0 + b) * a.seg[0].ldy + j] = ex_silu(s) * u;
        }
      }
    }
    return;
  }
  if (tid < Lc) {
    const uint32_t b = tid / R, r = tid - b * R;
    const float* wp;
    uint32_t sg, lr;
    if (b < nb && gemv_row(a, blockIdx.x, r, &wp, &sg, &lr)) {
      float y = s;
      if (a.mode == GM_RESID) y = a.R[(size_t)(b0 + b) * a.ldr + lr] + s;
      a.seg[sg].Y[(size_t)(b0 + b) * a.seg[sg].ldy + lr] = y;
    }
  }
}

static size_t gemv_lds(uint32_t R, uint32_t BT, uint32_t QC) {
  const uint32_t Q4 = QC / 4, Lc = R * BT;
  return ((size_t)R * Q4 + (size_t)BT * Q4 + (size_t)Lc * (Q4 + 1)) * 16 + (BT + Lc) * 4;
}

void gemv_shape(uint32_t rows, uint32_t K, uint32_t B, uint32_t mode, GemvArgs* a) {
  // batch rows per workgroup, then rows per workgroup so that a launch has
  // about 256+ workgroups (one per CU) while R*BT chain lanes stay <= 256
  const uint32_t BT = B <= 64 ? B : 64;
  uint32_t tiles_b = (B + BT - 1) / BT;
  uint32_t R = 256 / BT;
  uint32_t want = rows / (256 / tiles_b > 0 ? 256 / tiles_b : 1);
  if (want < 1) want = 1;
  if (R > want) R = want;
  if (R > 64) R = 64;
  if (mode == GM_SILU) {
    R = R < 2 ? 2 : (R & ~1u);
    if (R * BT > 256) R = (256 / BT) & ~1u;
    if (R < 2) R = 2;
  }
  // K chunk: as large as fits 64 KB of LDS
  uint32_t QC = K;
  while (QC > 4 && gemv_lds(R, BT, QC) > 65536) QC = ((QC / 2) + 3) & ~3u;
  a->rows_wg = R;
  a->bt = BT;
  a->qc = QC;
}

hipError_t launch_gemv(const GemvArgs& a0, hipStream_t st) {
  GemvArgs a = a0;
  uint32_t rows = a.mode == GM_SILU ? a.seg[0].rows * 2 : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  if (a.rows_wg == 0) gemv_shape(rows, a.K, a.B, a.mode, &a);
  const uint32_t per = a.mode == GM_SILU ? a.rows_wg / 2 : a.rows_wg;
  const uint32_t tiles = a.mode == GM_SILU ? (a.seg[0].rows + per - 1) / per : (rows + per - 1) / per;
  dim3 grid(tiles, (a.B + a.bt - 1) / a.bt);
  hipLaunchKernelGGL(k_gemv_exact, grid, dim3(256), gemv_lds(a.rows_wg, a.bt, a.qc), st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ embed

__global__ void k_embed(const float* __restrict__ E, const uint32_t* __restrict__ tok, uint32_t d,
                        float* __restrict__ X) {
  const uint32_t b = blockIdx.x;
  const float* src = E + (size_t)tok[b] * d;
  for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) X[(size_t)b * d + j] = src[j];
}

hipError_t launch_embed(const float* E, const uint32_t* tok, uint32_t d, uint32_t B, float* X,
                        hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(B), dim3(256), 0, st, E, tok, d, X);
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
__global__ __launch_bounds__(256) void k_gla(const float* __restrict__ QKV,
                                              const float* __restrict__ Z,
                                              const float* __restrict__ lam, StateRef S,
                                              const uint32_t* __restrict__ seq, uint32_t seq0,
                                              float* __restrict__ O, uint32_t d, uint32_t hd,
                                              uint32_t rglru, uint32_t nT) {
  __shared__ float q[64], k[64], v[64], z[64], al[64], kh[64], qh[64], sq[2];
  __shared__ float Sl[64 * 65];
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const uint32_t sl = seq ? seq[b] : seq0;
  float* Sg = S.base + (size_t)sl * S.seq_stride + S.layer_off + (size_t)h * hd * hd;
  const uint32_t hh2 = hd * hd;
  for (uint32_t e = tid; e < hh2; e += 256) Sl[(e / hd) * 65 + (e % hd)] = Sg[e];
  for (uint32_t t = 0; t < nT; t++) {
    const uint32_t row = seq ? b : t;   // batch row (step) or token row (chunk)
    const float* x = QKV + (size_t)row * 3 * d;
    __syncthreads();
    if (tid < hd) {
      q[tid] = x[h * hd + tid];
      k[tid] = x[d + h * hd + tid];
      v[tid] = x[2 * d + h * hd + tid];
      z[tid] = Z[(size_t)row * d + h * hd + tid];
    }
    __syncthreads();
    if (tid == 0) {
      float s = 0.0f;
      for (uint32_t i = 0; i < hd; i++) s = s + q[i] * q[i];
      sq[0] = s;
    } else if (tid == 64) {
      float s = 0.0f;
      for (uint32_t i = 0; i < hd; i++) s = s + k[i] * k[i];
      sq[1] = s;
    }
    __syncthreads();
    if (tid < hd) {
      qh[tid] = q[tid] / csqrt(1.0e-6f + sq[0]);
      const float kn = k[tid] / csqrt(1.0e-6f + sq[1]);
      if (rglru) {
        const float la = ex_rglru_log_gate(z[tid], lam[h * hd + tid]);
        kh[tid] = kn * ex_rglru_write_scale(la);
        al[tid] = dexp(la);
      } else {
        al[tid] = ex_sigmoid(z[tid]);
        kh[tid] = kn;
      }
    }
    __syncthreads();
    for (uint32_t e = tid; e < hh2; e += 256) {
      const uint32_t ia = e / hd, ib = e - ia * hd;
      float* p = &Sl[ia * 65 + ib];
      *p = (al[ia] * *p) + (kh[ia] * v[ib]);
    }
    __syncthreads();
    if (tid < hd) {
      float acc = 0.0f;
      for (uint32_t i = 0; i < hd; i++) acc = acc + qh[i] * Sl[i * 65 + tid];
      O[(size_t)row * d + h * hd + tid] = acc;
    }
  }
  __syncthreads();
  for (uint32_t e = tid; e < hh2; e += 256) Sg[e] = Sl[(e / hd) * 65 + (e % hd)];
}

hipError_t launch_gla_step(const float* QKV, const float* Z, const float* lam, StateRef S,
                           const uint32_t* seq, float* O, uint32_t d, uint32_t heads,
                           uint32_t rglru, uint32_t B, hipStream_t st) {
  hipLaunchKernelGGL(k_gla, dim3(heads, B), dim3(256), 0, st, QKV, Z, lam, S, seq, 0u, O, d,
                     d / heads, rglru, 1u);
  return hipGetLastError();
}

hipError_t launch_gla_chunk(const float* QKV, const float* Z, const float* lam, float* Sbase,
                            float* O, uint32_t d, uint32_t heads, uint32_t rglru, uint32_t T,
                            hipStream_t st) {
  StateRef S{Sbase, 0, 0};
  hipLaunchKernelGGL(k_gla, dim3(heads, 1), dim3(256), 0, st, QKV, Z, lam, S,
                     (const uint32_t*)nullptr, 0u, O, d, d / heads, rglru, T);
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

// qk-norm for one head (M.qkn, bend/Dense/Model.bend:39-42), in place;
// lanes < hd hold x, the chain runs in lane `chain`.
__device__ __forceinline__ void qk_norm(float* x, const float* g, uint32_t hd, float* ssum,
                                        uint32_t tid, uint32_t chain) {
  if (tid == chain) {
    float s = 0.0f;
    for (uint32_t i = 0; i < hd; i++) s = s + x[i] * x[i];
    *ssum = ex_rms_scale(s, (float)hd);
  }
  __syncthreads();
  if (tid < hd) x[tid] = (x[tid] * *ssum) * (1.0f + g[tid]);
  __syncthreads();
}

#define ATTN_TC 128

// dd.sm.attend (bend/Dense/Decode.bend:321-353) for one (row, head): scores
// over the live slots t' <= npos, the masked max (with the sink), exp,
// se = sum e in slot order, den (+ exp(sink - m)), oi = sum_t' e*V in slot
// order, o = (1/den) * oi. Masked slots are skipped: the reference adds
// exactly +0 to each sum there (e = 0 and, with finite V, 0*V = +-0 to a
// sum that is never -0) and -inf to the max.
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
  extern __shared__ float dyn[];
  __shared__ float q[64], k[64], v[64], red[4], nrm[2];
  const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const uint32_t d = a.d, hd = d / a.heads, ctx = a.ctx;
  const uint32_t pos = a.pos ? a.pos[b] : a.pos0 + b;
  const uint32_t slot = pos % ctx, npos = pos < ctx - 1 ? pos : ctx - 1;
  const uint32_t sl = a.seq ? a.seq[b] : a.seq0;
  float* Kr = a.KV.base + (size_t)sl * a.KV.seq_stride + a.KV.layer_off;
  float* Vr = Kr + (size_t)ctx * d;
  float* ss = dyn;                          // [ctx]: sc*s, then e
  float* P = dyn + ctx;                     // [hd][ATTN_TC + 4]
  const float* x = a.QKV + (size_t)b * 3 * d;
  if (tid < hd) {
    q[tid] = x[h * hd + tid];
    k[tid] = x[d + h * hd + tid];
    v[tid] = x[2 * d + h * hd + tid];
  }
  __syncthreads();
  if (a.gq) {
    qk_norm(q, a.gq, hd, &nrm[0], tid, 0);
    if (a.write_kv) qk_norm(k, a.gk, hd, &nrm[1], tid, 64);
  }
  if (a.write_kv && tid < hd) {
    Kr[(size_t)slot * d + h * hd + tid] = k[tid];
    Vr[(size_t)slot * d + h * hd + tid] = v[tid];
  }
  const float sc = 1.0f / csqrt((float)hd);
  // scores: s = sum_c q_c K[t'][c] (a gemm chain over c), kept as sc*s
  for (uint32_t t = tid; t <= npos; t += 256) {
    const float* kr = (a.write_kv && t == slot) ? k : Kr + (size_t)t * d + h * hd;
    float acc = 0.0f;
    for (uint32_t c = 0; c < hd; c++) acc = acc + q[c] * kr[c];
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
  const uint32_t PS = ATTN_TC + 4;
  for (uint32_t t0 = 0; t0 <= npos; t0 += ATTN_TC) {
    const uint32_t tc = min((uint32_t)ATTN_TC, npos + 1 - t0);
    for (uint32_t i = tid; i < tc * hd; i += 256) {
      const uint32_t t = i / hd, c = i - t * hd, tt = t0 + t;
      const float vv = (a.write_kv && tt == slot) ? v[c] : Vr[(size_t)tt * d + h * hd + c];
      P[c * PS + t] = ss[tt] * vv;
    }
    __syncthreads();
    if (tid < hd) {
      const float* p = P + tid * PS;
      uint32_t t = 0;
      for (; t + 4 <= tc; t += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(p + t);
        oi = oi + w4.x;
        oi = oi + w4.y;
        oi = oi + w4.z;
        oi = oi + w4.w;
      }
      for (; t < tc; t++) oi = oi + p[t];
    } else if (tid == 64) {
      for (uint32_t t = 0; t < tc; t++) se = se + ss[t0 + t];
    }
    __syncthreads();
  }
  if (tid == 64) red[0] = a.sink ? se + dexp(sink - m) : se;
  __syncthreads();
  if (tid < hd) a.O[(size_t)b * d + h * hd + tid] = (1.0f / red[0]) * oi;
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t st) {
  const size_t lds = ((size_t)a.ctx + (size_t)(a.d / a.heads) * (ATTN_TC + 4)) * 4;
  hipLaunchKernelGGL(k_attn, dim3(a.heads, a.B), dim3(256), lds, st, a);
  return hipGetLastError();
}

// a chunk's k (qk-normed) and v into their slots (dd.sm.writes)
__global__ __launch_bounds__(64) void k_kv_write(const float* __restrict__ QKV,
                                                 const float* __restrict__ gk, StateRef KV,
                                                 uint32_t seq, uint32_t pos0, uint32_t d,
                                                 uint32_t hd, uint32_t ctx) {
  __shared__ float k[64], nrm;
  const uint32_t h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const float* x = QKV + (size_t)t * 3 * d;
  if (tid < hd) k[tid] = x[d + h * hd + tid];
  __syncthreads();
  if (gk) {
    if (tid == 0) {
      float s = 0.0f;
      for (uint32_t i = 0; i < hd; i++) s = s + k[i] * k[i];
      nrm = ex_rms_scale(s, (float)hd);
    }
    __syncthreads();
    if (tid < hd) k[tid] = (k[tid] * nrm) * (1.0f + gk[tid]);
  }
  const uint32_t slot = (pos0 + t) % ctx;
  float* Kr = KV.base + (size_t)seq * KV.seq_stride + KV.layer_off;
  if (tid < hd) {
    Kr[(size_t)slot * d + h * hd + tid] = k[tid];
    Kr[(size_t)ctx * d + (size_t)slot * d + h * hd + tid] = x[2 * d + h * hd + tid];
  }
}

hipError_t launch_kv_write(const float* QKV, const float* gk, StateRef KV, uint32_t seq,
                           uint32_t pos0, uint32_t d, uint32_t heads, uint32_t ctx, uint32_t T,
                           hipStream_t st) {
  hipLaunchKernelGGL(k_kv_write, dim3(heads, T), dim3(64), 0, st, QKV, gk, KV, seq, pos0, d,
                     d / heads, ctx);
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

// the token loop's step end: record the pick, feed it next at pos + 1
__global__ void k_advance(uint32_t* pos, uint32_t* tok, const uint32_t* pick, uint32_t* out,
                          uint32_t steps, uint32_t step, uint32_t B) {
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  out[(size_t)b * steps + step] = pick[b];
  tok[b] = pick[b];
  pos[b] = pos[b] + 1;
}

hipError_t launch_advance(uint32_t* pos, uint32_t* tok, const uint32_t* pick, uint32_t* out,
                          uint32_t steps, uint32_t step, uint32_t B, hipStream_t st) {
  hipLaunchKernelGGL(k_advance, dim3((B + 255) / 256), dim3(256), 0, st, pos, tok, pick, out,
                     steps, step, B);
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

}  // namespace ana

// ANA_BF16 prefill products on wide wave tiles (gfx950).
//
// Y[m][n] = sum_k A[m][k] W[n][k] for the layer products of a prefill step
// of thousands of rows: A the activations in bf16 (k_split, or the bf16
// hidden rows gate|up leaves), W the bf16 weights; norm scale, SiLU and
// residual in the epilogue.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "ana_internal.h"
#include "mfma.h"

namespace ana {

namespace {

constexpr int kWideBK = 64;

// A (WM * NI * 16) x (WN * NJ * 16) tile of WM x WN waves, each
// (NI * 16) x (NJ * 16) (NI x NJ v_mfma_f32_16x16x32_bf16 tiles). K goes
// through two LDS stages of 64 k, each filled by global_load_lds one stage
// ahead: the A and weight tiles as 1 KB chunks of 8 rows, each row's whole
// 128-byte line, its eight 16-byte k pieces at slot piece ^ (row & 7), so
// the 16 rows of a fragment read touch distinct 16-byte bank groups eight
// at a time. (Loads of 16 rows x 64 bytes, half lines, for stages of 32 k
// moved the same bytes at two thirds the rate: 652 against 434 ns a 32-k
// step for a round of 256 tiles, no MFMAs.) Each wave reads one 32-k
// half's fragments of a stage, then runs its MFMAs, then the other half;
// the other wave of its SIMD computes meanwhile. Norm scale, residual and
// SiLU in the
// epilogue (SiLU, a compile-time choice so the other products' code and
// its schedule do not carry it: the tile's first half of columns are gate
// rows, the second half the matching up rows).
template <int WM, int WN, int NI, int NJ, bool SILU>
__global__ __launch_bounds__(WM * WN * 64, WM * WN / 4) void k_gemm_wide(GemvArgs a, const __bf16* __restrict__ Ahg,
                                                                         const float* __restrict__ rscg) {
  constexpr int NW = WM * WN, NT = NW * 64;
  constexpr int BM = WM * NI * 16, BN = WN * NJ * 16, BK = kWideBK;
  constexpr int ACH = BM / 8, WCH = BN / 8;       // 1 KB chunks a stage
  // of them a wave fills: the A chunks split evenly; the weight chunks
  // round up, the spare slots loading chunks 0, 1, .. again (the same
  // bytes to the same place), so every wave issues the same count
  constexpr int AW = ACH / NW, BW = (WCH + NW - 1) / NW;
  static_assert(AW * NW == ACH, "A chunks split evenly over the waves");
  static_assert(BM == 256, "one norm scale a thread of the first 256");
  constexpr int SO = (ACH + WCH) * 512;           // bf16 elements of a stage object
  static_assert(SO >= 64 * (BN / 2) * 4, "half a stage object holds 64 rows of the SiLU exchange");
  __shared__ __align__(1024) __bf16 st0[SO], st1[SO];
  __shared__ float rsl[BM];
  auto stage = [&](auto B) -> __bf16* {
    if constexpr (decltype(B)::value == 0) return st0;
    else return st1;
  };
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t wm = wv / WN, wn = wv % WN;
  uint32_t ntile, mtile;
  xcd_tile(&ntile, &mtile);
  const uint32_t m0 = mtile * BM;
  const uint32_t nb = min((uint32_t)BM, a.B - m0);
  const uint32_t K = a.K, nst = K / BK;
  const Segs sgs(a);
  // wave wv fills A chunks AW wv .. and weight chunks BW wv .. of each
  // stage (chunk c: tile rows 8 c .. 8 c + 7), this lane's 16-byte piece of
  // each: row lane / 8 of the chunk, slot lane % 8 holding k piece
  // (lane % 8) ^ row (as 32-bit byte offsets from a uniform base, so each
  // load is the base in SGPRs plus one VGPR: the weights' base is the lower
  // of the two segments', which lie in one buffer)
  const uint32_t pr = lane >> 3, pq = (lane & 7) ^ pr;
  const char* const abase = reinterpret_cast<const char*>(Ahg);
  const uint16_t* const wlo = a.nseg > 1 && a.Wh1 < a.Wh0 ? a.Wh1 : a.Wh0;
  const char* const wbase = reinterpret_cast<const char*>(wlo);
  uint32_t aoff[AW], boff[BW];
#pragma unroll
  for (int h = 0; h < AW; h++) {
    const uint32_t r = 8 * (AW * wv + h) + pr;
    aoff[h] = 2 * ((m0 + (r < nb ? r : 0)) * K + 8 * pq);
  }
#pragma unroll
  for (int h = 0; h < BW; h++) {
    const uint32_t r = 8 * ((BW * wv + h) % WCH) + pr;
    const float* w;
    uint32_t sg, lr;
    const bool ok = sgs.row(BN, ntile, r, &w, &sg, &lr);
    const uint16_t* p = ok ? (sg ? a.Wh1 : a.Wh0) + (size_t)lr * K + 8 * pq : a.Wh0 + 8 * pq;
    boff[h] = (uint32_t)(reinterpret_cast<const char*>(p) - wbase);
  }
  // AW + BW loads a wave a stage
  auto issue = [&](uint32_t s, auto B) {
    const uint32_t kb = s * BK * 2;
#pragma unroll
    for (int h = 0; h < AW; h++)
      __builtin_amdgcn_global_load_lds((const void*)(abase + (aoff[h] + kb)), (lds_void*)(stage(B) + (AW * wv + h) * 512), 16, 0, 0);
#pragma unroll
    for (int h = 0; h < BW; h++)
      __builtin_amdgcn_global_load_lds((const void*)(wbase + (boff[h] + kb)), (lds_void*)(stage(B) + (ACH + (BW * wv + h) % WCH) * 512), 16, 0, 0);
  };
  f32x4_t acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t r16 = lane & 15, g4 = lane >> 4;
  // a 16-row MFMA tile is two chunks; this lane's row r16 and 32-k half kh
  // (k piece 4 kh + g4)
  const uint32_t fbase = (r16 >> 3) * 512 + (r16 & 7) * 64;
  const uint32_t foff0 = fbase + 8 * (g4 ^ (r16 & 7)), foff1 = fbase + 8 * ((4 + g4) ^ (r16 & 7));
  bf16x8_t fa[NI], fb[NJ];
  auto lread = [&](auto B, uint32_t foff) {
    const __bf16* S = stage(B);
#pragma unroll
    for (int i = 0; i < NI; i++) fa[i] = *reinterpret_cast<const bf16x8_t*>(S + (wm * NI + i) * 1024 + foff);
#pragma unroll
    for (int j = 0; j < NJ; j++) fb[j] = *reinterpret_cast<const bf16x8_t*>(S + ACH * 512 + (wn * NJ + j) * 1024 + foff);
  };
  auto mma = [&]() {
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
      for (int j = 0; j < NJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
  };
  // the waits and the barrier, with nothing moved across them: a memory
  // clobber so no LDS access crosses (the barrier builtin alone orders no
  // memory), and scheduling barriers so no MFMA does
  auto step_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    ANA_LGKMCNT0();
    ANA_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // stage s (object B): this wave's loads of it (the only ones in flight)
  // and its fragment reads of the other object are done; the barrier makes
  // every wave's loads of s visible and says every wave is done reading the
  // other object, which stage s + 1 then fills; then each 32-k half's
  // fragments and MFMAs (the SIMD's other wave computes while this one
  // waits on its reads)
  auto step = [&](uint32_t s, auto B, auto Bn) {
    step_barrier();
    if (s + 1 < nst) issue(s + 1, Bn);
    lread(B, foff0);
    mma();
    lread(B, foff1);
    mma();
  };
  constexpr std::integral_constant<int, 0> S0{};
  constexpr std::integral_constant<int, 1> S1{};
  issue(0, S0);
  for (uint32_t s = 0; s < nst; s += 2) {
    step(s, S0, S1);
    step(s + 1, S1, S0);
  }
  const bool norm = a.ng != nullptr;
  // results: tile (i, j) of the wave holds rows wm*NI*16 + 16i + 4*g4 + r,
  // column wn*NJ*16 + 16j + r16; the row norm scales go to LDS first (every
  // wave's fragment reads and loads are done at the barrier)
  ANA_VMCNT(0);
  __syncthreads();
  if (norm) {
    for (uint32_t t = tid; t < (uint32_t)BM; t += NT) {
      const uint32_t m = m0 + (t < nb ? t : 0);
      rsl[t] = a.sspi ? norm_from_partials(a.sspi + (size_t)m * a.nspi, a.nspi, K) : rscg[m];
    }
    __syncthreads();
  }
  auto rs = [&](int i, int r) { return norm ? rsl[wm * NI * 16 + 16 * i + 4 * g4 + r] : 1.0f; };
  // full tiles (every row and column valid; every tile of the 8192-row
  // prefill products) store without a check or a load among the stores:
  // with per-element bounds checks, per-element scale lookups and loads
  // between the stores, the compiler drained the stores (vmcnt(0)) again
  // and again, and the epilogue took longer than the k loop
  const uint32_t wrows = SILU ? a.seg[0].rows : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  const uint32_t wper = SILU ? BN / 2 : BN;
  const bool full = nb == (uint32_t)BM && (ntile + 1) * wper <= wrows && a.mode != GM_RESID;
  if (full) {
    float sc[NI][4];
    if (norm) {
#pragma unroll
      for (int i = 0; i < NI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) sc[i][r] = rsl[wm * NI * 16 + 16 * i + 4 * g4 + r];
    } else {
#pragma unroll
      for (int i = 0; i < NI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) sc[i][r] = 1.0f;
    }
    const size_t mrow = m0 + wm * NI * 16 + 4 * g4;   // this lane's first row
    if constexpr (SILU) {
      constexpr int HB = BN / 2;
      // tile rows 64 q .. 64 q + 63 in half q & 1 of stage object q >> 1
      auto upat = [&](uint32_t m) -> float* {
        const uint32_t q = m >> 6;
        return reinterpret_cast<float*>((q >> 1 ? st1 : st0) + (q & 1) * (SO / 2)) + (m & 63) * HB;
      };
      // each gate wave and its up wave (same rows, matching columns) swap
      // half their rows: the gate wave hands over its gate values of rows
      // i >= NI / 2, the up wave its up values of rows i < NI / 2; then each
      // forms silu(gate) * up and stores for its own half of the rows
      const bool gate = wn < (uint32_t)(WN / 2);
      const uint32_t cw = (gate ? wn : wn - WN / 2) * NJ * 16 + r16;   // column in the half
#pragma unroll
      for (int i = 0; i < NI; i++) {
        if ((i >= NI / 2) != gate) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          float* x = upat(wm * NI * 16 + 16 * i + 4 * g4 + r) + cw;
#pragma unroll
          for (int j = 0; j < NJ; j++) x[16 * j] = acc[i][j][r] * sc[i][r];
        }
      }
      __syncthreads();
      // the gate row of this lane's columns: the tile's column n is gate
      // row ntile * HB + n
      const uint32_t lr0 = ntile * HB + cw;
      float hv[NI / 2][4][NJ];
#pragma unroll
      for (int ii = 0; ii < NI / 2; ii++) {
        const int i = gate ? ii : ii + NI / 2;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float* x = upat(wm * NI * 16 + 16 * i + 4 * g4 + r) + cw;
#pragma unroll
          for (int j = 0; j < NJ; j++) {
            const float own = acc[i][j][r] * sc[i][r], other = x[16 * j];
            hv[ii][r][j] = gate ? fast_silu(own) * other : fast_silu(other) * own;
          }
        }
      }
      const size_t mh = mrow + (gate ? 0 : 16 * (NI / 2));   // this lane's first row of its half
      if (a.Yh) {
        __bf16* yb = a.Yh + mh * a.seg[0].rows + lr0;
#pragma unroll
        for (int ii = 0; ii < NI / 2; ii++)
#pragma unroll
          for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < NJ; j++) yb[(size_t)(16 * ii + r) * a.seg[0].rows + 16 * j] = (__bf16)hv[ii][r][j];
      } else {
        float* yb = a.seg[0].Y + mh * a.seg[0].ldy + lr0;
#pragma unroll
        for (int ii = 0; ii < NI / 2; ii++)
#pragma unroll
          for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < NJ; j++) yb[(size_t)(16 * ii + r) * a.seg[0].ldy + 16 * j] = hv[ii][r][j];
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      // this lane's column: the segment and row it falls in, by selects
      const uint32_t v = ntile * BN + wn * NJ * 16 + 16 * j + r16;
      const bool s1 = v >= a.seg[0].rows;
      float* const Yb = s1 ? a.seg[1].Y : a.seg[0].Y;
      const uint32_t ld = s1 ? a.seg[1].ldy : a.seg[0].ldy;
      float* yb = Yb + mrow * ld + (s1 ? v - a.seg[0].rows : v);
#pragma unroll
      for (int i = 0; i < NI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) yb[(size_t)(16 * i + r) * ld] = acc[i][j][r] * sc[i][r];
    }
    return;
  }
  if constexpr (SILU) {
    // up columns (the second half of the waves' columns) through LDS to the
    // gate columns: tile rows 64 q .. 64 q + 63 in stage object q
    constexpr int HB = BN / 2;
    auto upat = [&](uint32_t m) -> float* {
      const uint32_t q = m >> 6;
      return reinterpret_cast<float*>((q >> 1 ? st1 : st0) + (q & 1) * (SO / 2)) + (m & 63) * HB;
    };
    if (wn >= (uint32_t)(WN / 2)) {
#pragma unroll
      for (int i = 0; i < NI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t m = wm * NI * 16 + 16 * i + 4 * g4 + r;
          float* up = upat(m);
          const float sc = rs(i, r);
#pragma unroll
          for (int j = 0; j < NJ; j++) up[(wn - WN / 2) * NJ * 16 + 16 * j + r16] = acc[i][j][r] * sc;
        }
    }
    __syncthreads();
    if (wn < (uint32_t)(WN / 2)) {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const uint32_t n = wn * NJ * 16 + 16 * j + r16;
        const float* w_;
        uint32_t sg, lr;
        if (!sgs.row(BN, ntile, n, &w_, &sg, &lr)) continue;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const uint32_t m = wm * NI * 16 + 16 * i + 4 * g4 + r;
            if (m >= nb) continue;
            const float y = acc[i][j][r] * rs(i, r);
            const float hv = fast_silu(y) * upat(m)[n];
            if (a.Yh) a.Yh[(size_t)(m0 + m) * a.seg[0].rows + lr] = (__bf16)hv;
            else a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = hv;
          }
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    // one column block's residuals live at a time
    asm volatile("" ::: "memory");
    const uint32_t n = wn * NJ * 16 + 16 * j + r16;
    const float* w_;
    uint32_t sg, lr;
    if (!sgs.row(BN, ntile, n, &w_, &sg, &lr)) continue;
    float res[NI][4];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = wm * NI * 16 + 16 * i + 4 * g4 + r;
        res[i][r] = a.mode == GM_RESID && m < nb ? a.R[(size_t)(m0 + m) * a.ldr + lr] : 0.0f;
      }
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = wm * NI * 16 + 16 * i + 4 * g4 + r;
        if (m >= nb) continue;
        float y = acc[i][j][r] * rs(i, r);
        if (a.mode == GM_RESID) y = res[i][r] + y;
        if (sg) a.seg[1].Y[(size_t)(m0 + m) * a.seg[1].ldy + lr] = y;
        else a.seg[0].Y[(size_t)(m0 + m) * a.seg[0].ldy + lr] = y;
      }
  }
}

// the configurations launched: 2 x 4 waves of 128 x 64 on a 256 x 256 tile,
// two waves a SIMD (128 accumulators and two fragment sets of 12 in 256
// registers); each wave reads 12 KB of fragments a 32-k stage for 32 MFMAs,
// against 8 KB for 16 in sixteen waves of 64 x 64. Four waves of 128 x 96
// ran at two thirds of this rate: with one wave a SIMD nothing covered a
// stall, and their 192 accumulators sat in AGPRs, where the allocator moved
// them between MFMAs. And 4 x 2 waves of 64 x 96 on a 256 x 192 tile, for
// products whose 256-wide tiles leave the last round of workgroups part
// empty (q|k|v|z at 3072 output rows: 384 tiles, a round and a half on 256
// CUs, against 512 of three quarters the work)
constexpr int kWideBM = 256;
constexpr int kBN256 = 256, kBN192 = 192;

uint32_t wide_tiles(const GemvArgs& a, uint32_t BN) {
  const uint32_t rows = a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  return a.mode == GM_SILU ? (a.seg[0].rows + BN / 2 - 1) / (BN / 2) : (rows + BN - 1) / BN;
}

// rounds of one workgroup a CU times the work of a tile, in 64-column units
uint32_t wide_cost(const GemvArgs& a, uint32_t BN, uint32_t cus) {
  const uint32_t t = wide_tiles(a, BN) * ((a.B + kWideBM - 1) / kWideBM);
  return (t + cus - 1) / cus * (BN / 64);
}

}  // namespace

bool gemm_wide_takes(const GemvArgs& a) {
  const uint32_t rows = a.mode == GM_SILU ? 2 * a.seg[0].rows
                                          : a.seg[0].rows + (a.nseg > 1 ? a.seg[1].rows : 0);
  return rows >= 2048 && wide_tiles(a, kBN256) * ((a.B + kWideBM - 1) / kWideBM) >= 256 && a.K % 128 == 0;
}

hipError_t launch_gemm_wide(const GemvArgs& a, const __bf16* Ah, const float* rsc, hipStream_t st) {
  if (!gemm_wide_takes(a) || a.amax || !a.Wh0 || (a.nseg > 1 && !a.Wh1)) return hipErrorInvalidValue;
  // the A and weight offsets are 32-bit byte offsets
  if (2ull * a.B * a.K >= (1ull << 32)) return hipErrorInvalidValue;
  {
    const uint16_t* lo = a.nseg > 1 && a.Wh1 < a.Wh0 ? a.Wh1 : a.Wh0;
    const uint16_t* e0 = a.Wh0 + (size_t)a.seg[0].rows * a.K;
    const uint16_t* e1 = a.nseg > 1 ? a.Wh1 + (size_t)a.seg[1].rows * a.K : e0;
    const uint16_t* hi = e1 > e0 ? e1 : e0;
    if ((uint64_t)(hi - lo) * 2 >= (1ull << 32)) return hipErrorInvalidValue;
  }
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return hipErrorInvalidDevice;
    cus = n;
  }
  const uint32_t mt = (a.B + kWideBM - 1) / kWideBM;
  if (wide_cost(a, kBN192, cus) < wide_cost(a, kBN256, cus))
    if (a.mode == GM_SILU) hipLaunchKernelGGL((k_gemm_wide<4, 2, 4, 6, true>), dim3(wide_tiles(a, kBN192), mt), dim3(512), 0, st, a, Ah, rsc);
    else hipLaunchKernelGGL((k_gemm_wide<4, 2, 4, 6, false>), dim3(wide_tiles(a, kBN192), mt), dim3(512), 0, st, a, Ah, rsc);
  else
    if (a.mode == GM_SILU) hipLaunchKernelGGL((k_gemm_wide<2, 4, 8, 4, true>), dim3(wide_tiles(a, kBN256), mt), dim3(512), 0, st, a, Ah, rsc);
    else hipLaunchKernelGGL((k_gemm_wide<2, 4, 8, 4, false>), dim3(wide_tiles(a, kBN256), mt), dim3(512), 0, st, a, Ah, rsc);
  return hipGetLastError();
}

}  // namespace ana

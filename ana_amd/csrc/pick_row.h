// S.pick (bend/Sample.bend:95-254) for one row on one workgroup, and the
// tree reductions it is built from; k_pick runs it a row per workgroup, the
// LM head's fused form (k_head_pw with PICK) on the workgroups that finish
// a row block last.
//
// The reference keeps the logits in a left-packed binary tree of depth
// dv = depth(vocab) (bend/Tensor.bend) and every sum and max is that tree's
// pairwise reduction. Here a thread owns LPT consecutive leaves; it reduces
// them pairwise in registers, then lanes combine with xor partners (level m
// joins the groups that differ in lane bit m, left group first) and waves
// combine the same way through LDS: each partial is a node of the
// reference's tree, so the results are its bits. Absent leaves (index >=
// vocab, the tree's VZ) count 0.0 in sums and -3e38 in the max, as V.sum and
// V.max give VZ; Sample.argmax gives VZ the pair (-3e38, 0).
#pragma once
#include <type_traits>

#include "ana_internal.h"
#include "numerics.h"

#pragma clang fp contract(off)

namespace ana {

namespace {


struct Add { __device__ float operator()(float a, float b) const { return a + b; } };
// F32.max a b = (a < b ? b : a): a is the left subtree
struct Max { __device__ float operator()(float a, float b) const { return a < b ? b : a; } };

// x[i] = row[base + i] for i < LPT (0 past v or when inactive): a thread's
// LPT consecutive logits, as 16-byte loads when the run is whole and
// aligned (each load of a wave then covers whole cache-line pieces instead
// of one float of 64 lines)
template <int LPT>
__device__ __forceinline__ void load_run(const float* __restrict__ row, uint32_t base, uint32_t v, bool active,
                                         float (&x)[LPT]) {
  if constexpr (LPT % 4 == 0) {
    if (active && base + LPT <= v && (reinterpret_cast<uintptr_t>(row + base) & 15) == 0) {
      const float4* r4 = reinterpret_cast<const float4*>(row + base);
#pragma unroll
      for (int i = 0; i < LPT / 4; i++) {
        const float4 f = r4[i];
        x[4 * i + 0] = f.x;
        x[4 * i + 1] = f.y;
        x[4 * i + 2] = f.z;
        x[4 * i + 3] = f.w;
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < LPT; i++) x[i] = (active && base + i < v) ? row[base + i] : 0.0f;
}

template <int LPT, class Op>
__device__ __forceinline__ float local_reduce(const float (&x)[LPT], Op op) {
  float t[LPT];
#pragma unroll
  for (int i = 0; i < LPT; i++) t[i] = x[i];
#pragma unroll
  for (int s = 1; s < LPT; s *= 2)
#pragma unroll
    for (int i = 0; i < LPT; i += 2 * s) t[i] = op(t[i], t[i + s]);
  return t[0];
}

// The tree above the threads: NT = leaves/LPT threads, a power of two.
template <class Op>
__device__ float tree_up(float v, Op op, float* red, uint32_t tid, uint32_t NT) {
  const uint32_t lane = tid & 63;
  for (uint32_t m = 1; m < 64 && m < NT; m <<= 1) {
    const float o = __shfl_xor(v, m, 64);
    v = (lane & m) ? op(o, v) : op(v, o);
  }
  if (NT <= 64) {
    // every lane of the first group holds the root; share lane 0's
    if (tid == 0) red[0] = v;
    __syncthreads();
    const float r = red[0];
    __syncthreads();
    return r;
  }
  const uint32_t nw = NT >> 6;   // a power of two, at most 16
  if (lane == 0 && (tid >> 6) < nw) red[tid >> 6] = v;
  __syncthreads();
  // the wave partials' tree, unrolled over the 16 possible leaves (a
  // runtime-bounded loop would keep w in scratch memory)
  float w[16];
#pragma unroll
  for (uint32_t i = 0; i < 16; i++) w[i] = i < nw ? red[i] : 0.0f;
#pragma unroll
  for (uint32_t s = 1; s < 16; s *= 2)
#pragma unroll
    for (uint32_t i = 0; i < 16; i += 2 * s)
      if (i + s < nw) w[i] = op(w[i], w[i + s]);
  __syncthreads();
  return w[0];
}

// Sample.argmax's pairs: the right one wins only when strictly greater
__device__ __forceinline__ void best_join(float& av, uint32_t& ai, float bv, uint32_t bi) {
  if (bv > av) { av = bv; ai = bi; }
}

template <int LPT>
__device__ uint32_t tree_argmax(const float (&x)[LPT], uint32_t base, uint32_t vocab, float* redf,
                                uint32_t* redi, uint32_t tid, uint32_t NT) {
  float v[LPT];
  uint32_t ix[LPT];
#pragma unroll
  for (int i = 0; i < LPT; i++) {
    const bool here = base + i < vocab;
    v[i] = here ? x[i] : -3.0e38f;
    ix[i] = here ? base + i : 0u;
  }
#pragma unroll
  for (int s = 1; s < LPT; s *= 2)
#pragma unroll
    for (int i = 0; i < LPT; i += 2 * s) best_join(v[i], ix[i], v[i + s], ix[i + s]);
  float bv = v[0];
  uint32_t bi = ix[0];
  const uint32_t lane = tid & 63;
  for (uint32_t m = 1; m < 64 && m < NT; m <<= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const uint32_t oi = __shfl_xor(bi, m, 64);
    if (lane & m) {  // partner is the left subtree
      float lv = ov;
      uint32_t li = oi;
      best_join(lv, li, bv, bi);
      bv = lv;
      bi = li;
    } else {
      best_join(bv, bi, ov, oi);
    }
  }
  if (NT <= 64) {
    if (tid == 0) redi[0] = bi;
    __syncthreads();
    const uint32_t r = redi[0];
    __syncthreads();
    return r;
  }
  const uint32_t nw = NT >> 6;
  if (lane == 0 && (tid >> 6) < nw) {
    redf[tid >> 6] = bv;
    redi[tid >> 6] = bi;
  }
  __syncthreads();
  float wv[16];
  uint32_t wi[16];
  for (uint32_t i = 0; i < nw; i++) { wv[i] = redf[i]; wi[i] = redi[i]; }
  for (uint32_t s = 1; s < nw; s *= 2)
    for (uint32_t i = 0; i < nw; i += 2 * s) best_join(wv[i], wi[i], wv[i + s], wi[i + s]);
  __syncthreads();
  return wi[0];
}

// wave reductions by DPP within rows of 16 lanes (lane ^ 1, lane ^ 2, the
// mirrored quad, the mirrored half-row), then the four rows by lane reads:
// a few cycles a step where a lane shuffle waits on LDS
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
// a whole number over the wave (every lane gets it)
__device__ __forceinline__ uint32_t wave_count(uint32_t c) {
  int v = (int)c;
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  v += dpp_i<0x141>(v);
  v += dpp_i<0x140>(v);
  return (uint32_t)((__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
                    (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48)));
}
// the least of a wave's floats (every lane gets it)
__device__ __forceinline__ float wave_minf(float x) {
  auto mn = [](float a, float b) { return b < a ? b : a; };
  auto d = [](float a, auto c) {
    return __builtin_bit_cast(float, dpp_i<decltype(c)::value>(__builtin_bit_cast(int, a)));
  };
  x = mn(x, d(x, std::integral_constant<int, 0xB1>{}));
  x = mn(x, d(x, std::integral_constant<int, 0x4E>{}));
  x = mn(x, d(x, std::integral_constant<int, 0x141>{}));
  x = mn(x, d(x, std::integral_constant<int, 0x140>{}));
  auto rl = [](float a, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), l)); };
  return mn(mn(rl(x, 0), rl(x, 16)), mn(rl(x, 32), rl(x, 48)));
}

// N whole numbers, each summed over the workgroup's 16 waves (every thread
// gets them)
template <int N>
__device__ void block_counts(uint32_t (&c)[N], uint32_t (*redn)[16], uint32_t tid) {
#pragma unroll
  for (int i = 0; i < N; i++) c[i] = wave_count(c[i]);
  if ((tid & 63) == 0)
#pragma unroll
    for (int i = 0; i < N; i++) redn[tid >> 6][i] = c[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; i++) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < 16; w++) t += redn[w][i];
    c[i] = t;
  }
  __syncthreads();
}

__device__ __forceinline__ uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

// Rng.next (bend/Sample.bend:57-66): the file's transition, which is not
// textbook xoshiro256** (s0' and s1' differ)
__device__ uint64_t rng_next(uint64_t* r) {
  const uint64_t s0 = r[0], s1 = r[1], s2 = r[2], s3 = r[3];
  const uint64_t t = s1 << 17;
  const uint64_t w = rotl64(s1 * 5, 7) * 9;
  r[0] = (s0 ^ s3) ^ (s1 ^ s2);
  r[1] = s1 ^ s2;
  r[2] = (s2 ^ s0) ^ t;
  r[3] = rotl64(s3 ^ s1, 45);
  return w;
}


// candidates a wave finishes the top-k bisection on; survivors of a top-k
// the top-p bisection takes in one wave, and its fold's stack depth (the
// tree's levels, at most 16 for a vocabulary of 65536, plus one)
constexpr int kCand = 1024, kSurv = 64, kSurvDepth = 18;
// top-k steps a pass over the whole row resolves, and its midpoints
constexpr int kPass = 2, kNodes = (1 << kPass) - 1;

// row b of a.logits (read from `rowp` when given: a copy in LDS), on all
// threads of the workgroup (NT of them own leaves, LPT each): the pick into
// a.tok[b], the row's RNG words advanced
template <int LPT>
__device__ __forceinline__ void pick_row(const PickArgs& a, uint32_t b, uint32_t NT, uint32_t dv,
                                         const float* rowp = nullptr) {
  __shared__ float red[16];
  __shared__ uint32_t redi[16];
  __shared__ float heap[2048];
  __shared__ float leafh[2 * LPT];
  __shared__ uint32_t who;
  __shared__ uint32_t redn[16][16], nc_s, off_s[16];
  __shared__ float lo_s;
  __shared__ uint32_t sidx[kSurv];
  __shared__ float sw[kSurv], stk[kSurvDepth][64];
  __shared__ uint32_t ops[kSurvDepth];
  const uint32_t tid = threadIdx.x;
  const uint32_t v = a.vocab;
  const uint32_t base = tid * LPT;
  const bool active = tid < NT;
  const float* lg = rowp ? rowp : a.logits + (size_t)b * v;
  float x[LPT];
  load_run<LPT>(lg, base, v, active, x);

  // greedy on the store (dc.px.top, bend/Decode.bend:407-418): dd.pick's
  // least index reaching the max; only a NaN max falls back to argmax
  if (a.temp <= 0.0f && a.store_first) {
    float r = -INFINITY;
#pragma unroll
    for (int i = 0; i < LPT; i++)
      if (active && base + i < v) r = x[i] > r ? x[i] : r;
    for (uint32_t m = 1; m < 64; m <<= 1) {
      const float o = __shfl_xor(r, m, 64);
      r = o > r ? o : r;
    }
    if ((tid & 63) == 0) red[tid >> 6] = r;
    __syncthreads();
    float top = red[0];
    for (int w = 1; w < 16; w++) top = red[w] > top ? red[w] : top;
    uint32_t best = v;
#pragma unroll
    for (int i = LPT - 1; i >= 0; i--)
      if (active && base + i < v && top <= x[i]) best = base + i;
    for (uint32_t m = 1; m < 64; m <<= 1) {
      const uint32_t o = __shfl_xor(best, m, 64);
      best = o < best ? o : best;
    }
    __syncthreads();
    if ((tid & 63) == 0) redi[tid >> 6] = best;
    __syncthreads();
    uint32_t bb = redi[0];
    for (int w = 1; w < 16; w++) bb = redi[w] < bb ? redi[w] : bb;
    __syncthreads();
    if (bb < v) {
      if (tid == 0) a.tok[b] = bb;
      return;
    }
  }
  // greedy: Sample.argmax over the tree, the rng untouched
  if (a.temp <= 0.0f) {
    const uint32_t t = tree_argmax<LPT>(x, base, v, red, redi, tid, NT);
    if (tid == 0) a.tok[b] = t;
    return;
  }
  // peak = V.max(logits)
  float pm[LPT];
#pragma unroll
  for (int i = 0; i < LPT; i++) pm[i] = (active && base + i < v) ? x[i] : -3.0e38f;
  const float peak = tree_up(local_reduce<LPT>(pm, Max()), Max(), red, tid, NT);

  // top-k: the largest t in [peak-100, peak] (40 bisection steps) keeping
  // at least k logits >= t; the rest go to -3e38 (sample.topk). A count is
  // a whole number below 2^24, so its tree sum is exact and may be formed
  // in any order: the steps run over the whole row while more than kCand
  // logits lie in [lo, hi), then those candidates go to LDS and wave 0 takes
  // the remaining steps (count(x >= mid) = count(x >= hi0) + the candidates
  // >= mid) with no barrier. nsurv = count(x >= lo) after the last step.
  uint32_t nsurv = 0;
  if (a.topk < v) {
    const float need = (float)a.topk;
    float lo = peak - 100.0f, hi = peak;
    auto cnt_ge = [&](float t) {
      uint32_t c = 0;
#pragma unroll
      for (int i = 0; i < LPT; i++) c += (active && base + i < v && x[i] >= t) ? 1u : 0u;
      return c;
    };
    uint32_t c0[2] = {cnt_ge(lo), cnt_ge(hi)};
    block_counts<2>(c0, redn, tid);
    uint32_t c_lo = c0[0], c_hi = c0[1];
    int it = 0;
    // kPass steps a pass over the row: the kNodes midpoints the next kPass
    // steps could take (node i's lower child 2 i + 1 halves [lo, mid], its
    // upper child 2 i + 2 halves [mid, hi], each midpoint the same float
    // 0.5 (lo + hi) the step itself forms), all counted at once, then the path
    while (it + kPass <= 40 && c_lo - c_hi > kCand) {
      float mids[kNodes], los[kNodes], his[kNodes];
      los[0] = lo;
      his[0] = hi;
#pragma unroll
      for (int n = 0; n < kNodes; n++) {
        mids[n] = 0.5f * (los[n] + his[n]);
        if (2 * n + 2 < kNodes) {
          los[2 * n + 1] = los[n];
          his[2 * n + 1] = mids[n];
          los[2 * n + 2] = mids[n];
          his[2 * n + 2] = his[n];
        }
      }
      uint32_t cs[kNodes];
#pragma unroll
      for (int n = 0; n < kNodes; n++) cs[n] = cnt_ge(mids[n]);
      block_counts<kNodes>(cs, redn, tid);
      int node = 0;
#pragma unroll
      for (int st = 0; st < kPass; st++) {
        // (a uniform walk: select by index without dynamic register indexing)
        float mid = 0.0f;
        uint32_t c = 0;
#pragma unroll
        for (int n = 0; n < kNodes; n++)
          if (n == node) { mid = mids[n]; c = cs[n]; }
        if ((float)c >= need) { lo = mid; c_lo = c; node = 2 * node + 2; } else { hi = mid; c_hi = c; node = 2 * node + 1; }
      }
      it += kPass;
    }
    if (it < 40) {
      float* cand = heap;   // (the draw's heap is filled only later)
      if (tid == 0) nc_s = 0;
      __syncthreads();
      {
        // one atomic a wave for its candidates' places, then each thread's
        // after the lanes before it
        uint32_t mine = 0;
#pragma unroll
        for (int i = 0; i < LPT; i++) mine += (active && base + i < v && x[i] >= lo && x[i] < hi) ? 1u : 0u;
        const uint32_t lane = tid & 63;
        uint32_t incl = mine;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
          const uint32_t o = __shfl_up(incl, m, 64);
          if (lane >= (uint32_t)m) incl += o;
        }
        uint32_t at = 0;
        if (lane == 63) at = atomicAdd(&nc_s, incl);
        at = (uint32_t)__builtin_amdgcn_readlane((int)at, 63) + incl - mine;
#pragma unroll
        for (int i = 0; i < LPT; i++)
          if (active && base + i < v && x[i] >= lo && x[i] < hi) cand[at++] = x[i];
      }
      __syncthreads();
      if (tid < 64) {
        const uint32_t nc = nc_s;
        float cv[kCand / 64];
#pragma unroll
        for (int e = 0; e < kCand / 64; e++) cv[e] = tid + 64 * e < nc ? cand[tid + 64 * e] : 0.0f;
        for (; it < 40; it++) {
          const float mid = 0.5f * (lo + hi);
          uint32_t c = 0;
#pragma unroll
          for (int e = 0; e < kCand / 64; e++) c += (tid + 64 * e < nc && cv[e] >= mid) ? 1u : 0u;
          c = c_hi + wave_count(c);   // (c_hi: count(x >= hi) when the candidates were taken)
          if ((float)c >= need) { lo = mid; c_lo = c; } else { hi = mid; }
        }
        if (tid == 0) {
          lo_s = lo;
          nc_s = c_lo;
        }
      }
      __syncthreads();
      lo = lo_s;
      c_lo = nc_s;
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < LPT; i++) x[i] = x[i] >= lo ? x[i] : -3.0e38f;
    nsurv = c_lo;
  }
  // w = exp((x - peak) / temp) (exp.at); absent leaves stay 0. Every logit
  // the top-k dropped is -3e38 now, so its weight is one value, formed once
  const float wz = dexp((-3.0e38f - peak) / a.temp);
  float w[LPT];
#pragma unroll
  for (int i = 0; i < LPT; i++)
    w[i] = (active && base + i < v) ? (x[i] == -3.0e38f ? wz : dexp((x[i] - peak) / a.temp)) : 0.0f;

  // top-p: the largest t in [0, 1] whose kept mass reaches p of the total.
  // After a top-k that kept 1..kSurv logits only those weights are not 0,
  // and a 0 leaf leaves every sum of the reference's tree unchanged, so
  // each mass is the tree sum over the survivors alone: wave 0 forms, per
  // survivor L, the tree-ordered mass of {w >= w_L} once, and each step's
  // mass is the one of the least w_L >= mid (0 when there is none).
  // (every logit the top-k dropped now weighs dexp((-3e38 - peak) / temp),
  // which must be 0 for the survivors to be the only leaves that count)
  if (a.topp < 1.0f && a.topk < v && nsurv >= 1 && nsurv <= (uint32_t)kSurv && wz == 0.0f) {
    // the leaves of non-zero weight (at most the survivors) in index order:
    // a thread's own, after those of the threads before it
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < LPT; i++) mine += w[i] > 0.0f ? 1u : 0u;
    const uint32_t lane = tid & 63;
    uint32_t incl = mine;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const uint32_t o = __shfl_up(incl, m, 64);
      if (lane >= (uint32_t)m) incl += o;
    }
    if (lane == 63) off_s[tid >> 6] = incl;
    __syncthreads();
    uint32_t off = incl - mine;
    for (uint32_t w2 = 0; w2 < (tid >> 6); w2++) off += off_s[w2];
#pragma unroll
    for (int i = 0; i < LPT; i++)
      if (w[i] > 0.0f) {
        sidx[off] = base + i;
        sw[off] = w[i];
        off++;
      }
    uint32_t n = 0;
#pragma unroll
    for (int w2 = 0; w2 < 16; w2++) n += off_s[w2];
    __syncthreads();
    if (tid < 64 && n == 0) {
      // no weight above 0: every mass is 0, which reaches need = 0, so lo
      // climbs to the last midpoint
      float lo = 0.0f, hi = 1.0f;
      for (int it = 0; it < 40; it++) {
        const float mid = 0.5f * (lo + hi);
        if (0.0f >= a.topp * 0.0f) lo = mid; else hi = mid;
      }
      if (tid == 0) lo_s = lo;
    } else if (tid < 64) {
      const bool valid = tid < n;
      const float wl = valid ? sw[tid] : 0.0f;
      // lane L's mass: the leaves in index order with w < w_L as 0, summed
      // as the tree nests them. Consecutive leaves meet at level
      // h = 32 - clz(i ^ j); a smaller h binds first, so a stack of pending
      // levels (uniform across the wave) folds them left to right
      // (ops: the pending levels, the same in every lane, which all write
      // them; the stack's top value stays in a register, the rest in stk)
      const uint32_t myi = valid ? sidx[tid] : 0u;
      int sp = 0;   // values on the stack; sp - 1 pending levels
      uint32_t prev = 0;
      float cur = 0.0f;
      for (uint32_t j = 0; j < n; j++) {
        const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)myi, (int)j);
        const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), (int)j));
        const float val = wj >= wl ? wj : 0.0f;
        if (j > 0) {
          const uint32_t h = 32u - __builtin_clz(prev ^ ij);
          while (sp > 1 && ops[sp - 2] < h) {
            cur = stk[sp - 2][tid] + cur;
            sp--;
          }
          ops[sp - 1] = h;
          stk[sp - 1][tid] = cur;
        }
        cur = val;
        sp++;
        prev = ij;
      }
      while (sp > 1) {
        cur = stk[sp - 2][tid] + cur;
        sp--;
      }
      const float ml = cur;
      // the total: the mass of the least weight (every survivor)
      const float mn = wave_minf(valid ? wl : INFINITY);
      const unsigned long long at0 = __ballot(valid && wl == mn);
      const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml), __builtin_ctzll(at0)));
      const float need = a.topp * total;
      float lo = 0.0f, hi = 1.0f;
      for (int it = 0; it < 40; it++) {
        const float mid = 0.5f * (lo + hi);
        const float k2 = wave_minf(valid && wl >= mid ? wl : INFINITY);
        float mass = 0.0f;
        if (k2 != INFINITY) {
          const unsigned long long at = __ballot(valid && wl == k2);
          mass = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml), __builtin_ctzll(at)));
        }
        if (mass >= need) lo = mid; else hi = mid;
      }
      if (tid == 0) lo_s = lo;
    }
    __syncthreads();
    const float lo = lo_s;
#pragma unroll
    for (int i = 0; i < LPT; i++) w[i] = w[i] >= lo ? w[i] : 0.0f;
  } else if (a.topp < 1.0f) {
    const float need = a.topp * tree_up(local_reduce<LPT>(w, Add()), Add(), red, tid, NT);
    float lo = 0.0f, hi = 1.0f;
    for (int it = 0; it < 40; it++) {
      const float mid = 0.5f * (lo + hi);
      float c[LPT];
#pragma unroll
      for (int i = 0; i < LPT; i++) c[i] = w[i] >= mid ? w[i] : 0.0f;
      const float mass = tree_up(local_reduce<LPT>(c, Add()), Add(), red, tid, NT);
      if (mass >= need) lo = mid; else hi = mid;
    }
#pragma unroll
    for (int i = 0; i < LPT; i++) w[i] = w[i] >= lo ? w[i] : 0.0f;
  }

  // the draw: thread sums into a heap of the tree above the threads (node n
  // = node 2 n + node 2 n + 1), then draw.go walks from the root (left iff
  // u < sum(left) or the right is VZ). The levels inside a wave join lanes
  // by xor partners, left + right; those above, wave 0 alone
  {
    float hv = active ? local_reduce<LPT>(w, Add()) : 0.0f;
    if (active) heap[NT + tid] = hv;
    const uint32_t lane = tid & 63;
    for (uint32_t m = 1; m < 64 && m < NT; m <<= 1) {
      const float o = __shfl_xor(hv, m, 64);
      hv = (lane & m) ? o + hv : hv + o;
      if (active && (lane & (2 * m - 1)) == 0) heap[(NT + tid) / (2 * m)] = hv;
    }
    __syncthreads();
    if (NT > 64 && tid < 64)
      for (uint32_t n = NT >> 7; n >= 1; n >>= 1) {
        if (tid < n) heap[n + tid] = heap[2 * (n + tid)] + heap[2 * (n + tid) + 1];
        __builtin_amdgcn_wave_barrier();   // (one wave: its LDS ops keep their order)
      }
    __syncthreads();
  }
  uint32_t pbase = 0;
  float u = 0.0f;
  int p = (int)dv;
  if (tid == 0) {
    uint64_t* r = a.rng + (size_t)b * 4;
    const uint64_t word = rng_next(r);
    const float unit = (float)(uint32_t)((word >> 32) >> 8) / 16777216.0f;
    u = unit * heap[1];
    const uint32_t lptlog = __builtin_ctz(LPT);
    while (p > (int)lptlog) {
      const uint32_t half = 1u << (p - 1);
      const float ml = heap[(NT * LPT) / half + pbase / half];
      const bool left = (u < ml) || (pbase + half >= v);
      if (!left) { u = u - ml; pbase += half; }
      p--;
    }
    who = pbase / LPT;
  }
  __syncthreads();
  if (tid == who) {
    // the run's own tree in LDS: leaves at LPT + i, node n = node 2 n +
    // node 2 n + 1 (the pairs local_reduce forms)
#pragma unroll
    for (int i = 0; i < LPT; i++) leafh[LPT + i] = w[i];
#pragma unroll
    for (int st = 1; st < LPT; st *= 2)
#pragma unroll
      for (int i = 0; i < LPT; i += 2 * st) {
        w[i] = w[i] + w[i + st];
        leafh[(LPT + i) / (2 * st)] = w[i];
      }
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t n = 1;
    while (p > 0) {
      const uint32_t half = 1u << (p - 1);
      const float ml = leafh[2 * n];
      const bool left = (u < ml) || (pbase + half >= v);
      if (!left) { u = u - ml; pbase += half; n = 2 * n + 1; } else { n = 2 * n; }
      p--;
    }
    a.tok[b] = pbase;
  }
}

}  // namespace

}  // namespace ana

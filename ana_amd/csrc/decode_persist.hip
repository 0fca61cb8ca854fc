// The fast-mode token loop of one sequence (ANA_FAST_FP32, B = 1) as one
// persistent launch per ana_generate call.
//
// A decode step is ~65 dependent phases (per layer: q|k|v|z, the mix, Wo,
// gate|up, down; the head; the pick). As separate graph nodes each phase
// pays a kernel boundary (~1.9 us) plus the start of its own weight stream
// (~1-3 us). Here one workgroup per CU runs every phase of every step, and
// a phase's inputs arrive by a flag-in-data exchange: each producer writes
// its outputs as 8-byte entries (the value's bits, the step's epoch above)
// with device-coherent stores, and each consumer polls the entries it needs
// with device-coherent loads until every one carries the epoch it waits
// for. There is no grid barrier. Each workgroup loads the weights of the
// phase after the current one into registers before it waits, so the weight
// stream runs under the exchanges instead of after them.
//
// Entries of one (layer, phase) have their own slots, and slots alternate
// between two sets by the epoch's parity: a producer can only reach step
// s + 2 after every workgroup has produced for step s + 1, so no consumer
// of step s still reads a slot it overwrites.
//
// Every wait is bounded in time (the device's constant-rate clock, against a
// limit the host passes): a workgroup that waits too long, or sees another
// one give up, raises the abort word and leaves, and the host reports a
// time-out (the sequence's state is then partly advanced).
// A step whose logits have no maximum (NaN) stops the launch before its
// pick; the host picks by Sample.argmax and launches again.
#include <hip/hip_runtime.h>

#include "ana_internal.h"
#include "numerics.h"
#include "wave.h"

namespace ana {

namespace {

constexpr uint32_t kPT = 256;           // threads per workgroup
constexpr uint32_t kMaxPLayers = 64;    // layers the persistent kernel takes
constexpr uint32_t kMaxTracePhases = 6 * 32 + 2;       // phases a traced step may have (32 layers)

// the device's constant-rate clock (s_memrealtime: 100 MHz on gfx950)
__device__ __forceinline__ uint64_t rtc() { return __builtin_amdgcn_s_memrealtime(); }


__device__ __forceinline__ void ll_put(unsigned long long* p, float v, uint32_t ep) {
  __hip_atomic_store(p, ((unsigned long long)ep << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ll_ld(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool aborted(uint32_t* ctl) {
  return __hip_atomic_load(&ctl[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Poll n entries (entry i at base[map(i)]) until each carries epoch ep
// (tag(entry) == ep), then dst[i] = the value. PE entries a thread at most.
// Returns false for the whole workgroup when a wait ran out or the launch
// was aborted (and raises the abort word).
template <int PE, class Map, class Tag>
__device__ bool ll_gather(const unsigned long long* base, uint32_t n, uint32_t ep, Map map, Tag tag, float* dst,
                          uint32_t* ctl, uint32_t* bad_s, uint64_t tmo) {
  const uint32_t tid = threadIdx.x;
  const uint64_t t0 = rtc();
  unsigned long long v[PE];
#pragma unroll
  for (int e = 0; e < PE; e++) {
    const uint32_t i = tid + kPT * e;
    v[e] = i < n ? ll_ld(base + map(i)) : 0ull;
  }
  bool ok = true;
  for (uint32_t it = 1;; it++) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < PE; e++) {
      const uint32_t i = tid + kPT * e;
      if (i < n && tag(v[e]) != ep) {
        all = false;
        v[e] = ll_ld(base + map(i));
      }
    }
    if (all) break;
    if ((it & 127) == 0 && (rtc() - t0 > tmo || aborted(ctl))) {
      ok = false;
      break;
    }
  }
#pragma unroll
  for (int e = 0; e < PE; e++) {
    const uint32_t i = tid + kPT * e;
    if (i < n) dst[i] = __uint_as_float((uint32_t)v[e]);
  }
  if (!ok) *bad_s = 1;
  __syncthreads();
  if (*bad_s) {
    if (tid == 0) {
      if (!aborted(ctl)) atomicOr(&ctl[0], 1u);   // this workgroup's wait timed out
      __hip_atomic_store(&ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);   // no load into LDS outlives the workgroup
    return false;
  }
  return true;
}

struct Ident {
  uint64_t o;
  __device__ uint64_t operator()(uint32_t i) const { return o + i; }
};
struct Tag32 {
  __device__ uint32_t operator()(unsigned long long v) const { return (uint32_t)(v >> 32); }
};

// block-wide sum of one value per thread (all threads get it)
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wsum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
  acc = fmaf(a.x, b.x, acc);
  acc = fmaf(a.y, b.y, acc);
  acc = fmaf(a.z, b.z, acc);
  return fmaf(a.w, b.w, acc);
}


__device__ __forceinline__ float p_sigmoid(float z) {
  if (0.0f <= z) return 1.0f / (1.0f + expf(-z));
  const float e = expf(z);
  return e / (1.0f + e);
}
__device__ __forceinline__ float p_log_sigmoid(float z) { return -(fmaxf(-z, 0.0f) + log1pf(expf(-fabsf(z)))); }

}  // namespace


// an LDS address for global_load_lds
typedef __attribute__((address_space(3))) void lds_void;

// HD the head dimension; NFD float4s a lane holds of a K = d row (d <= 256
// NFD); NFF of a K = f row (f <= 256 NFF). One workgroup of kPT threads
// (four waves) a CU.
//
// A phase's weights (and an attention unit's K and V rows) go from HBM
// straight into one of two 64 KB LDS buffers (global_load_lds_dwordx4: a
// wave instruction moves one 1 KB piece, lane l's 16 bytes to byte 16 l),
// issued at the start of the phase before; the other buffer holds the
// current phase's. A wave's weight pieces are laid out as it reads them
// back: (row, k chunk j) at piece (row_i NF + j), lane l's float4 at k =
// 4 (l + 64 j). Loads retire in issue order, so a phase waits for all of
// its wave's loads (vmcnt 0) before it reads its buffer: the next phase's
// pieces, issued before this phase's input polls, have landed by then too.
//
// TR: the trace build. Wave 0's first lane stamps four clock readings a
// phase (the clock's low 32 bits) into LDS (the phase's start; its inputs all seen; its weights
// landed; its outputs published) and the workgroup copies a step's stamps
// to a.trace after the pick, for the first a.trace_steps steps.
template <int HD, int NFD, int NFF, bool TR>
__global__ __launch_bounds__(kPT, 1) void k_decode1(PersistArgs a) {
  constexpr int QD = HD / 4;            // attention: dims a score lane holds (4 lanes a slot)
  constexpr int C4 = HD / 4;            // float4 columns of a head
  constexpr int GS = kPT / C4;          // attention V lanes: slot groups
  constexpr int KPASS = 2;              // 64 slots a pass: pieces of up to 128 slots
  constexpr int MAXP = 2;               // gate|up pairs a wave (f <= 8 G)
  constexpr int HBR = 4;                // head rows a wave a batch
  constexpr uint32_t WB = 4096;         // float4s a weight buffer (64 KB)
  constexpr uint32_t KV_V = KPASS * 64 * C4;   // V's float4 offset in an attention buffer
  __shared__ __align__(16) float4 wbuf[2][WB];
  __shared__ __align__(16) float xs[256 * NFF];
  __shared__ float red[8], qv[HD], kvv[HD], vvv[HD], al[HD], kh[HD], es[KPASS * 64], lgs[4][32];
  __shared__ float4 part4[4][C4];
  __shared__ float o16[4][4][4];
  __shared__ uint32_t bad_s;
  __shared__ unsigned long long key_s[4];
  __shared__ uint32_t tr_s[TR ? kMaxTracePhases : 1][4];
  uint32_t ph = 0;   // the step's phase (trace)
#define TS(i)                                       \
  do {                                              \
    if constexpr (TR) {                             \
      if (tid == 0) tr_s[ph][i] = (uint32_t)rtc();  \
    }                                               \
  } while (0)
#define TS_END()                                    \
  do {                                              \
    TS(3);                                          \
    ph++;                                           \
  } while (0)
  const uint32_t w = blockIdx.x, G = gridDim.x, tid = threadIdx.x, lane = tid & 63;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // (a scalar: the wave's branches are uniform)
  const uint32_t d = a.d, f = a.f, H = a.heads, ctx = a.ctx, L = a.L;
  if (tid == 0) bad_s = 0;
  __syncthreads();
  const float* W = a.W;
  float* Sseq = a.state + (size_t)a.seq[0] * a.seq_stride;
  uint32_t pos = a.pos[0], tok = a.tok[0];
  const uint32_t st0 = a.step[0];
  const uint32_t RO = (d + G - 1) / G;          // Wo / down rows a workgroup (one a wave)
  const uint32_t RGp = (f + G - 1) / G;         // gate|up pairs a workgroup
  const uint32_t orow = w * RO + wv;            // this wave's Wo / down row
  const bool orow_ok = wv < RO && orow < d;
  float x_own = 0.0f, xa_own = 0.0f;            // this wave's rows of x and xa
  const float sc = 1.0f / sqrtf((float)HD);
  const uint32_t np = a.np, PL = (ctx + np - 1) / np;
  const uint32_t v = a.vocab, RH = (v + G - 1) / G, h0 = w * RH, h1 = min(v, h0 + RH);
  const uint32_t nhb = (RH + 4 * HBR - 1) / (4 * HBR);   // head batches (each wave HBR rows a batch)
  // the layer table in LDS: its fields are read there (a global copy would
  // be re-read after every store the compiler cannot tell apart from it)
  __shared__ PLayer lays[kMaxPLayers];
  for (uint32_t i = tid; i < L * (uint32_t)(sizeof(PLayer) / 8); i += kPT)
    reinterpret_cast<uint64_t*>(lays)[i] = reinterpret_cast<const uint64_t*>(a.lay)[i];
  __syncthreads();
  const PLayer* Ls = lays;
  auto zero4 = []() { return make_float4(0.f, 0.f, 0.f, 0.f); };
  auto piece = [&](const float* src, uint32_t buf, uint32_t at) {
    // one 1 KB piece: lane l's 16 bytes from src (this lane's address) to
    // float4 at * 64 + l of the buffer
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)&wbuf[buf][at * 64], 16, 0, 0);
  };
  // ---- the pieces of each phase (this wave's)
  auto qkv_rows = [&](const PLayer& P) { return P.gla ? 4 * d : 3 * d; };
  auto dma_qkv = [&](const PLayer& P, uint32_t buf) {
    const uint32_t R = qkv_rows(P), RQ = (R + G - 1) / G;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t r = w * RQ + wv + 4 * i;
      if ((uint32_t)(wv + 4 * i) < RQ && r < R) {
        const float* row = W + (r < 3 * d ? P.wq + (size_t)r * d : P.wa + (size_t)(r - 3 * d) * d);
#pragma unroll
        for (int j = 0; j < NFD; j++) {
          const uint32_t k = 4 * (lane + 64 * j);
          piece(row + (k < d ? k : 0), buf, (wv * 4 + i) * NFD + j);
        }
      }
    }
  };
  auto dma_wo = [&](const PLayer& P, uint32_t buf) {
    if (!orow_ok) return;
    const float* row = W + P.wo + (size_t)orow * d;
#pragma unroll
    for (int j = 0; j < NFD; j++) {
      const uint32_t k = 4 * (lane + 64 * j);
      piece(row + (k < d ? k : 0), buf, wv * NFD + j);
    }
  };
  auto dma_gu = [&](const PLayer& P, uint32_t buf) {
#pragma unroll
    for (int i = 0; i < MAXP; i++) {
      const uint32_t jp = w * RGp + wv + 4 * i;
      if ((uint32_t)(wv + 4 * i) < RGp && jp < f) {
        const float* g = W + P.wg + (size_t)jp * d;
        const float* u = g + (size_t)f * d;
#pragma unroll
        for (int j = 0; j < NFD; j++) {
          const uint32_t k = 4 * (lane + 64 * j), kk = k < d ? k : 0;
          piece(g + kk, buf, ((wv * MAXP + i) * 2 + 0) * NFD + j);
          piece(u + kk, buf, ((wv * MAXP + i) * 2 + 1) * NFD + j);
        }
      }
    }
  };
  auto dma_wd = [&](const PLayer& P, uint32_t buf) {
    if (!orow_ok) return;
    const float* row = W + P.wd + (size_t)orow * f;
#pragma unroll
    for (int j = 0; j < NFF; j++) {
      const uint32_t k = 4 * (lane + 64 * j);
      piece(row + (k < f ? k : 0), buf, wv * NFF + j);
    }
  };
  // an attention unit's K rows then V rows of its piece of the ring: slot i
  // of the piece at float4 i C4 .. (V from KV_V); slots past the ring or the
  // piece read slot t0 (never used)
  auto dma_kv = [&](const PLayer& P, uint32_t buf) {
    if (P.gla || w >= H * np) return;
    const uint32_t h = w / np, t0 = (w % np) * PL;
    const float* Kr = Sseq + P.soff;
    const float* Vr = Kr + (size_t)ctx * d;
    const uint32_t nq = KPASS * 64 * C4 / 64;   // pieces of K (and of V)
    for (uint32_t q = wv; q < nq; q += 4) {
      const uint32_t i = q * (64 / C4) + lane / C4, t = t0 + i;
      const uint32_t tt = (i < PL && t < ctx) ? t : t0;
      const size_t off = (size_t)tt * d + h * HD + 4 * (lane % C4);
      piece(Kr + off, buf, q);
      piece(Vr + off, buf, KV_V / 64 + q);
    }
  };
  auto dma_head = [&](uint32_t batch, uint32_t buf) {
#pragma unroll
    for (int i = 0; i < HBR; i++) {
      const uint32_t r = h0 + wv + 4 * (batch * HBR + i);
      const uint32_t rr = r < h1 ? r : 0u;   // (row 0 stands in; its result is not used)
#pragma unroll
      for (int j = 0; j < NFD; j++) {
        const uint32_t k = 4 * (lane + 64 * j);
        piece(W + (size_t)rr * d + (k < d ? k : 0), buf, (wv * HBR + i) * NFD + j);
      }
    }
  };
  auto wb4 = [&](uint32_t buf, uint32_t at) { return wbuf[buf][at * 64 + lane]; };
  auto land = [&]() {
    __builtin_amdgcn_s_waitcnt(0);   // every load of this wave retired (LDS written)
    __syncthreads();
  };
  // xs[0..n) times the RMSNorm scale and the gains at gain[] (thread tid owns
  // entries tid + 256 e)
  auto norm_xs = [&](uint32_t n, const float (&g)[4]) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t i = tid + kPT * e;
      if (i < n) ss += xs[i] * xs[i];
    }
    ss = block_sum(ss, red);
    const float rs = 1.0f / sqrtf(ss / (float)n + 1.0e-5f);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t i = tid + kPT * e;
      if (i < n) xs[i] = (xs[i] * rs) * g[e];
    }
    __syncthreads();
  };
  auto load_gain = [&](float (&g)[4], uint64_t off) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t i = tid + kPT * e;
      g[e] = i < d ? W[off + i] : 0.0f;
    }
  };
  // this lane's float4 j of xs[0..n) (zero past n)
  auto xs4 = [&](uint32_t j, uint32_t n) {
    const uint32_t k = 4 * (lane + 64 * j);
    return k < n ? *reinterpret_cast<const float4*>(&xs[k]) : zero4();
  };
  auto fail_wg = [&]() {
    if (tid == 0) {
      if (!aborted(a.ctl)) atomicOr(&a.ctl[0], 1u);
      __hip_atomic_store(&a.ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  uint32_t pb = 0;          // the buffer holding the current phase's pieces
  dma_qkv(Ls[0], pb);
  uint32_t k = 0;
  bool nan_stop = false;
  for (; k < a.steps; k++) {
    const uint32_t ep = a.epoch0 + k + 1;
    unsigned long long* LL = a.ll + (size_t)(ep & 1) * a.ll_par;
    ph = 0;
    // layer 0's residual input is the token's embedding row
    if (orow_ok) x_own = W[(size_t)tok * d + orow];
    for (uint32_t l = 0; l < L; l++) {
      const PLayer P = Ls[l];
      float gra[4], grf[4];
      float svr = 0.0f, lamr = 0.0f, gqr = 0.0f, gkr = 0.0f, sinkr = 0.0f;
      // ---- norm, then q|k|v (|z): rows w RQ .. w RQ + RQ - 1
      __syncthreads();
      TS(0);
      dma_kv(P, pb ^ 1);
      load_gain(gra, P.ra);
      // the mix's own inputs that do not depend on this token
      if (P.gla) {
        if (w < H * C4) {
          const uint32_t h = w / C4, cb = w % C4, ar = tid >> 2, c = tid & 3;
          if ((int)ar < HD) svr = Sseq[P.soff + (size_t)h * HD * HD + (size_t)ar * HD + 4 * cb + c];
          if (a.rglru && (int)tid < HD) lamr = W[P.lam + h * HD + tid];
        }
      } else {
        if (a.qk && w < H * np && (int)tid < HD) {
          gqr = W[P.gq + tid];
          gkr = W[P.gk + tid];
        }
        if (a.sinks && w < H * C4) sinkr = W[P.sink + w / C4];
      }
      if (l == 0) {
        for (uint32_t i = tid; i < d; i += kPT) xs[i] = W[(size_t)tok * d + i];
      } else if (!ll_gather<4>(LL, d, ep, Ident{Ls[l - 1].e_x}, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) {
        return;
      }
      TS(1);
      land();
      TS(2);
      norm_xs(d, gra);
      {
        float4 xr[NFD];
#pragma unroll
        for (int j = 0; j < NFD; j++) xr[j] = xs4(j, d);
        const uint32_t R = qkv_rows(P), RQ = (R + G - 1) / G;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t r = w * RQ + wv + 4 * i;
          if ((uint32_t)(wv + 4 * i) < RQ && r < R) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < NFD; j++) acc = dot4(wb4(pb, (wv * 4 + i) * NFD + j), xr[j], acc);
            acc = wsum(acc);
            if (lane == 0) ll_put(LL + P.e_qkv + r, acc, ep);
          }
        }
      }
      TS_END();
      pb ^= 1;
      // ---- the mix (pieces: an attention unit's K and V, in pb)
      __syncthreads();
      TS(0);
      dma_wo(P, pb ^ 1);
      if (P.gla) {
        if (w < H * C4) {
          const uint32_t h = w / C4, cb = w % C4;
          // q, k, z of head h, then v's four columns of this block
          const uint64_t base = P.e_qkv;
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < (uint32_t)HD) return base + h * HD + i;
            if (i < 2u * HD) return base + d + h * HD + (i - HD);
            if (i < 3u * HD) return base + 3 * d + h * HD + (i - 2 * HD);
            return base + 2 * d + h * HD + 4 * cb + (i - 3 * HD);
          };
          if (!ll_gather<1>(LL, 3 * HD + 4, ep, map, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
          TS(1);
          TS(2);
          const uint32_t ar = tid >> 2, c = tid & 3;
          const float q = (int)tid < HD ? xs[tid] : 0.0f, kk = (int)tid < HD ? xs[HD + tid] : 0.0f;
          const float q2 = block_sum(q * q, red);
          const float k2 = block_sum(kk * kk, red);
          if ((int)tid < HD) {
            qv[tid] = q / sqrtf(1.0e-6f + q2);
            const float kn = kk / sqrtf(1.0e-6f + k2);
            const float z = xs[2 * HD + tid];
            if (a.rglru) {
              // dd.gate's RG-LRU arm (bend/Dense/Ex.bend:158-162), in float
              const float la = fminf(ANA_CAP, (8.0f * p_sigmoid(z)) * p_log_sigmoid(lamr));
              kh[tid] = kn * sqrtf(1.0f - expf(2.0f * la));
              al[tid] = expf(la);
            } else {
              al[tid] = p_sigmoid(z);
              kh[tid] = kn;
            }
          }
          __syncthreads();
          float o = 0.0f;
          if ((int)ar < HD) {
            const float s = fmaf(al[ar], svr, kh[ar] * xs[3 * HD + c]);
            Sseq[P.soff + (size_t)h * HD * HD + (size_t)ar * HD + 4 * cb + c] = s;
            o = qv[ar] * s;
          }
          // over the rows: lanes of one column (lane & 3) in a row of 16 by
          // rotations of 4 and 8, then the wave's four rows and the four
          // waves through LDS
          o += dpp<0x124>(o);   // row_ror:4
          o += dpp<0x128>(o);   // row_ror:8
          if ((lane & 15) < 4) o16[wv][lane >> 4][lane & 3] = o;
          __syncthreads();
          if (tid < 4) {
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) acc += o16[q >> 2][q & 3][tid];
            ll_put(LL + P.e_o + h * HD + 4 * cb + tid, acc, ep);
          }
        } else {
          TS(1);
          TS(2);
        }
        TS_END();
        land();
      } else {
        const uint32_t npos = pos < ctx - 1 ? pos : ctx - 1, slot = pos % ctx;
        if (w < H * np) {
          const uint32_t h = w / np, p = w % np, t0 = p * PL;
          const uint64_t base = P.e_qkv;
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < (uint32_t)HD) return base + h * HD + i;
            if (i < 2u * HD) return base + d + h * HD + (i - HD);
            return base + 2 * d + h * HD + (i - 2 * HD);
          };
          if (!ll_gather<1>(LL, 3 * HD, ep, map, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
          TS(1);
          land();
          TS(2);
          float q = (int)tid < HD ? xs[tid] : 0.0f, kx = (int)tid < HD ? xs[HD + tid] : 0.0f;
          if (a.qk) {
            // M.qkn (bend/Dense/Model.bend:39-42): gains 1 + g
            const float q2 = block_sum(q * q, red), k2 = block_sum(kx * kx, red);
            q = (q * (1.0f / sqrtf(q2 / (float)HD + 1.0e-5f))) * (1.0f + gqr);
            kx = (kx * (1.0f / sqrtf(k2 / (float)HD + 1.0e-5f))) * (1.0f + gkr);
          }
          if ((int)tid < HD) {
            qv[tid] = q;
            kvv[tid] = kx;
            vvv[tid] = xs[2 * HD + tid];
          }
          __syncthreads();
          // dd.sm.write: the piece holding this step's slot writes k and v
          if (slot >= t0 && slot < t0 + PL && (int)tid < HD) {
            float* Kr = Sseq + P.soff;
            Kr[(size_t)slot * d + h * HD + tid] = kvv[tid];
            Kr[(size_t)ctx * d + (size_t)slot * d + h * HD + tid] = vvv[tid];
          }
          // scores, 4 lanes a slot; the step's own slot from kvv
          float mloc = -INFINITY;
#pragma unroll
          for (int ps = 0; ps < KPASS; ps++) {
            const uint32_t i = (tid >> 2) + 64 * ps, t = t0 + i, qq = tid & 3;
            float acc = 0.0f;
            if (t == slot) {
#pragma unroll
              for (int c = 0; c < QD; c++) acc = fmaf(qv[qq * QD + c], kvv[qq * QD + c], acc);
            } else {
#pragma unroll
              for (int u = 0; u < QD / 4; u++) {
                const float4 k4 = wbuf[pb][i * C4 + qq * (QD / 4) + u];
                const uint32_t c = qq * QD + 4 * u;
                acc = fmaf(qv[c], k4.x, acc);
                acc = fmaf(qv[c + 1], k4.y, acc);
                acc = fmaf(qv[c + 2], k4.z, acc);
                acc = fmaf(qv[c + 3], k4.w, acc);
              }
            }
            acc += dpp<0xB1>(acc);
            acc += dpp<0x4E>(acc);
            const bool live = i < PL && t <= npos;
            const float y = live ? sc * acc : -INFINITY;
            if ((tid & 3) == 0) es[i] = y;
            mloc = fmaxf(mloc, y);
          }
          mloc = wmax(mloc);
          if (lane == 0) red[4 + wv] = mloc;
          __syncthreads();
          const float m = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
          float e = 0.0f;
          if (tid < KPASS * 64) {
            const float y = es[tid];
            e = y == -INFINITY ? 0.0f : __expf(y - m);
          }
          const float lsum = block_sum(e, red);   // (its first barrier orders the reads of es above)
          if (tid < KPASS * 64) es[tid] = e;
          __syncthreads();
          // o over the piece: thread (c4, g) takes slots g, g + GS, ...
          const uint32_t c4 = tid % C4, g = tid / C4;
          float4 o = zero4();
          for (uint32_t i = g; i < PL && i < KPASS * 64; i += GS) {
            float4 v4 = wbuf[pb][KV_V + i * C4 + c4];
            if (t0 + i == slot) v4 = make_float4(vvv[4 * c4], vvv[4 * c4 + 1], vvv[4 * c4 + 2], vvv[4 * c4 + 3]);
            const float ev = es[i];
            o.x = fmaf(ev, v4.x, o.x);
            o.y = fmaf(ev, v4.y, o.y);
            o.z = fmaf(ev, v4.z, o.z);
            o.w = fmaf(ev, v4.w, o.w);
          }
#pragma unroll
          for (int s2 = C4; s2 < 64; s2 <<= 1) {
            o.x += __shfl_xor(o.x, s2, 64);
            o.y += __shfl_xor(o.y, s2, 64);
            o.z += __shfl_xor(o.z, s2, 64);
            o.w += __shfl_xor(o.w, s2, 64);
          }
          if (lane < (uint32_t)C4) part4[wv][lane] = o;
          __syncthreads();
          unsigned long long* out = LL + P.e_part + (size_t)(h * np + p) * (HD + 2);
          if ((int)tid < HD) {
            const uint32_t c = tid / 4, e4 = tid % 4;
            float s2 = 0.0f;
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
              const float4 p4 = part4[q4][c];
              s2 += e4 == 0 ? p4.x : e4 == 1 ? p4.y : e4 == 2 ? p4.z : p4.w;
            }
            ll_put(out + 2 + tid, s2, ep);
          }
          if (tid == 0) {
            ll_put(out, m, ep);
            ll_put(out + 1, lsum, ep);
          }
        } else {
          TS(1);
          land();
          TS(2);
        }
        TS_END();
        TS(0);
        // ---- the pieces and the sink combined: o of head h, columns 4 cb ..
        if (w < H * C4) {
          const uint32_t h = w / C4, cb = w % C4;
          const uint64_t base = P.e_part + (uint64_t)h * np * (HD + 2);
          // entries: np maxima, np sums, then np x 4 columns
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < np) return base + (uint64_t)i * (HD + 2);
            if (i < 2 * np) return base + (uint64_t)(i - np) * (HD + 2) + 1;
            const uint32_t j = i - 2 * np;
            return base + (uint64_t)(j / 4) * (HD + 2) + 2 + 4 * cb + (j % 4);
          };
          if (!ll_gather<1>(LL, 6 * np, ep, map, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
          TS(1);
          TS(2);
          if (tid < 4) {
            float M = -INFINITY;
            for (uint32_t i = 0; i < np; i++) M = fmaxf(M, xs[i]);
            if (a.sinks) M = fmaxf(M, sinkr);
            float den = 0.0f, acc = 0.0f;
            for (uint32_t i = 0; i < np; i++) {
              const float mi = xs[i];
              const float wgt = mi == -INFINITY ? 0.0f : __expf(mi - M);
              den = fmaf(xs[np + i], wgt, den);
              acc = fmaf(xs[2 * np + 4 * i + tid], wgt, acc);
            }
            if (a.sinks) den += __expf(sinkr - M);
            ll_put(LL + P.e_o + h * HD + 4 * cb + tid, acc / den, ep);
          }
        } else {
          TS(1);
          TS(2);
        }
        TS_END();
      }
      pb ^= 1;
      // ---- xa = x + Wo o
      __syncthreads();
      TS(0);
      dma_gu(P, pb ^ 1);
      load_gain(grf, P.rf);
      if (!ll_gather<4>(LL, d, ep, Ident{P.e_o}, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
      TS(1);
      land();
      TS(2);
      {
        float acc = 0.0f;
        if (orow_ok) {
#pragma unroll
          for (int j = 0; j < NFD; j++) acc = dot4(wb4(pb, wv * NFD + j), xs4(j, d), acc);
        }
        acc = wsum(acc);
        xa_own = x_own + acc;
        if (lane == 0 && orow_ok) ll_put(LL + P.e_xa + orow, xa_own, ep);
      }
      TS_END();
      pb ^= 1;
      // ---- hh = silu(g) u on norm(xa)
      __syncthreads();
      TS(0);
      dma_wd(P, pb ^ 1);
      if (!ll_gather<4>(LL, d, ep, Ident{P.e_xa}, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
      TS(1);
      land();
      TS(2);
      norm_xs(d, grf);
      {
        float4 xr[NFD];
#pragma unroll
        for (int j = 0; j < NFD; j++) xr[j] = xs4(j, d);
#pragma unroll
        for (int i = 0; i < MAXP; i++) {
          const uint32_t jp = w * RGp + wv + 4 * i;
          if ((uint32_t)(wv + 4 * i) < RGp && jp < f) {
            float g = 0.0f, u = 0.0f;
#pragma unroll
            for (int j = 0; j < NFD; j++) {
              g = dot4(wb4(pb, ((wv * MAXP + i) * 2 + 0) * NFD + j), xr[j], g);
              u = dot4(wb4(pb, ((wv * MAXP + i) * 2 + 1) * NFD + j), xr[j], u);
            }
            g = wsum(g);
            u = wsum(u);
            if (lane == 0) ll_put(LL + P.e_hh + jp, g / (1.0f + __expf(-g)) * u, ep);
          }
        }
      }
      TS_END();
      pb ^= 1;
      // ---- x = xa + Wd hh
      __syncthreads();
      TS(0);
      if (l + 1 < L) dma_qkv(Ls[l + 1], pb ^ 1);
      else dma_head(0, pb ^ 1);
      if (!ll_gather<NFF>(LL, f, ep, Ident{P.e_hh}, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
      TS(1);
      land();
      TS(2);
      {
        float acc = 0.0f;
        if (orow_ok) {
#pragma unroll
          for (int j = 0; j < NFF; j++) acc = dot4(wb4(pb, wv * NFF + j), xs4(j, f), acc);
        }
        acc = wsum(acc);
        x_own = xa_own + acc;
        if (lane == 0 && orow_ok) ll_put(LL + P.e_x + orow, x_own, ep);
      }
      TS_END();
      pb ^= 1;
    }
    // ---- the head: logits of rows h0 .. h1 - 1 (wave wv: rows h0 + wv + 4 i),
    // batch b (rows h0 + wv + 4 (b HBR + i)) in buffer pb ^ (b & 1)
    {
      TS(0);
      float gfin[4];
      load_gain(gfin, a.fin);
      if (!ll_gather<4>(LL, d, ep, Ident{Ls[L - 1].e_x}, Tag32{}, xs, a.ctl, &bad_s, a.tmo)) return;
      TS(1);
      land();
      TS(2);
      norm_xs(d, gfin);
      float4 xr[NFD];
#pragma unroll
      for (int j = 0; j < NFD; j++) xr[j] = xs4(j, d);
      unsigned long long best = 0ull;
      for (uint32_t b = 0; b < nhb; b++) {
        const uint32_t cur = pb ^ (b & 1);
        if (b + 1 < nhb) {
          dma_head(b + 1, cur ^ 1);
          // batch b retired, batch b + 1 (HBR NFD pieces) may be in flight
          __builtin_amdgcn_s_waitcnt((HBR * NFD & 15) | (((HBR * NFD) >> 4) << 14) | (7 << 4) | (15 << 8));
        } else {
          __builtin_amdgcn_s_waitcnt(0);
        }
#pragma unroll
        for (int i = 0; i < HBR; i++) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < NFD; j++) acc = dot4(wb4(cur, (wv * HBR + i) * NFD + j), xr[j], acc);
          acc = wsum(acc);
          const uint32_t r = h0 + wv + 4 * (b * HBR + i);
          if (lane == 0 && r < h1) {
            lgs[wv][b * HBR + i] = acc;
            const unsigned long long kk = argmax_key(acc, r);
            best = kk > best ? kk : best;
          }
        }
      }
      if (lane == 0) key_s[wv] = best;
      __syncthreads();
      // the rows' logits, then (once they are stored) the key
      for (uint32_t i = tid; i < RH; i += kPT) {
        const uint32_t r = h0 + i;
        if (r < h1) __hip_atomic_store(a.LG + r, lgs[i & 3][i >> 2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) {
        unsigned long long b2 = key_s[0];
        for (int i = 1; i < 4; i++) b2 = key_s[i] > b2 ? key_s[i] : b2;
        // (value bits, 0xFFFF - index) in 48 bits, over a 16-bit epoch tag
        const uint32_t ix = 0xFFFFFFFFu - (uint32_t)(b2 & 0xFFFFFFFFull);
        const unsigned long long k48 = b2 ? ((b2 >> 32) << 16) | (0xFFFFull - ix) : 0ull;
        __hip_atomic_store(LL + a.e_key + w, (k48 << 16) | (ep & 0xFFFFu), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      TS_END();
      pb ^= (nhb & 1);
    }
    // ---- the pick (dd.pick's order): every workgroup reads every key; the
    // next step's first product loads meanwhile
    {
      __syncthreads();
      TS(0);
      dma_qkv(Ls[0], pb);
      unsigned long long kv = 0ull;
      bool ok = true;
      if (tid < G) {
        const uint64_t t0 = rtc();
        kv = ll_ld(LL + a.e_key + tid);
        for (uint32_t it = 1; (uint32_t)(kv & 0xFFFFu) != (ep & 0xFFFFu); it++) {
          if ((it & 127) == 0 && (rtc() - t0 > a.tmo || aborted(a.ctl))) {
            ok = false;
            break;
          }
          kv = ll_ld(LL + a.e_key + tid);
        }
      }
      if (!ok) bad_s = 1;
      unsigned long long mk = tid < G ? kv >> 16 : 0ull;
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(mk, m, 64);
        mk = o > mk ? o : mk;
      }
      __syncthreads();
      if (bad_s) {
        fail_wg();
        __builtin_amdgcn_s_waitcnt(0);
        return;
      }
      if (lane == 0) key_s[wv] = mk;
      __syncthreads();
      mk = key_s[0];
      for (int i = 1; i < 4; i++) mk = key_s[i] > mk ? key_s[i] : mk;
      __syncthreads();
      TS(1);
      TS(2);
      TS_END();
      if constexpr (TR) {
        // this step's stamps: [step][phase][workgroup][4]
        if (k < a.trace_steps) {
          for (uint32_t i = tid; i < ph * 4; i += kPT)
            a.trace[(((size_t)k * a.trace_phases + i / 4) * G + w) * 4 + i % 4] = tr_s[i / 4][i % 4];
        }
      }
      if (mk == 0ull) {
        // no logit reaches the maximum (NaN): the host picks by Sample.argmax
        nan_stop = true;
        break;
      }
      const uint32_t t = 0xFFFFu - (uint32_t)(mk & 0xFFFFull);
      if (w == 0 && tid == 0) a.out[(size_t)(st0 + k)] = t;
      tok = t;
      pos = pos + 1;
    }
  }
  // after the launch: the last fed token's residual row (this workgroup's
  // rows), and (workgroup 0) the loop's position, token, step and stop
  __builtin_amdgcn_s_waitcnt(0);   // no load into LDS outlives the workgroup
  if (orow_ok && lane == 0) a.X[orow] = x_own;
  if (w == 0 && tid == 0) {
    a.pos[0] = pos;
    a.tok[0] = tok;
    a.step[0] = st0 + k;
    if (nan_stop) a.pick[0] = v;
    a.ctl[2] = k;
    a.ctl[3] = nan_stop ? 1u : 0u;
  }
#undef TS
#undef TS_END
}


uint32_t decode1_pieces(const ana_config& c, uint32_t G) {
  if (c.heads == 0) return 0;
  uint32_t np = 16;
  while (np > 1 && c.heads * np > G) np >>= 1;
  while (np < 32 && (c.ctx + np - 1) / np > 128 && c.heads * np * 2 <= G) np <<= 1;
  return np;
}

bool decode1_fits(const ana_config& c, uint32_t G) {
  const uint32_t hd = c.heads ? c.d / c.heads : 0;
  if (G == 0 || G > 256 || c.layers == 0) return false;
  if (hd != 16 && hd != 32 && hd != 64) return false;
  if (c.d > 768 || c.d % 4 || c.f % 4 || c.f > 2048) return false;
  if ((4 * c.d + G - 1) / G > 16 || (c.d + G - 1) / G > 4) return false;   // q|k|v|z rows, Wo/down rows
  if ((c.f + G - 1) / G > 8) return false;                                  // gate|up pairs (two a wave)
  if ((c.vocab + G - 1) / G > 128) return false;                            // head rows (their logits in LDS)
  if (c.heads * (hd / 4) > G) return false;                                 // GLA and combine units
  const uint32_t np = decode1_pieces(c, G);
  if (np == 0 || c.heads * np > G || (c.ctx + np - 1) / np > 128 || 6 * np > 256) return false;
  if (c.vocab > 65536 || c.layers > kMaxPLayers) return false;
  return true;
}

uint32_t decode1_phases(const ana_config& c) {
  const uint32_t sm = c.layers / 4;
  return 5 * (c.layers - sm) + 6 * sm + 2;
}

hipError_t launch_decode1(const PersistArgs& a, uint32_t G, hipStream_t st) {
  void* args[] = {const_cast<PersistArgs*>(&a)};
  const uint32_t hd = a.d / a.heads;
  if (a.f > 2048) return hipErrorInvalidValue;
  const bool tr = a.trace && a.trace_steps;
  if (tr && a.trace_phases > kMaxTracePhases) return hipErrorInvalidValue;
#define L_(H)                                                                                                     \
  return hipLaunchCooperativeKernel(tr ? (const void*)k_decode1<H, 3, 8, true> : (const void*)k_decode1<H, 3, 8, false>, \
                                    dim3(G), dim3(kPT), args, 0, st)
  if (hd == 64) L_(64);
  if (hd == 32) L_(32);
  if (hd == 16) L_(16);
#undef L_
  return hipErrorInvalidValue;
}

}  // namespace ana


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
// for. There is no grid barrier.
//
// Each wave first issues its share of the next phase's weights (1 KB pieces
// streamed into LDS by global_load_lds), then polls its share of the
// current phase's inputs. A wave's loads retire in issue order, so its polls
// return only after its pieces have landed: the first poll then usually
// finds the inputs already published (polling at once, in waves of their
// own beside the stream, took a second round trip and ran slower; issuing
// the pieces after the inputs were in, before the compute, ran slower too),
// and when the inputs are in, both buffers are ready. The two 64 KB weight buffers
// are separate LDS objects and every phase knows at compile time which one
// it reads and which one its loads fill (a layer is compiled for each
// starting buffer), so the compiler never holds a read of one buffer behind
// the loads filling the other.
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

#include <type_traits>

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

// s_waitcnt with vmcnt = k (expcnt and lgkmcnt not waited on)
#define ANA_VM(k) (((k) & 15) | (((k) >> 4) << 14) | (7 << 4) | (15 << 8))

// a workgroup barrier that waits for this wave's LDS operations only: the
// weight pieces streaming into the other LDS buffer stay in flight (a
// __syncthreads() fence would wait for them), and no LDS access moves
// across it. Global memory is ordered where it matters by explicit waits
// (a wave's polls retire after its pieces; the head's logit stores).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt and expcnt not waited on
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The workgroup's threads poll n entries (entry i at base[map(i)]; thread t
// takes i = t + 256 e, e < PE) until each carries epoch ep in its upper
// half, then dst[i] = the value (and sq[i] its square, when sq is given).
// False (for this wave) when the wait passed tmo ticks or another
// workgroup gave up.
template <int PE, class Map>
__device__ __forceinline__ bool poll_gather(const unsigned long long* base, uint32_t n, uint32_t ep, Map map, float* dst,
                                            uint32_t* ctl, uint64_t tmo, float* sq = nullptr) {
  uint32_t pt = threadIdx.x;
  asm volatile("" : "+v"(pt));   // (its addresses are built here, not hoisted out of the caller's loop)
  unsigned long long v[PE];
#pragma unroll
  for (int e = 0; e < PE; e++) {
    const uint32_t i = pt + kPT * e;
    v[e] = i < n ? ll_ld(base + map(i)) : 0ull;
  }
  const uint64_t t0 = rtc();
  bool ok = true;
  for (uint32_t it = 1;; it++) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < PE; e++) {
      const uint32_t i = pt + kPT * e;
      if (i < n && (uint32_t)(v[e] >> 32) != ep) {
        all = false;
        v[e] = ll_ld(base + map(i));
      }
    }
    if (__all(all)) break;
    if ((it & 31) == 0 && (rtc() - t0 > tmo || aborted(ctl))) {
      ok = false;
      break;
    }
  }
#pragma unroll
  for (int e = 0; e < PE; e++) {
    const uint32_t i = pt + kPT * e;
    if (i < n) {
      const float f = __uint_as_float((uint32_t)v[e]);
      dst[i] = f;
      if (sq) sq[i] = f * f;
    }
  }
  return ok;
}

struct Ident {
  uint64_t o;
  __device__ uint64_t operator()(uint32_t i) const { return o + i; }
};

// block-wide sum of one value per thread (all threads get it)
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wsum(v);
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_barrier();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
  acc = fmaf(a.x, b.x, acc);
  acc = fmaf(a.y, b.y, acc);
  acc = fmaf(a.z, b.z, acc);
  return fmaf(a.w, b.w, acc);
}
// four bf16 (two a word, the lower half first) as floats
__device__ __forceinline__ float4 bf4(uint32_t a, uint32_t b) {
  return make_float4(__uint_as_float(a << 16), __uint_as_float(a & 0xFFFF0000u), __uint_as_float(b << 16),
                     __uint_as_float(b & 0xFFFF0000u));
}
__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

// the gates in the fast mode's float: exp and log on the hardware's
// base-2 units, the division as a reciprocal
__device__ __forceinline__ float p_sigmoid(float z) {
  const float e = __expf(-fabsf(z));
  const float r = __builtin_amdgcn_rcpf(1.0f + e);
  return 0.0f <= z ? r : e * r;
}
__device__ __forceinline__ float p_log_sigmoid(float z) { return -(fmaxf(-z, 0.0f) + __logf(1.0f + __expf(-fabsf(z)))); }

template <int B>
using IC = std::integral_constant<int, B>;

// the hardware's reciprocal and reciprocal square root (about 1 ulp): the
// fast mode's norms, gates and sums take them in place of IEEE division
__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float rsq(float x) { return __builtin_amdgcn_rsqf(x); }

// ---- the exact build's reductions: one lane's chain in the reference's
// order, a product and the sum it joins two roundings (bulk.c's product
// loop)

// s + v(0).x + v(0).y + ... + v(n4 - 1).w in order (numerics.h's block
// chain), every term a product the workgroup formed beforehand: a product
// formed next to its add puts its latency in the chain too
template <class F>
__device__ __forceinline__ float chain4(float s, uint32_t n4, F at) {
  return chain4_lds(s, n4, at, [](float x) { return x; });
}

// a wave's maximum by r = t > r ? t : r (a NaN never wins), as the exact
// attention takes its maxima
__device__ __forceinline__ float wmax_gt(float r) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float t = __shfl_xor(r, m, 64);
    r = t > r ? t : r;
  }
  return r;
}

}  // namespace


// an LDS address for global_load_lds
typedef __attribute__((address_space(3))) void lds_void;

// HD the head dimension; NFD float4s a lane holds of a K = d row (d <= 256
// NFD); NFF of a K = f row (f <= 256 NFF). One workgroup of kPT threads
// (four waves) a CU.
//
// A weight piece is 1 KB: a wave's global_load_lds_dwordx4 moves lane l's
// 16 bytes to byte 16 l of the piece. In fp32 a row of K = d is NFD pieces,
// lane l's float4 of piece j at k = 4 (l + 64 j); in bf16 (the first layer
// aside) it is (NFD + 1) / 2 pieces, lane l's eight values of piece j at
// k = 8 (l + 64 j). Each phase's pieces are numbered 0 .. P - 1 and wave u
// issues pieces u, u + 4, ....
//
// WT: the weights' type past the first layer and in the head (0 fp32 from
// a.W; 1 bf16, the layers' matrices at the PLayer h* addresses and the tied
// embedding at a.Wh); gains, lambdas and the first layer are fp32 from a.W
// in either build.
//
// TR: the trace build. Four clock readings a phase (the clock's low 32
// bits) go into LDS by thread 0: the phase's start; its inputs all seen;
// all waves met after their waits; its outputs published. The workgroup copies a step's stamps to a.trace
// after the pick, for the first a.trace_steps steps.
//
// EX: the exact build (ANA_EXACT_FP32, fp32 weights): every output takes
// the F32 steps of the exact kernels, in their order: the norms' sums of
// squares, the products, the GLA and attention sums as in-order chains in
// one lane each, exp/log/sqrt through double, IEEE division. The phases,
// the exchange and the weight stream are the fast build's; the attention
// publishes its raw scores and a second phase runs the softmax's chains
// over the whole window (its V columns streamed as slices of 4 columns).
template <int HD, int NFD, int NFF, bool TR, int WT, bool EX>
__global__ __launch_bounds__(kPT, 1) void k_decode1(PersistArgs a) {
  constexpr int QD = HD / 4;            // attention: dims a score lane holds (4 lanes a slot)
  constexpr int C4 = HD / 4;            // float4 columns of a head
  constexpr int GS = kPT / C4;          // attention V lanes: slot groups
  constexpr int KPASS = 2;              // 64 slots a pass: pieces of up to 128 slots
  constexpr int HBR = WT ? 8 : 5;       // head rows a wave a batch (its pieces fill a buffer)
  // a bf16 row's pieces: 512 values each (lane l's eight at k = 8 (l + 64 j))
  constexpr int PDH = (NFD + 1) / 2, PFH = (NFF + 1) / 2;
  constexpr int XN = NFD > 2 * PDH ? NFD : 2 * PDH;   // float4s a lane holds of a d vector
  constexpr uint32_t WB = 4096;         // float4s a weight buffer (64 KB)
  constexpr uint32_t KVQ = KPASS * C4;  // pieces of an attention unit's K (and of its V)
  constexpr uint32_t KV_V = KVQ * 64;   // V's float4 offset in an attention buffer
  constexpr int PEX = NFD;              // entries a thread polls of a d vector
  constexpr int PEF = NFF;              // of an f vector
  constexpr int PES = 1;                // of up to 256 entries
  __shared__ __align__(16) float4 wbA[WB];
  __shared__ __align__(16) float4 wbB[WB];
  __shared__ __align__(16) float xs[256 * NFF + (EX ? 256 : 0)];   // (exact: a window's scores and 4 values)
  __shared__ __align__(16) float qv[HD];
  __shared__ __align__(16) float kvv[HD];
  __shared__ __align__(16) float vvv[HD];
  __shared__ float red[8], es[KPASS * 64], lgs[4][40];
  __shared__ float4 part4[4][C4];
  __shared__ uint32_t bad_s;
  __shared__ unsigned long long key_s[4], pick_s[4];
  __shared__ uint32_t tr_s[TR ? kMaxTracePhases : 1][4];
  uint32_t ph = 0;   // the step's phase (trace)
#define TS(i)                                       \
  do {                                              \
    if constexpr (TR) {                             \
      if (tid == 0) tr_s[ph][i] = (uint32_t)rtc();  \
    }                                               \
  } while (0)
  // a phase's start: the barrier, its stamp, the thread index made opaque
#define BEGIN() \
  do {                  \
    lds_barrier();      \
    TS(0);              \
    fresh();            \
  } while (0)
  const uint32_t w = blockIdx.x, G = gridDim.x;
  // the thread's index and lane, made opaque again at every phase's start
  // (fresh()): what the compiler derives from them (addresses, masks) is
  // then rebuilt in each phase (a few instructions) instead of hoisted out
  // of the step loop, where ~140 such values held registers across every
  // phase (the build used all 256 VGPRs and spilled to AGPRs; 178 now)
  uint32_t tid = threadIdx.x, lane = tid & 63;
  auto fresh = [&]() {
    asm volatile("" : "+v"(tid));
    lane = tid & 63;
  };
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // (a scalar: the wave's branches are uniform)

  const uint32_t d = a.d, f = a.f, H = a.heads, ctx = a.ctx, L = a.L;
  if (tid == 0) bad_s = 0;
  const float* W = a.W;
  float* Sseq = a.state + (size_t)a.seq[0] * a.seq_stride;
  uint32_t pos = a.pos[0], tok = a.tok[0];
  const uint32_t st0 = a.step[0];
  const uint32_t RO = (d + G - 1) / G;          // Wo / down rows a workgroup (one a wave)
  const uint32_t RGp = (f + G - 1) / G;         // gate|up pairs a workgroup
  const uint32_t orow = w * RO + wv;            // this wave's Wo / down row
  const bool orow_ok = wv < RO && orow < d;
  float x_own = 0.0f, xa_own = 0.0f;            // this wave's rows of x and xa
  const float sc = 1.0f / sqrtf((float)HD), invd = 1.0f / (float)d;
  const uint32_t np = a.np, PL = (ctx + np - 1) / np;
  const uint32_t v = a.vocab, RH = (v + G - 1) / G, h0 = w * RH, h1 = min(v, h0 + RH);
  // head batches (each wave HBR rows a batch; exact: 16 rows' chunks of 256)
  const uint32_t nhb = EX ? ((RH + 63) / 64) * ((d + 255) / 256) : (RH + 4 * HBR - 1) / (4 * HBR);
  const bool gla_unit = w < H * C4, att_unit = w < H * np;
  // the layer table in LDS: its fields are read there (a global copy would
  // be re-read after every store the compiler cannot tell apart from it)
  __shared__ PLayer lays[kMaxPLayers];
  for (uint32_t i = tid; i < L * (uint32_t)(sizeof(PLayer) / 8); i += kPT)
    reinterpret_cast<uint64_t*>(lays)[i] = reinterpret_cast<const uint64_t*>(a.lay)[i];
  __syncthreads();
  const PLayer* Ls = lays;
  auto zero4 = []() { return make_float4(0.f, 0.f, 0.f, 0.f); };
  // the buffer of parity B
  auto bufp = [&](auto B) -> float4* {
    if constexpr (decltype(B)::value) return wbB;
    else return wbA;
  };
  // one 1 KB piece: lane l's 16 bytes from src (this lane's address) to
  // float4 at * 64 + l of the buffer. Weights take the non-temporal hint
  // (cache policy 2, nt): each is read once a step, and the step's stream
  // is larger than the caches (fast_fp32: 4707 -> 4815 tok/s on one box;
  // bf16, whose weights would fit the MALL, unchanged). K and V do not: the
  // rings are read again every step (+0.8% in either mode)
  auto piece = [&](const void* src, float4* buf, uint32_t at) {
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)&buf[at * 64], 16, 0, 2);
  };
  auto piece_kv = [&](const void* src, float4* buf, uint32_t at) {
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)&buf[at * 64], 16, 0, 0);
  };
  // ---- weights in either layout: WL 0 fp32 (a row of K is K / 256
  // pieces, lane l's float4 of piece j at k = 4 (l + 64 j)), WL 1 bf16 (a
  // row of K is K / 512 pieces, rounded up, lane l's eight values of piece j
  // at k = 8 (l + 64 j)). Every row takes the build's count of pieces (d <=
  // 256 NFD, f <= 256 NFF): lanes past K read the row's start, L2-resident
  // already, and meet zeros on the activation side
  auto npd = [&](auto WLc) -> uint32_t { return decltype(WLc)::value ? PDH : NFD; };   // a K = d row
  auto npf = [&](auto WLc) -> uint32_t { return decltype(WLc)::value ? PFH : NFF; };   // a K = f row
  auto kof = [&](auto WLc, uint32_t j) -> uint32_t {
    return decltype(WLc)::value ? 8 * (lane + 64 * j) : 4 * (lane + 64 * j);
  };
  // this lane's part of row r (rows of K), piece j, of the matrix at
  // parameter offset off (fp32) or at device address hp (bf16)
  auto wsrc = [&](auto WLc, uint64_t off, uint64_t hp, size_t r, uint32_t K, uint32_t j) -> const void* {
    const uint32_t k = kof(WLc, j);
    const size_t e = r * K + (k < K ? k : 0);
    if constexpr (decltype(WLc)::value) return reinterpret_cast<const uint16_t*>(hp) + e;
    else return W + off + e;
  };
  // ---- the pieces of each phase (issued by the loading waves)
  auto qkv_rows = [&](const PLayer& P) { return P.gla ? 4 * d : 3 * d; };
  auto dma_qkv = [&](auto WLc, const PLayer& P, float4* buf) {
    const uint32_t PD = npd(WLc);
    const uint32_t R = qkv_rows(P), RQ = (R + G - 1) / G, NP = RQ * PD;
    for (uint32_t q = wv; q < NP; q += 4) {
      const uint32_t i = q / PD, j = q % PD, r = min(w * RQ + i, R - 1);
      piece(r < 3 * d ? wsrc(WLc, P.wq, P.hq, r, d, j) : wsrc(WLc, P.wa, P.ha, r - 3 * d, d, j), buf, q);
    }
  };
  // an attention unit's K rows then V rows of its piece of the ring: slot i
  // of the piece at float4 i C4 .. (V from KV_V); slots past the ring or the
  // piece read slot t0 (never used)
  // (exact: K only, then the combine unit's V slices: piece KVQ + j, lane
  // l holds slot 64 j + l's 4 columns 4 cb .. of head h, read past the L2
  // (sc1): the unit holding a slot writes it, another XCD may read it)
  auto dma_kv = [&](const PLayer& P, float4* buf) {
    if (P.gla) return;
    const float* Kr = Sseq + P.soff;
    const float* Vr = Kr + (size_t)ctx * d;
    if constexpr (EX) {
      if (gla_unit) {
        const uint32_t h = w / C4, cb = w % C4, NS = (ctx + 63) / 64;
        for (uint32_t q = wv; q < NS; q += 4) {
          const uint32_t t = 64 * q + lane, tt = t < ctx ? t : 0u;
          __builtin_amdgcn_global_load_lds((const void*)(Vr + (size_t)tt * d + h * HD + 4 * cb),
                                           (lds_void*)&buf[(KVQ + q) * 64], 16, 0, 16);
        }
      }
    }
    if (!att_unit) return;
    const uint32_t h = w / np, t0 = (w % np) * PL;
    for (uint32_t q = wv; q < (EX ? 1u : 2u) * KVQ; q += 4) {
      const uint32_t qq = q < KVQ ? q : q - KVQ;
      const uint32_t i = qq * (64 / C4) + lane / C4, t = t0 + i;
      const uint32_t tt = (i < PL && t < ctx) ? t : t0;
      const size_t off = (size_t)tt * d + h * HD + 4 * (lane % C4);
      piece_kv((q < KVQ ? Kr : Vr) + off, buf, q);
    }
  };
  auto dma_wo = [&](auto WLc, const PLayer& P, float4* buf) {
    const uint32_t PD = npd(WLc), NP = RO * PD;
    for (uint32_t q = wv; q < NP; q += 4) {
      const uint32_t i = q / PD, j = q % PD, r = min(w * RO + i, d - 1);
      piece(wsrc(WLc, P.wo, P.ho, r, d, j), buf, q);
    }
  };
  // gate|up's pieces in three parts (part k: pieces [gu_cut(k), gu_cut(k +
  // 1))), issued over the phases before Wo's where its buffer is free: a
  // GLA layer's q|k|v|z and mix phases, a softmax layer's combine, then
  // Wo's phase itself, so no phase's stream is much longer than the
  // exchange it overlaps
  auto gu_cut = [&](auto WLc, uint32_t k) -> uint32_t {
    const uint32_t NP = RGp * 2 * npd(WLc), n1 = ((NP + 11) / 12) * 4;
    return min(NP, k * n1);
  };
  auto dma_gu = [&](auto WLc, const PLayer& P, float4* buf, uint32_t k0, uint32_t k1) {
    const uint32_t PD = npd(WLc), NP = k1 >= 3 ? RGp * 2 * PD : gu_cut(WLc, k1);
    for (uint32_t q = gu_cut(WLc, k0) + wv; q < NP; q += 4) {
      const uint32_t pi = q / (2 * PD), gu = (q / PD) & 1, j = q % PD, jp = min(w * RGp + pi, f - 1);
      const uint64_t up = gu ? (uint64_t)f * d : 0;   // up's rows follow gate's: up values on
      piece(wsrc(WLc, P.wg + up, P.hg + sizeof(uint16_t) * up, jp, d, j), buf, q);   // (hg: a byte address)
    }
  };
  auto dma_wd = [&](auto WLc, const PLayer& P, float4* buf) {
    const uint32_t PF = npf(WLc), NP = RO * PF;
    for (uint32_t q = wv; q < NP; q += 4) {
      const uint32_t i = q / PF, j = q % PF, r = min(w * RO + i, d - 1);
      piece(wsrc(WLc, P.wd, P.hd, r, f, j), buf, q);
    }
  };
  // the head's rows of batch b for wave u: h0 + u + 4 (b HBR + i), at
  // pieces (u HBR + i) HPD + j (row 0 stands in past h1; its result is not
  // used). Batch 0 of every wave, by the loading waves:
  constexpr IC<WT> HW{};                 // the head's layout (the mode's)
  constexpr int HPD = WT ? PDH : NFD;     // its pieces a row
  // (exact: batch b of wave u holds chunk c = b % NC (k = 256 c ..; NC
  // chunks a row) of its rows h0 + u + 4 (16 (b / NC) + i), i < 16, at
  // pieces 16 u + i)
  auto dma_headx = [&](uint32_t u, uint32_t b, float4* buf) {
    const uint32_t NC = (d + 255) / 256, g = b / NC, c = b % NC;
    for (uint32_t i = 0; i < 16; i++) {
      const uint32_t r = h0 + u + 4 * (16 * g + i), rr = r < h1 ? r : 0u;
      piece(wsrc(IC<0>{}, 0, 0, rr, d, c), buf, 16 * u + i);
    }
  };
  auto dma_head0 = [&](float4* buf) {
    if constexpr (EX) {
      dma_headx(wv, 0, buf);
      return;
    }
    const uint32_t NP = 4 * HBR * HPD;
    for (uint32_t q = wv; q < NP; q += 4) {
      const uint32_t rl = q / HPD, j = q % HPD, u = rl / HBR, i = rl % HBR;
      const uint32_t r = h0 + u + 4 * i, rr = r < h1 ? r : 0u;
      piece(wsrc(HW, 0, (uint64_t)a.Wh, rr, d, j), buf, q);
    }
  };
  // ... and batch b of this wave's own rows, by the wave itself
  auto dma_head_own = [&](uint32_t b, float4* buf) {
#pragma unroll
    for (int i = 0; i < HBR; i++) {
      const uint32_t r = h0 + wv + 4 * (b * HBR + i), rr = r < h1 ? r : 0u;
#pragma unroll
      for (int j = 0; j < HPD; j++) piece(wsrc(HW, 0, (uint64_t)a.Wh, rr, d, j), buf, (wv * HBR + i) * HPD + j);
    }
  };
  // this lane's float4 i of a vector in layout WL: fp32 at k = 4 (l + 64 i)
  // (piece i), bf16 at k = 8 (l + 64 (i / 2)) + 4 (i % 2) (half i % 2 of
  // piece i / 2); XW of them cover a d vector
  auto kx = [&](auto WLc, uint32_t i) -> uint32_t {
    return decltype(WLc)::value ? 8 * (lane + 64 * (i >> 1)) + 4 * (i & 1) : 4 * (lane + 64 * i);
  };
  // this lane's float4 i of xs[0..n) in layout WL (zero past n)
  auto xsw = [&](auto WLc, uint32_t i, uint32_t n) {
    const uint32_t k = kx(WLc, i);
    return k < n ? *reinterpret_cast<const float4*>(&xs[k]) : zero4();
  };
  // this lane's float4s of a gain vector at W + off (d entries; gains are
  // fp32 in every mode)
  auto load_g = [&](auto WLc, float4 (&g)[XN], uint64_t off) {
    constexpr int XW = decltype(WLc)::value ? 2 * PDH : NFD;
#pragma unroll
    for (int i = 0; i < XN; i++) {
      const uint32_t k = kx(WLc, i);
      g[i] = i < XW ? *reinterpret_cast<const float4*>(W + off + (k < d ? k : 0u)) : zero4();
    }
  };
  // this lane's float4s of xs[0..n) in layout WL (XV of them)
  auto xload = [&](auto WLc, auto& xv, uint32_t n) {
    constexpr int XV = sizeof(xv) / sizeof(float4);
#pragma unroll
    for (int i = 0; i < XV; i++) xv[i] = xsw(WLc, i, n);
  };
  // the RMSNorm of a d vector (this lane's float4s xv) folded into the
  // products: xg = x g, and the scale 1 / sqrt(mean(x^2) + 1e-5), which
  // every wave forms from the whole row itself
  auto norm_fold = [&](auto WLc, const float4 (&g)[XN], const float4 (&xv)[XN], float4 (&xg)[XN]) -> float {
    constexpr int XW = decltype(WLc)::value ? 2 * PDH : NFD;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < XW; i++) {
      ss = dot4(xv[i], xv[i], ss);
      xg[i] = mul4(xv[i], g[i]);
    }
    ss = wsum(ss);
    return rsq(ss * invd + 1.0e-5f);
  };
  // this lane's 16 bytes of piece pc of buf
  auto ldp = [&](const float4* buf, uint32_t pc) -> uint4 {
    return reinterpret_cast<const uint4*>(buf)[pc * 64 + lane];
  };
  // acc + those 16 bytes (four fp32 or eight bf16 weights) times x (this
  // lane's float4s of the piece: one in fp32, two in bf16)
  auto dotp = [&](auto WLc, uint4 u, const float4* x, float acc) -> float {
    if constexpr (decltype(WLc)::value) {
      acc = dot4(bf4(u.x, u.y), x[0], acc);
      return dot4(bf4(u.z, u.w), x[1], acc);
    } else {
      return dot4(make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                              __uint_as_float(u.w)),
                  x[0], acc);
    }
  };
  // Each phase's compute reads its x and its pieces out of LDS first, all
  // of them, then computes: the scheduler (which takes an LDS read to be a
  // few cycles) would otherwise put each read next to its use, and with one
  // wave a SIMD nothing would hide the reads' real latency
#define ISSUED() __builtin_amdgcn_sched_barrier(0)
  auto fail_wg = [&]() {
    if (tid == 0) {
      if (!aborted(a.ctl)) atomicOr(&a.ctl[0], 1u);
      __hip_atomic_store(&a.ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  // the meeting after the polls: the phase's inputs are in xs and its
  // pieces in LDS (each wave's polls retired after its pieces). False
  // (every wave) when a wait failed.
  auto meet = [&]() -> bool {
    lds_barrier();
    __builtin_amdgcn_s_waitcnt(ANA_VM(0));
    TS(2);
    if (bad_s) {
      fail_wg();
      __builtin_amdgcn_s_waitcnt(0);   // no load into LDS outlives the workgroup
      return false;
    }
    return true;
  };
  // a wave's poll verdict, before the meeting
  auto gathered = [&](bool ok) {
    if (!ok && lane == 0) bad_s = 1;
    if constexpr (TR) {
      if (tid == 0) tr_s[ph][1] = (uint32_t)rtc();
    }
  };
  auto pub = [&]() {
    TS(3);
    ph++;
  };

  // ---- exact build: M.norm (bend/Dense/Model.bend:27-30) of the d vector
  // in xs: ss = x0 x0 + x1 x1 + ... in order (one wave's chain over the
  // squares the gather left at xs + 1024), then rs = 1 / sqrt(ss / d +
  // 1e-5); the normed values (x rs) g are formed where they are used
  float* const sqx = EX ? xs + 1024 : nullptr;
  auto xrs = [&]() -> float {
    if (wv == 0) {
      const float ss = chain_sum_lds(0.0f, xs + 1024, d);   // (every lane the same chain)
      if (lane == 0) red[0] = ex_rms_scale(ss, (float)d);
    }
    lds_barrier();
    return red[0];
  };
  // ... the products of nrow rows (row i from piece i NP, K values each) in
  // place of the weights: x_k w_k, or with the norm (NORM) ((x_k rs) g_k)
  // w_k, g the gains at k = 4 tid (the only float4 of x its thread takes
  // then). With ROT row i's float4 k4 goes to (k4 + i mod 16) mod RP of
  // the row, so the rows one wave chains at once start on different LDS
  // banks (every row starts on bank 0: four such rows a wave on four waves
  // took 16 cycles a dependent add against 7); gate|up takes it (four rows
  // a wave), the others keep their places (one to three rows a wave, where
  // the rotation's barriers cost more than it saved). Thread t takes k4 = t
  // (and t + 256) of GR rows at a time: their reads, (ROT: a barrier,) their
  // writes
  auto xprod_rows = [&](float4* buf, uint32_t nrow, auto NPc, uint32_t K, auto NORMc, float rs, float4 g,
                        auto ROTc) {
    constexpr bool ROT = decltype(ROTc)::value;
    constexpr uint32_t RP = decltype(NPc)::value * 64, KT = (RP + kPT - 1) / kPT, GR = ROT ? 8 : 4;
    const float4* x4 = reinterpret_cast<const float4*>(xs);
    float4 x[KT];
#pragma unroll
    for (uint32_t kt = 0; kt < KT; kt++) {
      const uint32_t k4 = tid + kPT * kt;
      x[kt] = k4 < RP && 4 * k4 < K ? x4[k4] : zero4();
      if constexpr (decltype(NORMc)::value)
        x[kt] = make_float4((x[kt].x * rs) * g.x, (x[kt].y * rs) * g.y, (x[kt].z * rs) * g.z, (x[kt].w * rs) * g.w);
    }
    for (uint32_t i0 = 0; i0 < nrow; i0 += GR) {
      float4 pr[GR][KT];
#pragma unroll
      for (uint32_t j = 0; j < GR; j++) {
#pragma unroll
        for (uint32_t kt = 0; kt < KT; kt++) {
          const uint32_t k4 = tid + kPT * kt;
          const float4 w4 = i0 + j < nrow && k4 < RP ? buf[(i0 + j) * RP + k4] : zero4();
          pr[j][kt] = make_float4(x[kt].x * w4.x, x[kt].y * w4.y, x[kt].z * w4.z, x[kt].w * w4.w);
        }
      }
      if constexpr (ROT) lds_barrier();
#pragma unroll
      for (uint32_t j = 0; j < GR; j++) {
#pragma unroll
        for (uint32_t kt = 0; kt < KT; kt++) {
          const uint32_t k4 = tid + kPT * kt, i = i0 + j, q = k4 + (ROT ? i & 15 : 0);
          if (i < nrow && k4 < RP && 4 * k4 < K) buf[i * RP + (q < RP ? q : q - RP)] = pr[j][kt];
        }
      }
    }
    lds_barrier();
  };
  auto xprod_n = [&](float4* buf, uint32_t nrow, auto NPc, float rs, float4 g, auto ROTc) {
    xprod_rows(buf, nrow, NPc, d, std::true_type{}, rs, g, ROTc);
  };
  auto xprod = [&](float4* buf, uint32_t nrow, auto NPc, uint32_t K) {
    xprod_rows(buf, nrow, NPc, K, std::false_type{}, 1.0f, zero4(), std::false_type{});
  };
  // ... and row i's sum of its products (so placed), (((0 + p0) + p1) +
  // ...), k ascending
  auto xrow = [&](const float4* buf, uint32_t i, auto NPc, uint32_t K, auto ROTc) -> float {
    constexpr uint32_t RP = decltype(NPc)::value * 64;
    // (two contiguous runs: float4s 0 .. RP - r - 1 at r .., the rest from
    // the row's start; an index wrapped at each read put its VALU work in
    // the chain)
    const float4* row = buf + i * RP;
    const uint32_t r = decltype(ROTc)::value ? i & 15 : 0u, K4 = K >> 2, n1 = K4 < RP - r ? K4 : RP - r;
    const float4* a = row + r;
    const float s1 = chain4(0.0f, n1, [&](uint32_t q) { return a[q]; });
    return chain4(s1, K4 - n1, [&](uint32_t q) { return row[q]; });
  };

  // one layer, compiled for the buffer parity its first phase reads (B)
  // and the layout of its weights (WLc); false when a wait failed
  auto layer = [&](auto B, auto WLc, uint32_t l, uint32_t ep, unsigned long long* LL) -> bool {
    constexpr int PB = decltype(B)::value;
    constexpr bool WL = decltype(WLc)::value;
    constexpr int PDc = WL ? PDH : NFD;           // pieces of a K = d row
    constexpr int PFc = WL ? PFH : NFF;           // of a K = f row
    constexpr int XW = WL ? 2 * PDH : NFD;        // float4s a lane holds of a d vector
    constexpr int XF = WL ? 2 * PFH : NFF;        // of an f vector
    constexpr int XS = WL ? 2 : 1;                // float4s a lane holds of a piece
    float4* bufB = bufp(IC<PB>{});
    float4* bufN = bufp(IC<1 - PB>{});
    const PLayer P = Ls[l];
    // ---- norm, then q|k|v (|z) (in bufB): rows w RQ .. w RQ + RQ - 1,
    // wave wv the rows wv + 4 i
    BEGIN();
    float4 g4[XN];
    if constexpr (EX) g4[0] = 4 * tid < d ? *reinterpret_cast<const float4*>(W + P.ra + 4 * tid) : zero4();
    else load_g(WLc, g4, P.ra);
    float svr, lamr, gqr, gkr, sinkr;
    // the mix's own inputs that do not depend on this token: GLA column
    // 4 cb + wv of head h (lane a: row a of S) and the RG-LRU lambdas; the
    // attention's qk gains and sink
    // (loaded by every thread, from a valid place where the thread has none:
    // a load that only some paths make leaves the compiler unsure which
    // registers still await one, and it then waits for every load in
    // flight, this phase's weight pieces included, at the next write to
    // such a register)
    {
      const uint32_t h = gla_unit ? w / C4 : 0u, cb = w % C4, la = (int)lane < HD ? lane : 0u;
      const uint32_t tq = (int)tid < HD ? tid : 0u;
      svr = Sseq[(P.gla ? P.soff : 0u) + (size_t)h * HD * HD + (size_t)la * HD + 4 * cb + wv];
      lamr = W[(P.gla && a.rglru ? P.lam : 0u) + h * HD + la];
      gqr = W[(!P.gla && a.qk ? P.gq : 0u) + tq];
      gkr = W[(!P.gla && a.qk ? P.gk : 0u) + tq];
      sinkr = W[(!P.gla && a.sinks ? P.sink : 0u) + h];
    }
    if (l == 0 && orow_ok) x_own = W[(size_t)tok * d + orow];
    dma_kv(P, bufN);
    if (P.gla) dma_gu(WLc, P, bufN, 0, 1);
    {
      bool ok = true;
      if (l == 0) {
        // layer 0's input is the token's embedding row
        for (uint32_t i = tid; i < d; i += kPT) {
          const float v = W[(size_t)tok * d + i];
          xs[i] = v;
          if (EX) xs[1024 + i] = v * v;
        }
      } else {
        ok = poll_gather<PEX>(LL, d, ep, Ident{Ls[l - 1].e_x}, xs, a.ctl, a.tmo, sqx);
      }
      gathered(ok);
    }
    if (!meet()) return false;
    if constexpr (EX) {
      const uint32_t R = qkv_rows(P), RQ = (R + G - 1) / G;
      xprod_n(bufB, RQ, IC<NFD>{}, xrs(), g4[0], std::false_type{});
      // row i on wave i % 4, lane i / 4: one chain over k (every lane
      // runs one, those past the rows the last row's: a dependent add
      // takes about half again the cycles with most lanes masked off)
      const uint32_t i = wv + 4 * lane, ic = i < RQ ? i : RQ - 1;
      const float s = xrow(bufB, ic, IC<NFD>{}, d, std::false_type{});
      const uint32_t r = w * RQ + i;
      if (lane < 4 && i < RQ && r < R) ll_put(LL + P.e_qkv + r, s, ep);
    } else {
      const uint32_t R = qkv_rows(P), RQ = (R + G - 1) / G;
      float4 xv[XN], xg[XN];
      xload(WLc, xv, d);
      uint4 pw[4][PDc];
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const uint32_t i = min(wv + 4 * kk, RQ - 1);
#pragma unroll
        for (int j = 0; j < PDc; j++) pw[kk][j] = ldp(bufB, i * PDc + j);
      }
      ISSUED();
      const float rs = norm_fold(WLc, g4, xv, xg);
      float res[4];
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < PDc; j++) acc = dotp(WLc, pw[kk][j], &xg[XS * j], acc);
        res[kk] = acc;
      }
      wsum_n(res);
#pragma unroll
      for (int kk = 0; kk < 4; kk++) res[kk] *= rs;
      if (lane < 4) {
        const uint32_t i = wv + 4 * lane, r = w * RQ + i;
        const float val = lane == 0 ? res[0] : lane == 1 ? res[1] : lane == 2 ? res[2] : res[3];
        if (i < RQ && r < R) ll_put(LL + P.e_qkv + r, val, ep);
      }
    }
    pub();
    // ---- the mix (an attention unit's K and V pieces in bufN)
    BEGIN();
    dma_wo(WLc, P, bufB);
    if (P.gla) {
      dma_gu(WLc, P, bufN, 1, 2);
      {
        bool ok = true;
        if (gla_unit) {
          const uint32_t h = w / C4, cb = w % C4;
          // q, k, z of head h, then v's four columns of this block
          const uint64_t base = P.e_qkv;
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < (uint32_t)HD) return base + h * HD + i;
            if (i < 2u * HD) return base + d + h * HD + (i - HD);
            if (i < 3u * HD) return base + 3 * d + h * HD + (i - 2 * HD);
            return base + 2 * d + h * HD + 4 * cb + (i - 3 * HD);
          };
          ok = poll_gather<PES>(LL, 3 * HD + 4, ep, map, xs, a.ctl, a.tmo);
        }
        gathered(ok);
      }
      if (!meet()) return false;
      // (the layer's constants, opaque from here: nothing computed from them
      // is moved up to where they were loaded, which would wait for them there)
      asm volatile("" : "+v"(svr), "+v"(lamr), "+v"(gqr), "+v"(gkr), "+v"(sinkr));
      if (EX && gla_unit) {
        // dd.gla.tok as the exact kernels take it (k_gla_w): every lane
        // runs the norms' chains over q and k; S'_ac = (al_a S_ac) + (kh_a
        // v_c); o_c = ((0 + qh_0 S'_0c) + qh_1 S'_1c) + ..., a ascending
        // (wave wv: column c = 4 cb + wv, lane a: row a)
        const uint32_t h = w / C4, cb = w % C4, c = 4 * cb + wv;
        const bool on = (int)lane < HD;
        // q's and k's sums of squares: the squares by waves 0 and 1, one
        // lane's chain each
        if (wv < 2 && on) xs[1024 + 64 * wv + lane] = xs[HD * wv + lane] * xs[HD * wv + lane];
        lds_barrier();
        if (wv < 2) {
          const float ss = chain_sum_lds(0.0f, xs + 1024 + 64 * wv, HD);
          if (lane == 0) red[wv] = ss;
        }
        lds_barrier();
        const float s0 = red[0], s1 = red[1];
        const float qa = on ? xs[lane] : 0.0f, ka = on ? xs[HD + lane] : 0.0f;
        const float z = on ? xs[2 * HD + lane] : 0.0f, vc = xs[3 * HD + wv];
        const float kn = ka / csqrt(1.0e-6f + s1);
        float al, kh;
        if (a.rglru) {
          const float la = ex_rglru_log_gate(z, lamr);
          kh = kn * ex_rglru_write_scale(la);
          al = dexp(la);
        } else {
          al = ex_sigmoid(z);
          kh = kn;
        }
        const float qh = qa / csqrt(1.0e-6f + s0);
        const float sn = (al * svr) + (kh * vc);
        if (on) Sseq[P.soff + (size_t)h * HD * HD + (size_t)lane * HD + c] = sn;
        float* pr = xs + 256 + 64 * wv;   // this wave's qh_a S'_ac (past the gathered values)
        if (on) pr[lane] = qh * sn;
        __builtin_amdgcn_wave_barrier();
        const float o = chain_sum_lds(0.0f, pr, HD);
        if (lane == 0) ll_put(LL + P.e_o + h * HD + c, o, ep);
      } else if (gla_unit) {
        // wave wv: column c = 4 cb + wv of head h's state, lane a its row a
        const uint32_t h = w / C4, cb = w % C4, c = 4 * cb + wv;
        const bool on = (int)lane < HD;
        const float qa = on ? xs[lane] : 0.0f, ka = on ? xs[HD + lane] : 0.0f;
        const float q2 = wsum(qa * qa), k2 = wsum(ka * ka);
        const float qn = qa * rsq(1.0e-6f + q2), kn = ka * rsq(1.0e-6f + k2);
        const float z = on ? xs[2 * HD + lane] : 0.0f, vc = xs[3 * HD + wv];
        float al, kh;
        if (a.rglru) {
          // dd.gate's RG-LRU arm (bend/Dense/Ex.bend:158-162), in float
          const float la = fminf(ANA_CAP, (8.0f * p_sigmoid(z)) * p_log_sigmoid(lamr));
          kh = kn * sqrtf(1.0f - expf(2.0f * la));   // (1 - e^2la cancels: the exact exp)
          al = __expf(la);
        } else {
          al = p_sigmoid(z);
          kh = kn;
        }
        const float s = fmaf(al, svr, kh * vc);
        if (on) Sseq[P.soff + (size_t)h * HD * HD + (size_t)lane * HD + c] = s;
        const float o = wsum(on ? qn * s : 0.0f);
        if (lane == 0) ll_put(LL + P.e_o + h * HD + c, o, ep);
      }
      pub();
    } else {
      const uint32_t npos = pos < ctx - 1 ? pos : ctx - 1, slot = pos % ctx;
      {
        bool ok = true;
        if (att_unit) {
          const uint32_t h = w / np;
          const uint64_t base = P.e_qkv;
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < (uint32_t)HD) return base + h * HD + i;
            if (i < 2u * HD) return base + d + h * HD + (i - HD);
            return base + 2 * d + h * HD + (i - 2 * HD);
          };
          ok = poll_gather<PES>(LL, 3 * HD, ep, map, xs, a.ctl, a.tmo);
        }
        gathered(ok);
      }
      if (!meet()) return false;
      // (the layer's constants, opaque from here: nothing computed from them
      // is moved up to where they were loaded, which would wait for them there)
      asm volatile("" : "+v"(svr), "+v"(lamr), "+v"(gqr), "+v"(gkr), "+v"(sinkr));
      if (EX && att_unit) {
        // k_attn_scores' steps: M.qkn (bend/Dense/Model.bend:39-42) by the
        // norms' chains, dd.sm.write of the row's k and v by the unit
        // holding the slot, then each live slot's score sc (q . k) (one
        // chain a slot, c ascending), published raw (dead slots -inf)
        const uint32_t h = w / np, p = w % np, t0 = p * PL;
        if ((int)tid < HD) {
          qv[tid] = xs[tid];
          kvv[tid] = xs[HD + tid];
          vvv[tid] = xs[2 * HD + tid];
        }
        lds_barrier();
        if (a.qk) {
          if ((int)tid < HD) {
            xs[1024 + tid] = qv[tid] * qv[tid];
            xs[1088 + tid] = kvv[tid] * kvv[tid];
          }
          lds_barrier();
          if (wv < 2) {
            const float ss = chain_sum_lds(0.0f, xs + 1024 + 64 * wv, HD);
            if (lane == 0) red[wv] = ex_rms_scale(ss, (float)HD);
          }
          lds_barrier();
          if ((int)tid < HD) {
            qv[tid] = (qv[tid] * red[0]) * (1.0f + gqr);
            kvv[tid] = (kvv[tid] * red[1]) * (1.0f + gkr);
          }
          lds_barrier();
        }
        if (slot >= t0 && slot < t0 + PL && (int)tid < HD) {
          float* Kr = Sseq + P.soff;
          __hip_atomic_store(Kr + (size_t)slot * d + h * HD + tid, kvv[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(Kr + (size_t)ctx * d + (size_t)slot * d + h * HD + tid, vvv[tid], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
        // the products q_c K_tc in place of K, slot i's float4 u at i C4 +
        // (u + i) mod C4 (so the slots' chains read different banks), and
        // the own slot's q_c k_c
        {
          const float4* q4 = reinterpret_cast<const float4*>(qv);
          constexpr uint32_t NQ = (KPASS * 64 * C4 + kPT - 1) / kPT;
          float4 pk[NQ];
#pragma unroll
          for (uint32_t j = 0; j < NQ; j++) {
            const uint32_t e = tid + kPT * j, u = e % C4;
            const float4 k4 = e < KPASS * 64 * C4 ? bufN[e] : zero4(), q = q4[u];
            pk[j] = make_float4(q.x * k4.x, q.y * k4.y, q.z * k4.z, q.w * k4.w);
          }
          if ((int)tid < HD) xs[1152 + tid] = qv[tid] * kvv[tid];
          lds_barrier();
#pragma unroll
          for (uint32_t j = 0; j < NQ; j++) {
            const uint32_t e = tid + kPT * j, i = e / C4, u = e % C4;
            if (e < KPASS * 64 * C4) bufN[i * C4 + (u + i) % C4] = pk[j];
          }
          lds_barrier();
        }
        if (tid < PL) {
          const uint32_t t = t0 + tid;
          float acc;
          if (t == slot) {
            acc = chain_sum_lds(0.0f, xs + 1152, HD);
          } else {
            const float4* k4 = bufN + tid * C4;
            acc = chain4(0.0f, C4, [&](uint32_t u) { return k4[(u + tid) % C4]; });
          }
          const float sc = 1.0f / csqrt((float)HD);
          ll_put(LL + P.e_part + (size_t)(h * np + p) * PL + tid, t <= npos ? sc * acc : -INFINITY, ep);
        }
      } else if (att_unit) {
        const uint32_t h = w / np, p = w % np, t0 = p * PL;
        float q = (int)tid < HD ? xs[tid] : 0.0f, kx = (int)tid < HD ? xs[HD + tid] : 0.0f;
        if (a.qk) {
          // M.qkn (bend/Dense/Model.bend:39-42): gains 1 + g (wave 0 holds
          // the head's dims)
          const float q2 = wsum(q * q), k2 = wsum(kx * kx);
          q = (q * rsq(q2 * (1.0f / HD) + 1.0e-5f)) * (1.0f + gqr);
          kx = (kx * rsq(k2 * (1.0f / HD) + 1.0e-5f)) * (1.0f + gkr);
        }
        if ((int)tid < HD) {
          qv[tid] = q;
          kvv[tid] = kx;
          vvv[tid] = xs[2 * HD + tid];
        }
        lds_barrier();
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
              const float4 k4 = bufN[i * C4 + qq * (QD / 4) + u];
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
        lds_barrier();
        const float m = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
        float e = 0.0f;
        if (tid < KPASS * 64) {
          const float y = es[tid];
          e = y == -INFINITY ? 0.0f : __expf(y - m);
        }
        const float lsum = block_sum(e, red);   // (its first barrier orders the reads of es above)
        if (tid < KPASS * 64) es[tid] = e;
        lds_barrier();
        // o over the piece: thread (c4, g) takes slots g, g + GS, ...
        const uint32_t c4 = tid % C4, g = tid / C4;
        float4 o = zero4();
        for (uint32_t i = g; i < PL && i < KPASS * 64; i += GS) {
          float4 v4 = bufN[KV_V + i * C4 + c4];
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
        lds_barrier();
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
      }
      pub();
      // ---- the pieces and the sink combined: o of head h, columns 4 cb ..
      // (the K and V pieces are read: gate|up's first two parts go to their
      // buffer)
      BEGIN();
      if constexpr (!EX) dma_gu(WLc, P, bufN, 0, 2);   // (exact: the V slices in that buffer are read here)
      if constexpr (EX) {
        // exact: v's 4 columns into xs[0 .. 4), the head's scores of slots
        // 0 .. npos into xs[4 ..)
        bool ok = true;
        if (gla_unit) {
          const uint32_t h = w / C4, cb = w % C4;
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < 4) return P.e_qkv + 2 * d + h * HD + 4 * cb + i;
            const uint32_t t = i - 4;
            return P.e_part + (uint64_t)(h * np + t / PL) * PL + t % PL;
          };
          ok = poll_gather<NFF + 1>(LL, npos + 5, ep, map, xs, a.ctl, a.tmo);
        }
        gathered(ok);
      } else {
        bool ok = true;
        if (gla_unit) {
          const uint32_t h = w / C4, cb = w % C4;
          const uint64_t base = P.e_part + (uint64_t)h * np * (HD + 2);
          // entries: np maxima, np sums, then np x 4 columns
          auto map = [&](uint32_t i) -> uint64_t {
            if (i < np) return base + (uint64_t)i * (HD + 2);
            if (i < 2 * np) return base + (uint64_t)(i - np) * (HD + 2) + 1;
            const uint32_t j = i - 2 * np;
            return base + (uint64_t)(j / 4) * (HD + 2) + 2 + 4 * cb + (j % 4);
          };
          ok = poll_gather<PES>(LL, 6 * np, ep, map, xs, a.ctl, a.tmo);
        }
        gathered(ok);
      }
      if (!meet()) return false;
      if (EX && gla_unit) {
        // k_attn_out's steps over the whole window: m (a maximum: any
        // order), dd.sm.max with the sink, e_t = exp(y_t - m), then one chain
        // a column oi_c = ((0 + e_0 V_0c) + e_1 V_1c) + ... and se = ((0 +
        // e_0) + e_1) + ..., t ascending; o_c = (1 / (se (+ exp(sink - m))))
        // oi_c. The own slot's V comes from the gathered v.
        const uint32_t h = w / C4, cb = w % C4, nl = npos + 1;
        float* e = xs + 4;
        float mloc = -INFINITY;
        for (uint32_t t = tid; t < nl; t += kPT) {
          const float y = e[t];
          mloc = y > mloc ? y : mloc;
        }
        mloc = wmax_gt(mloc);
        if (lane == 0) red[4 + wv] = mloc;
        lds_barrier();
        float m = red[4];
        for (int u = 1; u < 4; u++) m = red[4 + u] > m ? red[4 + u] : m;
        if (a.sinks) m = ex_max(m, sinkr);
        for (uint32_t t = tid; t < nl; t += kPT) e[t] = dexp(e[t] - m);
        const float4* vs = bufN + KVQ * 64;   // slot t's 4 columns
        if (tid < 4) reinterpret_cast<float*>(bufN + KVQ * 64)[4 * slot + tid] = xs[tid];
        lds_barrier();
        // the products e_t V_tc, column c at pc + c PC (past Wo's pieces in
        // the other buffer, which this phase neither reads nor loads)
        constexpr uint32_t PC = 2048 + 4;
        float* pc = reinterpret_cast<float*>(bufB) + 4096;
        for (uint32_t t0 = tid; t0 < nl; t0 += 4 * kPT) {
          float4 v[4];
          float et[4];
#pragma unroll
          for (uint32_t j = 0; j < 4; j++) {
            const uint32_t t = t0 + kPT * j < nl ? t0 + kPT * j : t0;
            v[j] = vs[t];
            et[j] = e[t];
          }
#pragma unroll
          for (uint32_t j = 0; j < 4; j++) {
            const uint32_t t = t0 + kPT * j;
            if (t < nl) {
              pc[t] = et[j] * v[j].x;
              pc[PC + t] = et[j] * v[j].y;
              pc[2 * PC + t] = et[j] * v[j].z;
              pc[3 * PC + t] = et[j] * v[j].w;
            }
          }
        }
        lds_barrier();
        if (wv == 0) {
          const float oi = chain_sum_lds(0.0f, pc + (lane & 3) * PC, nl);
          if (lane < 4) part4[0][lane].x = oi;
        } else if (wv == 1) {
          const float se = chain_sum_lds(0.0f, e, nl);
          if (lane == 0) red[0] = a.sinks ? se + dexp(sinkr - m) : se;
        }
        lds_barrier();
        if (wv == 0 && lane < 4) ll_put(LL + P.e_o + h * HD + 4 * cb + lane, (1.0f / red[0]) * part4[0][lane].x, ep);
      } else if (gla_unit && wv == 0) {
        // lane i: piece i (np <= 64)
        const uint32_t h = w / C4, cb = w % C4;
        const bool on = lane < np;
        const float mi = on ? xs[lane] : -INFINITY;
        float M = wmax(mi);
        if (a.sinks) M = fmaxf(M, sinkr);
        const float wgt = on && mi != -INFINITY ? __expf(mi - M) : 0.0f;
        float den = wsum(on ? xs[np + lane] * wgt : 0.0f);
        if (a.sinks) den += __expf(sinkr - M);
        float acc[4];
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] = wsum(on ? xs[2 * np + 4 * lane + c] * wgt : 0.0f);
        if (lane < 4) {
          const float val = lane == 0 ? acc[0] : lane == 1 ? acc[1] : lane == 2 ? acc[2] : acc[3];
          ll_put(LL + P.e_o + h * HD + 4 * cb + lane, val * rcp(den), ep);
        }
      }
      pub();
    }
    // ---- xa = x + Wo o (Wo in bufB)
    BEGIN();
    float4 gf[XN];
    if constexpr (EX) gf[0] = 4 * tid < d ? *reinterpret_cast<const float4*>(W + P.rf + 4 * tid) : zero4();
    else load_g(WLc, gf, P.rf);
    dma_gu(WLc, P, bufN, EX && !P.gla ? 0 : 2, 3);
    gathered(poll_gather<PEX>(LL, d, ep, Ident{P.e_o}, xs, a.ctl, a.tmo));
    if (!meet()) return false;
    if constexpr (EX) {
      // add2 (bend/Dense/Model.bend:44-45): x + (the row's chain), lane 0
      xprod(bufB, RO, IC<NFD>{}, d);
      const float s = xrow(bufB, wv < RO ? wv : 0u, IC<NFD>{}, d, std::false_type{});
      if (orow_ok) {
        xa_own = x_own + s;
        if (lane == 0) ll_put(LL + P.e_xa + orow, xa_own, ep);
      }
    } else if (orow_ok) {
      float4 xv[XW];
      xload(WLc, xv, d);
      uint4 pw[PDc];
#pragma unroll
      for (int j = 0; j < PDc; j++) pw[j] = ldp(bufB, wv * PDc + j);
      ISSUED();
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < PDc; j++) acc = dotp(WLc, pw[j], &xv[XS * j], acc);
      xa_own = x_own + wsum(acc);
      if (lane == 0) ll_put(LL + P.e_xa + orow, xa_own, ep);
    }
    pub();
    // ---- hh = silu(g) u on norm(xa) (gate|up in bufN): wave wv the pairs
    // wv + 4 i
    BEGIN();
    dma_wd(WLc, P, bufB);
    gathered(poll_gather<PEX>(LL, d, ep, Ident{P.e_xa}, xs, a.ctl, a.tmo, sqx));
    if (!meet()) return false;
    if constexpr (EX) {
      // M.norm, then lane 2 i + u: gate (u 0) or up (u 1) of pair wv + 4 i;
      // hh = silu(g) u (bend/Dense/Model.bend:58-59)
      xprod_n(bufN, 2 * RGp, IC<NFD>{}, xrs(), gf[0], std::true_type{});
      const uint32_t pi = wv + 4 * ((lane & 3) >> 1), u = lane & 1, pc = pi < RGp ? pi : RGp - 1;
      const float s = xrow(bufN, pc * 2 + u, IC<NFD>{}, d, std::true_type{});
      const float up = __shfl_down(s, 1, 64);
      if (lane < 4 && u == 0) {
        const uint32_t jp = w * RGp + pi;
        if (pi < RGp && jp < f) ll_put(LL + P.e_hh + jp, ex_silu(s) * up, ep);
      }
    } else {
      float4 xv[XN], xg[XN];
      xload(WLc, xv, d);
      uint4 pw[2][2][PDc];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t pi = min(wv + 4 * i, RGp - 1);
#pragma unroll
        for (int j = 0; j < PDc; j++) {
          pw[i][0][j] = ldp(bufN, (pi * 2 + 0) * PDc + j);
          pw[i][1][j] = ldp(bufN, (pi * 2 + 1) * PDc + j);
        }
      }
      ISSUED();
      const float rs = norm_fold(WLc, gf, xv, xg);
      float hv[2], gu4[4];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int j = 0; j < PDc; j++) {
          g = dotp(WLc, pw[i][0][j], &xg[XS * j], g);
          u = dotp(WLc, pw[i][1][j], &xg[XS * j], u);
        }
        gu4[2 * i] = g;
        gu4[2 * i + 1] = u;
      }
      wsum_n(gu4);
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const float g = gu4[2 * i] * rs, u = gu4[2 * i + 1] * rs;
        hv[i] = g * rcp(1.0f + __expf(-g)) * u;
      }
      if (lane < 2) {
        const uint32_t pi = wv + 4 * lane, jp = w * RGp + pi;
        if (pi < RGp && jp < f) ll_put(LL + P.e_hh + jp, lane == 0 ? hv[0] : hv[1], ep);
      }
    }
    pub();
    // ---- x = xa + Wd hh (Wd in bufB)
    BEGIN();
    if (l + 1 < L) dma_qkv(IC<WT>{}, Ls[l + 1], bufN);   // (layers past the first: the mode's layout)
    else dma_head0(bufN);
    gathered(poll_gather<PEF>(LL, f, ep, Ident{P.e_hh}, xs, a.ctl, a.tmo));
    if (!meet()) return false;
    if constexpr (EX) {
      xprod(bufB, RO, IC<NFF>{}, f);
      const float s = xrow(bufB, wv < RO ? wv : 0u, IC<NFF>{}, f, std::false_type{});
      if (orow_ok) {
        x_own = xa_own + s;
        if (lane == 0) ll_put(LL + P.e_x + orow, x_own, ep);
      }
    } else if (orow_ok) {
      float4 xv[XF];
      xload(WLc, xv, f);
      uint4 pw[PFc];
#pragma unroll
      for (int j = 0; j < PFc; j++) pw[j] = ldp(bufB, wv * PFc + j);
      ISSUED();
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < PFc; j++) acc = dotp(WLc, pw[j], &xv[XS * j], acc);
      x_own = xa_own + wsum(acc);
      if (lane == 0) ll_put(LL + P.e_x + orow, x_own, ep);
    }
    pub();
    return true;
  };

  // the head: logits of rows h0 .. h1 - 1 (wave wv: rows h0 + wv + 4 i),
  // batch b (rows h0 + wv + 4 (b HBR + i)) in the buffer of parity B ^ (b &
  // 1); batch 0 came from the loading waves, the rest each wave loads itself
  auto head = [&](auto B, uint32_t ep, unsigned long long* LL) -> bool {
    constexpr int PB = decltype(B)::value;
    float4* b0 = bufp(IC<PB>{});
    float4* b1 = bufp(IC<1 - PB>{});
    BEGIN();
    float4 gf[XN];
    if constexpr (EX) gf[0] = 4 * tid < d ? *reinterpret_cast<const float4*>(W + a.fin + 4 * tid) : zero4();
    else load_g(HW, gf, a.fin);
    gathered(poll_gather<PEX>(LL, d, ep, Ident{Ls[L - 1].e_x}, xs, a.ctl, a.tmo, sqx));
    if (!meet()) return false;
    unsigned long long best = 0ull;
    if constexpr (EX) {
      // the final M.norm, then each row's chain over k (lane i < 16 of wave
      // wv: row h0 + wv + 4 (16 g + i), its chunks c = 0 .. NC - 1 in
      // batches g NC + c, the chain carried across them)
      {
        const float rs = xrs();
        if (4 * tid < d) {
          float4* x4 = reinterpret_cast<float4*>(xs) + tid;
          const float4 v = *x4, g = gf[0];
          *x4 = make_float4((v.x * rs) * g.x, (v.y * rs) * g.y, (v.z * rs) * g.z, (v.w * rs) * g.w);
        }
        lds_barrier();
      }
      const uint32_t NC = (d + 255) / 256;
      float hacc = 0.0f;
      auto rowsx = [&](float4* cur, uint32_t b) {
        const uint32_t g = b / NC, c = b % NC;
        const uint32_t n4 = min(64u, (d - 256 * c) >> 2);
        // the wave's products x_k w_k in place of its 16 pieces, piece i's
        // float4 q at (q + i) mod 64 (so the 16 rows' chains read
        // different banks): every lane's reads first, then its writes
        {
          float4* base = cur + 16 * wv * 64;
          const float4 xv = lane < n4 ? reinterpret_cast<const float4*>(xs)[64 * c + lane] : zero4();
          float4 pv[16];
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const float4 w4 = base[i * 64 + lane];
            pv[i] = make_float4(xv.x * w4.x, xv.y * w4.y, xv.z * w4.z, xv.w * w4.w);
          }
          __builtin_amdgcn_sched_barrier(0);
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int i = 0; i < 16; i++) base[i * 64 + ((lane + i) & 63)] = pv[i];
          __builtin_amdgcn_wave_barrier();
        }
        {
          const uint32_t li = lane & 15;   // (lanes 16 .. 63 repeat lanes 0 .. 15's chains)
          const float4* wr = cur + (16 * wv + li) * 64;
          hacc = chain4(hacc, n4, [&](uint32_t q) { return wr[(q + li) & 63]; });
        }
        if (c == NC - 1) {
          const uint32_t i = 16 * g + lane, r = h0 + wv + 4 * i;
          if (lane < 16 && r < h1) {
            lgs[wv][i] = hacc;
            const unsigned long long kk = argmax_key(hacc, r);
            best = kk > best ? kk : best;
          }
          hacc = 0.0f;
        }
      };
      for (uint32_t b = 0; b < nhb; b += 2) {
        if (b + 1 < nhb) {
          dma_headx(wv, b + 1, b1);
          if (b > 0) __builtin_amdgcn_s_waitcnt(ANA_VM(16));
        } else if (b > 0) {
          __builtin_amdgcn_s_waitcnt(0);
        }
        rowsx(b0, b);
        if (b + 1 < nhb) {
          if (b + 2 < nhb) {
            dma_headx(wv, b + 2, b0);
            __builtin_amdgcn_s_waitcnt(ANA_VM(16));
          } else {
            __builtin_amdgcn_s_waitcnt(0);
          }
          rowsx(b1, b + 1);
        }
      }
      for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(best, m, 64);
        best = o > best ? o : best;
      }
    } else {
    float4 xv[XN], xg[XN];
    xload(HW, xv, d);
    const float rs = norm_fold(HW, gf, xv, xg);
    auto rows = [&](float4* cur, uint32_t b) {
      uint4 pw[HBR][HPD];
#pragma unroll
      for (int i = 0; i < HBR; i++) {
#pragma unroll
        for (int j = 0; j < HPD; j++) pw[i][j] = ldp(cur, (wv * HBR + i) * HPD + j);
      }
      ISSUED();
      float hs[HBR];
#pragma unroll
      for (int i = 0; i < HBR; i++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < HPD; j++) acc = dotp(HW, pw[i][j], &xg[(WT ? 2 : 1) * j], acc);
        hs[i] = acc;
      }
      wsum_n(hs);
#pragma unroll
      for (int i = 0; i < HBR; i++) {
        const float acc = hs[i] * rs;
        const uint32_t r = h0 + wv + 4 * (b * HBR + i);
        if (lane == 0 && r < h1) {
          lgs[wv][b * HBR + i] = acc;
          const unsigned long long kk = argmax_key(acc, r);
          best = kk > best ? kk : best;
        }
      }
    };
    // batch b in b0 and b + 1 in b1, each issued one batch ahead (this
    // wave's rows, which it alone reads: its own count suffices, no
    // barrier)
    for (uint32_t b = 0; b < nhb; b += 2) {
      if (b + 1 < nhb) {
        dma_head_own(b + 1, b1);
        if (b > 0) __builtin_amdgcn_s_waitcnt(ANA_VM(HBR * HPD));
      } else if (b > 0) {
        __builtin_amdgcn_s_waitcnt(0);
      }
      rows(b0, b);
      if (b + 1 < nhb) {
        if (b + 2 < nhb) {
          dma_head_own(b + 2, b0);
          __builtin_amdgcn_s_waitcnt(ANA_VM(HBR * HPD));
        } else {
          __builtin_amdgcn_s_waitcnt(0);
        }
        rows(b1, b + 1);
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
    pub();
    return true;
  };

  // the pick (dd.pick's order): the poll wave reads every workgroup's key
  // while the loading waves load the next step's first product into the
  // buffer of parity B; the best key (0: no logit reached the maximum)
  auto pick = [&](auto B, uint32_t ep, unsigned long long* LL, bool& ok) -> unsigned long long {
    constexpr int PB = decltype(B)::value;
    BEGIN();
    dma_qkv(IC<0>{}, Ls[0], bufp(IC<PB>{}));   // (the first layer: fp32 in every mode)
    {
      const uint32_t pt = tid;
      unsigned long long kv[PES];
      bool good = true;
#pragma unroll
      for (int e = 0; e < PES; e++) {
        const uint32_t i = pt + kPT * e;
        kv[e] = i < G ? ll_ld(LL + a.e_key + i) : 0ull;
      }
      const uint64_t t0 = rtc();
      for (uint32_t it = 1;; it++) {
        bool all = true;
#pragma unroll
        for (int e = 0; e < PES; e++) {
          const uint32_t i = pt + kPT * e;
          if (i < G && (uint32_t)(kv[e] & 0xFFFFu) != (ep & 0xFFFFu)) {
            all = false;
            kv[e] = ll_ld(LL + a.e_key + i);
          }
        }
        if (__all(all)) break;
        if ((it & 31) == 0 && (rtc() - t0 > a.tmo || aborted(a.ctl))) {
          good = false;
          break;
        }
      }
      unsigned long long mk = 0ull;
#pragma unroll
      for (int e = 0; e < PES; e++) {
        const uint32_t i = pt + kPT * e;
        const unsigned long long k = i < G ? kv[e] >> 16 : 0ull;
        mk = k > mk ? k : mk;
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(mk, m, 64);
        mk = o > mk ? o : mk;
      }
      if (lane == 0) pick_s[wv] = mk;
      gathered(good);
    }
    ok = meet();
    unsigned long long r = 0ull;
    for (uint32_t u = 0; u < 4; u++) r = pick_s[u] > r ? pick_s[u] : r;
    pub();
    return r;
  };

  dma_qkv(IC<0>{}, Ls[0], wbA);
  __builtin_amdgcn_s_waitcnt(0);
  uint32_t pb = 0;          // the buffer parity the next phase reads
  uint32_t k = 0;
  bool nan_stop = false;
  for (; k < a.steps; k++) {
    const uint32_t ep = a.epoch0 + k + 1;
    unsigned long long* LL = a.ll + (size_t)(ep & 1) * a.ll_par;
    ph = 0;
    for (uint32_t l = 0; l < L; l++) {
      // the first layer's weights are fp32 in every mode, the rest the mode's
      bool ok;
      if (l == 0) ok = pb ? layer(IC<1>{}, IC<0>{}, l, ep, LL) : layer(IC<0>{}, IC<0>{}, l, ep, LL);
      else ok = pb ? layer(IC<1>{}, IC<WT>{}, l, ep, LL) : layer(IC<0>{}, IC<WT>{}, l, ep, LL);
      if (!ok) return;
      pb ^= 1;   // five buffer phases a layer
    }
    if (!(pb ? head(IC<1>{}, ep, LL) : head(IC<0>{}, ep, LL))) return;
    pb ^= (nhb & 1);
    bool ok = true;
    const unsigned long long mk = pb ? pick(IC<1>{}, ep, LL, ok) : pick(IC<0>{}, ep, LL, ok);
    if (!ok) return;
    if constexpr (TR) {
      // this step's stamps: [step][phase][workgroup][4]
      lds_barrier();
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
#undef BEGIN
#undef ISSUED
}


uint32_t decode1_pieces(const ana_config& c, uint32_t G) {
  if (c.heads == 0) return 0;
  uint32_t np = 16;
  while (np > 1 && c.heads * np > G) np >>= 1;
  while (np < 32 && (c.ctx + np - 1) / np > 128 && c.heads * np * 2 <= G) np <<= 1;
  return np;
}

bool decode1_fits(const ana_config& c, uint32_t G, bool exact) {
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
  // exact: a head's scores of the whole window in LDS, and its K pieces
  // with the combine's V slices in one buffer
  if (exact && (c.ctx > 2048 || 2 * (hd / 4) + (c.ctx + 63) / 64 > 64)) return false;
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
  // bf16 weights: 16-byte pieces of eight values, so rows of K = d and
  // K = f start on 16 bytes when d and f are multiples of 8 (the host places
  // every matrix on 16 bytes)
  const bool bf = a.Wh != nullptr;
  if (bf && (a.d % 8 || a.f % 8)) return hipErrorInvalidValue;
  if (a.exact && (bf || a.ctx > 2048)) return hipErrorInvalidValue;
#define K_(H, T)                                                        \
  (a.exact ? (const void*)k_decode1<H, 3, 8, T, 0, true>               \
   : bf    ? (const void*)k_decode1<H, 3, 8, T, 1, false>              \
           : (const void*)k_decode1<H, 3, 8, T, 0, false>)
#define L_(H) return hipLaunchCooperativeKernel(tr ? K_(H, true) : K_(H, false), dim3(G), dim3(kPT), args, 0, st)
  if (hd == 64) L_(64);
  if (hd == 32) L_(32);
  if (hd == 16) L_(16);
#undef L_
#undef K_
  return hipErrorInvalidValue;
}

}  // namespace ana

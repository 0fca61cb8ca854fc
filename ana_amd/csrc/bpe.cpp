// The fast BPE tokenizer of bend/Tokenizer.bend on the host: the .bpe
// artifact, its identity, pretokenization, encode and decode, and the
// SHA-256 the identity digests with (bend/Sha256.bend).
//
// Tokens: 0 = BOS, 1 = EOS, 2..257 the 256 bytes, then one token per merge
// in id order (a merge's id is its token and its rank).
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ana.h"

namespace {

// ------------------------------------------------------------------ SHA-256

// FIPS 180-4. The round constants and the initial hash are defined as the
// first 32 bits of the fractional parts of the cube roots of the first 64
// primes and of the square roots of the first 8; they are computed from
// that definition once (long double carries the 35 significant bits each
// needs, and the known-answer tests pin the result).
struct ShaConst {
  uint32_t k[64], h0[8];
  ShaConst() {
    uint32_t primes[64];
    int n = 0;
    for (uint32_t c = 2; n < 64; c++) {
      bool p = true;
      for (int i = 0; i < n && primes[i] * primes[i] <= c; i++)
        if (c % primes[i] == 0) p = false;
      if (p) primes[n++] = c;
    }
    for (int i = 0; i < 64; i++) {
      long double r = cbrtl((long double)primes[i]);
      k[i] = (uint32_t)(uint64_t)floorl((r - floorl(r)) * 4294967296.0L);
    }
    for (int i = 0; i < 8; i++) {
      long double r = sqrtl((long double)primes[i]);
      h0[i] = (uint32_t)(uint64_t)floorl((r - floorl(r)) * 4294967296.0L);
    }
  }
};

const ShaConst& sha_const() {
  static const ShaConst c;
  return c;
}

inline uint32_t ror(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

std::string sha256_hex(const uint8_t* p, size_t n) {
  const ShaConst& C = sha_const();
  uint32_t h[8];
  memcpy(h, C.h0, sizeof h);
  // the message, a 1 bit, zeros to 56 mod 64, the 64-bit bit length
  std::vector<uint8_t> m(p, p + n);
  m.push_back(0x80);
  while (m.size() % 64 != 56) m.push_back(0);
  const uint64_t bits = (uint64_t)n * 8;
  for (int i = 7; i >= 0; i--) m.push_back((uint8_t)(bits >> (8 * i)));
  for (size_t off = 0; off < m.size(); off += 64) {
    uint32_t w[64];
    for (int t = 0; t < 16; t++)
      w[t] = (uint32_t)m[off + 4 * t] << 24 | (uint32_t)m[off + 4 * t + 1] << 16 |
             (uint32_t)m[off + 4 * t + 2] << 8 | (uint32_t)m[off + 4 * t + 3];
    for (int t = 16; t < 64; t++) {
      const uint32_t s0 = ror(w[t - 15], 7) ^ ror(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = ror(w[t - 2], 17) ^ ror(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int t = 0; t < 64; t++) {
      const uint32_t S1 = ror(e, 6) ^ ror(e, 11) ^ ror(e, 25);
      const uint32_t ch = (e & f) ^ (~e & g);
      const uint32_t t1 = hh + S1 + ch + C.k[t] + w[t];
      const uint32_t S0 = ror(a, 2) ^ ror(a, 13) ^ ror(a, 22);
      const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
      const uint32_t t2 = S0 + mj;
      hh = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
  }
  // eight lowercase hex digits a word, zeros kept (U32.hex8)
  char out[65];
  for (int i = 0; i < 8; i++) snprintf(out + 8 * i, 9, "%08x", h[i]);
  return std::string(out, 64);
}

// ------------------------------------------------------------------ artifact

constexpr uint32_t kNone = 0xffffffffu;

inline bool is_sp(uint8_t c) { return c == 32 || c == 13 || c == 9; }   // skip.sp's blanks
inline bool is_digit(uint8_t c) { return c >= 48 && c <= 57; }

}  // namespace

struct ana_bpe {
  uint32_t vocab = 258;
  bool v2 = true;
  std::vector<uint32_t> a, b;                  // merge i (token 258 + i) = (a[i], b[i])
  std::unordered_map<uint32_t, uint32_t> rank; // pair key (a << 16 | b) -> merge id (the latest)

  uint32_t rank_of(uint32_t x, uint32_t y) const {
    auto it = rank.find(x << 16 | y);
    return it == rank.end() ? kNone : it->second;
  }
};

namespace {

// Bpe.parse (bend/Tokenizer.bend:146-295): "BPE <vocab> [v2]", then one
// "a b new" row per merge; ids contiguous from 258 and vocab = 258 + rows,
// else no tokenizer. Rows are read as the reference reads them: blanks
// skipped, a missing number reads 0, the rest of the line dropped.
bool parse_bpe(const uint8_t* s, size_t n, ana_bpe* t) {
  size_t i = 0;
  if (n == 0 || s[0] != 'B') return false;
  auto skip_sp = [&]() { while (i < n && is_sp(s[i])) i++; };
  auto num = [&]() {
    uint32_t v = 0;
    while (i < n && is_digit(s[i])) v = v * 10 + (s[i++] - 48);
    return v;
  };
  auto skip_line = [&]() {
    while (i < n && s[i] != 10) i++;
    if (i < n) i++;
  };
  i = n < 3 ? n : 3;
  skip_sp();
  const uint32_t vocab = num();
  size_t j = i;
  while (j < n && is_sp(s[j])) j++;
  t->v2 = j + 1 < n && s[j] == 'v' && s[j + 1] == '2';
  skip_line();
  t->a.clear();
  t->b.clear();
  t->rank.clear();
  uint32_t next = 258;
  bool ok = true;
  while (i < n && t->a.size() < 65536) {
    skip_sp();
    if (i >= n) break;
    const uint32_t x = num();
    skip_sp();
    const uint32_t y = num();
    skip_sp();
    const uint32_t z = num();
    skip_line();
    if (z != next) ok = false;
    next++;
    t->a.push_back(x);
    t->b.push_back(y);
    // the rank table lists a pair's merge ids latest first; a lookup takes
    // the first
    t->rank[x << 16 | y] = z;
  }
  t->vocab = vocab;
  return ok && (uint64_t)258 + t->a.size() == vocab;
}

const char* rule_name(bool v2) { return v2 ? "ascii-space-run+lf-prefix-v2" : "ascii-space-prefix+lf-boundary"; }

// Bpe.identity (bend/Tokenizer.bend:330-336)
std::string identity(const ana_bpe* t) {
  std::string canon = "fastbpe-word-v1\nvocab " + std::to_string(t->vocab) + "\n";
  for (size_t k = 0; k < t->a.size(); k++)
    canon += std::to_string(t->a[k]) + " " + std::to_string(t->b[k]) + " " + std::to_string(258 + k) + "\n";
  return std::string("fastbpe-word-v1:bos=0:eos=1:bytes=2..257:pretoken=") + rule_name(t->v2) +
         ":vocab=" + std::to_string(t->vocab) + ":sha256=" +
         sha256_hex(reinterpret_cast<const uint8_t*>(canon.data()), canon.size());
}

// ------------------------------------------------------------------ pretokenize

inline bool ordinary(uint8_t c) { return c != 32 && c != 10; }

// pretokenize (bend/Tokenizer.bend:338-472): words as [begin, end) spans of
// the input, except that V2 words may join a kept space with the run after
// it, which is contiguous in the input as well, so spans suffice.
void pretokenize(const uint8_t* s, size_t n, bool v2, std::vector<std::pair<size_t, size_t>>* out) {
  size_t i = 0;
  auto ord_end = [&](size_t k) {
    while (k < n && ordinary(s[k])) k++;
    return k;
  };
  while (i < n) {
    const uint8_t h = s[i];
    if (!v2) {
      // V1: a newline alone, a space and the ordinary run after it, or an
      // ordinary run
      if (h == 10) {
        out->push_back({i, i + 1});
        i += 1;
      } else if (h == 32) {
        const size_t e = ord_end(i + 1);
        out->push_back({i, e});
        i = e;
      } else {
        const size_t e = ord_end(i);
        out->push_back({i, e});
        i = e;
      }
      continue;
    }
    if (h != 10 && h != 32) {
      const size_t e = ord_end(i);
      out->push_back({i, e});
      i = e;
      continue;
    }
    // V2's whitespace words (v2.ws): an optional leading newline, then the
    // run of spaces; a run followed by content hands its last space to the
    // content's word
    const size_t lead = i;
    size_t k = h == 10 ? i + 1 : i;
    const size_t sp0 = k;
    while (k < n && s[k] == 32) k++;
    const size_t sp1 = k;
    if (k < n && ordinary(s[k])) {
      const size_t keep = sp1 > sp0 ? sp1 - 1 : sp1;   // the last space, if any
      if (keep > lead) out->push_back({lead, keep});
      const size_t e = ord_end(k);
      out->push_back({keep, e});
      i = e;
    } else {
      out->push_back({lead, sp1});
      i = sp1;
    }
  }
}

// ------------------------------------------------------------------ encode

// encode.word (bend/Tokenizer.bend:567-621): while some adjacent pair has a
// merge, the lowest merge id among them replaces every occurrence of its
// pair, left to right without overlap. Each symbol carries the id of the
// pair it starts; a sweep recomputes only what a merge touched.
void encode_word(const ana_bpe* t, const uint8_t* s, size_t n, std::vector<uint32_t>* out) {
  std::vector<uint32_t> tok(n), r(n), nt, nr;
  std::vector<uint8_t> merged;
  for (size_t i = 0; i < n; i++) tok[i] = (uint32_t)s[i] + 2;
  for (size_t i = 0; i < n; i++) r[i] = i + 1 < n ? t->rank_of(tok[i], tok[i + 1]) : kNone;
  for (;;) {
    uint32_t m = kNone;
    for (uint32_t x : r) m = x < m ? x : m;
    if (m == kNone) break;
    // the sweep: a symbol whose pair has id m starts a merge and takes its
    // right neighbour with it
    nt.clear();
    nr.clear();
    merged.clear();
    for (size_t i = 0; i < tok.size();) {
      if (r[i] == m && i + 1 < tok.size()) {
        nt.push_back(m);
        nr.push_back(kNone);
        merged.push_back(1);
        i += 2;
      } else {
        nt.push_back(tok[i]);
        nr.push_back(r[i]);
        merged.push_back(0);
        i += 1;
      }
    }
    // pairs that changed: a merged symbol's, and a kept symbol's whose right
    // neighbour was merged (sw.merged, sw.kept)
    for (size_t k = 0; k < nt.size(); k++) {
      const bool last = k + 1 == nt.size();
      if (merged[k]) nr[k] = last ? kNone : t->rank_of(nt[k], nt[k + 1]);
      else if (!last && merged[k + 1]) nr[k] = t->rank_of(nt[k], nt[k + 1]);
    }
    nt.swap(tok);
    nr.swap(r);
  }
  out->insert(out->end(), tok.begin(), tok.end());
}

// Bpe.decode (bend/Tokenizer.bend:642-665): a token's bytes
void decode_tok(const ana_bpe* t, uint32_t tok, int fuel, std::vector<uint8_t>* out) {
  if (tok < 258) {
    if (tok >= 2) out->push_back((uint8_t)(tok - 2));
    return;
  }
  if (fuel == 0) return;
  // the decode table is keyed by the id's low 16 bits (a depth-16 tree);
  // an id with no merge there expands to nothing
  const uint32_t key = tok & 0xffffu;
  if (key < 258 || key - 258 >= t->a.size()) return;
  const size_t k = key - 258;
  decode_tok(t, t->a[k], fuel - 1, out);
  decode_tok(t, t->b[k], fuel - 1, out);
}

}  // namespace

extern "C" {

int ana_bpe_open(const char* path, ana_bpe** out) {
  if (!path || !out) return ANA_EINVAL;
  *out = nullptr;
  FILE* fp = fopen(path, "rb");
  if (!fp) return ANA_ETOK;
  std::vector<uint8_t> buf;
  uint8_t tmp[1 << 16];
  size_t k;
  while ((k = fread(tmp, 1, sizeof tmp, fp)) > 0) buf.insert(buf.end(), tmp, tmp + k);
  fclose(fp);
  ana_bpe* t = new ana_bpe;
  if (!parse_bpe(buf.data(), buf.size(), t)) {
    delete t;
    return ANA_ETOK;
  }
  *out = t;
  return ANA_OK;
}

int ana_bpe_bytes(ana_bpe** out) {
  // the byte tokenizer: a BPE with no merges, V2 (dc.tok.btc, bend/Decode.bend:264-268)
  if (!out) return ANA_EINVAL;
  *out = new ana_bpe;
  return ANA_OK;
}

void ana_bpe_close(ana_bpe* t) { delete t; }

uint32_t ana_bpe_vocab(const ana_bpe* t) { return t ? t->vocab : 0; }

int ana_bpe_identity(const ana_bpe* t, char* buf, size_t cap) {
  if (!t || !buf) return ANA_EINVAL;
  const std::string s = identity(t);
  if (s.size() + 1 > cap) return ANA_EINVAL;
  memcpy(buf, s.c_str(), s.size() + 1);
  return ANA_OK;
}

int ana_bpe_encode(const ana_bpe* t, const uint8_t* bytes, size_t n, uint32_t* ids, size_t cap,
                   size_t* nids) {
  if (!t || (!bytes && n) || !nids) return ANA_EINVAL;
  std::vector<std::pair<size_t, size_t>> words;
  pretokenize(bytes, n, t->v2, &words);
  std::vector<uint32_t> out;
  for (const auto& w : words) encode_word(t, bytes + w.first, w.second - w.first, &out);
  *nids = out.size();
  if (out.size() > cap || (!ids && !out.empty())) return ANA_EINVAL;
  if (!out.empty()) memcpy(ids, out.data(), 4 * out.size());
  return ANA_OK;
}

int ana_bpe_decode(const ana_bpe* t, const uint32_t* ids, size_t n, uint8_t* bytes, size_t cap,
                   size_t* nbytes) {
  if (!t || (!ids && n) || !nbytes) return ANA_EINVAL;
  std::vector<uint8_t> out;
  for (size_t i = 0; i < n; i++) decode_tok(t, ids[i], 64, &out);
  *nbytes = out.size();
  if (out.size() > cap || (!bytes && !out.empty())) return ANA_EINVAL;
  if (!out.empty()) memcpy(bytes, out.data(), out.size());
  return ANA_OK;
}

int ana_sha256_hex(const uint8_t* bytes, size_t n, char* out65) {
  if ((!bytes && n) || !out65) return ANA_EINVAL;
  const std::string h = sha256_hex(bytes, n);
  memcpy(out65, h.c_str(), 65);
  return ANA_OK;
}

}  // extern "C"

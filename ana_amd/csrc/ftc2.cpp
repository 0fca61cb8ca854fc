// FTC2 checkpoints and the parameter layout, host side.
//
// Format: bend/Checkpoint.bend (magic, Data.Binary manifest v4) and
// bend/Dense/Ckpt.bend:21-34 (u64 count, P big-endian f32, Adam step, ...).
// Validation and messages: Manifest.problem (bend/Checkpoint.bend:162-170)
// and dd.load (bend/Dense/Decode.bend:664-699).
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "ana_internal.h"

namespace ana {

uint64_t params_of(const ana_config& c) {
  const uint64_t d = c.d, f = c.f, v = c.vocab, L = c.layers, h = c.heads;
  const uint64_t hd = h ? d / h : 0, sm = L / 4, gla = L - sm;
  uint64_t p = v * d + L * (4 * d * d + 3 * f * d + 2 * d) + gla * d * d;
  if (c.rglru) p += gla * d;
  if (c.qk) p += sm * 2 * hd;
  if (c.sinks) p += sm * h;
  p += d;
  if (!c.tied) p += v * d;
  return p;
}

std::string model_id_of(const ana_config& c) {
  char buf[1024];
  snprintf(buf, sizeof buf,
           "formal-transformer-futhark-hybrid-gla-v3:Config {vocabSize = %u, contextSize = %u, "
           "modelDim = %u, ffDim = %u, layerCount = %u, headCount = %u, gateKind = %s, "
           "qkNorm = %s, headSinks = %s, tiedHead = %s}",
           c.vocab, c.ctx, c.d, c.f, c.layers, c.heads, c.rglru ? "GateRgLru" : "GateSigmoid",
           c.qk ? "True" : "False", c.sinks ? "True" : "False", c.tied ? "True" : "False");
  return buf;
}

std::vector<Blk> layout_of(const ana_config& c, uint64_t* fin) {
  const uint64_t d = c.d, f = c.f, dd = d * d, hd = c.heads ? d / c.heads : 0;
  uint64_t o = (uint64_t)c.vocab * d;
  std::vector<Blk> out(c.layers);
  for (uint32_t i = 0; i < c.layers; i++) {
    Blk& b = out[i];
    b = Blk{};
    b.gla = i % 4 != 3;  // the hybrid rule, bend/Config.bend:213-227
    b.ra = o;
    const uint64_t q = o + d;
    b.wq = q; b.wk = q + dd; b.wv = q + 2 * dd; b.wo = q + 3 * dd;
    if (b.gla) {
      b.wa = q + 4 * dd;
      b.lam = q + 5 * dd;
      b.rf = b.lam + (c.rglru ? d : 0);
    } else {
      b.gq = q + 4 * dd;
      b.gk = b.gq + (c.qk ? hd : 0);
      b.sink = b.gk + (c.qk ? hd : 0);
      b.rf = b.sink + (c.sinks ? c.heads : 0);
    }
    b.wg = b.rf + d;
    b.wu = b.wg + f * d;
    b.wd = b.wg + 2 * f * d;
    b.end = b.wd + d * f;
    o = b.end;
  }
  *fin = o;
  return out;
}

namespace {

struct Cur {
  const uint8_t* p;
  size_t n, at;
  bool bad;
  uint64_t be(int k) {
    if (at + (size_t)k > n) { bad = true; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < k; i++) v = (v << 8) | p[at + i];
    at += (size_t)k;
    return v;
  }
  uint32_t nat() { return (uint32_t)be(8); }  // Load.nat: an Int64's low word
  std::string str() {                          // Load.string: char count, UTF-8
    const uint32_t n_ = nat();
    std::string s;
    for (uint32_t i = 0; i < n_ && !bad; i++) {
      const uint32_t b = (uint32_t)be(1);
      const int extra = b < 128 ? 0 : b < 224 ? 1 : b < 240 ? 2 : 3;
      s.push_back((char)b);
      for (int j = 0; j < extra; j++) s.push_back((char)be(1));
    }
    return s;
  }
  // Load.double (bend/Checkpoint.bend:54-81): an Integer (tag 0: Int32;
  // tag 1: sign byte, byte count, little-endian bytes) times 2 to an Int64,
  // in F32 as the reference forms it: signed.f32 and le.f32
  // (bend/Parse.bend:71-79,171-186), then m * F32.pow(2, e)
  float dbl() {
    float m;
    if (be(1) == 0) {
      m = signed_f32((uint32_t)be(4));
    } else {
      const uint32_t s = (uint32_t)be(1);
      const uint32_t k = nat();
      std::vector<uint8_t> bs;
      for (uint32_t i = 0; i < k && !bad; i++) bs.push_back((uint8_t)be(1));
      float f = 0.0f;
      for (size_t i = bs.size(); i-- > 0;) f = (float)bs[i] + 256.0f * f;
      m = s == 1 ? f : -f;
    }
    const float e = signed_f32((uint32_t)be(8));
    return m * (float)pow(2.0, (double)e);
  }
  static float signed_f32(uint32_t x) { return x >= 2147483648u ? -(float)(~x + 1u) : (float)x; }
};

void copy_str(char* dst, const std::string& s) {
  const size_t n = s.size() < ANA_MANIFEST_STR - 1 ? s.size() : ANA_MANIFEST_STR - 1;
  memcpy(dst, s.data(), n);
  dst[n] = 0;
}

// Load.header's manifest after the magic (bend/Checkpoint.bend:100-136)
void parse_manifest(Cur& c, ana_manifest* m) {
  memset(m, 0, sizeof *m);
  m->version = (uint32_t)c.be(4);
  ana_config& cf = m->cfg;
  cf.vocab = c.nat(); cf.ctx = c.nat(); cf.d = c.nat(); cf.f = c.nat();
  cf.layers = c.nat(); cf.heads = c.nat();
  cf.rglru = c.be(1) != 0; cf.qk = c.be(1) != 0; cf.sinks = c.be(1) != 0; cf.tied = c.be(1) != 0;
  m->count = c.nat();
  copy_str(m->layout, c.str());
  m->layout_version = (uint32_t)c.be(4);
  m->lr = c.dbl(); m->beta1 = c.dbl(); m->beta2 = c.dbl(); m->eps = c.dbl(); m->weight_decay = c.dbl();
  m->warmup = c.nat();
  m->total_steps = c.nat();
  m->has_muon = c.be(1) != 0;
  if (m->has_muon) m->muon = c.dbl();
  copy_str(m->model_id, c.str());
  copy_str(m->tokenizer_id, c.str());
  copy_str(m->dataset_id, c.str());
  m->clip = c.dbl();
  m->numerics = (uint32_t)c.be(1);
}

}  // namespace

std::string read_manifest(const char* path, ana_manifest* out) {
  FILE* fp = fopen(path, "rb");
  if (!fp) return std::string("checkpoint: cannot open ") + path;
  std::vector<uint8_t> head(1 << 16);
  head.resize(fread(head.data(), 1, head.size(), fp));
  fclose(fp);
  Cur c{head.data(), head.size(), 0, false};
  if ((uint32_t)c.be(4) != 1179927346u || c.bad) return "not a compact checkpoint (magic is not FTC2)";
  parse_manifest(c, out);
  if (c.bad) return "checkpoint: short read";
  return "";
}

std::string read_ftc2(const char* path, Ftc2* out) {
  FILE* fp = fopen(path, "rb");
  if (!fp) return std::string("checkpoint: cannot open ") + path;
  // the header is small; read a generous prefix first
  std::vector<uint8_t> head(1 << 16);
  const size_t got = fread(head.data(), 1, head.size(), fp);
  head.resize(got);
  Cur c{head.data(), head.size(), 0, false};
  if ((uint32_t)c.be(4) != 1179927346u || c.bad) {
    fclose(fp);
    return "not a compact checkpoint (magic is not FTC2)";
  }
  ana_manifest man;
  parse_manifest(c, &man);
  const uint32_t version = man.version;
  const ana_config cf = man.cfg;
  const uint32_t count = man.count;
  const std::string lay = man.layout, mid = man.model_id;
  const uint32_t lv = man.layout_version;
  if (c.bad) { fclose(fp); return "checkpoint: short read"; }
  const size_t h = c.at;
  if (version != 4) { fclose(fp); return "checkpoint: unsupported checkpoint manifest version (this branch reads version 4)"; }
  if (lay != "hybrid-gla-decoder-flat-parameters") { fclose(fp); return "checkpoint: unsupported checkpoint model layout identity"; }
  if (lv != 3) { fclose(fp); return "checkpoint: unsupported checkpoint model layout version"; }
  if ((uint64_t)count != params_of(cf)) { fclose(fp); return "checkpoint: manifest parameter count does not match config"; }
  if (mid != model_id_of(cf)) { fclose(fp); return "checkpoint: checkpoint model identity is not supported by this host"; }
  if (!cf.tied) { fclose(fp); return "checkpoint: the dense decoder needs a tied head"; }
  const uint64_t P = params_of(cf);
  // the decoder reads the count (8 bytes at h), the step (16 bytes at
  // h + 8 + 4P) and the parameters; a file shorter than that is a short read
  if (fseek(fp, 0, SEEK_END) != 0) { fclose(fp); return "checkpoint: short read"; }
  const long size = ftell(fp);
  const uint64_t stp = h + 8 + 4 * P;
  if (size < 0 || (uint64_t)size < stp + 16) { fclose(fp); return "checkpoint: short read"; }
  uint8_t cnt[8], step[16];
  fseek(fp, (long)h, SEEK_SET);
  if (fread(cnt, 1, 8, fp) != 8) { fclose(fp); return "checkpoint: short read"; }
  uint32_t lo = ((uint32_t)cnt[4] << 24) | ((uint32_t)cnt[5] << 16) | ((uint32_t)cnt[6] << 8) | cnt[7];
  if (lo != (uint32_t)P) { fclose(fp); return "checkpoint: checkpoint parameter vector length is not the parameter count"; }
  out->raw.resize(4 * P);
  if (fread(out->raw.data(), 1, 4 * P, fp) != 4 * P) { fclose(fp); return "checkpoint: short read"; }
  if (fread(step, 1, 16, fp) != 16) { fclose(fp); return "checkpoint: short read"; }
  fclose(fp);
  uint64_t s = 0;
  for (int i = 0; i < 8; i++) s = (s << 8) | step[i];
  out->cfg = cf;
  out->step = (uint32_t)s;
  return "";
}

}  // namespace ana

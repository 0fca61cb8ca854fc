// Host-side capacity checks of libana's launchers, driven without a GPU.
//
// Each case hands a launcher a grid that its scratch buffer (or the switched
// off decode path) cannot take and expects hipErrorInvalidValue, returned
// before any launch. The same arguments at a size the buffer does take must
// get past the check (the launch itself then fails with hipErrorNoDevice).
//
// Every pointer here is host memory standing in for a device buffer, so the
// probe runs only where no device is visible: if HIP reports one, it prints
// "skip" and exits 0 before calling any launcher (a launcher whose check had
// regressed would otherwise launch a kernel on host addresses).
//
// Prints one line per case, "ok <name>" or "FAIL <name> ...", and exits 0
// when every case holds.
#include <cstdio>

#include "ana_internal.h"

using namespace ana;

static int fails = 0;

static void expect(const char* name, hipError_t got, bool reject) {
  const bool ok = reject ? got == hipErrorInvalidValue : got != hipErrorInvalidValue;
  if (!ok) fails++;
  printf("%s %s (got %d)\n", ok ? "ok" : "FAIL", name, (int)got);
}

int main() {
  int n = 0;
  if (hipGetDeviceCount(&n) == hipSuccess && n > 0) {
    printf("skip: %d device(s) visible; this probe runs on the CPU only\n", n);
    return 0;
  }
  static float buf[1 << 16];
  static uint32_t ids[64];

  // split attention of decode rows: per (row, head, split) hd + 2 floats
  AttnArgs a{};
  a.QKV = buf; a.O = buf; a.d = 64; a.heads = 4; a.ctx = 128; a.write_kv = 1;
  a.seq = ids; a.pos = ids;
  a.part = buf;
  const size_t per_row = (size_t)a.heads * (a.ctx / kFastTS) * (16 + 2);
  a.B = 3; a.part_cap = 3 * per_row - 1;
  expect("attn_fast: partials one float short", launch_attn_fast(a, nullptr), true);
  a.B = 5; a.part_cap = 100 * per_row;
  expect("attn_fast: decode step above kSmallB rows", launch_attn_fast(a, nullptr), true);
  a.write_kv = 0; a.B = 12; a.part_cap = 12 * per_row - 1;
  expect("attn_fast: prefill chunk of 12 rows, partials short", launch_attn_fast(a, nullptr), true);
  a.part_cap = 12 * per_row;
  expect("attn_fast: prefill chunk of 12 rows fits", launch_attn_fast(a, nullptr), false);

  // the wide decode attention in kRowsSplit-slot pieces
  AttnArgs r{};
  r.QKV = buf; r.O = buf; r.d = 256; r.heads = 4; r.ctx = 1024; r.write_kv = 1;
  r.seq = ids; r.pos = ids; r.part = buf; r.B = 9;
  const size_t rneed = (size_t)r.B * r.heads * (r.ctx / kRowsSplit) * (64 + 2);
  r.part_cap = rneed - 1;
  expect("attn_rows split: partials one float short", launch_attn_rows(r, true, nullptr), true);
  r.part_cap = rneed;
  expect("attn_rows split: partials fit", launch_attn_rows(r, true, nullptr), false);

  // exact split attention: scores and maxima for ss_rows rows
  AttnArgs e{};
  e.QKV = buf; e.O = buf; e.d = 64; e.heads = 4; e.ctx = 64; e.write_kv = 1;
  e.ss = buf; e.pm = buf; e.B = 6; e.ss_rows = 5;
  expect("attn exact: 6 rows, scratch for 5", launch_attn(e, nullptr), true);

  // fast GLA step: off above kSmallB rows
  StateRef S{buf, 0, 0};
  expect("gla_fast: 5 rows", launch_gla_fast(buf, buf, nullptr, S, ids, buf, 64, 4, 0, 5, nullptr), true);

  // GLA scan: sub-chunks beyond what the scratch was carved for
  GlaScratch g = gla_scan_carve(buf, 64, 4, 2, 64, 4);
  expect("gla_scan: 5 sub-chunks, carved for 4",
         launch_gla_scan(buf, buf, nullptr, S, buf, g, nullptr, 5, 64, 4, 0, nullptr), true);

  // bf16 prefill products: the split activations hold cap_rows rows
  GemvArgs p{};
  p.X = buf; p.ldx = 64; p.K = 64; p.seg[0] = GemvSeg{buf, 64, buf, 64}; p.nseg = 1;
  p.B = 200; p.Wh0 = reinterpret_cast<const uint16_t*>(buf);
  expect("gemm_dl: 200 rows, split buffers for 199",
         launch_gemm_dl(p, reinterpret_cast<__bf16*>(buf), buf, 199, nullptr),
         true);

  printf("%d failed\n", fails);
  return fails ? 1 : 0;
}

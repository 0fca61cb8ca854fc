"""Decode throughput of libana on one MI355X (BASELINE.json's metric).

Workload: the reference's 115M model at ctx 2048 (fp100m: d 768, f 2048,
12 layers 9 GLA + 3 softmax, 12 heads, vocab 32768, RG-LRU, qk-norm, sinks),
random-init weights in an FTC2 file this script writes, synthetic prompts.
A step is one token for every sequence of the batch: the whole decode step
(embedding, 12 layers, LM head, greedy pick on the device), run by
ana_generate's on-device token loop with inputs already in HBM.

B = 1 (the headline `value`): a 1920-token prompt through chunked prefill,
an untimed priming call of 8 steps (graph capture, or the persistent
kernel's first launch), then W warm-up and K timed decode steps at
positions 1928+ (the full 2048-slot window).
Reported beside it: B = 1 in the other modes, B = 64 (128-token prompts) in
every mode, B = 64 x 512 prefill and window scoring, 64 agent episodes, and
BASELINE's other decode configs (next: B = 32 at 1920+; v3: B = 64 sampled;
bf16: B = 256), the last in a child process of their own.

The roofline entry is the dominant kernel of the B = 1 step: the
persistent step kernel k_decode1 (one launch runs every step of a call;
every mode has a build of it), or, where it does not run, the layer
products with the LM head. `achieved` is their
algorithmic bytes (every weight once a step, the GLA states read and
written, the live K/V rows read and the new ones written) over their
launches' HIP-event time on the library's stream, against 8 TB/s;
`traffic` the HBM bytes a launch fetched and wrote (rocprofv3 FETCH_SIZE +
WRITE_SIZE, calibrated on a copy kernel), from profiles/traffic.json.
cpu_baseline: the CPU oracle (a restatement of the reference's dense
decoder; the reference's Bend toolchain is absent) on a bounded sample.
"""
from __future__ import annotations

import argparse
import subprocess
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import ana_amd  # noqa: E402
from ana_amd import ckpt  # noqa: E402
from ana_amd import config as cf  # noqa: E402

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def ensure_ckpt(c: cf.Config, path: str) -> str:
    want = len(ckpt.manifest_bytes(c)) + 8 + 4 * c.params + 16
    if not (os.path.exists(path) and os.path.getsize(path) == want):
        t = time.perf_counter()
        ckpt.write(path, c, ckpt.init_params(c, "normal", 0))
        log(f"wrote {path} ({want / 1e6:.0f} MB) in {time.perf_counter() - t:.1f}s")
    return path


def run_bytes(c: cf.Config, positions, steps: int, wbytes: float = 4.0) -> float:
    """Algorithmic HBM bytes of `steps` decode steps: every weight once per
    step (the tied head reads all of E; the gather reads one row per
    sequence), and per (sequence, position) the GLA states read and written
    and the live K/V rows read."""
    w = wbytes * (c.params - c.vocab * c.d + c.vocab * c.d) * steps
    per = 0.0
    for p in positions:
        live = min(p, c.ctx - 1) + 1
        per += c.gla_layers * 2 * c.heads * c.hd * c.hd * 4.0
        per += c.softmax_layers * (2 * live * c.d * 4.0 + 2 * c.d * 4.0)
    return w + per


PRIME = 8   # steps of the untimed priming call before any warm-up

MODES = {"exact": ana_amd.EXACT_FP32, "fast_fp32": ana_amd.FAST_FP32, "bf16": ana_amd.BF16}


def run_batch(path: str, c: cf.Config, B: int, prompt: int, warmup: int, steps: int, prof_steps: int,
              mode: str = "exact", chunk: int = 64):
    seqs = list(range(B))
    with ana_amd.Decoder(path, max_seqs=B, prefill_chunk=chunk, numerics=MODES[mode]) as dec:
        prs = [ckpt.prompt(b, prompt, c.vocab) for b in seqs]
        first = [int(pr[-1]) for pr in prs]
        pos = [prompt - 1] * B
        t = time.perf_counter()
        if B == 1:
            dec.feeds(0, 0, prs[0][:-1])
        else:
            dec.feeds_n(seqs, [0] * B, [pr[:-1] for pr in prs])
        t_pre = time.perf_counter() - t
        log(f"B={B} {mode}: prefill {B}x{prompt - 1} tokens in {t_pre:.3f}s")
        tok = np.array(first, dtype=np.uint32)
        pos = np.array(pos, dtype=np.uint32)
        # an untimed priming call, not counted as warm-up: it captures the
        # step graphs (one step and eight) or makes the persistent kernel's
        # first launch, so the timed call replays what it would in a loop
        out = dec.generate(seqs, pos, tok, PRIME)
        tok, pos = out[:, -1].copy(), pos + PRIME
        if warmup:
            out = dec.generate(seqs, pos, tok, warmup)
            tok, pos = out[:, -1].copy(), pos + warmup
        t0 = time.perf_counter()
        out = dec.generate(seqs, pos, tok, steps)
        t1 = time.perf_counter()
        positions = [int(p) + k for k in range(steps) for p in pos]
        tok, pos = out[:, -1].copy(), pos + steps
        stats = {}
        if prof_steps:
            dec.prof(True)
            dec.generate(seqs, pos, tok, prof_steps)
            stats = dec.prof_read()
            dec.prof(False)
    dt = t1 - t0
    sb = run_bytes(c, positions, steps, 2.0 if mode == "bf16" else 4.0) / steps
    return {
        "tok_s": B * steps / dt,
        "ms_per_step": 1000.0 * dt / steps,
        "prefill_tok_s": B * (prompt - 1) / t_pre,
        "step_bytes": sb,
        "step_gbs": sb * steps / dt / 1e9,
        "stats": stats,
    }


def run_configs(path: str, c, only: str = "") -> dict:
    """BASELINE's other decode configs on the same checkpoint (ctx 2048):
    "next" (B=32, 1920-token prompts, 128 greedy steps, fast_fp32, past the
    ring's wrap at the end), "v3" (B=64, 128-token prompts, 128 sampled steps
    at T 0.8 / top-k 40 / top-p 0.9, seed b per sequence, fast_fp32) and
    "bf16" (B=256, 512-token prompts, 256 greedy steps, bf16)."""
    out = {}
    for key, B, prompt, steps, mode, sampled in (("cfg_next", 32, 1920, 128, "fast_fp32", False),
                                                 ("cfg_v3", 64, 128, 128, "fast_fp32", True),
                                                 ("cfg_bf16", 256, 512, 256, "bf16", False)):
        if only and key != "cfg_" + only:
            continue
        seqs = list(range(B))
        with ana_amd.Decoder(path, max_seqs=B, prefill_chunk=128, numerics=MODES[mode]) as dec:
            prs = [ckpt.prompt(5000 + b, prompt, c.vocab) for b in seqs]
            t = time.perf_counter()
            dec.feeds_n(seqs, [0] * B, [pr[:-1] for pr in prs])
            t_pre = time.perf_counter() - t
            tok = np.array([int(pr[-1]) for pr in prs], dtype=np.uint32)
            pos = np.full(B, prompt - 1, dtype=np.uint32)
            st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9))) if sampled else None
            rng = np.ascontiguousarray(np.stack([ana_amd.rng_seeded(b) for b in seqs])) if sampled else None
            tok = dec.generate(seqs, pos, tok, 8, st, rng)[:, -1].copy()   # graph capture, untimed
            t0 = time.perf_counter()
            dec.generate(seqs, pos + 8, tok, steps, st, rng)
            dt = time.perf_counter() - t0
        positions = [int(prompt - 1 + 8 + k) for k in range(steps) for _ in seqs]
        sb = run_bytes(c, positions, steps, 2.0 if mode == "bf16" else 4.0) / steps
        out[key] = {"tok_s": round(B * steps / dt, 1), "ms_per_step": round(1000.0 * dt / steps, 4),
                    "step_gbs": round(sb * steps / dt / 1e9, 2), "prefill_tok_s": round(B * (prompt - 1) / t_pre, 1),
                    "workload": f"B={B}, {prompt}-token prompts (ana_feeds_n, chunk 128), {steps} "
                                f"{'sampled (T 0.8, top-k 40, top-p 0.9)' if sampled else 'greedy'} steps; "
                                + NUMERICS[mode]}
        log(f"{key}: {out[key]['tok_s']} tok/s, prefill {out[key]['prefill_tok_s']} tok/s")
    return out


def cpu_baseline(path: str, c: cf.Config, seconds: float) -> dict:
    """The oracle's dense decode on the host cores, bounded to ~`seconds`:
    one thread per core this process may run on, capped by OMP_NUM_THREADS
    where the host sets it (a GPU box's share of its host cores)."""
    from oracle import oracle as O
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    share = os.environ.get("OMP_NUM_THREADS", "")
    threads = max(1, min(cores, int(share))) if share.isdigit() and int(share) > 0 else max(1, cores)
    O.set_threads(threads)
    m = O.Model(path)
    st = O.State(m)
    pr = ckpt.prompt(0, 8, c.vocab)
    for p, t in enumerate(pr):
        st.feed(p, int(t))
    pos, n = len(pr), 0
    tok = O.top(st.logits())
    t0 = time.perf_counter()
    while True:
        st.feed(pos, tok)
        tok = O.top(st.logits())
        pos += 1
        n += 1
        if time.perf_counter() - t0 > seconds or n >= 512:
            break
    dt = time.perf_counter() - t0
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": n / dt, "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": (f"CPU oracle (C restatement of the reference's dense decoder, AVX2 no-FMA, "
                   f"pthreads) greedy decode of {n} tokens at positions 8..{pos - 1}, B=1, same "
                   f"115M ctx-2048 checkpoint; it scores every ring slot as the reference does, so "
                   f"a token costs the same at any position; {threads} threads of the {cores} cores "
                   f"this process may use (OMP_NUM_THREADS={share or 'unset'}); {cpu}"),
    }


KERNEL_PERSIST = {
    "exact": ("k_decode1 (exact build, one greedy sequence: every phase of every step in one cooperative "
              "launch of one workgroup per CU, each output an in-order chain in one lane; weights streamed "
              "into LDS a phase ahead)"),
    "fast_fp32": ("k_decode1 (fast fp32, one greedy sequence: every phase of every step in one "
                  "cooperative launch of one workgroup per CU; weights streamed into LDS a phase ahead)"),
    "bf16": ("k_decode1 (bf16 weights past the first layer and in the head, one greedy sequence: every "
             "phase of every step in one cooperative launch of one workgroup per CU; weights streamed "
             "into LDS a phase ahead)")}
KERNEL = {"exact": "k_gemv_small<1> (exact products, norm/residual/SiLU/argmax fused) + LM head",
          "fast_fp32": "k_gemv_fast<fp32> (split-K products, norm/residual/SiLU/argmax fused) + LM head",
          "bf16": "k_gemv_fast<bf16> (split-K products over bf16 weights) + LM head"}
NUMERICS = {"exact": "exact_fp32: bit-exact with the reference's CPU kernels",
            "fast_fp32": "fast_fp32: fp32 with reassociated sums; logits within 1e-4 of the reference",
            "bf16": "bf16 weights, fp32 activations/accumulation/state; logits within 2e-2"}


def phase_names(c) -> list:
    """k_decode1's phases of a step, in order: per layer q|k|v(|z), the mix
    (GLA; or the attention pieces, then their combination), Wo, gate|up,
    down; then the LM head and the pick."""
    names = []
    for i in range(c.layers):
        if c.is_softmax(i):
            names += [(i, "qkv"), (i, "att"), (i, "comb"), (i, "wo"), (i, "gu"), (i, "down")]
        else:
            names += [(i, "qkvz"), (i, "gla"), (i, "wo"), (i, "gu"), (i, "down")]
    return names + [(-1, "head"), (-1, "pick")]


def run_phase_trace(path: str, c, steps: int, mode: int = ana_amd.FAST_FP32) -> str:
    """The bench's B=1 workload in a fast mode (fast_fp32, or bf16 with
    --numerics bf16; 1920-token prompt, decode from 1919) with k_decode1's
    phase stamps armed for `steps` steps of one call; returns a markdown
    summary. Per (phase, workgroup) the stamps
    split a phase into: wait (start to every input seen: the exchange, and
    the weight loads issued before it, which retire first), land (to the
    phase's weights in LDS), compute (to the outputs published), and the gap
    to the next phase's start. Figures are means over workgroups and over
    the traced steps after the first two."""
    TICK_US = 0.01   # the constant-rate clock runs at 100 MHz
    pr = ckpt.prompt(0, 1920, c.vocab)
    with ana_amd.Decoder(path, max_seqs=1, numerics=mode) as dec:
        dec.feeds(0, 0, pr[:-1])
        pos, tok = 1919, int(pr[-1])
        o = dec.generate([0], [pos], [tok], PRIME)[0]
        pos, tok = pos + PRIME, int(o[-1])
        t = time.perf_counter()
        o = dec.generate([0], [pos], [tok], 64)[0]
        untraced = (time.perf_counter() - t) / 64 * 1e6
        pos, tok = pos + 64, int(o[-1])
        dec.trace(steps)
        t = time.perf_counter()
        o = dec.generate([0], [pos], [tok], 64)[0]
        traced = (time.perf_counter() - t) / 64 * 1e6
        tr = dec.trace_read().astype(np.int64)
    S, P, G, _ = tr.shape
    names = phase_names(c)
    if len(names) != P:
        raise RuntimeError(f"phase trace: {P} phases, expected {len(names)}")
    # ticks relative to each step's first stamp (the low 32 bits wrap)
    t = (tr - tr[:, 0:1, :, 0:1]) % (1 << 32)
    t = np.where(t > (1 << 31), t - (1 << 32), t) * TICK_US
    ss = list(range(2, S)) if S > 2 else list(range(S))
    a = t[ss]                                        # [s, P, G, 4]
    wait = a[..., 1] - a[..., 0]
    land = a[..., 2] - a[..., 1]
    comp = a[..., 3] - a[..., 2]
    gap = np.concatenate([a[:, 1:, :, 0] - a[:, :-1, :, 3], np.zeros_like(a[:, :1, :, 0])], axis=1)
    span = [float(a[i, -1, :, 3].max() - a[i, 0, :, 0].min()) for i in range(len(ss))]
    out = [f"k_decode1 phase stamps: {len(ss)} steps (of {S} traced) x {P} phases x {G} workgroups; "
           f"one step {np.mean(span):.1f} us from its first phase's start to its pick's last publish "
           f"(ana_generate: {untraced:.1f} us a step untraced, {traced:.1f} traced)", "",
           "| phase | count | wait us | land us | compute us | gap us | total us | x count |",
           "|---|---|---|---|---|---|---|---|"]
    kinds = []
    for _, k in names:
        if k not in kinds:
            kinds.append(k)
    tot = np.zeros(5)
    for k in kinds:
        idx = [p for p, (_, kk) in enumerate(names) if kk == k]
        w, la, co, g = (float(x[:, idx].mean()) for x in (wait, land, comp, gap))
        n = len(idx)
        tot += np.array([w, la, co, g, w + la + co + g]) * n
        out.append(f"| {k} | {n} | {w:.2f} | {la:.2f} | {co:.2f} | {g:.2f} | {w + la + co + g:.2f} | "
                   f"{(w + la + co + g) * n:.1f} |")
    out.append(f"| step | {P} | {tot[0]:.1f} | {tot[1]:.1f} | {tot[2]:.1f} | {tot[3]:.1f} | {tot[4]:.1f} | |")
    return "\n".join(out)


def run_agent(path: str, c, mode: str) -> dict:
    """Many agent episodes decoded together (ana_amd.agent): 64 episodes of
    a 128-token prompt, the v3 sampling settings, 48 draws a stretch, two
    calls each; a call is a drawn id = 7 mod 61 and the stand-in tool's
    echo is 24 ids, fed as unsampled tokens."""
    from ana_amd import agent
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9)))
    eps = [agent.Episode([int(x) for x in ckpt.prompt(3000 + b, 128, c.vocab)], seed=b, budget=48, calls=2)
           for b in range(64)]
    is_call = lambda i, t: t[-1] % 61 == 7  # noqa: E731
    echoed = [0]   # the echoes' tokens (fed, and not among an outcome's tokens)

    def tool(i, t):
        e = [2 + (t[-1] * 31 + j) % (c.vocab - 2) for j in range(24)]
        echoed[0] += len(e)
        return e
    with ana_amd.Decoder(path, max_seqs=64, prefill_chunk=128, numerics=MODES[mode]) as dec:
        agent.run(dec, eps[:8], st, is_call, tool)   # warm-up
        echoed[0] = 0
        t = time.perf_counter()
        out = agent.run(dec, eps, st, is_call, tool)
        dt = time.perf_counter() - t
    drawn = sum(sum(o.drawn) for o in out)
    fed = sum(len(o.drawn) - sum(o.drawn) for o in out) + echoed[0]
    log(f"agent {mode}: {drawn} drawn + {fed} fed tokens over 64 episodes in {dt:.3f}s")
    return {"episodes": 64, "seconds": round(dt, 4), "drawn": drawn, "fed": fed, "echoed": echoed[0],
            "drawn_tok_s": round(drawn / dt, 1), "tok_s": round((drawn + fed) / dt, 1),
            "endings": {w: sum(1 for o in out if o.why == w) for w in ("eos", "budget", "calls", "tool")},
            "workload": "64 episodes (128-token prompts, T 0.8 / top-k 40 / top-p 0.9, 48 draws a stretch, "
                        "2 calls; a call: drawn id = 7 mod 61; echo 24 ids fed unsampled; fed counts given "
                        "tokens and echoes); " + NUMERICS[mode]}


def run_prefill(path: str, c, reps: int = 5) -> dict:
    """B=64 prefill on the matrix cores: 64 prompts of 512 tokens through
    ana_feeds_n at chunk 128 (8192 rows a product), in both fast modes; the
    median of `reps` timed passes (one pass is about 25 ms, short enough for
    clock ramps to move it by a fifth)."""
    extra = {}
    for m in ("bf16", "fast_fp32"):
        with ana_amd.Decoder(path, max_seqs=64, prefill_chunk=128, numerics=MODES[m]) as dec:
            prs = [ckpt.prompt(1000 + b, 512, c.vocab) for b in range(64)]
            dec.feeds_n(list(range(64)), [0] * 64, [pr[:64] for pr in prs])   # warm-up
            runs = []
            for _ in range(reps):
                for b in range(64):
                    dec.reset(b)
                t = time.perf_counter()
                dec.feeds_n(list(range(64)), [0] * 64, prs)
                runs.append(time.perf_counter() - t)
            dt = float(np.median(runs))
        ntok, L = 64 * 512, 512
        # the products, plus causal attention in the softmax layers
        # (q k and p v over the live slots: 2 x 2 x L^2 / 2 x d per
        # sequence and layer)
        n_sm = sum(1 for i in range(c.layers) if i % 4 == 3)
        flops = 2.0 * (c.params - c.vocab * c.d) * ntok + n_sm * 2.0 * 64 * L * L * c.d
        peak = 2500.0 if m == "bf16" else 157.3
        extra[f"prefill_b64_{m}"] = {
            "tok_s": round(ntok / dt, 1), "seconds": round(dt, 4),
            "runs_s": [round(x, 4) for x in runs],
            "tflops": round(flops / dt / 1e12, 2), "peak_tflops": peak,
            "frac": round(flops / dt / 1e12 / peak, 4),
            "workload": "64 prompts x 512 tokens through ana_feeds_n, chunk 128; flops = 2 x "
                        "(P - v d) per token (the products) + causal attention 2 B L^2 d per "
                        "softmax layer (the GLA scan not counted)",
            "kernels": ("products k_split + k_gemm_wide / k_gemm_dl (256 x 256 and 128 x 128 MFMA tiles, "
                        "bf16 weights x bf16 activations, both streamed straight into LDS)" if m == "bf16" else
                        "products k_gemm_big (128 x 128 MFMA tiles, fp32 MFMA)")
                       + ", attention k_attn_flash (fp32 MFMA), GLA k_gla_sub + k_gla_carry",
        }
        log(f"prefill B=64 x 512 {m}: {ntok / dt:.0f} tok/s")
        # window scoring (Evaluate.bend's window.go through ana_score_n): 64
        # windows of 513 tokens, the head and G.lse after each of 512
        with ana_amd.Decoder(path, max_seqs=64, prefill_chunk=128, numerics=MODES[m]) as dec:
            ws = [ckpt.prompt(2000 + b, 513, c.vocab) for b in range(64)]
            dec.score_n(list(range(64)), [0] * 64, [w[:65] for w in ws])   # warm-up
            runs = []
            for _ in range(reps):
                for b in range(64):
                    dec.reset(b)
                t = time.perf_counter()
                ce = dec.score_n(list(range(64)), [0] * 64, ws)
                runs.append(time.perf_counter() - t)
            dt = float(np.median(runs))
        loss = float(np.mean([ana_amd.window_mean(x) for x in ce]))
        extra[f"score_b64_{m}"] = {
            "tok_s": round(ntok / dt, 1), "seconds": round(dt, 4), "mean_window_loss": round(loss, 4),
            "runs_s": [round(x, 4) for x in runs],
            "workload": "64 windows x 513 tokens through ana_score_n, chunk 128: prefill plus the "
                        "head and G.lse - logit[next] on every one of the 32768 positions",
        }
        log(f"score B=64 x 512 {m}: {ntok / dt:.0f} tok/s (mean window loss {loss:.4f})")
    return extra


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8, help="untimed steps first (8 or more also capture the 8-step graph)")
    ap.add_argument("--prompt", type=int, default=1920)
    ap.add_argument("--numerics", choices=list(MODES), default="fast_fp32",
                    help="the mode `value` is measured in")
    ap.add_argument("--others", type=int, default=1, help="also measure B=1 in the other modes (1/0)")
    ap.add_argument("--b64", type=int, default=1, help="also measure B=64 (1/0)")
    ap.add_argument("--prefill", type=int, default=1, help="also measure B=64 x 512 prefill (1/0)")
    ap.add_argument("--prefill-only", type=int, default=0,
                    help="measure only the B=64 x 512 prefill and print its figures (1/0)")
    ap.add_argument("--reps", type=int, default=5, help="timed passes of each prefill and scoring figure (the median is reported)")
    ap.add_argument("--agent", type=int, default=1, help="also measure 64 agent episodes (1/0)")
    ap.add_argument("--configs", type=int, default=1, help="also measure BASELINE's next, v3 and bf16 decode configs (1/0)")
    ap.add_argument("--configs-only", type=int, default=0, help="print only those configs' JSON (the child run)")
    ap.add_argument("--config", choices=["", "next", "v3", "bf16"], default="",
                    help="with --configs-only: just this one config")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--ckpt", default=os.environ.get("ANA_BENCH_CKPT", "/tmp/ana_bench_fp100m.ftc2"))
    ap.add_argument("--mall-probe", type=int, default=0,
                    help="only print the re-read rate of device buffers from 32 MiB to 1 GiB (1/0)")
    ap.add_argument("--phase-trace", type=int, default=0,
                    help="only print k_decode1's per-phase stamp summary over this many traced steps (1..64)")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py: this build measures one GPU only; the decode path shards by sequence "
              "with no collective, so run --gpus 1.", file=sys.stderr)
        return 2
    c = cf.FP100M
    path = ensure_ckpt(c, a.ckpt)
    mode = a.numerics
    if a.mall_probe:
        # the cache levels by their re-read rates: eight 4 MB L2s (one an
        # XCD), the 256 MB Infinity Cache, then HBM
        print("| buffer | re-read rate |\n|---|---|")
        for mib in (16, 32, 64, 128, 192, 256, 320, 512, 1024):
            print(f"| {mib} MiB | {ana_amd.probe_reread(mib << 20, 20) / 1e3:.2f} TB/s |", flush=True)
        return 0
    if a.phase_trace:
        print(run_phase_trace(path, c, a.phase_trace, MODES[a.numerics]), flush=True)
        release_device()
        return 0
    if a.prefill_only:
        print(json.dumps(run_prefill(path, c, a.reps)), flush=True)
        release_device()
        return 0
    if a.configs_only:
        print(json.dumps(run_configs(path, c, a.config)), flush=True)
        release_device()
        return 0
    cfg_lines = {}
    if a.configs:
        # first, in a child process of its own (before this one touches the
        # GPU), so a failure there costs only these lines
        cmd = [sys.executable, os.path.abspath(__file__), "--configs-only", "1", "--ckpt", path]
        try:
            pr = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=600)   # its progress on stderr
            lines = [ln for ln in pr.stdout.splitlines() if ln.startswith("{")]
            if pr.returncode == 0 and lines:
                cfg_lines = json.loads(lines[-1])
            else:
                cfg_lines = {"configs_error": f"child exited {pr.returncode}"}
        except subprocess.TimeoutExpired:
            cfg_lines = {"configs_error": "child timed out"}
    prof_steps = min(a.steps, 32)
    r1 = run_batch(path, c, 1, a.prompt, a.warmup, a.steps, prof_steps, mode)
    # the dominant kernel: the persistent step kernel where it ran (every
    # phase of every step in one launch), else the products and the head
    persistent = r1["stats"]["step"][0] > 0
    if persistent:
        launches, ms, by = r1["stats"]["step"]
        kernel = KERNEL_PERSIST[mode]
    else:
        g, h = r1["stats"]["gemv"], r1["stats"]["head"]
        launches, ms, by = g[0] + h[0], g[1] + h[1], g[2] + h[2]
        kernel = KERNEL[mode]
    achieved = by / (ms / 1e3) / 1e9 if ms > 0 else 0.0
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        try:
            tj = json.load(open(tpath))
            if persistent:
                per_step = tj.get(f"decode1_{mode}_bytes_per_step")
                traffic = round(per_step * prof_steps / max(launches, 1)) if per_step else None
            else:
                traffic = tj.get(f"gemv_{mode}_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    extra = {}
    if a.others:
        for m in MODES:
            if m == mode:
                continue
            r = run_batch(path, c, 1, a.prompt, a.warmup, a.steps, 0, m)
            extra[f"b1_{m}"] = {"tok_s": round(r["tok_s"], 2), "ms_per_step": round(r["ms_per_step"], 4),
                                "step_gbs": round(r["step_gbs"], 2), "prefill_tok_s": round(r["prefill_tok_s"], 1),
                                "numerics": NUMERICS[m]}
    if a.b64:
        for m in [mode] + ([x for x in MODES if x != mode] if a.others else []):
            r64 = run_batch(path, c, 64, 128, 8, 32, 8, m)
            key = "b64" if m == mode else f"b64_{m}"
            extra[key] = {k: round(r64[k], 3) for k in ("tok_s", "ms_per_step", "step_gbs", "prefill_tok_s")}
            extra[key]["workload"] = ("B=64, 128-token prompts (ana_feeds_n, chunk 64), 8 untimed then 32 "
                                      "timed greedy steps at positions 135+; " + NUMERICS[m])
        # the same batch deep in the window: every step's attention reads
        # ~1940 live slots a sequence instead of ~150
        r = run_batch(path, c, 64, 1920, 8, 32, 0, mode, chunk=128)
        extra["b64_ctx2048"] = {k: round(r[k], 3) for k in ("tok_s", "ms_per_step", "step_gbs", "prefill_tok_s")}
        extra["b64_ctx2048"]["workload"] = (f"B=64, 1920-token prompts (ana_feeds_n, chunk 128), {PRIME} + 8 untimed "
                                            f"then 32 timed greedy steps at positions {1919 + PRIME + 8}+; "
                                            + NUMERICS[mode])
    if a.prefill:
        extra.update(run_prefill(path, c, a.reps))
    if a.agent:
        extra["agent"] = run_agent(path, c, mode)
    extra.update(cfg_lines)
    cpu = cpu_baseline(path, c, a.cpu_seconds) if a.cpu_seconds > 0 else None
    kern = {k: {"launches": v[0], "ms": round(v[1], 4), "gb": round(v[2] / 1e9, 4)}
            for k, v in r1["stats"].items()}
    line = {
        "metric": "decode tok/s for 115M ctx2048 at B=1 and B=64; % of HBM roofline",
        "value": round(r1["tok_s"], 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if mode == "bf16" else "f32",
        "data": "synthetic: random-init N(0,0.02) FTC2 checkpoint (seed 0), uniform-random prompts",
        "config": {
            "workload": "115M fp100m (d768 f2048 L12 h12 v32768, RG-LRU, qk-norm, sinks) ctx 2048 "
                        "greedy decode, B=1, 1920-token prompt (chunked prefill), then decode at "
                        "positions 1920+; " + NUMERICS[mode],
            "batch": 1, "prompt": a.prompt, "ctx": c.ctx, "numerics": mode,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5),
            "traffic": traffic,
            "launches": launches,
            "avg_launch_us": round(1e3 * ms / max(launches, 1), 3),
            "steps_per_launch": round(prof_steps / max(launches, 1), 3) if persistent else None,
        },
        "step_gbs": round(r1["step_gbs"], 2),
        "step_frac": round(r1["step_gbs"] / HBM_PEAK_GBS, 5),
        "prefill_tok_s": round(r1["prefill_tok_s"], 1),
        "kernels": kern,
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)
    release_device()
    return 0


def release_device() -> None:
    """hipDeviceReset before the interpreter exits: the runtime's queues
    and signals go while a profiler attached to this process (rocprofv3)
    can still write its records; left to the exit handlers, the profiler's
    finalisation has read them after the runtime tore them down."""
    import ctypes
    try:
        ctypes.CDLL("libamdhip64.so").hipDeviceReset()
    except OSError:
        pass


if __name__ == "__main__":
    rc = main()
    if rc:
        sys.exit(rc)

"""BASELINE.json's five configs at their own workloads, on the GPU, against
the CPU oracle.

Each test runs the whole workload through the C ABI (prompts through
ana_feeds_n, then the on-device token loop ana_generate) and holds watched
sequences to the oracle:

- v1 (d 256, 4 layers, ctx 256): B = 1, a 32-token prompt, 64 greedy steps;
  exact mode bit for bit (ids and the last logits), fast_fp32 within 1e-4.
- v2 (the 115M, arms off, ctx 256): B = 1, a 64-token prompt, 192 greedy
  steps; the same two bars.
- v3 (the 115M, arms on, ctx 256): B = 64, 128-token prompts, 128 sampled
  steps at temperature 0.8, top-k 40, top-p 0.9, seed 0 + b; exact mode, four
  watched sequences' ids and final RNG words bit for bit. Its checkpoint
  carries trained-like vectors (norm gains 1 + N(0, 0.1^2), qk gains
  N(0, 0.1^2), sinks N(0, 1)) so the arms the config names are live.
- next (the 115M, ctx 2048): B = 32, 1920-token prompts, 128 greedy steps
  (the softmax rings fill and wrap); one watched sequence bit for bit in exact
  mode, and in fast_fp32 every pick within tolerance of the oracle's max,
  teacher-forced, with the final logits within 1e-4.
- bf16 (the 115M, ctx 2048, ANA_BF16): B = 256, 512-token prompts, 256 greedy
  steps in four calls; two watched sequences' logits within 2e-2 after each
  call and every pick within tolerance of the oracle's max.

Prompts are BOS then uniform ids (ckpt.prompt, seed b); weights are
N(0, 0.02^2) from seed 0 (ckpt.init_params). EOS does not stop the loop
(the BASELINE workloads are fixed-length).
"""
import os

import numpy as np
import pytest

import ana_amd
from ana_amd import ckpt
from ana_amd import config as cf

pytestmark = pytest.mark.gpu

TOL = {ana_amd.FAST_FP32: 1e-4, ana_amd.BF16: 2e-2}


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rel_err(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.abs(got - want).max() / np.abs(want).max())


def _threads(oracle):
    oracle.set_threads(max(1, min(16, os.cpu_count() or 1)))


def _ckpt(tmp_path, c, name, trained=False):
    path = str(tmp_path / f"{name}.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "normal", 0, trained=trained))
    return path


def _prompts(c, n, length):
    return [ckpt.prompt(b, length, c.vocab) for b in range(n)]


def _greedy(oracle, st, steps, vocab):
    """Generate.bend's greedy loop on the oracle from a state whose last fed
    token is the one before the first pick: the picks, and the logits the
    last pick came from."""
    out, lg = [], None
    for k in range(steps):
        lg = st.logits()
        t = oracle.top(lg)
        if t == vocab:
            t = oracle.tree_argmax(lg)
        out.append(int(t))
        if k + 1 < steps:
            st.feed(st.pos, int(t))
            st.pos += 1
    return out, lg


def _teacher(oracle, st, picks, tol, where):
    """Each device pick, fed to the oracle in turn, is within tolerance of
    the oracle's largest logit at that step; returns the logits the last
    pick came from."""
    lg = None
    for k, t in enumerate(picks):
        lg = st.logits()
        scale = float(np.abs(lg).max())
        assert lg[t] >= lg.max() - 2 * tol * scale, (where, k, int(t), int(np.argmax(lg)))
        if k + 1 < len(picks):
            st.feed(st.pos, int(t))
            st.pos += 1
    return lg


def _oracle_prompt(oracle, m, pr):
    st = oracle.State(m)
    for p, t in enumerate(pr):
        st.feed(p, int(t))
    st.pos = len(pr)
    return st


def _single(oracle, tmp_path, c, name, plen, steps):
    """B = 1: a plen-token prompt, then steps greedy picks, exact and fast."""
    path = _ckpt(tmp_path, c, name)
    _threads(oracle)
    m = oracle.Model(path)
    pr = _prompts(c, 1, plen)[0]
    st = _oracle_prompt(oracle, m, pr)
    st_fast = st.clone()
    st_fast.pos = st.pos
    want, want_lg = _greedy(oracle, st, steps, c.vocab)
    for mode in (ana_amd.EXACT_FP32, ana_amd.FAST_FP32):
        print(f"case config {name} mode {mode}: prompt {plen}, {steps} greedy steps", flush=True)
        with ana_amd.Decoder(path, max_seqs=1, numerics=mode) as dec:
            dec.feeds_n([0], [0], [pr[:-1]])
            out = dec.generate([0], [plen - 1], [pr[-1]], steps)[0]
            lg = dec.logits([0])[0]
        if mode == ana_amd.EXACT_FP32:
            assert [int(t) for t in out] == want
            assert np.array_equal(bits(lg), bits(want_lg))
        else:
            ref = _teacher(oracle, st_fast, [int(t) for t in out], TOL[mode], name)
            e = rel_err(lg, ref)
            print(f"final relative error {e:.3e}", flush=True)
            assert e <= TOL[mode], e


def test_config_v1(oracle, tmp_path):
    _single(oracle, tmp_path, cf.V1, "v1", 32, 64)


def test_config_v2(oracle, tmp_path):
    _single(oracle, tmp_path, cf.V2, "v2", 64, 192)


def test_config_v3_sampled(oracle, tmp_path):
    c = cf.BPE100M_V3
    path = _ckpt(tmp_path, c, "v3", trained=True)
    _threads(oracle)
    m = oracle.Model(path)
    n, plen, steps = 64, 128, 128
    temp, topk, topp = float(np.float32(0.8)), 40, float(np.float32(0.9))
    prompts = _prompts(c, n, plen)
    rng = np.ascontiguousarray(np.stack([ana_amd.rng_seeded(b) for b in range(n)]).astype(np.uint64))
    print(f"case config v3: B {n}, prompt {plen}, {steps} sampled steps, exact", flush=True)
    with ana_amd.Decoder(path, max_seqs=n, numerics=ana_amd.EXACT_FP32) as dec:
        dec.feeds_n(list(range(n)), [0] * n, [p[:-1] for p in prompts])
        st = ana_amd.Settings(temp, topk, topp)
        out = dec.generate(list(range(n)), [plen - 1] * n, [int(p[-1]) for p in prompts], steps, st, rng)
    for b in (0, 21, 42, 63):
        o = _oracle_prompt(oracle, m, prompts[b])
        r = oracle.rng_seeded(b)
        want = []
        for k in range(steps):
            t = oracle.pick(o.logits(), temp, topk, topp, r)
            want.append(int(t))
            if k + 1 < steps:
                o.feed(o.pos, int(t))
                o.pos += 1
        assert [int(t) for t in out[b]] == want, b
        assert np.array_equal(rng[b], r), b


def test_config_next(oracle, tmp_path):
    c = cf.FP100M
    path = _ckpt(tmp_path, c, "next")
    _threads(oracle)
    m = oracle.Model(path)
    n, plen, steps = 32, 1920, 128
    prompts = _prompts(c, n, plen)
    seqs = list(range(n))
    print("case config next: oracle prompt", flush=True)
    st = _oracle_prompt(oracle, m, prompts[0])
    st_fast = st.clone()
    st_fast.pos = st.pos
    want, want_lg = _greedy(oracle, st, steps, c.vocab)
    for mode in (ana_amd.EXACT_FP32, ana_amd.FAST_FP32):
        print(f"case config next mode {mode}: B {n}, prompt {plen}, {steps} greedy steps", flush=True)
        with ana_amd.Decoder(path, max_seqs=n, numerics=mode) as dec:
            dec.feeds_n(seqs, [0] * n, [p[:-1] for p in prompts])
            out = dec.generate(seqs, [plen - 1] * n, [int(p[-1]) for p in prompts], steps)
            lg = dec.logits([0])[0]
        if mode == ana_amd.EXACT_FP32:
            assert [int(t) for t in out[0]] == want
            assert np.array_equal(bits(lg), bits(want_lg))
        else:
            ref = _teacher(oracle, st_fast, [int(t) for t in out[0]], TOL[mode], "next")
            e = rel_err(lg, ref)
            print(f"final relative error {e:.3e}", flush=True)
            assert e <= TOL[mode], e


def test_config_bf16(oracle, tmp_path):
    c = cf.FP100M
    path = _ckpt(tmp_path, c, "bf16")
    _threads(oracle)
    m = oracle.Model(path)
    n, plen, steps, calls = 256, 512, 256, 4
    prompts = _prompts(c, n, plen)
    seqs = list(range(n))
    watch = (0, 255)
    print(f"case config bf16: B {n}, prompt {plen}, {steps} greedy steps in {calls} calls", flush=True)
    outs, lgs = [], []
    with ana_amd.Decoder(path, max_seqs=n, numerics=ana_amd.BF16) as dec:
        dec.feeds_n(seqs, [0] * n, [p[:-1] for p in prompts])
        pos = np.full(n, plen - 1, dtype=np.uint32)
        tok = np.array([int(p[-1]) for p in prompts], dtype=np.uint32)
        for _ in range(calls):
            o = dec.generate(seqs, pos, tok, steps // calls)
            outs.append(o)
            lgs.append(dec.logits(list(watch)))
            pos, tok = pos + steps // calls, o[:, -1].copy()
    worst = 0.0
    for i, b in enumerate(watch):
        st = _oracle_prompt(oracle, m, prompts[b])
        for j in range(calls):
            picks = [int(t) for t in outs[j][b]]
            ref = _teacher(oracle, st, picks, TOL[ana_amd.BF16], ("bf16", b, j))
            worst = max(worst, rel_err(lgs[j][i], ref))
            # the next call starts by feeding this call's last pick
            st.feed(st.pos, picks[-1])
            st.pos += 1
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[ana_amd.BF16], worst

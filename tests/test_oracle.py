"""The CPU oracle pinned against the reference's own known answers and laws.

These run without a GPU. They hold the oracle (oracle/ana_oracle.c) to:
- the U64 known answers of bend/tests/num.bend and the file's RNG transition;
- greedy's tie vectors (bend/tests/decode-dense.bend:199-220);
- the dense step within 1e-5 relative of the tree meaning before and after
  the ring wraps, reset => same bits, store pick = tree argmax
  (bend/tests/decode-dense.bend:13-22);
- closed forms on hand-built weights (uniform attention, zero blocks,
  the sink in the denominator, the GLA state recurrence), so a mistake
  shared by both restatements still fails;
- the sampler's thresholds against brute force and its draw against the
  cumulative mass.
"""
import json
import math
import os
import struct

import numpy as np
import pytest

from ana_amd import ckpt
from ana_amd import config as cf

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = json.load(open(os.path.join(HERE, "golden", "reference_vectors.json")))
M64 = (1 << 64) - 1


def u64(hl):
    return (hl[0] << 32) | hl[1]


def rotl(x, k):
    return ((x << k) | (x >> (64 - k))) & M64


def test_num_kats(oracle):
    k = VEC["num_kats"]
    assert f"{(u64(k['mul']['a']) * u64(k['mul']['b'])) & M64:016x}" == k["mul"]["hex"]
    assert f"{rotl(u64(k['rotl45']['a']), 45):016x}" == k["rotl45"]["hex"]
    assert f"{u64(k['shr30']['a']) >> 30:016x}" == k["shr30"]["hex"]
    assert f"{(u64(k['add']['a']) + u64(k['add']['b'])) & M64:016x}" == k["add"]["hex"]
    assert f"{oracle.u64_read(k['read']['s']):016x}" == k["read"]["hex"]
    assert struct.unpack(">f", bytes(k["f32_from_bits"]["bytes"]))[0] == k["f32_from_bits"]["value"]
    # U64.read: a non-digit poisons, the empty string is None, overflow wraps
    assert oracle.u64_read("12a") is None
    assert oracle.u64_read("") is None
    assert oracle.u64_read("18446744073709551616") == 0


def _splitmix(s):
    s2 = (s + 0x9E3779B97F4A7C15) & M64
    z = ((s2 ^ (s2 >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31), s2


def test_rng_is_the_files_transition(oracle):
    """Rng.seeded and Rng.next expanded by hand from bend/Sample.bend:57-93,
    with the two constants of the transition that differ from textbook
    xoshiro256** (s0' includes s2, s1' excludes s0)."""
    for seed in (0, 1, 42, 2 ** 63 + 5):
        st, s = [], seed
        for _ in range(4):
            z, s = _splitmix(s)
            st.append(z)
        r = oracle.rng_seeded(seed)
        assert [int(x) for x in r] == st
        for _ in range(5):
            s0, s1, s2, s3 = st
            w = (rotl((s1 * 5) & M64, 7) * 9) & M64
            st = [s0 ^ s3 ^ s1 ^ s2, s1 ^ s2, s2 ^ s0 ^ ((s1 << 17) & M64), rotl(s3 ^ s1, 45)]
            assert oracle.rng_next(r) == w
            assert [int(x) for x in r] == st
    # and it is not textbook xoshiro: the second draw differs
    r = oracle.rng_seeded(7)
    s0, s1, s2, s3 = [int(x) for x in r]
    oracle.rng_next(r)
    tb1 = s1 ^ s2 ^ s0
    assert int(r[1]) != tb1 or s0 == 0


def test_tie_vectors(oracle):
    for xs, want in zip(VEC["ties"], VEC["tie_picks"]):
        lg = np.array([float(x) for x in xs], dtype=np.float32)
        assert oracle.top(lg) == want
        assert oracle.tree_argmax(lg) == want


def test_store_pick_nan_and_inf(oracle):
    lg = np.array([np.nan, 5.0, 5.0, 1.0], dtype=np.float32)
    assert oracle.top(lg) == 1           # NaN never reaches the max
    assert oracle.top(np.full(4, np.nan, dtype=np.float32)) == 4  # vocab: the fallback signal
    lg = np.array([-np.inf, -np.inf, -np.inf], dtype=np.float32)
    assert oracle.top(lg) == 0


def _ckpt(tmp_path, c, kind="hash", seed=0, name="m.ftc2", trained=False):
    p = ckpt.init_params(c, kind, seed, trained=trained)
    path = str(tmp_path / name)
    ckpt.write(path, c, p)
    return path, p


@pytest.mark.parametrize("c,trained", [(cf.SMALL4_V3, False), (cf.SMALL4_NOARMS, False), (cf.SMALL4_V3, True)],
                         ids=["v3-arms", "no-arms", "v3-trained"])
def test_dense_matches_meaning(oracle, tmp_path, c, trained):
    """bend/tests/decode-dense.bend: 96 positions on ctx 64 (the ring wraps);
    dense vs tree within 1e-5 relative on each side of the wrap; a reset
    reproduces the bits; the store pick is the tree argmax at every position.
    v3-trained carries non-unit norm gains, qk gains and per-head sinks."""
    path, _ = _ckpt(tmp_path, c, trained=trained)
    m = oracle.Model(path)
    st, tr = oracle.State(m), oracle.Tree(m)
    ts = VEC["window"]
    dense, tree = [], []
    for pos, t in enumerate(ts):
        st.feed(pos, t)
        dense.append(st.logits())
        tree.append(tr.step(pos, t))
    dense, tree = np.array(dense), np.array(tree)
    for seg in (slice(0, c.ctx), slice(c.ctx, None)):
        d = np.abs(dense[seg] - tree[seg]).max()
        s = np.abs(tree[seg]).max()
        assert d / s <= 1e-5, (seg, d, s)
    st.reset()
    again = []
    for pos, t in enumerate(ts):
        st.feed(pos, t)
        again.append(st.logits())
    assert np.array_equal(np.array(again).view(np.uint32), dense.view(np.uint32))
    for lg in dense:
        assert oracle.top(lg) == oracle.tree_argmax(lg)


def _blank(c):
    """Parameters with every matrix zero, gains 1, nothing else set."""
    blocks, fin = cf.layout(c)
    p = np.zeros(c.params, dtype=np.float32)
    for b in blocks:
        p[b.ra:b.ra + c.d] = 1.0
        p[b.rf:b.rf + c.d] = 1.0
    p[fin:fin + c.d] = 1.0
    return p, blocks, fin


def test_zero_blocks_leave_the_residual(oracle):
    """With zero matrices every block adds exactly 0, so the logits are
    E . (rmsnorm(E[tok]) * final) (a closed form independent of summation
    order up to rounding). The block gains ra and rf are random too: with
    zero matrices they must change nothing, while the final gain must scale
    the head's input column by column."""
    c = cf.Config(64, 16, 32, 48, 4, 2, True, True, True)
    p, blocks, fin = _blank(c)
    rng = np.random.default_rng(1)
    E = rng.standard_normal((c.vocab, c.d)).astype(np.float32)
    p[: c.vocab * c.d] = E.reshape(-1)
    for b in blocks:
        p[b.ra:b.ra + c.d] = 1.0 + 0.3 * rng.standard_normal(c.d)
        p[b.rf:b.rf + c.d] = 1.0 + 0.3 * rng.standard_normal(c.d)
    g = (1.0 + 0.3 * rng.standard_normal(c.d)).astype(np.float32)
    p[fin:fin + c.d] = g
    m = oracle.Model(cfg=c, params=p)
    st = oracle.State(m)
    for pos, tok in enumerate([3, 9, 9, 1]):
        st.feed(pos, tok)
        x = E[tok].astype(np.float64)
        assert np.array_equal(st.x(), E[tok])
        want = E.astype(np.float64) @ (x / np.sqrt((x * x).mean() + 1e-5) * g)
        np.testing.assert_allclose(st.logits(), want, rtol=2e-6, atol=2e-6)


def _rms(x, g):
    return x / np.sqrt((x * x).mean() + 1e-5) * g


def test_softmax_layer_float64(oracle):
    """One softmax layer with every arm on and every parameter non-trivial:
    random Wq, Wk, Wv, Wo, norm gains ra, qk-norm gains gq and gk (one hd
    vector each, shared by the heads, applied as 1 + g), and a different
    sink per head; the GLA layers before it and the MLP are zero. The
    residual after each of 13 tokens on ctx 8 (the ring wraps) is held to
    a float64 evaluation of bend/Model.bend's sm.attend (scores scaled by
    1/sqrt(hd), the sink in the max and the denominator only). A gain
    without its 1 +, one gain vector used for both q and k, sink[0] for
    every head, or a missing 1/sqrt(hd) each fail it by far more than the
    tolerance."""
    c = cf.Config(32, 8, 16, 8, 4, 4, False, True, True)
    p, blocks, fin = _blank(c)
    rng = np.random.default_rng(12)
    d, hd, H = c.d, c.hd, c.heads
    E = rng.standard_normal((c.vocab, d)).astype(np.float32)
    p[: c.vocab * d] = E.reshape(-1)
    sm = blocks[3]
    W = {}
    for name, o in (("q", sm.wq), ("k", sm.wk), ("v", sm.wv), ("o", sm.wo)):
        W[name] = (rng.standard_normal((d, d)) * 0.6).astype(np.float32)
        p[o:o + d * d] = W[name].reshape(-1)
    ra = (1.0 + 0.3 * rng.standard_normal(d)).astype(np.float32)
    gq = (0.4 * rng.standard_normal(hd)).astype(np.float32)
    gk = (0.4 * rng.standard_normal(hd)).astype(np.float32)
    sinks = (1.5 * rng.standard_normal(H)).astype(np.float32)
    p[sm.ra:sm.ra + d] = ra
    p[sm.gq:sm.gq + hd] = gq
    p[sm.gk:sm.gk + hd] = gk
    p[sm.sink:sm.sink + H] = sinks
    m = oracle.Model(cfg=c, params=p)
    st = oracle.State(m)
    f8 = lambda a: np.asarray(a, dtype=np.float64)  # noqa: E731
    Ks, Vs = [], []
    toks = [int(t) for t in rng.integers(0, c.vocab, size=13)]
    for pos, t in enumerate(toks):
        st.feed(pos, t)
        x = f8(E[t])
        n = _rms(x, f8(ra))
        q, k, v = f8(W["q"]) @ n, f8(W["k"]) @ n, f8(W["v"]) @ n
        qh = np.concatenate([_rms(q[h * hd:(h + 1) * hd], 1.0 + f8(gq)) for h in range(H)])
        kh = np.concatenate([_rms(k[h * hd:(h + 1) * hd], 1.0 + f8(gk)) for h in range(H)])
        Ks.append(kh)
        Vs.append(v)
        K, V = np.array(Ks[-c.ctx:]), np.array(Vs[-c.ctx:])
        o = np.zeros(d)
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            s = K[:, sl] @ qh[sl] / math.sqrt(hd)
            mx = max(s.max(), float(sinks[h]))
            e = np.exp(s - mx)
            o[sl] = (e[:, None] * V[:, sl]).sum(0) / (e.sum() + math.exp(float(sinks[h]) - mx))
        want = x + f8(W["o"]) @ o
        np.testing.assert_allclose(st.x(), want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_mlp_float64(oracle):
    """The tail's MLP with a non-unit norm gain: one GLA layer whose mix is
    zero (Wq = Wk = Wv = Wa = Wo = 0), so x' = x + Wd (silu(Wg n) * (Wu n))
    with n = rmsnorm(x) * rf; rf random (ra too, which must not matter).
    Against float64; rf applied to the wrong norm, or gate and up swapped,
    fails it."""
    c = cf.Config(32, 8, 16, 24, 1, 2, False, False, False)
    p, blocks, fin = _blank(c)
    rng = np.random.default_rng(13)
    d, f = c.d, c.f
    E = rng.standard_normal((c.vocab, d)).astype(np.float32)
    p[: c.vocab * d] = E.reshape(-1)
    b = blocks[0]
    Wg = (rng.standard_normal((f, d)) * 0.5).astype(np.float32)
    Wu = (rng.standard_normal((f, d)) * 0.5).astype(np.float32)
    Wd = (rng.standard_normal((d, f)) * 0.5).astype(np.float32)
    p[b.wg:b.wg + f * d] = Wg.reshape(-1)
    p[b.wu:b.wu + f * d] = Wu.reshape(-1)
    p[b.wd:b.wd + d * f] = Wd.reshape(-1)
    rf = (1.0 + 0.3 * rng.standard_normal(d)).astype(np.float32)
    p[b.rf:b.rf + d] = rf
    p[b.ra:b.ra + d] = 1.0 + 0.3 * rng.standard_normal(d)
    m = oracle.Model(cfg=c, params=p)
    st = oracle.State(m)
    for pos, t in enumerate([5, 1, 30, 7]):
        st.feed(pos, t)
        x = E[t].astype(np.float64)
        n = _rms(x, rf.astype(np.float64))
        g, u = Wg.astype(np.float64) @ n, Wu.astype(np.float64) @ n
        want = x + Wd.astype(np.float64) @ (g / (1.0 + np.exp(-g)) * u)
        np.testing.assert_allclose(st.x(), want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_attention_closed_form(oracle):
    """Wq = Wk = 0 makes every score 0: the softmax is uniform over the live
    slots, and with sinks each head's denominator gains exp(sink - max(0,
    sink)). Wv = I and Wo = I then put the mean of the live values (scaled
    by the sink) into the residual; the MLP is off (Wd = 0)."""
    c = cf.Config(16, 8, 8, 8, 4, 2, False, False, True)
    p, blocks, fin = _blank(c)
    rng = np.random.default_rng(2)
    E = rng.standard_normal((c.vocab, c.d)).astype(np.float32)
    p[: c.vocab * c.d] = E.reshape(-1)
    sm = blocks[3]
    d = c.d
    p[sm.wv:sm.wv + d * d] = np.eye(d, dtype=np.float32).reshape(-1)
    p[sm.wo:sm.wo + d * d] = np.eye(d, dtype=np.float32).reshape(-1)
    sinks = np.array([0.5, -1.0], dtype=np.float32)
    p[sm.sink:sm.sink + c.heads] = sinks
    m = oracle.Model(cfg=c, params=p)
    st = oracle.State(m)
    toks = [1, 4, 7, 2, 9, 11, 3, 5, 6, 8, 10]    # 11 tokens on ctx 8: wraps
    for pos, t in enumerate(toks):
        st.feed(pos, t)
        x = E[t].astype(np.float64)
        nrm = x / np.sqrt((x * x).mean() + 1e-5)
        live = [E[u].astype(np.float64) / np.sqrt((E[u].astype(np.float64) ** 2).mean() + 1e-5)
                for u in toks[max(0, pos - c.ctx + 1): pos + 1]]
        V = np.array(live)
        want = x.copy()
        hd = c.hd
        for h in range(c.heads):
            mx = max(0.0, float(sinks[h]))
            w = np.exp(0.0 - mx)
            den = w * len(live) + math.exp(float(sinks[h]) - mx)
            want[h * hd:(h + 1) * hd] += (w * V[:, h * hd:(h + 1) * hd]).sum(0) / den
        np.testing.assert_allclose(st.x(), want, rtol=2e-5, atol=2e-6)
        del nrm


def test_gla_state_closed_form(oracle):
    """One GLA layer with sigmoid gates: Wa = 0 gives alpha = 1/2 exactly;
    Wq = Wk = Wv = I. Then S_t = S_{t-1}/2 + k^ v^T with k^ the per-head L2
    normalised key, and the state is checked against that recurrence in
    float64 (the residual stream is irrelevant: Wo = Wd = 0)."""
    c = cf.Config(16, 8, 8, 8, 1, 2, False, False, False)
    p, blocks, fin = _blank(c)
    rng = np.random.default_rng(3)
    E = rng.standard_normal((c.vocab, c.d)).astype(np.float32)
    p[: c.vocab * c.d] = E.reshape(-1)
    b = blocks[0]
    d, hd = c.d, c.hd
    for w in (b.wq, b.wk, b.wv):
        p[w:w + d * d] = np.eye(d, dtype=np.float32).reshape(-1)
    m = oracle.Model(cfg=c, params=p)
    st = oracle.State(m)
    S = np.zeros((c.heads, hd, hd))
    for pos, t in enumerate([2, 5, 5, 13, 0, 7]):
        st.feed(pos, t)
        x = E[t].astype(np.float64)
        n = x / np.sqrt((x * x).mean() + 1e-5)
        for h in range(c.heads):
            k = n[h * hd:(h + 1) * hd]
            kh = k / np.sqrt(1e-6 + (k * k).sum())
            S[h] = 0.5 * S[h] + np.outer(kh, k)
        np.testing.assert_allclose(st.layer(0).reshape(S.shape), S, rtol=1e-5, atol=1e-6)


def test_rglru_state_closed_form(oracle):
    """One GLA layer with the RG-LRU gate: Wa = 0 gives z = 0, sigmoid(z) =
    1/2, so la = min(-1e-4, 4 log sigmoid(lam)) (Griffin's gate at c = 8),
    alpha = exp(la) and the key is scaled by sqrt(1 - alpha^2). With
    Wq = Wk = Wv = I the state follows S_t = alpha S_{t-1} + (s k^) v^T,
    checked in float64."""
    c = cf.Config(16, 8, 8, 8, 1, 2, True, False, False)
    p, blocks, fin = _blank(c)
    rng = np.random.default_rng(6)
    E = rng.standard_normal((c.vocab, c.d)).astype(np.float32)
    p[: c.vocab * c.d] = E.reshape(-1)
    b = blocks[0]
    d, hd = c.d, c.hd
    for w in (b.wq, b.wk, b.wv):
        p[w:w + d * d] = np.eye(d, dtype=np.float32).reshape(-1)
    lam = np.array([4.0, 2.0, 0.5, -1.0, 9.0, 12.0, 0.0, 3.0], dtype=np.float32)
    p[b.lam:b.lam + d] = lam
    m = oracle.Model(cfg=c, params=p)
    st = oracle.State(m)
    lam64 = lam.astype(np.float64)
    la = np.minimum(-1e-4, 4.0 * -np.log1p(np.exp(-lam64)))
    alpha, scale = np.exp(la), np.sqrt(1 - np.exp(2 * la))
    S = np.zeros((c.heads, hd, hd))
    for pos, t in enumerate([2, 5, 5, 13, 0, 7]):
        st.feed(pos, t)
        x = E[t].astype(np.float64)
        n = x / np.sqrt((x * x).mean() + 1e-5)
        for h in range(c.heads):
            k = n[h * hd:(h + 1) * hd]
            kh = k / np.sqrt(1e-6 + (k * k).sum()) * scale[h * hd:(h + 1) * hd]
            S[h] = alpha[h * hd:(h + 1) * hd, None] * S[h] + np.outer(kh, k)
        np.testing.assert_allclose(st.layer(0).reshape(S.shape), S, rtol=1e-5, atol=1e-6)


def test_sampler_thresholds_and_draw(oracle):
    rng = np.random.default_rng(4)
    for v in (258, 1000, 4096, 32768):
        lg = (rng.standard_normal(v) * 3).astype(np.float32)
        for k in (1, 5, 40):
            t = oracle.topk_threshold(lg, k)
            kth = np.sort(lg)[::-1][k - 1]
            assert (lg >= t).sum() >= k
            # the bisection stops within float spacing below the k-th largest
            assert kth - 100 * 2.0 ** -39 - 8 * np.spacing(np.abs(kth)) <= t <= kth
        w = np.exp((lg - lg.max()) / 0.8).astype(np.float32)
        for p_ in (0.5, 0.9):
            t = oracle.topp_threshold(w, p_)
            assert w[w >= t].astype(np.float64).sum() >= p_ * w.astype(np.float64).sum() * (1 - 1e-5)
        # top-k 1 is the argmax, whatever the temperature and top-p
        r = oracle.rng_seeded(9)
        assert oracle.pick(lg, 1.3, 1, 0.9, r) == int(np.argmax(lg))
        # greedy leaves the rng untouched
        r0 = r.copy()
        assert oracle.pick(lg, 0.0, 40, 0.9, r) == oracle.tree_argmax(lg)
        assert np.array_equal(r, r0)


def test_bisections_take_forty_steps(oracle):
    """Sample.bend's thresholds bisect 40 times: top-k over [peak - 100,
    peak] (a final width of 100 / 2^40 = 9.09e-11) and top-p over [0, 1]
    (2^-40 = 9.09e-13). So when the value just below the boundary sits
    further below it than that width, exactly the true set survives; with
    a gap between one and two widths, a bisection of 39 steps (twice the
    width) keeps the value below the boundary for some placements. Values
    near zero keep float32 spacing far below either width."""
    rng = np.random.default_rng(40)
    v, k = 64, 3
    for trial in range(64):
        # top-k: the peak at 0, the k-th largest at -x, the next 1.35 widths
        # below it, every other logit far below
        x = float(rng.uniform(1e-10, 3e-9))
        gap = 1.35 * 100.0 * 2.0 ** -40
        lg = np.full(v, -60.0, np.float32)
        lg[5], lg[17] = 0.0, -1e-11
        lg[30] = -x
        lg[41] = -(x + gap)
        assert np.float32(-(x + gap)) < np.float32(-x)
        t = oracle.topk_threshold(lg, k)
        assert (lg >= t).sum() == k, (trial, x, t)
        # top-p: weights of magnitude 1e-11, the boundary weight b and the
        # next 1.35 widths below it; the mass needed lies between the top
        # two's and the top three's
        b = float(rng.uniform(3e-12, 6e-12))
        w = np.full(v, 1e-14, np.float32)
        w[7], w[20] = 9e-12, b
        w[33] = b - 1.35 * 2.0 ** -40
        total = float(w.astype(np.float64).sum())
        need = 9e-12 + 0.5 * b
        t = oracle.topp_threshold(w, np.float32(need / total))
        assert (w >= t).sum() == 2, (trial, b, t)


def test_draw_follows_cumulative_mass(oracle):
    """With top-k and top-p off the draw is inverse CDF over index order:
    the pick i satisfies cum[i-1] <= u*total < cum[i] up to rounding."""
    rng = np.random.default_rng(5)
    v = 512
    lg = rng.standard_normal(v).astype(np.float32)
    seeds = range(200)
    counts = np.zeros(v)
    for s in seeds:
        r = oracle.rng_seeded(s)
        r2 = r.copy()
        word = oracle.rng_next(r2)
        unit = ((word >> 32) >> 8) / 16777216.0
        w = np.exp((lg.astype(np.float64) - lg.max()) / 1.0)
        cum = np.cumsum(w)
        u = unit * cum[-1]
        i = oracle.pick(lg, 1.0, 0xFFFFFFFF, 1.0, r)
        assert np.array_equal(r, r2)
        lo = cum[i - 1] if i else 0.0
        assert lo - 1e-4 * cum[-1] <= u <= cum[i] + 1e-4 * cum[-1]
        counts[i] += 1
    assert counts.sum() == len(seeds)


def test_ftc2_round_trip_and_errors(oracle, tmp_path):
    c = cf.SMALL4_V3
    path, p = _ckpt(tmp_path, c, "normal", 3)
    assert ckpt.read_config(path) == c
    m = oracle.Model(path)
    assert m.vocab == c.vocab and m.step == 0
    assert oracle.params(c) == c.params
    assert oracle.model_id(c) == c.model_id
    raw = open(path, "rb").read()
    bad = tmp_path / "bad.ftc2"
    bad.write_bytes(b"FTC3" + raw[4:])
    with pytest.raises(ValueError, match="magic is not FTC2"):
        oracle.Model(str(bad))
    bad.write_bytes(raw[: len(raw) - 20])
    with pytest.raises(ValueError, match="short read"):
        oracle.Model(str(bad))


def test_params_formula():
    # bend/Config.bend:243-253 at the reference's 115M (arms off / on) and
    # BASELINE's f = 3072 variant
    assert cf.Config(32768, 2048, 768, 2048, 12, 12, False, False, False).params == 115_428_096
    assert cf.FP100M.params == 115_435_428
    assert cf.Config(32768, 2048, 768, 3072, 12, 12, False, False, False).params == 143_739_648
    assert cf.V1.params == 12_781_824


def _f32max(a, b):
    # F32.max a b = (a < b ? b : a)
    return b if a < b else a


def test_ce_tree_order(oracle):
    """or_ce, Evaluate.bend's summand G.lse(l) - l[y] (bend/Train/Grad.bend:
    795-797): pinned by uniform logits (the tree sum of ones is exact, so
    the value is log v), by a hand expansion of the depth-3 tree of 5
    leaves (a sequential sum or another max convention fails some of the
    random trials), and by a double-precision logsumexp at v = 32768."""
    f32 = np.float32
    for v in (258, 32768):
        lg = np.full(v, 1.25, np.float32)
        want = f32(f32(f32(1.25) + f32(np.log(np.float64(v)))) - f32(1.25))
        assert oracle.ce(lg, 7) == want
    rng = np.random.default_rng(31)
    for _ in range(200):
        x = (rng.standard_normal(5) * 3.0).astype(np.float32)
        y = int(rng.integers(0, 5))
        vz = f32(-3.0e38)
        m = _f32max(_f32max(_f32max(x[0], x[1]), _f32max(x[2], x[3])),
                    _f32max(_f32max(x[4], vz), _f32max(vz, vz)))
        e = [f32(np.exp(np.float64(f32(xi - m)))) for xi in x]
        s = f32(f32(f32(e[0] + e[1]) + f32(e[2] + e[3])) + f32(f32(e[4] + f32(0.0)) + f32(0.0)))
        want = f32(f32(m + f32(np.log(np.float64(s)))) - x[y])
        assert oracle.ce(x, y) == want, (x, y)
    x = (rng.standard_normal(32768) * 4.0).astype(np.float32)
    xd = x.astype(np.float64)
    ref = np.log(np.exp(xd - xd.max()).sum()) + xd.max() - xd[123]
    assert abs(oracle.ce(x, 123) - ref) <= 1e-5 * max(1.0, abs(ref))



def test_stat_prob_and_rival(oracle):
    """or_stat, dc.prob.of (bend/Decode.bend:199-202) and al.stat
    (bend/Agent/Loop.bend:284-288): p = exp(l[x] - m) / z over the tree
    sum z, the rival a = Sample.argmax with l[x] set to -3e38 (least index
    on a tie), pa its probability. Pinned by uniform logits (z = v exactly,
    so p = 1/v and the rival is index 0, or 1 when x is 0), by the 5-leaf
    depth-3 tree expanded by hand (the sum's order and the max's
    convention), by logits near 1e4 (the sum overflows unless the max comes
    off first), and by a double-precision softmax at v = 32768."""
    f32 = np.float32
    for v in (256, 32768):
        lg = np.full(v, 2.5, np.float32)
        for x in (0, 5):
            p, a, pa = oracle.stat(lg, x)
            assert p == f32(1.0) / f32(v) and pa == p
            assert a == (1 if x == 0 else 0)
    rng = np.random.default_rng(7)
    vz = f32(-3.0e38)
    for _ in range(200):
        lg = (rng.standard_normal(5) * 3.0).astype(np.float32)
        x = int(rng.integers(0, 5))
        m = _f32max(_f32max(_f32max(lg[0], lg[1]), _f32max(lg[2], lg[3])),
                    _f32max(_f32max(lg[4], vz), _f32max(vz, vz)))
        e = [f32(np.exp(np.float64(f32(xi - m)))) for xi in lg]
        z = f32(f32(f32(e[0] + e[1]) + f32(e[2] + e[3])) + f32(f32(e[4] + f32(0.0)) + f32(0.0)))
        others = [(float(lg[i]) if i != x else -3.0e38, -i) for i in range(5)]
        a_want = -max(others)[1]
        p, a, pa = oracle.stat(lg, x)
        assert p == f32(e[x] / z) and a == a_want and pa == f32(e[a_want] / z), (lg, x)
    big = np.full(300, 1.0e4, np.float32)
    big[17] = 1.0e4 + 2.0
    p, a, pa = oracle.stat(big, 17)
    assert np.isfinite(p) and abs(float(p) - np.exp(2.0) / (np.exp(2.0) + 299)) < 1e-6 and a == 0
    lg = (rng.standard_normal(32768) * 4.0).astype(np.float32)
    x = int(np.argsort(lg)[-1])
    d = lg.astype(np.float64)
    sm = np.exp(d - d.max())
    sm /= sm.sum()
    p, a, pa = oracle.stat(lg, x)
    second = int(np.argsort(lg)[-2])
    assert a == second
    assert abs(float(p) - sm[x]) <= 1e-6 * sm[x] and abs(float(pa) - sm[second]) <= 1e-6 * sm[second]
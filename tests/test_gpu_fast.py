"""libana's fast numerics modes on the GPU against the CPU oracle.

ANA_FAST_FP32 reassociates the decode step's sums (split-K products, tree
reductions, fused multiply-adds); ANA_BF16 also reads the matrices as
bfloat16. Neither can be bit-exact, so these tests hold them to the
tolerances the north star states, measured on the logits of every decode
step, teacher-forced on the same tokens as the oracle:

    max_i |got_i - want_i| / max_i |want_i|  <=  1e-4 (fp32-fast), 2e-2 (bf16)

and check the greedy token loop's picks are argmaxes of the oracle's logits
up to that tolerance (a near-tie may pick either side of it).

Every checkpoint here carries trained-like vectors (norm gains 1 + N(0, 0.1^2),
qk-norm gains N(0, 0.1^2), per-head sinks N(0, 1)), so the gains the fast
modes fold into their packed weights, the (1 + g) qk factor and per-head
sink indexing are all exercised.
"""
import json
import os

import numpy as np
import pytest

import ana_amd
from ana_amd import ckpt
from ana_amd import config as cf

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = json.load(open(os.path.join(HERE, "golden", "reference_vectors.json")))
TOL = {ana_amd.FAST_FP32: 1e-4, ana_amd.BF16: 2e-2}
MODES = [pytest.param(ana_amd.FAST_FP32, id="fast_fp32"), pytest.param(ana_amd.BF16, id="bf16")]


def rel_err(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.abs(got - want).max() / np.abs(want).max())


@pytest.fixture(scope="module")
def small_ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckf")
    p = str(d / "v3.ftc2")
    ckpt.write(p, cf.SMALL4_V3, ckpt.init_params(cf.SMALL4_V3, "normal", 3, trained=True))
    return p


# d and f multiples of 128 (the packed decode-batch products take K = 256
# and 1024 here; gate|up at 120 rows takes two weight tiles a workgroup),
# every arm on, hd 64
MID = cf.Config(vocab=258, ctx=64, d=256, f=1024, layers=4, heads=4, rglru=True, qk=True, sinks=True, tied=True)


@pytest.fixture(scope="module")
def mid_ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckm")
    p = str(d / "mid.ftc2")
    ckpt.write(p, MID, ckpt.init_params(MID, "normal", 5, trained=True))
    return p


@pytest.fixture(scope="module")
def big_ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckb")
    p = str(d / "fp100m.ftc2")
    ckpt.write(p, cf.FP100M, ckpt.init_params(cf.FP100M, "normal", 0, trained=True))
    return p


@pytest.mark.parametrize("mode", MODES)
def test_fast_small_decode(oracle, small_ckpt, mode):
    """small4_v3 (all arms, ctx 64): 96 tokens of the LCG window fed one at a
    time through the fast step, across the ring wrap; logits every step."""
    print(f"case fast small mode {mode}", flush=True)
    m = oracle.Model(small_ckpt)
    st = oracle.State(m)
    worst = 0.0
    with ana_amd.Decoder(small_ckpt, numerics=mode) as dec:
        for pos, t in enumerate(VEC["window"]):
            dec.feed([0], [pos], [t])
            st.feed(pos, t)
            e = rel_err(dec.logits([0])[0], st.logits())
            worst = max(worst, e)
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
def test_fast_115m_batch6(oracle, big_ckpt, mode):
    """fp100m at ctx 2048, six sequences: decode steps of more than four
    rows, so every layer product (K 768 and 2048) and the head run on the
    packed matrix-core GEMM; logits against each sequence's oracle run."""
    print(f"case fast 115m batch6 mode {mode}", flush=True)
    oracle.set_threads(8)
    m = oracle.Model(big_ckpt)
    n, pre, steps = 6, [5, 9, 14, 20, 3, 11], 4
    prompts = [[int(t) for t in ckpt.prompt(17 + i, pre[i] + steps, m.vocab)] for i in range(n)]
    sts = [oracle.State(m) for _ in range(n)]
    worst = 0.0
    with ana_amd.Decoder(big_ckpt, max_seqs=n, numerics=mode) as dec:
        for i in range(n):
            dec.feeds(i, 0, prompts[i][: pre[i]])
            for p in range(pre[i]):
                sts[i].feed(p, prompts[i][p])
        for k in range(steps):
            pos = [pre[i] + k for i in range(n)]
            tok = [prompts[i][pos[i]] for i in range(n)]
            dec.feed(list(range(n)), pos, tok)
            for i in range(n):
                sts[i].feed(pos[i], tok[i])
            if k in (0, steps - 1):
                got = dec.logits(list(range(n)))
                for i in range(n):
                    worst = max(worst, rel_err(got[i], sts[i].logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
def test_fast_115m_batch(oracle, big_ckpt, mode):
    """fp100m at ctx 2048: four sequences prefilled (exact chunks), then 6
    fast decode steps together; every sequence's logits against its own
    oracle run."""
    print(f"case fast 115m batch mode {mode}", flush=True)
    oracle.set_threads(8)
    m = oracle.Model(big_ckpt)
    n, pre, steps = 4, [5, 9, 14, 20], 6
    prompts = [[int(t) for t in ckpt.prompt(7 + i, pre[i] + steps, m.vocab)] for i in range(n)]
    sts = [oracle.State(m) for _ in range(n)]
    worst = 0.0
    with ana_amd.Decoder(big_ckpt, max_seqs=n, numerics=mode) as dec:
        for i in range(n):
            dec.feeds(i, 0, prompts[i][: pre[i]])
            for p in range(pre[i]):
                sts[i].feed(p, prompts[i][p])
        for k in range(steps):
            pos = [pre[i] + k for i in range(n)]
            tok = [prompts[i][pos[i]] for i in range(n)]
            dec.feed(list(range(n)), pos, tok)
            for i in range(n):
                sts[i].feed(pos[i], tok[i])
            if k in (0, steps - 1):
                got = dec.logits(list(range(n)))
                for i in range(n):
                    worst = max(worst, rel_err(got[i], sts[i].logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
def test_fast_token_loop(oracle, small_ckpt, mode):
    """ana_generate in a fast mode: each pick, teacher-forced into the oracle,
    is within tolerance of the oracle's maximum logit at that step."""
    print(f"case fast generate mode {mode}", flush=True)
    m = oracle.Model(small_ckpt)
    pr = VEC["window"][:9]
    steps = 60
    with ana_amd.Decoder(small_ckpt, max_seqs=1, prefill_chunk=16, numerics=mode) as dec:
        dec.feeds(0, 0, pr[:-1])
        out = dec.generate([0], [len(pr) - 1], [pr[-1]], steps)[0]
    st = oracle.State(m)
    for p, t in enumerate(pr):
        st.feed(p, t)
    pos = len(pr)
    for t in out:
        lg = st.logits()
        scale = np.abs(lg).max()
        assert lg[t] >= lg.max() - 2 * TOL[mode] * scale, (pos, t, int(lg.argmax()))
        st.feed(pos, int(t))
        pos += 1


@pytest.mark.skip(reason="its first run faulted the GPU (an illegal memory access reported at the "
                         "first ana_logits of 8 sequences); no cause found yet, so the paths it "
                         "covered (fast decode of more than 4 sequences, the matrix-core head, "
                         "fast products in prefill chunks of 4 rows or fewer) are switched off")
@pytest.mark.parametrize("mode", MODES)
def test_fast_batch8_matrix_cores(oracle, small_ckpt, mode):
    """Eight sequences decoded together: the products run on the matrix cores
    (B > 4), GLA and attention on the fast kernels; each sequence's logits
    against its own oracle run, across the ring wrap."""
    print(f"case fast batch8 mode {mode}", flush=True)
    m = oracle.Model(small_ckpt)
    n, steps = 8, 72
    rng = np.random.default_rng(5)
    streams = rng.integers(0, m.vocab, size=(n, steps + 8)).astype(np.uint32)
    starts = [0, 1, 2, 3, 5, 8, 4, 6]
    sts = [oracle.State(m) for _ in range(n)]
    worst = 0.0
    with ana_amd.Decoder(small_ckpt, max_seqs=n, numerics=mode, prefill_chunk=8) as dec:
        for i in range(n):
            if starts[i]:
                dec.feeds(i, 0, streams[i, : starts[i]])
            for p in range(starts[i]):
                sts[i].feed(p, int(streams[i, p]))
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tok = [int(streams[i, pos[i]]) for i in range(n)]
            dec.feed(list(range(n)), pos, tok)
            for i in range(n):
                sts[i].feed(pos[i], tok[i])
            if k % 12 == 11:
                got = dec.logits(list(range(n)))
                for i in range(n):
                    worst = max(worst, rel_err(got[i], sts[i].logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.fixture(scope="module")
def noarms_ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckn")
    p = str(d / "noarms.ftc2")
    ckpt.write(p, cf.SMALL4_NOARMS, ckpt.init_params(cf.SMALL4_NOARMS, "normal", 4, trained=True))
    return p


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("arms", ["v3", "noarms"])
@pytest.mark.parametrize("chunk", [16, 48])
def test_fast_prefill(oracle, small_ckpt, noarms_ckpt, mode, arms, chunk):
    """An 88-token prompt through chunked prefill (matrix-core products, the
    GLA chunk as a scan over 32-token sub-chunks, split attention; chunks past
    the ring wrap at ctx 64 take the per-token attention), then 8 fast decode
    steps; logits against the oracle fed the same tokens."""
    path = small_ckpt if arms == "v3" else noarms_ckpt
    print(f"case fast prefill {arms} chunk {chunk} mode {mode}", flush=True)
    m = oracle.Model(path)
    st = oracle.State(m)
    ts = VEC["window"]
    worst = 0.0
    with ana_amd.Decoder(path, prefill_chunk=chunk, numerics=mode) as dec:
        dec.feeds(0, 0, ts[:88])
        for p in range(88):
            st.feed(p, ts[p])
        worst = max(worst, rel_err(dec.logits([0])[0], st.logits()))
        for p in range(88, 96):
            dec.feed([0], [p], [ts[p]])
            st.feed(p, ts[p])
            worst = max(worst, rel_err(dec.logits([0])[0], st.logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("shape", ["ragged5", "wide6", "rows120"])
@pytest.mark.parametrize("model", ["small", "mid"])
def test_fast_feeds_n(oracle, small_ckpt, mid_ckpt, mode, shape, model):
    """ana_feeds_n in a fast mode: ragged prompts prefilled together
    (matrix-core products over all their rows: 93 rows a step; 288 for the
    128 x 128 tiles; 120, where gate|up takes two weight tiles a
    workgroup), then a decode step each; logits against the oracle."""
    print(f"case fast feeds_n {model} {shape} mode {mode}", flush=True)
    path = small_ckpt if model == "small" else mid_ckpt
    m = oracle.Model(path)
    if shape == "ragged5":
        seqs, lens, chunk = [3, 0, 2, 4, 1], [40, 3, 17, 70, 9], 32
    elif shape == "rows120":
        seqs, lens, chunk = [1, 3, 0, 2], [60, 45, 30, 90], 30
    else:
        seqs, lens, chunk = [5, 0, 2, 4, 1, 3], [60, 100, 49, 77, 90, 63], 48
    n = len(seqs)
    rng = np.random.default_rng(22)
    toks = [rng.integers(0, m.vocab, size=k + 1).astype(np.uint32) for k in lens]
    worst = 0.0
    with ana_amd.Decoder(path, max_seqs=n, prefill_chunk=chunk, numerics=mode) as dec:
        dec.feeds_n(seqs, [0] * n, [t[:-1] for t in toks])
        for i, s in enumerate(seqs):
            dec.feed([s], [lens[i]], [int(toks[i][-1])])
        got = dec.logits(seqs)
    for i in range(n):
        st = oracle.State(m)
        for p, t in enumerate(toks[i]):
            st.feed(p, int(t))
        worst = max(worst, rel_err(got[i], st.logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
def test_fast_score_n(oracle, small_ckpt, mode):
    """ana_score_n in a fast mode: five windows (300 rows in the first
    step, so the head runs on the 128 x 128 matrix-core tiles); every
    summand within 2 x tolerance x max|logit| of the oracle's."""
    print(f"case fast score_n mode {mode}", flush=True)
    m = oracle.Model(small_ckpt)
    seqs, lens = [4, 0, 2, 3, 1], [64, 61, 50, 64, 65]
    rng = np.random.default_rng(43)
    toks = [rng.integers(0, m.vocab, size=k).astype(np.uint32) for k in lens]
    with ana_amd.Decoder(small_ckpt, max_seqs=5, prefill_chunk=64, numerics=mode) as dec:
        got = dec.score_n(seqs, [0] * 5, toks)
    worst = 0.0
    for i in range(5):
        st = oracle.State(m)
        for k in range(lens[i] - 1):
            st.feed(k, int(toks[i][k]))
            lg = st.logits()
            want = oracle.ce(lg, int(toks[i][k + 1]))
            worst = max(worst, abs(float(got[i][k]) - want) / float(np.abs(lg).max()))
    print(f"worst |d ce| / max|logit| {worst:.3e}", flush=True)
    assert worst <= 2 * TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("model", ["small", "mid"])
def test_fast_decode_batch_products(oracle, small_ckpt, mid_ckpt, mode, model):
    """Decode steps of more than kSmallB sequences in a fast mode: the layer
    products and the head on the matrix cores (the packed GEMM where K is a
    multiple of 128, the mid model; the tiled fallback for the small model's
    K = 64 and 192), GLA and attention exact. Seven sequences from ragged
    starts, 70 teacher-forced steps across the ring wrap; every sequence's
    logits against its own oracle run at four steps."""
    print(f"case fast decode batch products {model} mode {mode}", flush=True)
    path = small_ckpt if model == "small" else mid_ckpt
    m = oracle.Model(path)
    n, steps = 7, 70
    starts = [3, 1, 6, 2, 8, 5, 4]
    seqs = [2, 0, 3, 6, 5, 1, 4]
    rng = np.random.default_rng(17)
    toks = rng.integers(0, m.vocab, size=(n, steps + 8)).astype(np.uint32)
    sts = [oracle.State(m) for _ in range(n)]
    worst = 0.0
    with ana_amd.Decoder(path, max_seqs=n, prefill_chunk=8, numerics=mode) as dec:
        for i in range(n):
            dec.feeds(seqs[i], 0, toks[i, : starts[i]])
            for p in range(starts[i]):
                sts[i].feed(p, int(toks[i, p]))
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tk = [int(toks[i, pos[i]]) for i in range(n)]
            dec.feed(seqs, pos, tk)
            for i in range(n):
                sts[i].feed(pos[i], tk[i])
            if k in (0, 30, 58, steps - 1):
                got = dec.logits(seqs)
                for i in range(n):
                    worst = max(worst, rel_err(got[i], sts[i].logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
def test_fast_greedy_batch_keys(mid_ckpt, mode):
    """Greedy picks of more than four sequences in a fast mode come from the
    head's argmax keys (no pass over the stored logits): ana_generate's
    tokens equal the first index of the max of the logits a twin decoder
    reads after feeding the same tokens, and ana_top equals that argmax."""
    print(f"case fast greedy batch keys mode {mode}", flush=True)
    n, steps = 7, 6
    rng = np.random.default_rng(31)
    with ana_amd.Decoder(mid_ckpt, max_seqs=n, numerics=mode) as dec, \
            ana_amd.Decoder(mid_ckpt, max_seqs=n, numerics=mode) as twin:
        v = dec.vocab
        prompts = [rng.integers(2, v, size=3 + i).astype(np.uint32) for i in range(n)]
        for d in (dec, twin):
            d.feeds_n(list(range(n)), [0] * n, [p[:-1] for p in prompts])
        pos = np.array([len(p) - 1 for p in prompts], dtype=np.uint32)
        tok = np.array([p[-1] for p in prompts], dtype=np.uint32)
        got = dec.generate(list(range(n)), pos, tok, steps)
        t, p = tok.copy(), pos.copy()
        for k in range(steps):
            twin.feed(list(range(n)), p, t)
            lg = twin.logits(list(range(n)))
            want = lg.argmax(axis=1).astype(np.uint32)
            assert np.array_equal(twin.top(list(range(n))), want), k
            assert np.array_equal(got[:, k], want), (k, got[:, k], want)
            t, p = want, p + 1


@pytest.mark.parametrize("mode", MODES)
def test_fast_decode_wide_batch(oracle, mid_ckpt, mode):
    """Decode steps of 160 sequences (above the prefill products' 128-row
    tiles, still on the packed products, the wide head and its greedy keys):
    ragged starts, six steps; five sequences' logits against their own oracle
    runs, and the greedy picks of a generate step are the argmax of a twin
    decoder's logits."""
    print(f"case fast decode wide batch mode {mode}", flush=True)
    m = oracle.Model(mid_ckpt)
    n, steps = 160, 6
    rng = np.random.default_rng(29)
    starts = [1 + i % 5 for i in range(n)]
    toks = rng.integers(2, m.vocab, size=(n, 16)).astype(np.uint32)
    watch = [0, 37, 81, 128, 159]
    sts = {i: oracle.State(m) for i in watch}
    seqs = list(range(n))
    worst = 0.0
    with ana_amd.Decoder(mid_ckpt, max_seqs=n, prefill_chunk=8, numerics=mode) as dec, \
            ana_amd.Decoder(mid_ckpt, max_seqs=n, prefill_chunk=8, numerics=mode) as twin:
        for d_ in (dec, twin):
            d_.feeds_n(seqs, [0] * n, [toks[i, : starts[i]] for i in range(n)])
        for i in watch:
            for p in range(starts[i]):
                sts[i].feed(p, int(toks[i, p]))
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tk = [int(toks[i, pos[i]]) for i in range(n)]
            dec.feed(seqs, pos, tk)
            twin.feed(seqs, pos, tk)
            for i in watch:
                sts[i].feed(pos[i], tk[i])
        got = dec.logits(seqs)
        for i in watch:
            worst = max(worst, rel_err(got[i], sts[i].logits()))
        # one greedy step at the next position against the twin's argmax
        nxt = [starts[i] + steps for i in range(n)]
        tn = [int(toks[i, nxt[i]]) for i in range(n)]
        picks = dec.generate(seqs, nxt, tn, 1)[:, 0]
        twin.feed(seqs, nxt, tn)
        lg = twin.logits(seqs)
        want = np.argmax(lg, axis=1)
        assert np.array_equal(picks, want.astype(np.uint32)), np.nonzero(picks != want)[0][:8]
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


LONG = cf.Config(vocab=258, ctx=1024, d=256, f=1024, layers=4, heads=4, rglru=True, qk=True, sinks=True, tied=True)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("chunk", [64, 320])
def test_fast_decode_long_split(oracle, tmp_path, mode, chunk):
    """Decode steps of 6 sequences at 600+ live slots (ctx 1024): the fast
    attention above four rows takes the window in 256-slot pieces and a
    combine. Ragged prompts through ana_feeds_n (chunks of 64 tokens take
    the GLA a workgroup per chunk, chunks of 320 the scan over sub-chunks),
    then teacher-forced steps through ana_feed; three sequences' logits
    against their own oracle runs after every step."""
    print(f"case fast decode long split chunk {chunk} mode {mode}", flush=True)
    p = str(tmp_path / "long.ftc2")
    ckpt.write(p, LONG, ckpt.init_params(LONG, "normal", 11, trained=True))
    m = oracle.Model(p)
    n, steps = 6, 4
    rng = np.random.default_rng(31)
    starts = [600 + 13 * i for i in range(n)]
    toks = rng.integers(2, m.vocab, size=(n, max(starts) + steps + 1)).astype(np.uint32)
    watch = [0, 3, 5]
    sts = {i: oracle.State(m) for i in watch}
    for i in watch:
        for q in range(starts[i]):
            sts[i].feed(q, int(toks[i, q]))
    seqs = list(range(n))
    worst = 0.0
    with ana_amd.Decoder(p, max_seqs=n, prefill_chunk=chunk, numerics=mode) as dec:
        dec.feeds_n(seqs, [0] * n, [toks[i, : starts[i]] for i in range(n)])
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tk = [int(toks[i, pos[i]]) for i in range(n)]
            dec.feed(seqs, pos, tk)
            got = dec.logits(seqs)
            for i in watch:
                sts[i].feed(pos[i], tk[i])
                worst = max(worst, rel_err(got[i], sts[i].logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


WRAP = cf.Config(vocab=258, ctx=512, d=256, f=1024, layers=4, heads=4, rglru=True, qk=True, sinks=True, tied=True)


@pytest.mark.parametrize("mode", MODES)
def test_fast_decode_split_after_wrap(oracle, tmp_path, mode):
    """The wide decode attention in 256-slot pieces after the ring wraps:
    6 sequences from positions 480-515 on ctx 512 (so two pieces, every slot
    live once the ring has wrapped), 40 teacher-forced decode steps that
    carry every sequence past position 512; three sequences' logits against
    their own oracle runs every fourth step."""
    print(f"case fast decode split after wrap mode {mode}", flush=True)
    p = str(tmp_path / "wrap.ftc2")
    ckpt.write(p, WRAP, ckpt.init_params(WRAP, "normal", 13, trained=True))
    m = oracle.Model(p)
    n, steps = 6, 40
    rng = np.random.default_rng(37)
    starts = [480 + 7 * i for i in range(n)]
    toks = rng.integers(2, m.vocab, size=(n, max(starts) + steps + 1)).astype(np.uint32)
    watch = [0, 2, 5]
    sts = {i: oracle.State(m) for i in watch}
    for i in watch:
        for q in range(starts[i]):
            sts[i].feed(q, int(toks[i, q]))
    seqs = list(range(n))
    worst = 0.0
    with ana_amd.Decoder(p, max_seqs=n, prefill_chunk=64, numerics=mode) as dec:
        dec.feeds_n(seqs, [0] * n, [toks[i, : starts[i]] for i in range(n)])
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tk = [int(toks[i, pos[i]]) for i in range(n)]
            dec.feed(seqs, pos, tk)
            for i in watch:
                sts[i].feed(pos[i], tk[i])
            if k % 4 == 3:
                got = dec.logits(seqs)
                for i in watch:
                    worst = max(worst, rel_err(got[i], sts[i].logits()))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst <= TOL[mode], worst


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("model", ["small", "mid", "115m"])
def test_fast_persistent_decode(oracle, small_ckpt, mid_ckpt, big_ckpt, model, mode):
    """The one-sequence greedy loop of a fast mode as one persistent launch
    per call (every phase of every step in one cooperative kernel, phases
    exchanging epoch-tagged entries; in bf16 the weights past the first
    layer and the head read as bf16 pieces): each pick, teacher-forced into
    the oracle, is within the mode's tolerance of the oracle's maximum
    logit, and the logits after the call (the residual row it leaves)
    within it of the oracle's; the same with the captured graphs
    (ANA_PERSIST=0) for comparison. Then the persistent launch against the
    step kernels on its own picks: the same tokens fed one step at a time
    give logits within 1e-4 of the launch's (the same weights, the sums in
    another order). The 115M case runs past the first 128 positions, so the
    attention pieces of 128 slots each get live slots one after another."""
    print(f"case fast persistent decode {model} mode {mode}", flush=True)
    path = {"small": small_ckpt, "mid": mid_ckpt, "115m": big_ckpt}[model]
    oracle.set_threads(8)
    m = oracle.Model(path)
    steps = {"small": 70, "mid": 70, "115m": 150}[model]
    pr = [int(t) for t in ckpt.prompt(3, 9, m.vocab)]
    runs = {}
    for persist in ("1", "0"):
        os.environ["ANA_PERSIST"] = persist
        try:
            with ana_amd.Decoder(path, max_seqs=1, prefill_chunk=16, numerics=mode) as dec:
                dec.feeds(0, 0, pr[:-1])
                out = dec.generate([0], [len(pr) - 1], [pr[-1]], steps)[0]
                lg = dec.logits([0])[0]
        finally:
            os.environ.pop("ANA_PERSIST", None)
        runs[persist] = (out, lg)
        st = oracle.State(m)
        for p, t in enumerate(pr):
            st.feed(p, t)
        pos = len(pr)
        for k, t in enumerate(out):
            want = st.logits()
            scale = np.abs(want).max()
            assert want[t] >= want.max() - 2 * TOL[mode] * scale, (persist, k, int(t), int(want.argmax()))
            if k + 1 < len(out):
                st.feed(pos, int(t))
                pos += 1
        e = rel_err(lg, want)
        print(f"persist {persist}: final relative error {e:.3e}", flush=True)
        assert e <= TOL[mode], (persist, e)
    out, lg = runs["1"]
    with ana_amd.Decoder(path, max_seqs=1, prefill_chunk=16, numerics=mode) as dec:
        dec.feeds(0, 0, pr[:-1])
        for k, t in enumerate([pr[-1]] + [int(x) for x in out[:-1]]):
            dec.feed([0], [len(pr) - 1 + k], [t])
        e = rel_err(lg, dec.logits([0])[0])
    print(f"persistent launch against the step kernels: relative difference {e:.3e}", flush=True)
    assert e <= 1e-4, e


@pytest.mark.parametrize("model", ["small", "mid", "115m"])
def test_exact_persistent_decode(oracle, small_ckpt, mid_ckpt, big_ckpt, model):
    """The exact mode's one-sequence greedy loop as one persistent launch a
    call (the exact build of the persistent kernel: the norms, products, GLA
    and attention sums as in-order chains, the attention's softmax over the
    whole window in a phase of its own): every id and the logits after the
    call bit for bit equal to the oracle's greedy loop, and to the captured
    graphs' (ANA_PERSIST=0). The small and mid cases (ctx 64) run past the
    ring's wrap; the 115M case past the first 128 positions, so each
    attention piece gets live slots in turn."""
    print(f"case exact persistent decode {model}", flush=True)
    path = {"small": small_ckpt, "mid": mid_ckpt, "115m": big_ckpt}[model]
    oracle.set_threads(8)
    m = oracle.Model(path)
    steps = {"small": 70, "mid": 70, "115m": 150}[model]
    pr = [int(t) for t in ckpt.prompt(3, 9, m.vocab)]
    st = oracle.State(m)
    for p, t in enumerate(pr):
        st.feed(p, t)
    want, lg = [], None
    for k in range(steps):
        lg = st.logits()
        t = int(oracle.top(lg))
        want.append(t)
        if k + 1 < steps:
            st.feed(len(pr) + k, t)
    for persist in ("1", "0"):
        os.environ["ANA_PERSIST"] = persist
        try:
            with ana_amd.Decoder(path, max_seqs=1, prefill_chunk=16, numerics=ana_amd.EXACT_FP32) as dec:
                dec.feeds(0, 0, pr[:-1])
                out = [int(t) for t in dec.generate([0], [len(pr) - 1], [pr[-1]], steps)[0]]
                got = dec.logits([0])[0]
        finally:
            os.environ.pop("ANA_PERSIST", None)
        first = next((k for k, (a, b) in enumerate(zip(out, want)) if a != b), None)
        assert first is None, (persist, first, out[first], want[first])
        assert np.array_equal(got.view(np.uint32), lg.view(np.uint32)), (persist, float(np.abs(got - lg).max()))
        print(f"persist {persist}: {steps} ids and the final logits bit-exact", flush=True)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("model,n", [("v1", 40), ("v1", 5), ("v1", 3)])
def test_fast_fused_head_sampler(oracle, mid_ckpt, tmp_path, mode, model, n):
    """Sampled steps of ana_generate in a fast mode run the LM head fused with
    the sampler above four rows (vocab 32768: 128 head workgroups a 32-row
    block, 40 rows being two blocks, 5 one); at three rows the head and
    k_pick run apart. Every step's picks, and the RNG words at the end,
    equal S.pick's (the oracle's) on the logits of a twin decoder fed the
    same tokens, and the unfused sampler's (ana_pick on the twin); the event
    timing shows the fused form's one pick-kind launch a step (the step
    end), or two apart."""
    print(f"case fused head sampler {model} n {n} mode {mode}", flush=True)
    if model == "v1":
        c = cf.V1
        path = str(tmp_path / "v1f.ftc2")
        ckpt.write(path, c, ckpt.init_params(c, "normal", 5, trained=True))
    else:
        path, c = mid_ckpt, MID
    oracle.set_threads(8)
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9)))
    steps = 3
    seqs = list(range(n))
    r = np.random.default_rng(41)
    prompts = [r.integers(2, c.vocab, size=2 + b % 5).astype(np.uint32) for b in range(n)]
    rng0 = np.ascontiguousarray(np.stack([ana_amd.rng_seeded(100 + b) for b in range(n)]))
    with ana_amd.Decoder(path, max_seqs=n, numerics=mode) as dec, \
            ana_amd.Decoder(path, max_seqs=n, numerics=mode) as twin:
        for d_ in (dec, twin):
            d_.feeds_n(seqs, [0] * n, [p[:-1] for p in prompts])
        pos = np.array([len(p) - 1 for p in prompts], dtype=np.uint32)
        tok = np.array([int(p[-1]) for p in prompts], dtype=np.uint32)
        rng = rng0.copy()
        out = dec.generate(seqs, pos, tok, steps, st, rng)
        r_or = [oracle.rng_seeded(100 + b) for b in range(n)]
        r_tw = rng0.copy()
        t, p = tok.copy(), pos.copy()
        for k in range(steps):
            twin.feed(seqs, p, t)
            lg = twin.logits(seqs)
            tw = twin.pick(seqs, st, r_tw)
            for b in range(n):
                want = oracle.pick(lg[b], st.temperature, st.top_k, st.top_p, r_or[b])
                assert int(out[b, k]) == int(want), (k, b)
            assert np.array_equal(tw, out[:, k]), k
            t, p = out[:, k].copy(), p + 1
        for b in range(n):
            assert np.array_equal(rng[b], r_or[b]), b
        assert np.array_equal(rng, r_tw)
        # one more step with event timing: the sampler ran inside the head
        dec.prof(True)
        dec.generate(seqs, p, t, 1, st, rng)
        stats = dec.prof_read()
        dec.prof(False)
        assert stats["pick"][0] == (1 if n > 4 else 2), stats["pick"]
        assert stats["head"][0] == 1, stats["head"]

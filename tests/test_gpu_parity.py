"""libana on the GPU against the CPU oracle, bit for bit (ANA_EXACT_FP32).

The cases are the reference's own (bend/tests/decode-dense.bend,
bend/tests/prefill-dense.bend): small4_v3 and its no-arms twin, 96 tokens of
the LCG window on ctx 64 (the ring wraps), the six chunked-prefill runs;
plus batches of sequences at staggered positions, the on-device token loop,
the sampler on the model's own logits, and the 115M shape.
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
# v3-trained: small4_v3 with the vectors a trained checkpoint carries (norm
# gains 1 + N(0, 0.1^2), qk-norm gains N(0, 0.1^2), a sink logit per head
# N(0, 1)), so gain offsets, the (1 + g) factor and per-head sinks are live
CFGS = {"v3-arms": cf.SMALL4_V3, "no-arms": cf.SMALL4_NOARMS, "v3-trained": cf.SMALL4_V3}
TRAINED = {"v3-trained"}


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ckpts(tmp_path_factory):
    d = tmp_path_factory.mktemp("ck")
    out = {}
    for name, c in CFGS.items():
        p = str(d / f"{name}.ftc2")
        ckpt.write(p, c, ckpt.init_params(c, "hash", 1, trained=name in TRAINED))
        out[name] = p
    return out


@pytest.mark.parametrize("name", list(CFGS))
def test_feed_bit_exact(oracle, ckpts, name):
    path = ckpts[name]
    print(f"case feed {name}", flush=True)
    m = oracle.Model(path)
    st = oracle.State(m)
    with ana_amd.Decoder(path) as dec:
        for pos, t in enumerate(VEC["window"]):
            dec.feed([0], [pos], [t])
            st.feed(pos, t)
            want = st.logits()
            got = dec.logits([0])[0]
            assert np.array_equal(bits(got), bits(want)), (pos, np.abs(got - want).max())
            assert dec.top([0])[0] == oracle.top(want)
        for l in range(m.layers):
            assert np.array_equal(bits(dec.state(0, l)), bits(st.layer(l))), l
        assert np.array_equal(bits(dec.state(0, m.layers)), bits(st.x()))
        # a reset then the same tokens: the same bits (decode-dense's law)
        dec.reset(0)
        for pos, t in enumerate(VEC["window"][:70]):
            dec.feed([0], [pos], [t])
        st.reset()
        for pos, t in enumerate(VEC["window"][:70]):
            st.feed(pos, t)
        assert np.array_equal(bits(dec.logits([0])[0]), bits(st.logits()))


@pytest.mark.parametrize("name", list(CFGS))
def test_chunked_prefill_is_feed(oracle, ckpts, name):
    """bend/tests/prefill-dense.bend's six runs at chunk 16: states, logits
    and the greedy pick bit for bit equal to feeding one token at a time."""
    path = ckpts[name]
    m = oracle.Model(path)
    ts = VEC["window"]
    with ana_amd.Decoder(path, prefill_chunk=VEC["prefill_chunk"]) as dec:
        for run in VEC["prefill_runs"]:
            print(f"case prefill {name} {run['name']}", flush=True)
            xs, pre = ts[: run["n"]], run["pre"]
            st = oracle.State(m)
            for pos, t in enumerate(xs):
                st.feed(pos, t)
            dec.reset(0)
            for pos in range(pre):
                dec.feed([0], [pos], [xs[pos]])
            dec.feeds(0, pre, xs[pre:])
            for l in range(m.layers + 1):
                want = st.layer(l) if l < m.layers else st.x()
                assert np.array_equal(bits(dec.state(0, l)), bits(want)), (run["name"], l)
            lg = st.logits()
            assert np.array_equal(bits(dec.logits([0])[0]), bits(lg))
            assert dec.top([0])[0] == oracle.top(lg)


@pytest.mark.parametrize("name", list(CFGS))
def test_batched_sequences(oracle, ckpts, name):
    """Four sequences at staggered positions fed together: each one's bits
    are its own single-sequence run's."""
    path = ckpts[name]
    print(f"case batch {name}", flush=True)
    m = oracle.Model(path)
    rng = np.random.default_rng(11)
    n, steps = 4, 80
    streams = rng.integers(0, m.vocab, size=(n, steps + 40)).astype(np.uint32)
    starts = [0, 3, 17, 40]
    sts = [oracle.State(m) for _ in range(n)]
    with ana_amd.Decoder(path, max_seqs=6) as dec:
        seqs = [5, 0, 2, 3]
        for i, s in enumerate(seqs):
            dec.feeds(s, 0, streams[i, : starts[i]])
            for p in range(starts[i]):
                sts[i].feed(p, int(streams[i, p]))
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tok = [int(streams[i, pos[i]]) for i in range(n)]
            dec.feed(seqs, pos, tok)
            for i in range(n):
                sts[i].feed(pos[i], tok[i])
        got = dec.logits(seqs)
        for i in range(n):
            assert np.array_equal(bits(got[i]), bits(sts[i].logits())), i
        tops = dec.top(seqs)
        for i in range(n):
            assert tops[i] == oracle.top(got[i])


@pytest.mark.parametrize("name", list(CFGS))
def test_batched_sequences_wide(oracle, ckpts, name):
    """Nine sequences at staggered positions, 70 steps across the ring's
    wrap (attention on one workgroup per head and row from eight rows on):
    each one's bits are its own single-sequence run's, at four steps."""
    path = ckpts[name]
    print(f"case wide batch {name}", flush=True)
    m = oracle.Model(path)
    rng = np.random.default_rng(23)
    n, steps = 9, 70
    streams = rng.integers(0, m.vocab, size=(n, steps + 40)).astype(np.uint32)
    starts = [0, 3, 17, 40, 5, 1, 29, 11, 8]
    seqs = [8, 0, 2, 3, 7, 5, 1, 6, 4]
    sts = [oracle.State(m) for _ in range(n)]
    with ana_amd.Decoder(path, max_seqs=9) as dec:
        for i, s in enumerate(seqs):
            dec.feeds(s, 0, streams[i, : starts[i]])
            for p in range(starts[i]):
                sts[i].feed(p, int(streams[i, p]))
        for k in range(steps):
            pos = [starts[i] + k for i in range(n)]
            tok = [int(streams[i, pos[i]]) for i in range(n)]
            dec.feed(seqs, pos, tok)
            for i in range(n):
                sts[i].feed(pos[i], tok[i])
            if k in (0, 23, 47, steps - 1):
                got = dec.logits(seqs)
                for i in range(n):
                    assert np.array_equal(bits(got[i]), bits(sts[i].logits())), (k, i)
        for i in range(n):
            for l in range(m.layers):
                assert np.array_equal(bits(dec.state(seqs[i], l)), bits(sts[i].layer(l))), (i, l)


@pytest.mark.parametrize("name", list(CFGS))
def test_token_loop_greedy(oracle, ckpts, name):
    """ana_generate's on-device loop = the host loop of Generate.bend on the
    oracle (feed, head, greedy pick on the store, feed the pick)."""
    path = ckpts[name]
    print(f"case generate {name}", flush=True)
    m = oracle.Model(path)
    prompts = [VEC["window"][:9], VEC["window"][20:33], VEC["window"][40:45]]
    steps = 70
    with ana_amd.Decoder(path, max_seqs=3, prefill_chunk=16) as dec:
        first, pos0 = [], []
        for i, pr in enumerate(prompts):
            dec.feeds(i, 0, pr[:-1])
            first.append(pr[-1])
            pos0.append(len(pr) - 1)
        out = dec.generate([0, 1, 2], pos0, first, steps)
    for i, pr in enumerate(prompts):
        st = oracle.State(m)
        for p, t in enumerate(pr):
            st.feed(p, t)
        want = []
        pos = len(pr)
        for _ in range(steps):
            lg = st.logits()
            t = oracle.top(lg)
            if t == m.vocab:
                t = oracle.tree_argmax(lg)
            want.append(t)
            st.feed(pos, t)
            pos += 1
        assert list(out[i]) == want, i


# (the device's top-k finishes its bisection in one wave once 1024 or fewer
# logits lie in the interval, and its top-p takes one wave after a top-k
# that kept 64 or fewer: 64 and 200 sit either side of that, 1000 keeps the
# whole-row steps going longer)
SETTINGS = [(0.8, 40, 0.9), (1.0, 0xFFFFFFFF, 0.95), (0.5, 5, 1.0), (0.8, 0xFFFFFFFF, 1.0),
            (1.5, 3, 0.5), (0.0, 40, 0.9), (0.7, 64, 0.95), (0.9, 200, 0.8), (1.2, 1000, 0.7)]


def _check_pick(oracle, dec, seqs, lgs):
    for temp, k, p in SETTINGS:
        st = ana_amd.Settings(float(np.float32(temp)), k, float(np.float32(p)))
        rng = np.stack([oracle.rng_seeded(100 + s) for s in seqs])
        want_rng = rng.copy()
        want = [oracle.pick(lgs[i], st.temperature, k, st.top_p, want_rng[i]) for i in range(len(seqs))]
        got = dec.pick(seqs, st, rng)
        assert list(got) == want, (temp, k, p)
        assert np.array_equal(rng, want_rng), (temp, k, p)


def test_sampler_small_vocab(oracle, ckpts):
    path = ckpts["v3-trained"]
    print("case pick v258", flush=True)
    with ana_amd.Decoder(path, max_seqs=4) as dec:
        for s in range(4):
            dec.feeds(s, 0, VEC["window"][s * 7: s * 7 + 12])
        seqs = [0, 1, 2, 3]
        _check_pick(oracle, dec, seqs, dec.logits(seqs))


def test_sampler_32k_vocab(oracle, tmp_path):
    """The v1 config (vocab 32768: a perfect depth-15 tree)."""
    c = cf.V1
    path = str(tmp_path / "v1.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "normal", 0, trained=True))
    print("case pick v32768", flush=True)
    oracle.set_threads(8)
    with ana_amd.Decoder(path, max_seqs=3) as dec:
        pr = ckpt.prompt(0, 16, c.vocab)
        for s in range(3):
            dec.feeds(s, 0, pr[s:])
        lgs = dec.logits([0, 1, 2])
        _check_pick(oracle, dec, [0, 1, 2], lgs)
        # the model's logits are the oracle's too
        m = oracle.Model(path)
        st = oracle.State(m)
        st.feeds(0, [int(t) for t in pr[1:]])
        assert np.array_equal(bits(lgs[1]), bits(st.logits()))


def test_115m_batch8(oracle, tmp_path):
    """fp100m, eight sequences decoded together from staggered positions:
    the GLA step on one wave per (head, sequence) and the one-workgroup
    attention at hd 64, bit for bit against each sequence's oracle run."""
    c = cf.FP100M
    path = str(tmp_path / "fp100m8.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "normal", 2, trained=True))
    print("case 115m batch8", flush=True)
    oracle.set_threads(8)
    m = oracle.Model(path)
    n, steps = 8, 3
    pre = [1, 4, 2, 6, 3, 5, 2, 7]
    prompts = [[int(t) for t in ckpt.prompt(30 + i, pre[i] + steps, c.vocab)] for i in range(n)]
    sts = [oracle.State(m) for _ in range(n)]
    with ana_amd.Decoder(path, max_seqs=n) as dec:
        for i in range(n):
            for p in range(pre[i]):
                dec.feed([i], [p], [prompts[i][p]])
                sts[i].feed(p, prompts[i][p])
        for k in range(steps):
            pos = [pre[i] + k for i in range(n)]
            tok = [prompts[i][pos[i]] for i in range(n)]
            dec.feed(list(range(n)), pos, tok)
            for i in range(n):
                sts[i].feed(pos[i], tok[i])
        got = dec.logits(list(range(n)))
    for i in range(n):
        want = sts[i].logits()
        assert np.array_equal(bits(got[i]), bits(want)), (i, np.abs(got[i] - want).max())


def test_115m_shape(oracle, tmp_path):
    """fp100m's dimensions (d 768, f 2048, 12 layers, 12 heads, vocab 32768,
    all arms) at ctx 2048: a prompt through feeds, then steps, bit for bit."""
    c = cf.FP100M
    path = str(tmp_path / "fp100m.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "normal", 0, trained=True))
    print("case 115m", flush=True)
    oracle.set_threads(8)
    m = oracle.Model(path)
    st = oracle.State(m)
    pr = [int(t) for t in ckpt.prompt(1, 12, c.vocab)]
    with ana_amd.Decoder(path, max_seqs=2) as dec:
        dec.feeds(1, 0, pr[:10])
        for p in range(10):
            st.feed(p, pr[p])
        for p in (10, 11):
            dec.feed([1], [p], [pr[p]])
            st.feed(p, pr[p])
            lg = st.logits()
            got = dec.logits([1])[0]
            assert np.array_equal(bits(got), bits(lg)), (p, np.abs(got - lg).max())
        out = dec.generate([1], [12], [int(oracle.top(lg))], 3)
    want = []
    pos, t = 12, int(oracle.top(lg))
    for _ in range(3):
        st.feed(pos, t)
        t = oracle.top(st.logits())
        want.append(t)
        pos += 1
    assert list(out[0]) == want


@pytest.mark.parametrize("name", list(CFGS))
def test_feeds_n_is_feeds(oracle, ckpts, name):
    """ana_feeds_n: five sequences of ragged lengths (one across the ring
    wrap, one starting mid-sequence) prefilled together at chunk 16 leave
    each sequence's states and logits bit for bit as the oracle fed one
    token at a time."""
    path = ckpts[name]
    print(f"case feeds_n {name}", flush=True)
    m = oracle.Model(path)
    seqs, pos, lens = [4, 0, 2, 5, 1], [0, 0, 3, 0, 60], [40, 3, 17, 70, 9]
    rng = np.random.default_rng(21)
    toks = [rng.integers(0, m.vocab, size=n).astype(np.uint32) for n in lens]
    pre = [rng.integers(0, m.vocab, size=p).astype(np.uint32) for p in pos]
    with ana_amd.Decoder(path, max_seqs=6, prefill_chunk=16) as dec:
        for s, p, pr in zip(seqs, pos, pre):
            if p:
                dec.feeds(s, 0, pr)
        dec.feeds_n(seqs, pos, toks)
        got = dec.logits(seqs)
        for i, s in enumerate(seqs):
            st = oracle.State(m)
            for p, t in enumerate(pre[i]):
                st.feed(p, int(t))
            for k, t in enumerate(toks[i]):
                st.feed(pos[i] + k, int(t))
            assert np.array_equal(bits(got[i]), bits(st.logits())), (i, s)
            for l in range(m.layers):
                assert np.array_equal(bits(dec.state(s, l)), bits(st.layer(l))), (i, l)


@pytest.mark.parametrize("name", list(CFGS))
def test_score_n_bit_exact(oracle, ckpts, name):
    """ana_score_n (Evaluate.bend's window.go): four windows of ragged
    length (one past the ring's wrap, one from a later position) scored
    together at chunk 16; every summand is, bit for bit, the oracle's
    G.lse - logit[next] after feeding the window token by token."""
    path = ckpts[name]
    print(f"case score_n {name}", flush=True)
    m = oracle.Model(path)
    seqs, pos, lens = [2, 0, 3, 1], [0, 0, 5, 0], [41, 2, 30, 80]
    rng = np.random.default_rng(41)
    toks = [rng.integers(0, m.vocab, size=n).astype(np.uint32) for n in lens]
    pre = [rng.integers(0, m.vocab, size=p).astype(np.uint32) for p in pos]
    with ana_amd.Decoder(path, max_seqs=4, prefill_chunk=16) as dec:
        for s, p, pr in zip(seqs, pos, pre):
            if p:
                dec.feeds(s, 0, pr)
        got = dec.score_n(seqs, pos, toks)
    for i in range(len(seqs)):
        assert got[i].size == lens[i] - 1
        st = oracle.State(m)
        for p, t in enumerate(pre[i]):
            st.feed(p, int(t))
        want = []
        for k in range(lens[i] - 1):
            st.feed(pos[i] + k, int(toks[i][k]))
            want.append(oracle.ce(st.logits(), int(toks[i][k + 1])))
        assert np.array_equal(bits(got[i]), bits(np.array(want, np.float32))), i
    # window.mean over the summands: F32 in order, over their count
    w = ana_amd.window_mean(got[3])
    acc = np.float32(0.0)
    for v in got[3]:
        acc = np.float32(acc + v)
    assert w == np.float32(acc / np.float32(got[3].size))


@pytest.mark.parametrize("name", list(CFGS))
def test_score_n_tree_engine(oracle, ckpts, name):
    """ana_score_n against the engine Evaluate.bend really scores with:
    window.go calls Md.decode, the tree meaning (bend/Evaluate.bend:33-42),
    while ana_score_n is bit-exact with the dense engine. One window of 90
    tokens (past the ring's wrap at ctx 64) scored on the device, against
    G.lse - logit[next] on the oracle's tree step (or_tree_step) at every
    position. The dense and tree logits agree within 1e-5 of the largest
    |logit| (decode-dense.bend's law), and a summand moves by at most twice
    that (lse and logit[next] each by at most the logits' difference), so
    each summand is held within 2e-5 of that position's largest |logit|,
    and the window means within the largest of those bounds."""
    path = ckpts[name]
    print(f"case score_n tree engine {name}", flush=True)
    m = oracle.Model(path)
    toks = np.array(VEC["window"][:90], np.uint32)
    with ana_amd.Decoder(path, max_seqs=1, prefill_chunk=16) as dec:
        got = dec.score_n([0], [0], [toks])[0]
    tr = oracle.Tree(m)
    worst, bounds, want = 0.0, [], []
    for k in range(toks.size - 1):
        lg = tr.step(k, int(toks[k]))
        want.append(oracle.ce(lg, int(toks[k + 1])))
        bound = 2e-5 * float(np.abs(lg).max())
        bounds.append(bound)
        d = abs(float(got[k]) - want[-1])
        worst = max(worst, d / bound)
        assert d <= bound, (k, float(got[k]), want[-1], bound)
    print(f"worst summand difference {worst:.3f} of its bound", flush=True)
    # window.mean on each engine's summands (F32 in order, over the count)
    d = abs(float(ana_amd.window_mean(got)) - float(ana_amd.window_mean(np.array(want, np.float32))))
    assert d <= max(bounds), (d, max(bounds))


def test_text_end_to_end(oracle, tmp_path):
    """Text in, text out: a checkpoint naming its tokenizer by identity
    (a synthetic artifact of 42 merges; model vocab 300); the manifest read,
    the tokenizer found by that identity (dc.tok.of), BOS plus the encoded
    prompt fed, 12 greedy ids from the device loop, bit for bit the oracle's
    greedy ids, decoded back to bytes."""
    print("case text end to end", flush=True)
    text = b"The history of the city of Paris"
    # merges: the prompt's most frequent adjacent byte pairs, then pairs of those
    xs = [b + 2 for b in text]
    rows, nxt = [], 258
    while nxt < 300:
        cnt = {}
        for i in range(len(xs) - 1):
            cnt[(xs[i], xs[i + 1])] = cnt.get((xs[i], xs[i + 1]), 0) + 1
        if not cnt:
            break
        pair = max(sorted(cnt), key=lambda p: cnt[p])
        rows.append((pair[0], pair[1], nxt))
        ys, i = [], 0
        while i < len(xs):
            if i + 1 < len(xs) and (xs[i], xs[i + 1]) == pair:
                ys.append(nxt); i += 2
            else:
                ys.append(xs[i]); i += 1
        xs, nxt = ys, nxt + 1
    while nxt < 300:   # pad with pairs of bytes the prompt lacks
        rows.append((200 + nxt - 258, 201, nxt)); nxt += 1
    art = tmp_path / "t.bpe"
    art.write_text("BPE 300 v2\n" + "".join(f"{a} {b} {n}\n" for a, b, n in rows))
    tok = ana_amd.Tokenizer(str(art))
    c = cf.Config(300, 64, 64, 192, 4, 4, True, True, True)
    path = str(tmp_path / "m.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "normal", 3, trained=True), tokenizer_id=tok.identity())
    man = ana_amd.read_manifest(path)
    t = ana_amd.find_tokenizer(man["tokenizer_id"], candidates=[str(art)])
    prompt = [ana_amd.Tokenizer.BOS] + [int(i) for i in t.encode(text)]
    assert t.decode(prompt) == text and len(prompt) < len(text)
    with ana_amd.Decoder(path, max_seqs=1, prefill_chunk=8) as dec:
        dec.feeds(0, 0, prompt[:-1])
        got = dec.generate([0], [len(prompt) - 1], [prompt[-1]], 12)[0]
    m = oracle.Model(path)
    st = oracle.State(m)
    for p, i in enumerate(prompt):
        st.feed(p, i)
    want, pos = [], len(prompt)
    nxt_id = oracle.top(st.logits())
    for _ in range(12):
        want.append(nxt_id)
        st.feed(pos, nxt_id)
        pos += 1
        nxt_id = oracle.top(st.logits())
    assert [int(x) for x in got] == want
    out = t.decode(got)
    assert isinstance(out, bytes)


@pytest.mark.parametrize("sampled", [False, True], ids=["greedy", "v3"])
@pytest.mark.parametrize("mode", [ana_amd.EXACT_FP32, ana_amd.FAST_FP32], ids=["exact", "fast_fp32"])
def test_generate_calls_of_any_length(ckpts, sampled, mode):
    """ana_generate replays its captured steps across calls of other step
    counts (the picks are step-major on the device, each row's step count
    its own): calls of 5, 9, 1 and 11 steps, each from where the last
    stopped with the RNG state handed back, give the tokens of one 26-step
    call on a twin decoder, bit for bit, greedy and sampled; so do 7 and 6
    rows (a capture per row count), and one row (in fast_fp32 the persistent
    one-sequence loop, whose state and exchange epochs carry across calls)."""
    print(f"case generate calls of any length mode {mode} sampled {sampled}", flush=True)
    path = ckpts["v3-trained"]
    lens = [5, 9, 1, 11]
    total = sum(lens)
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9))) if sampled else None
    for n in (7, 6, 1):
        seqs = list(range(n))
        rng0 = np.stack([ana_amd.rng_seeded(50 + s) for s in seqs]).astype(np.uint64) if sampled else None
        prompts = [VEC["window"][3 * i: 3 * i + 4 + i] for i in seqs]
        outs = []
        for split in (True, False):
            with ana_amd.Decoder(path, max_seqs=n, prefill_chunk=4, numerics=mode) as dec:
                for i, pr in enumerate(prompts):
                    dec.feeds(i, 0, pr[:-1])
                pos = np.array([len(pr) - 1 for pr in prompts], dtype=np.uint32)
                tok = np.array([pr[-1] for pr in prompts], dtype=np.uint32)
                rng = np.ascontiguousarray(rng0.copy()) if sampled else None
                got = []
                for k in (lens if split else [total]):
                    o = dec.generate(seqs, pos, tok, k, st, rng)
                    got.append(o)
                    tok, pos = o[:, -1].copy(), pos + k
                outs.append((np.concatenate(got, axis=1), None if rng is None else rng.copy()))
        assert np.array_equal(outs[0][0], outs[1][0]), n
        if sampled:
            assert np.array_equal(outs[0][1], outs[1][1]), n


NAN_MID = cf.Config(vocab=258, ctx=64, d=256, f=1024, layers=4, heads=4, rglru=True, qk=True, sinks=True, tied=True)


@pytest.mark.parametrize("n", [1, 6])
@pytest.mark.parametrize("mode", [ana_amd.EXACT_FP32, ana_amd.FAST_FP32, ana_amd.BF16],
                         ids=["exact", "fast_fp32", "bf16"])
def test_nan_logits_fall_back(oracle, tmp_path, mode, n):
    """dd.top's NaN answer and Decode.bend's fallback (bend/Dense/Decode.bend:
    475-484, bend/Decode.bend:407-418): one final norm gain is NaN, so every
    logit is NaN. ana_top answers vocab for every sequence, and each pick of
    the on-device loop is Sample.argmax over the NaN logits, as the oracle's
    host loop falls back to it (1 and 6 sequences: the small-batch head's
    argmax keys, and above four rows the wide head's keys or dd.top's pass
    over the stored logits)."""
    print(f"case nan fallback mode {mode} n {n}", flush=True)
    c = NAN_MID
    p = ckpt.init_params(c, "normal", 9, trained=True)
    _, fin = cf.layout(c)
    p[fin + 5] = np.nan
    path = str(tmp_path / "nan.ftc2")
    ckpt.write(path, c, p)
    m = oracle.Model(path)
    seqs = list(range(n))
    prompts = [[2 + 7 * i + k for k in range(3 + i)] for i in seqs]
    with ana_amd.Decoder(path, max_seqs=n, numerics=mode) as dec:
        dec.feeds_n(seqs, [0] * n, prompts)
        lg = dec.logits(seqs)
        assert np.isnan(lg).all()
        assert list(dec.top(seqs)) == [c.vocab] * n
        out = dec.generate(seqs, [len(pr) for pr in prompts], [1] * n, 3)
    for i in seqs:
        st = oracle.State(m)
        for q, t in enumerate(prompts[i] + [1]):
            st.feed(q, t)
        want, pos = [], len(prompts[i]) + 1
        for _ in range(3):
            w = st.logits()
            assert oracle.top(w) == c.vocab
            t = oracle.tree_argmax(w)
            want.append(t)
            st.feed(pos, t)
            pos += 1
        assert [int(x) for x in out[i]] == want, i


@pytest.mark.parametrize("mode", [ana_amd.EXACT_FP32, ana_amd.FAST_FP32, ana_amd.BF16], ids=["exact", "fast_fp32", "bf16"])
def test_stats_prob_and_rival(oracle, tmp_path, mode):
    """ana_stats (dc.prob.of and al.stat) after feeds, against the oracle's
    or_stat on its own logits: bit for bit in exact mode (with trained-like
    vectors at v = 32768 too), within the mode's tolerance in the fast ones
    (the rival then must be within tolerance of the best other logit)."""
    for name, c, trained in (("small", cf.SMALL4_V3, False), ("115m", cf.BPE100M_V3, True)):
        path = str(tmp_path / f"{name}.ftc2")
        ckpt.write(path, c, ckpt.init_params(c, "normal", 3, trained=trained))
        m = oracle.Model(path)
        rng = np.random.default_rng(5)
        n = 3
        prompts = [[0] + [int(x) for x in rng.integers(2, c.vocab, size=6 + 2 * b)] for b in range(n)]
        print(f"case stats {name} mode {mode}", flush=True)
        with ana_amd.Decoder(path, max_seqs=n, numerics=mode) as dec:
            dec.feeds_n(list(range(n)), [0] * n, prompts)
            want = []
            toks = []
            for b in range(n):
                st = oracle.State(m)
                for p_, t in enumerate(prompts[b]):
                    st.feed(p_, t)
                lg = st.logits()
                # the token: the best, a mid-ranked one, a random one
                x = [int(np.argmax(lg)), int(np.argsort(lg)[c.vocab // 2]), int(rng.integers(0, c.vocab))][b]
                toks.append(x)
                want.append((oracle.stat(lg, x), lg))
            p, a, pa = dec.stats(list(range(n)), toks)
        for b in range(n):
            (wp, wa, wpa), lg = want[b]
            if mode == ana_amd.EXACT_FP32:
                assert (p[b], int(a[b]), pa[b]) == (wp, wa, wpa), (name, b)
            else:
                tol = 1e-4 if mode == ana_amd.FAST_FP32 else 2e-2
                scale = float(np.abs(lg).max())
                # probabilities move by at most e^(2 tol scale) - 1 relative
                bound = np.expm1(2.5 * tol * scale)
                assert abs(float(p[b]) - float(wp)) <= bound * float(wp) + 1e-30, (name, b, p[b], wp)
                other = lg.copy()
                other[toks[b]] = -3e38
                assert lg[int(a[b])] >= other.max() - 2 * tol * scale and int(a[b]) != toks[b], (name, b)

"""ana_amd.agent's batching on a stand-in decoder (no GPU): every episode's
tokens, flags and ending are those of the one-episode restatement of
bend/Agent/Loop.bend (agent_loop_ref) on a stand-in engine with the same
rule for picks: positions, given tokens, RNG words, budgets and calls."""
import numpy as np
import pytest

from ana_amd import agent


class FakeDecoder:
    """Feeds must land at the next position of their slot; a drawn token is
    a function of the slot's fed tokens and its RNG words, which it
    advances (forced tokens leave them)."""

    def __init__(self, max_seqs, vocab=97):
        self.max_seqs, self.vocab = max_seqs, vocab
        self.hist = {}
        self.calls = []

    def reset(self, s):
        self.hist[s] = []

    def _put(self, s, p, toks):
        assert p == len(self.hist[s]), (s, p, len(self.hist[s]))
        self.hist[s] += [int(t) for t in toks]

    def feeds_n(self, seqs, pos, toks):
        self.calls.append(("feeds_n", len(seqs)))
        for s, p, t in zip(seqs, pos, toks):
            self._put(s, p, t)

    def feed(self, seqs, pos, toks):
        for s, p, t in zip(seqs, pos, toks):
            self._put(s, p, [t])

    def feeds(self, seq, pos, toks):
        self._put(seq, pos, toks)

    def stats(self, seqs, toks):
        """a stand-in al.stat: a function of the slot's fed tokens"""
        out = [fake_stat(self.hist[s], int(x), self.vocab) for s, x in zip(seqs, toks)]
        return (np.array([o[0] for o in out], np.float32), np.array([o[1] for o in out], np.uint32),
                np.array([o[2] for o in out], np.float32))

    def generate(self, seqs, pos, toks, steps, st, rng):
        assert steps == 1 and rng.shape == (len(seqs), 4) and rng.dtype == np.uint64
        self.calls.append(("generate", len(seqs)))
        out = np.zeros((len(seqs), 1), dtype=np.uint32)
        for k, (s, p, t) in enumerate(zip(seqs, pos, toks)):
            self._put(s, p, [t])
            h = (sum((i + 1) * x for i, x in enumerate(self.hist[s])) + int(rng[k, 0] % 1000003)) % self.vocab
            rng[k, 0] += np.uint64(7919)
            rng[k, 3] ^= np.uint64(h + 1)
            out[k, 0] = h
        return out


def fake_stat(hist, x, vocab=97):
    h = sum((i + 1) * t for i, t in enumerate(hist)) + 13 * x
    a = (h * 7 + 3) % vocab
    a = a if a != x else (a + 1) % vocab
    return np.float32((h % 89 + 1) / 100.0), a, np.float32(((h // 3) % 53 + 1) / 120.0)


def is_call(i, toks):
    return toks[-1] % 9 == 4


def tool(i, toks):
    if toks[-1] >= 60:
        return None
    return [2 + (toks[-1] * 3 + j + i) % 90 for j in range(1 + (i + len(toks)) % 4)]


EPS = [agent.Episode([0, 5, 9, 12], seed=3, budget=30, calls=3),
       agent.Episode([0], seed=11, budget=12, calls=1, first=[40, 41]),
       agent.Episode([0, 7, 7, 7, 7, 7, 2], seed=5, budget=25, calls=0),
       agent.Episode([0, 88, 3], seed=8, budget=40, calls=5, first=[17]),
       agent.Episode([0, 1 + 1, 60], seed=0, budget=5, calls=2),
       agent.Episode([0, 3], seed=2, budget=40, calls=2)]


def fake_engine(vocab=97, seed_rng=None):
    """One episode's stand-in engine: FakeDecoder's rule for one slot."""
    hist, rng = [], seed_rng.copy()

    def feed(t):
        hist.append(int(t))

    def pick():
        h = (sum((i + 1) * x for i, x in enumerate(hist)) + int(rng[0] % 1000003)) % vocab
        rng[0] += np.uint64(7919)
        rng[3] ^= np.uint64(h + 1)
        return h
    return feed, pick, hist


def test_batched_matches_loop():
    from ana_amd import rng_seeded
    from agent_loop_ref import episode
    for ct in (None, 11):
        dec = FakeDecoder(len(EPS))
        together = agent.run(dec, EPS, None, is_call, tool, call_token=ct)
        for i, e in enumerate(EPS):
            feed, pick, hist = fake_engine(seed_rng=rng_seeded(e.seed).astype(np.uint64))
            want = episode(feed, pick, e, lambda t, i=i: is_call(i, t), lambda t, i=i: tool(i, t), call_token=ct)
            assert together[i] == want, (ct, i)
            # the slot saw exactly the restatement's feeds (the last pick's
            # token is fed only when drawn)
            assert dec.hist[i] == hist, (ct, i)
        if ct is not None:
            # the call-ending picks (4 mod 9, never 11) were written as the
            # call's token: no written token ends a call, and some calls
            # were made
            assert not any(is_call(0, [t]) for o in together for t in o.tokens)
            assert sum(o.tokens.count(ct) for o in together) >= 3


def test_call_token_written_and_fed():
    """al.called: the pick that ends a call line is written as the newline
    and the newline token is fed in its place, so the tool and the engine
    both see call_token, never the pick."""
    seen = []

    def tool1(i, toks):
        seen.append(list(toks))
        return [5, 6] if len(seen) == 1 else None

    ep = agent.Episode([0, 3], seed=0, budget=40, calls=2)
    dec = FakeDecoder(1)
    out = agent.run(dec, [ep], None, is_call, tool1, call_token=11)[0]
    assert seen and all(s[-1] == 11 for s in seen)
    k = len(seen[0])
    assert out.tokens[k - 1] == 11
    # fed: the prompt, then the written tokens up to the call, with 11 at the
    # call's place, then the echo
    assert dec.hist[0][:len(ep.prompt) + k + 2] == list(ep.prompt) + out.tokens[:k] + [5, 6]


def test_endings_and_flags():
    out = agent.run(FakeDecoder(len(EPS)), EPS, None, is_call, tool)
    for e, o in zip(EPS, out):
        assert o.why in ("eos", "budget", "calls", "tool")
        assert len(o.tokens) == len(o.drawn)
        assert agent.EOS not in o.tokens
        # the given tokens lead, up to a call among them (al.resume drops
        # the rest), and are not drawn
        g = 0
        while g < len(o.tokens) and not o.drawn[g]:
            g += 1
        assert o.tokens[:g] == list(e.first)[:g] and (g == len(e.first) or is_call(0, [o.tokens[g - 1]]))
        # a stretch writes at most its budget of picks (given ones count)
        run_ = 0
        for t, d in zip(o.tokens, o.drawn):
            run_ += 1
            assert run_ <= e.budget
            if is_call(0, [t]):
                run_ = 0
    assert out[2].why in ("eos", "budget", "calls")
    # the scenario reaches every ending
    assert {o.why for o in out} == {"eos", "budget", "calls", "tool"}


def test_slots_and_errors():
    dec = FakeDecoder(8)
    a = agent.run(dec, EPS[:2], None, is_call, tool, slots=[6, 3])
    b = agent.run(FakeDecoder(2), EPS[:2], None, is_call, tool)
    assert a == b
    with pytest.raises(ValueError):
        agent.run(dec, EPS[:2], None, is_call, tool, slots=[1, 1])
    with pytest.raises(ValueError):
        agent.run(dec, [agent.Episode([0], 1, 4, first=[1])], None, is_call, tool)


def test_cut_by_hand():
    """al.cut.last / al.cut.step (Loop.bend:297-310) on hand cases: a
    one-token failed term is always left at its only token; at a step where
    the rival's b exceeds p (1 - q) (q the rest's probability) the term is
    left there, else kept."""
    f32 = np.float32
    q, d, a, b = agent.cut_of([(0.9, 5, 0.05)])
    assert (d, a) == (0, 5) and q == f32(0.9)
    # step 0: b0 = 0.5 > p0 (1 - p1) = 0.6 * 0.2 = 0.12: left at step 0
    q, d, a, b = agent.cut_of([(0.6, 11, 0.5), (0.8, 12, 0.1)])
    assert (d, a) == (0, 11) and q == f32(f32(0.6) * f32(0.8)) and b == f32(0.5)
    # step 0: b0 = 0.1 < 0.9 (1 - 0.3) = 0.63: kept, left at step 1's rival
    q, d, a, b = agent.cut_of([(0.9, 11, 0.1), (0.3, 12, 0.2)])
    assert (d, a, b) == (1, 12, f32(0.2))
    # three steps, left at the middle one: q folds every step's p
    q, d, a, b = agent.cut_of([(0.95, 1, 0.01), (0.4, 2, 0.55), (0.99, 3, 0.005)])
    assert (d, a) == (1, 2) and q == f32(f32(0.95) * f32(f32(0.4) * f32(0.99)))


def test_product_and_retry_match_the_loop():
    """agent.run with failed checks (Retry) and term starts, on the stand-in
    decoder, against the restatement: al.product's pass along the failed
    term, the replay and the given tokens, and the retry settings' draws."""
    from ana_amd import rng_seeded
    from agent_loop_ref import episode, product_ref

    def tool_r(i, toks):
        if toks[-1] >= 70:
            return None
        echo = [2 + (toks[-1] * 5 + j + i) % 80 for j in range(1 + (i + len(toks)) % 3)]
        return agent.Retry(echo, toks[-4:]) if (i + len(toks)) % 3 else echo

    def term_start(i, toks):
        return toks[-1] % 3 == 1

    dec = FakeDecoder(len(EPS))
    together = agent.run(dec, EPS, None, is_call, tool_r, term_start=term_start)
    n_products = 0
    for i, e in enumerate(EPS):
        feed, pick, hist = fake_engine(seed_rng=rng_seeded(e.seed).astype(np.uint64))

        def feed_at(pos, t, hist=hist):
            assert pos == len(hist)
            hist.append(int(t))

        def replay(fed, hist=hist):
            hist[:] = [int(t) for t in fed]

        def product(fed, term, hist=hist, feed_at=feed_at, replay=replay):
            nonlocal n_products
            n_products += 1
            return product_ref(feed_at, lambda x: fake_stat(hist, x), replay, fed, term)
        want = episode(feed, pick, e, lambda t, i=i: is_call(i, t), lambda t, i=i: tool_r(i, t),
                       term_start=lambda t, i=i: term_start(i, t), product=product)
        assert together[i] == want, i
        assert dec.hist[i] == hist, i
    assert n_products >= 3

"""ana_amd.agent's bookkeeping on a stand-in decoder (no GPU): positions,
forced runs, RNG words and endings, batched against one episode at a time."""
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
       agent.Episode([0, 1 + 1, 60], seed=0, budget=5, calls=2)]


def test_batched_is_alone():
    dec = FakeDecoder(len(EPS))
    together = agent.run(dec, EPS, None, is_call, tool)
    for i, e in enumerate(EPS):
        d1 = FakeDecoder(1)
        alone = agent.run(d1, [e], None, lambda _, t: is_call(i, t), lambda _, t: tool(i, t))[0]
        assert alone == together[i], i
        # every token but the last drawn one was fed at its position
        assert dec.hist[i] == list(e.prompt) + together[i].tokens[:-1]


def test_endings_and_flags():
    out = agent.run(FakeDecoder(len(EPS)), EPS, None, is_call, tool)
    for e, o in zip(EPS, out):
        assert o.why in ("eos", "budget", "calls", "tool")
        assert len(o.tokens) == len(o.drawn)
        assert o.tokens[: len(e.first)] == list(e.first) and not any(o.drawn[: len(e.first)])
        assert o.drawn[-1]
        # a stretch never draws more than its budget
        run_ = 0
        for d in o.drawn:
            run_ = run_ + 1 if d else 0
            assert run_ <= e.budget
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

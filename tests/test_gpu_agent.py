"""ana_amd.agent on the GPU (ANA_EXACT_FP32, the v3 sampling settings and
greedy): episodes decoded together, tool echoes and given tokens included,
take bit for bit the tokens, flags and endings of the one-episode
restatement of bend/Agent/Loop.bend (agent_loop_ref) driven by the CPU
oracle (its feed, its logits, S.pick with the episode's RNG words), and the
same tokens each takes alone."""
import numpy as np
import pytest

import ana_amd
from ana_amd import agent, ckpt
from ana_amd import config as cf

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def path(tmp_path_factory):
    d = tmp_path_factory.mktemp("cka")
    p = str(d / "v3.ftc2")
    ckpt.write(p, cf.SMALL4_V3, ckpt.init_params(cf.SMALL4_V3, "normal", 9))
    return p


def is_call(i, toks):
    return toks[-1] % 7 == 3


def is_call_len(i, toks):
    # (greedy picks on this model settle into repeats, so its calls come by
    # length instead)
    return len(toks) % 6 == 4 and len(toks) < 12


def tool(i, toks):
    # (keyed on every token written: with a call token, the last one is
    # always that token)
    key = sum(toks) % 251
    if key >= 190:
        return None
    return [2 + (key * 5 + j + i) % 250 for j in range(1 + (i + len(toks)) % 5)]


def episodes(vocab):
    rng = np.random.default_rng(4)
    eps = []
    for i in range(7):
        n = 1 + int(rng.integers(0, 20))
        prompt = [0] + [int(x) for x in rng.integers(2, vocab, size=n)]
        first = [int(x) for x in rng.integers(2, vocab, size=i % 3)]
        eps.append(agent.Episode(prompt, seed=100 + i, budget=10 + 3 * i, calls=i % 4, first=first))
    return eps


@pytest.mark.parametrize("call_token", [None, 10])
@pytest.mark.parametrize("sampling", ["v3", "greedy"])
def test_batched_episodes_are_the_loop(oracle, path, sampling, call_token):
    from agent_loop_ref import episode
    print(f"case agent {sampling} call token {call_token}", flush=True)
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9))) if sampling == "v3" else None
    call = is_call if sampling == "v3" else is_call_len
    m = oracle.Model(path)
    with ana_amd.Decoder(path, max_seqs=8, prefill_chunk=8) as dec:
        eps = episodes(dec.vocab)
        together = agent.run(dec, eps, st, call, tool, call_token=call_token)
        for i, e in enumerate(eps):
            s_ = oracle.State(m)
            at = [0]
            r = oracle.rng_seeded(e.seed)

            def feed(t):
                s_.feed(at[0], int(t))
                at[0] += 1

            def pick():
                lg = s_.logits()
                if st is None:
                    return oracle.top(lg)
                return oracle.pick(lg, st.temperature, st.top_k, st.top_p, r)
            want = episode(feed, pick, e, lambda t, i=i: call(i, t), lambda t, i=i: tool(i, t), call_token)
            assert together[i] == want, i
            if i < 3:
                alone = agent.run(dec, [e], st, lambda _, t, i=i: call(i, t), lambda _, t, i=i: tool(i, t),
                                  slots=[7], call_token=call_token)[0]
                assert alone == together[i], i
    whys = {o.why for o in together}
    print(f"endings {sorted(whys)}; tokens {[len(o.tokens) for o in together]}", flush=True)
    assert len(whys) >= 2


class OracleEngine:
    """One episode's engine on the CPU oracle: feed, the picks (the base
    settings and the retry ones share the episode's RNG words), al.stat on
    the last logits, and the replay after emptying the state."""

    def __init__(self, oracle, m, seed, st, rs):
        self.o, self.m, self.st, self.rs = oracle, m, st, rs
        self.s = oracle.State(m)
        self.at = 0
        self.r = oracle.rng_seeded(seed)

    def feed(self, t):
        self.s.feed(self.at, int(t))
        self.at += 1

    def feed_at(self, pos, t):
        assert pos == self.at
        self.feed(t)

    def _pick(self, st):
        lg = self.s.logits()
        if st is None:
            return self.o.top(lg)
        return self.o.pick(lg, st.temperature, st.top_k, st.top_p, self.r)

    def pick(self):
        return self._pick(self.st)

    def retry_pick(self):
        return self._pick(self.rs)

    def stat(self, x):
        return self.o.stat(self.s.logits(), x)

    def replay(self, fed):
        self.s = self.o.State(self.m)
        self.at = 0
        for t in fed:
            self.feed(t)


def test_product_is_the_reference(oracle, path):
    """agent.product (al.product: the pass along a failed term with
    ana_stats, the replay, the cut) bit for bit against its restatement on
    the oracle, in exact mode: the verdict (q, d, a, b), the given tokens,
    and the logits after the replay. The failed terms are the model's own
    greedy continuation with one token changed at different places, so the
    cut falls at the start and at several places along the term."""
    from agent_loop_ref import product_ref
    m = oracle.Model(path)
    rng = np.random.default_rng(11)
    with ana_amd.Decoder(path, max_seqs=2, prefill_chunk=8, numerics=ana_amd.EXACT_FP32) as dec:
        v = dec.vocab
        prompt = [0] + [int(x) for x in rng.integers(2, v, size=9)]
        eng = OracleEngine(oracle, m, 0, None, None)
        for t in prompt:
            eng.feed(t)
        greedy = []
        for _ in range(7):
            t = oracle.top(eng.s.logits())
            greedy.append(int(t))
            eng.feed(t)
        seen = set()
        for case, (k, length) in enumerate([(0, 1), (0, 6), (3, 6), (5, 6), (6, 6), (2, 3)]):
            term = list(greedy[1:1 + length])
            if k < length:
                term[k] = int(rng.integers(2, v))
            fed = prompt + [greedy[0]]
            print(f"case product {case}: term length {length}, changed at {k}", flush=True)
            dec.reset(1)
            dec.feeds(1, 0, prompt)
            got = agent.product(dec, 1, fed, term)
            e2 = OracleEngine(oracle, m, 0, None, None)
            for t in prompt:
                e2.feed(t)
            given, (q, d, a, b) = product_ref(e2.feed_at, e2.stat, e2.replay, fed, term)
            assert (got.q, got.d, got.a, got.b) == (q, d, a, b), (case, got, (q, d, a, b))
            assert got.given == given
            lg = dec.logits([1])[0]
            assert np.array_equal(lg.view(np.uint32), e2.s.logits().view(np.uint32)), case
            seen.add(d)
        assert len(seen) >= 3 and 0 in seen, seen


def test_retry_episodes_are_the_loop(oracle, path):
    """agent.run with failed checks (Retry answers with the term to avoid),
    term starts and retry settings, on the GPU in exact mode, bit for bit
    against the one-episode restatement driven by the oracle."""
    from agent_loop_ref import episode, product_ref
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9)))
    rs = ana_amd.Settings(float(np.float32(0.5)), 20, float(np.float32(0.95)))

    def tool_r(i, toks):
        key = sum(toks) % 251
        if key >= 215:
            return None
        echo = [2 + (key * 5 + j + i) % 250 for j in range(1 + (i + len(toks)) % 4)]
        return agent.Retry(echo, toks[-5:]) if (i + len(toks)) % 3 else echo

    def term_start(i, toks):
        return toks[-1] % 4 == 1

    m = oracle.Model(path)
    with ana_amd.Decoder(path, max_seqs=8, prefill_chunk=8, numerics=ana_amd.EXACT_FP32) as dec:
        eps = episodes(dec.vocab)
        print("case agent retry: 7 episodes, v3 then retry sampling", flush=True)
        together = agent.run(dec, eps, st, is_call, tool_r, term_start=term_start, retry=rs)
        products = 0
        for i, e in enumerate(eps):
            eng = OracleEngine(oracle, m, e.seed, st, rs)

            def product(fed, term, eng=eng):
                nonlocal products
                products += 1
                return product_ref(eng.feed_at, eng.stat, eng.replay, fed, term)
            want = episode(eng.feed, eng.pick, e, lambda t, i=i: is_call(i, t), lambda t, i=i: tool_r(i, t),
                           term_start=lambda t, i=i: term_start(i, t), product=product, retry_pick=eng.retry_pick)
            assert together[i] == want, i
    print(f"products {products}; endings {sorted({o.why for o in together})}", flush=True)
    assert products >= 2

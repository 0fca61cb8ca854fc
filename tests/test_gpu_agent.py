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

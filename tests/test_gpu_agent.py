"""ana_amd.agent on the GPU: episodes decoded together take exactly the
tokens each takes alone (ANA_EXACT_FP32, the v3 sampling settings and
greedy): tool echoes and first calls as forced runs through ana_feeds_n, one
ana_generate step for every live episode."""
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


def tool(i, toks):
    if toks[-1] >= 240:
        return None
    return [2 + (toks[-1] * 5 + j + i) % 250 for j in range(1 + (i + len(toks)) % 5)]


def episodes(vocab):
    rng = np.random.default_rng(4)
    eps = []
    for i in range(7):
        n = 1 + int(rng.integers(0, 20))
        prompt = [0] + [int(x) for x in rng.integers(2, vocab, size=n)]
        first = [int(x) for x in rng.integers(2, vocab, size=i % 3)]
        eps.append(agent.Episode(prompt, seed=100 + i, budget=10 + 3 * i, calls=i % 4, first=first))
    return eps


@pytest.mark.parametrize("sampling", ["v3", "greedy"])
def test_batched_episodes_are_alone(path, sampling):
    print(f"case agent batched {sampling}", flush=True)
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9))) if sampling == "v3" else None
    with ana_amd.Decoder(path, max_seqs=8, prefill_chunk=8) as dec:
        eps = episodes(dec.vocab)
        together = agent.run(dec, eps, st, is_call, tool)
        for i, e in enumerate(eps):
            alone = agent.run(dec, [e], st, lambda _, t, i=i: is_call(i, t), lambda _, t, i=i: tool(i, t),
                              slots=[7])[0]
            assert alone == together[i], i
    whys = {o.why for o in together}
    print(f"endings {sorted(whys)}; tokens {[len(o.tokens) for o in together]}", flush=True)
    assert len(whys) >= 2

"""Many agent episodes decoded together on one Decoder.

The engine's side of the agent tool loop (bend/Agent/Loop.bend), stretch by
stretch as al.gen runs it (Loop.bend:480-505):
- an episode feeds BOS and its prompt and draws a pick from the prompt's
  last logits (al.episode, Loop.bend:681-690, through dc.en.prefill.pick);
- given tokens to write first (AGENT_FIRST), that pick is drawn and set
  aside: the RNG moves past it, and the given tokens stand in as picks not
  drawn (al.start and al.forced.first, Loop.bend:275-277, 338-343);
- a stretch of budget N: a pick that is EOS ends the episode ("eos", the EOS
  not written); with N picks written, the next one ends it ("budget"); a
  pick that ends a call line is replaced by the call's token, written and
  fed in its place (al.called, Loop.bend:403-411, writes the newline and
  feeds the newline token, `call_token`), and the tool asked; any other pick is written, fed, and the next one drawn (or,
  while given tokens remain, taken from them: al.next, Loop.bend:375-383);
- a tool's echo is fed as unsampled tokens and a new stretch starts from a
  pick drawn from the echo's last logits (al.resume, Loop.bend:561-567);
  tokens still to be given are dropped there, as al.resume starts afresh.

What a call is and what the tool answers stay with the caller (`is_call`,
`tool`), as do the transcript, the repetition cut and the retry settings
after a failed check.

What this module adds is the batching: every live episode shares each engine
call. A round feeds, for each episode, the tokens written since its last
draw but the last one (ana_feeds_n), then takes one ana_generate step for
every episode that draws (the last token fed there, each episode with its
own RNG words). An episode's tokens do not depend on which others share its
calls; `test_agent` holds the batching to a one-episode restatement of the
loop on a stand-in decoder, and `test_gpu_agent` to the same restatement on
the CPU oracle, bit for bit in exact mode.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Sequence

import numpy as np

EOS = 1


@dataclass
class Episode:
    prompt: Sequence[int]          # BOS first (ids)
    seed: int                      # the episode's SAMPLE_SEED
    budget: int                    # tokens the model may draw a stretch
    calls: int = 4                 # tool calls answered (al.round's fuel / 2)
    first: Sequence[int] = ()      # fed as if drawn, before the first draw


@dataclass
class Outcome:
    tokens: list = field(default_factory=list)   # written after the prompt: drawn and given, in order (no EOS)
    drawn: list = field(default_factory=list)    # per token: drawn (True) or given (False)
    why: str = ""                                 # "eos", "budget", "calls" or "tool"


def run(dec, eps: Sequence[Episode], st, is_call: Callable[[int, list], bool],
        tool: Callable[[int, list], Sequence[int] | None], slots: Sequence[int] | None = None,
        call_token: int | None = None) -> list:
    """Decode episodes eps together on dec (sequence slots `slots`, default
    0..n-1; each is reset first) with sampling settings st (None: greedy).

    Each pick of episode i (tokens = everything it wrote so far): EOS ends
    it ("eos"); with the stretch's budget of picks written, it ends it
    ("budget"); else it is written, and is_call(i, tokens) asks whether it
    ends a call line. If it does, call_token (None: the pick itself) takes
    the pick's place among the tokens written, as al.called writes the
    newline in place of the pick's bytes; then, with calls left, tool(i,
    tokens) either ends the episode (None: "tool", the caller's verdict, as
    a passed check ends al.round) or gives the echo: the call's token is fed
    at the call's place, the echo after it, and a new stretch starts with a
    new budget; without calls left the episode ends ("calls")."""
    n = len(eps)
    slots = list(range(n)) if slots is None else [int(s) for s in slots]
    if len(slots) != n or len(set(slots)) != n:
        raise ValueError("agent.run: one distinct sequence slot per episode")
    if any(len(e.prompt) == 0 for e in eps):
        raise ValueError("agent.run: an empty prompt (BOS comes first)")
    if any(EOS in list(e.first) for e in eps):
        raise ValueError("agent.run: EOS among the tokens given as drawn")
    from . import rng_seeded
    out = [Outcome() for _ in eps]
    rng = np.ascontiguousarray(np.stack([rng_seeded(e.seed) for e in eps]).astype(np.uint64))
    pos = [0] * n                                 # where the next fed token goes
    pick = [(0, True)] * n                        # the pick in hand: (token, drawn)
    given = [list(e.first) for e in eps]          # given tokens after the one in hand
    left = [e.budget for e in eps]                # picks the stretch may still write
    calls = [e.calls for e in eps]
    for s in slots:
        dec.reset(s)

    def draw(idx, feeds):
        """For each episode idx[k]: feed feeds[k] from its position, the
        last token through one ana_generate step, whose pick comes back."""
        pre = [k for k in range(len(idx)) if len(feeds[k]) > 1]
        if pre:
            dec.feeds_n([slots[idx[k]] for k in pre], [pos[idx[k]] for k in pre], [feeds[k][:-1] for k in pre])
        r = np.ascontiguousarray(rng[idx])
        got = dec.generate([slots[i] for i in idx], [pos[i] + len(f) - 1 for i, f in zip(idx, feeds)],
                           [f[-1] for f in feeds], 1, st, r)
        rng[idx] = r
        for k, i in enumerate(idx):
            pos[i] += len(feeds[k])
        return [int(got[k, 0]) for k in range(len(idx))]

    # the prompts fed and each first pick drawn; given tokens set it aside
    first = draw(list(range(n)), [list(e.prompt) for e in eps])
    for i in range(n):
        pick[i] = (given[i].pop(0), False) if given[i] else (first[i], True)
    live = set(range(n))
    while live:
        idx, feeds = [], []
        for i in sorted(live):
            fed = []
            while True:
                t, drawn = pick[i]
                if t == EOS:
                    out[i].why = "eos"
                    break
                if left[i] == 0:
                    out[i].why = "budget"
                    break
                out[i].tokens.append(t)
                out[i].drawn.append(drawn)
                if is_call(i, out[i].tokens):
                    if call_token is not None:
                        t = out[i].tokens[-1] = int(call_token)
                    if calls[i] == 0:
                        out[i].why = "calls"
                        break
                    calls[i] -= 1
                    ans = tool(i, out[i].tokens)
                    if ans is None:
                        out[i].why = "tool"
                        break
                    echo = [int(x) for x in ans]
                    if EOS in echo:
                        raise ValueError("agent.run: EOS in a tool's echo")
                    fed += [t] + echo
                    given[i] = []
                    left[i] = eps[i].budget
                    idx.append(i)
                    feeds.append(fed)
                    break
                left[i] -= 1
                fed.append(t)
                if given[i]:
                    pick[i] = (given[i].pop(0), False)
                    continue
                idx.append(i)
                feeds.append(fed)
                break
            if out[i].why:
                live.discard(i)
        if idx:
            for i, t in zip(idx, draw(idx, feeds)):
                pick[i] = (t, True)
    return out

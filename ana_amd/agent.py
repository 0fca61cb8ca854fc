"""Many agent episodes decoded together on one Decoder.

The engine's side of the agent tool loop (bend/Agent/Loop.bend):
- an episode feeds BOS and its prompt, then draws from the prompt's last
  logits (al.episode, Loop.bend:681-690, through dc.en.prefill.pick);
- it draws one token a step (al.gen, through dc.en.step.pick);
- when a stretch ends a tool call, the tool's echo is fed as unsampled
  tokens, prefilled, and drawing resumes from the echo's last logits
  (al.called then al.resume, Loop.bend:561-567);
- tokens given as if the model had written them (AGENT_FIRST: al.start and
  al.forced.first, Loop.bend:275-277, 338-343) take the same route.

Forced tokens leave the episode's RNG where it was ("a pick not drawn",
Loop.bend:275). What a call is and what the tool answers stay with the
caller (`is_call`, `tool`), as do the transcript, the repetition cut and the
retry settings after a failed check.

What this module adds is the batching: every live episode shares each engine
call. A round is one ana_feeds_n for every episode with a forced run (the
pending token and the run but its last token, at each episode's own
position), then one ana_generate step for every live episode, each with its
own RNG words. An episode's tokens do not depend on which others share its
calls (`test_agent` and `test_gpu_agent` check that, the GPU one bit for
bit in exact mode).
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
    tokens: list = field(default_factory=list)   # after the prompt: drawn and fed, in order
    drawn: list = field(default_factory=list)    # per token: drawn (True) or fed (False)
    why: str = ""                                 # "eos", "budget", "calls" or "tool"


def run(dec, eps: Sequence[Episode], st, is_call: Callable[[int, list], bool],
        tool: Callable[[int, list], Sequence[int] | None], slots: Sequence[int] | None = None) -> list:
    """Decode episodes eps together on dec (sequence slots `slots`, default
    0..n-1; each is reset first) with sampling settings st (None: greedy).

    After every drawn token t of episode i (tokens = everything after its
    prompt so far): t == EOS ends it ("eos"); else is_call(i, tokens) asks
    for the tool: with calls left, tool(i, tokens) either ends the episode
    (None: "tool", the caller's verdict, as a passed check ends al.round) or
    gives the ids fed next, after which a new stretch begins with a new
    budget (al.resume); without calls left the episode ends ("calls"); else
    the stretch's budget of draws ends it ("budget")."""
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
    pos = [len(e.prompt) - 1 for e in eps]        # where the pending token goes
    nxt = [int(e.prompt[-1]) for e in eps]        # the pending token (fed, not yet)
    forced = [list(e.first) for e in eps]
    draws = [0] * n
    calls = [e.calls for e in eps]
    live = set(range(n))
    for s in slots:
        dec.reset(s)
    dec.feeds_n(slots, [0] * n, [list(e.prompt[:-1]) for e in eps])
    while live:
        fr = sorted(i for i in live if forced[i])
        if fr:
            dec.feeds_n([slots[i] for i in fr], [pos[i] for i in fr], [[nxt[i]] + forced[i][:-1] for i in fr])
            for i in fr:
                f, forced[i] = forced[i], []
                out[i].tokens += f
                out[i].drawn += [False] * len(f)
                pos[i] += len(f)
                nxt[i] = f[-1]
        dr = sorted(live)
        r = np.ascontiguousarray(rng[dr])
        got = dec.generate([slots[i] for i in dr], [pos[i] for i in dr], [nxt[i] for i in dr], 1, st, r)
        rng[dr] = r
        for k, i in enumerate(dr):
            t = int(got[k, 0])
            out[i].tokens.append(t)
            out[i].drawn.append(True)
            pos[i] += 1
            nxt[i] = t
            draws[i] += 1
            if t == EOS:
                out[i].why = "eos"
            elif is_call(i, out[i].tokens):
                if calls[i] == 0:
                    out[i].why = "calls"
                else:
                    calls[i] -= 1
                    ans = tool(i, out[i].tokens)
                    if ans is None:
                        out[i].why = "tool"
                    else:
                        echo = [int(x) for x in ans]
                        if EOS in echo:
                            raise ValueError("agent.run: EOS in a tool's echo")
                        forced[i] = echo
                        draws[i] = 0
            elif draws[i] >= eps[i].budget:
                out[i].why = "budget"
            if out[i].why:
                live.discard(i)
    return out

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
  tokens still to be given are dropped there, as al.resume starts afresh;
- a failed check (the tool answers `Retry(echo, term)`, al.round's AlFail,
  Loop.bend:622-627) resumes the same way, from then on with the retry
  settings, and with the failed term to avoid: when the caller's
  `term_start` says the token just written starts the new stretch's term,
  the next tokens come from the product rule instead of a draw (al.next.free
  and al.product, Loop.bend:284-357, `product` below): the model's
  probability of writing the failed term again is read step by step along
  it, the engine is emptied and every token fed so far replayed, and the
  failed term up to the first step where another token outweighs it, then
  that token, are given as if drawn.

What a call is, where a term starts and what the tool answers stay with
the caller (`is_call`, `term_start`, `tool`), as do the transcript and the
repetition cut.

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
class Retry:
    """A tool's failed check: its echo, and the failed term (the term's
    tokens, then the call's) the next stretch's term is to avoid."""
    echo: Sequence[int]
    term: Sequence[int]


@dataclass
class Cut:
    """al.product's verdict (AlC, Loop.bend:289-310): q, the model's
    probability of writing the whole failed term again from its start; d,
    the failed term's tokens kept; a, the token put at step d and b its
    probability; given, the failed term's first d tokens then a."""
    q: np.float32
    d: int
    a: int
    b: np.float32
    given: list


def cut_of(steps) -> tuple:
    """The pass along the failed term from its end back (al.cut.last and
    al.cut.step, Loop.bend:297-310, F32 arithmetic): steps[j] = (p, a, b),
    the model's probability of the term's token j at step j, the likeliest
    other token and its probability. T's own token weighs p (1 - q') (q' the
    rest's probability, after it), another its own probability; the first
    step where another outweighs T's is where T is left."""
    f32 = np.float32
    p, a, b = steps[-1]
    q, d, aa, bb = f32(p), 0, int(a), f32(b)
    for p, a, b in reversed(steps[:-1]):
        p, b = f32(p), f32(b)
        if b > f32(p * f32(f32(1.0) - q)):
            q, d, aa, bb = f32(p * q), 0, int(a), b
        else:
            q, d = f32(p * q), d + 1
    return q, d, aa, bb


def product(dec, slot: int, fed: Sequence[int], term: Sequence[int]) -> Cut:
    """al.product (Loop.bend:345-357) on one sequence slot: fed is every
    token the slot has taken so far, in order, with the term's first token
    (the pick that starts the new term) last and not yet fed; term is the
    failed term to avoid (at least one token). That token is fed, then
    along the failed term: at each step its token's probability and its
    likeliest rival (ana_stats: al.stat), each token fed but the last
    (al.pass). Then the slot is emptied and fed replayed (al.product.fin:
    the dense store has no rewind), so it stands after fed, and the cut
    says which tokens come next (given as if drawn; the RNG untouched)."""
    term = [int(x) for x in term]
    if not term:
        raise ValueError("agent.product: an empty failed term")
    pos = len(fed) - 1
    dec.feed([slot], [pos], [int(fed[-1])])
    steps = []
    for j, x in enumerate(term):
        p, a, b = dec.stats([slot], [x])
        steps.append((p[0], int(a[0]), b[0]))
        if j + 1 < len(term):
            dec.feed([slot], [pos + 1 + j], [x])
    q, d, a, b = cut_of(steps)
    dec.reset(slot)
    dec.feeds(slot, 0, [int(t) for t in fed])
    return Cut(q, d, a, b, term[:d] + [a])


@dataclass
class Outcome:
    tokens: list = field(default_factory=list)   # written after the prompt: drawn and given, in order (no EOS)
    drawn: list = field(default_factory=list)    # per token: drawn (True) or given (False)
    why: str = ""                                 # "eos", "budget", "calls" or "tool"


def run(dec, eps: Sequence[Episode], st, is_call: Callable[[int, list], bool],
        tool: Callable[[int, list], Sequence[int] | Retry | None], slots: Sequence[int] | None = None,
        call_token: int | None = None, term_start: Callable[[int, list], bool] | None = None,
        retry=None) -> list:
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
    new budget; without calls left the episode ends ("calls"). A
    Retry(echo, term) answer is a failed check: the same, and from then on
    the episode draws with the settings `retry` (None: st) and, when
    term_start(i, tokens) says the token just written starts the stretch's
    term (no given tokens pending), takes its next tokens from product()
    against that term."""
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
    hist = [[] for _ in eps]                      # every token fed, in order (al.k.fed)
    avoid = [None] * n                            # the failed term the next term avoids
    retried = [False] * n                         # drawing with the retry settings
    for s in slots:
        dec.reset(s)

    def draw(idx, feeds):
        """For each episode idx[k]: feed feeds[k] from its position, the
        last token through one ana_generate step, whose pick comes back
        (episodes after a failed check with the retry settings)."""
        pre = [k for k in range(len(idx)) if len(feeds[k]) > 1]
        if pre:
            dec.feeds_n([slots[idx[k]] for k in pre], [pos[idx[k]] for k in pre], [feeds[k][:-1] for k in pre])
        got = {}
        for sett, grp in ((st, [k for k, i in enumerate(idx) if not retried[i]]),
                          (st if retry is None else retry, [k for k, i in enumerate(idx) if retried[i]])):
            if not grp:
                continue
            ii = [idx[k] for k in grp]
            r = np.ascontiguousarray(rng[ii])
            o = dec.generate([slots[i] for i in ii], [pos[i] + len(feeds[k]) - 1 for i, k in zip(ii, grp)],
                             [feeds[k][-1] for k in grp], 1, sett, r)
            rng[ii] = r
            for j, k in enumerate(grp):
                got[k] = int(o[j, 0])
        for k, i in enumerate(idx):
            pos[i] += len(feeds[k])
            hist[i] += [int(t) for t in feeds[k]]
        return [got[k] for k in range(len(idx))]

    # the prompts fed and each first pick drawn; given tokens set it aside
    first = draw(list(range(n)), [list(e.prompt) for e in eps])
    for i in range(n):
        pick[i] = (given[i].pop(0), False) if given[i] else (first[i], True)
    live = set(range(n))
    tail = []
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
                    if isinstance(ans, Retry):
                        avoid[i] = [int(x) for x in ans.term] or None
                        retried[i] = True
                        ans = ans.echo
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
                if avoid[i] is not None and term_start is not None and term_start(i, out[i].tokens):
                    # al.next.free's product: what was written before t goes
                    # in, then t through the pass, the replay and the cut
                    if len(fed) > 1:
                        dec.feeds_n([slots[i]], [pos[i]], [fed[:-1]])
                        pos[i] += len(fed) - 1
                        hist[i] += [int(x) for x in fed[:-1]]
                    c = product(dec, slots[i], hist[i] + [int(t)], avoid[i])
                    hist[i].append(int(t))
                    pos[i] += 1
                    avoid[i] = None
                    fed = []
                    pick[i] = (c.given[0], False)
                    given[i] = c.given[1:]
                    continue
                idx.append(i)
                feeds.append(fed)
                break
            if out[i].why:
                live.discard(i)
                if fed:
                    # given tokens written before the end: fed, as al.next
                    # feeds each before the next one stands in
                    tail.append((i, fed))
        if tail:
            dec.feeds_n([slots[i] for i, _ in tail], [pos[i] for i, _ in tail], [f for _, f in tail])
            for i, f in tail:
                pos[i] += len(f)
                hist[i] += [int(t) for t in f]
            tail = []
        if idx:
            for i, t in zip(idx, draw(idx, feeds)):
                pick[i] = (t, True)
    return out

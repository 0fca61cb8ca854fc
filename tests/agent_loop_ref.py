"""One agent episode at a time, as bend/Agent/Loop.bend runs it (test
infrastructure: the restatement ana_amd.agent's batching is held to).

The engine is two callables: feed(t) feeds token t at the next position
(dc.en.feed), and pick() draws from the logits of the last token fed with
the episode's RNG (dc.en.step.pick; dc.en.prefill.pick is the feeds then
one pick); after a failed check, retry_pick() draws with the retry
settings, and product(fed, term) is al.product's engine side (product_ref
below, over the engine's own feed, stat and replay). Only the engine-side
control flow is restated; the call-line grammar, where a term starts, the
tools and the transcript are the caller's is_call, term_start and tool.
"""
import numpy as np

from ana_amd.agent import EOS, Outcome, Retry


def product_ref(feed_at, stat, replay, fed, term):
    """al.product with a failed term (bend/Agent/Loop.bend:345-357): the
    term's first token fed[-1] fed at its position with its logits
    (dc.en.step), then al.pass (:312-325) along the term: al.stat (:284-288,
    stat(x) on the logits the last feed answered) at each token, each fed
    but the last; the verdict folded from the end back (al.cut.last,
    al.cut.step, :297-310, in F32); then al.product.fin (:329-336): the
    engine emptied and every token fed so far replayed (replay(fed)), and
    the term up to d, then a, given. Returns (given, (q, d, a, b))."""
    f32 = np.float32
    pos = len(fed) - 1
    feed_at(pos, fed[-1])
    steps = []
    for j, x in enumerate(term):
        steps.append(stat(x))
        if j + 1 < len(term):
            feed_at(pos + 1 + j, x)
    # al.cut.last: AlC{p, 0, a, b}
    p, a, b = steps[-1]
    cut = (f32(p), 0, int(a), f32(b))
    for p, a, b in reversed(steps[:-1]):
        q, d, a2, b2 = cut
        # al.cut.step: another token outweighs T's (p (1 - q)) here?
        if f32(b) > f32(f32(p) * f32(f32(1.0) - q)):
            cut = (f32(f32(p) * q), 0, int(a), f32(b))
        else:
            cut = (f32(f32(p) * q), 1 + d, a2, b2)
    replay(fed)
    q, d, a, b = cut
    return [int(x) for x in term[:d]] + [a], cut


def episode(feed, pick, ep, is_call, tool, call_token=None, term_start=None, product=None, retry_pick=None):
    out = Outcome()
    hist = []
    feed0 = feed

    def feed(t):
        hist.append(int(t))
        feed0(t)
    avoid = None
    draw = pick
    # al.episode (Loop.bend:681-690): BOS and the prompt fed, a pick drawn
    for t in ep.prompt:
        feed(t)
    p = pick()
    # al.start / al.forced.first (Loop.bend:338-343): given tokens stand in
    # for that pick, which stays drawn (its RNG step is taken)
    force = list(ep.first)
    cur = (force.pop(0), False) if force else (p, True)
    calls = ep.calls
    while True:
        # al.gen (Loop.bend:480-505), a stretch of ep.budget picks
        n = ep.budget
        while True:
            t, drawn = cur
            if t == EOS:
                out.why = "eos"        # al.halt: the stop, EOS not written
                return out
            if n == 0:
                out.why = "budget"     # al.halt: the budget spent
                return out
            out.tokens.append(t)
            out.drawn.append(drawn)
            if is_call(out.tokens):
                # al.called (Loop.bend:403-411) writes the newline (10 <> out)
                # in place of the pick's bytes and feeds the newline token
                if call_token is not None:
                    out.tokens[-1] = t = call_token
                break
            n -= 1
            # al.next (Loop.bend:375-383): a given token next (t fed); else,
            # when t starts the term and a failed term is to be avoided, the
            # product's tokens (al.next.free, al.product); else t fed and a
            # pick drawn
            if force:
                feed(t)
                cur = (force.pop(0), False)
            elif avoid is not None and term_start is not None and term_start(out.tokens):
                given, _ = product(hist + [int(t)], avoid)
                hist.append(int(t))
                avoid = None
                cur = (given[0], False)
                force = given[1:]
            else:
                feed(t)
                cur = (draw(), True)
        # al.round answers the call while calls are left
        if calls == 0:
            out.why = "calls"
            return out
        calls -= 1
        echo = tool(out.tokens)
        if echo is None:
            out.why = "tool"
            return out
        if isinstance(echo, Retry):
            # al.round's AlFail (Loop.bend:622-627): the retry settings from
            # now on, the failed term to avoid (RETRY_AVOID)
            avoid = [int(x) for x in echo.term] or None
            if retry_pick is not None:
                draw = retry_pick
            echo = echo.echo
        feed(t)
        # al.resume (Loop.bend:561-567): the echo fed, a pick drawn, a new
        # stretch, nothing left to give
        for e in echo:
            feed(int(e))
        force = []
        cur = (draw(), True)

"""One agent episode at a time, as bend/Agent/Loop.bend runs it (test
infrastructure: the restatement ana_amd.agent's batching is held to).

The engine is two callables: feed(t) feeds token t at the next position
(dc.en.feed), and pick() draws from the logits of the last token fed with
the episode's RNG (dc.en.step.pick; dc.en.prefill.pick is the feeds then
one pick). Only the engine-side control flow is restated; the call-line
grammar, the tools and the transcript are the caller's is_call and tool.
"""
from ana_amd.agent import EOS, Outcome


def episode(feed, pick, ep, is_call, tool, call_token=None):
    out = Outcome()
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
            # al.next (Loop.bend:375-383): t fed; a given token next, else a
            # pick drawn
            feed(t)
            cur = (force.pop(0), False) if force else (pick(), True)
        # al.round answers the call while calls are left
        if calls == 0:
            out.why = "calls"
            return out
        calls -= 1
        echo = tool(out.tokens)
        if echo is None:
            out.why = "tool"
            return out
        feed(t)
        # al.resume (Loop.bend:561-567): the echo fed, a pick drawn, a new
        # stretch, nothing left to give
        for e in echo:
            feed(int(e))
        force = []
        cur = (pick(), True)

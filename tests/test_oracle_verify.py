"""The oracle's accept loop pinned by the reference's own speculative-step tests
(crates/engine/src/spec/step.rs:971-1059), restated on its scripted rows: whatever the drafts, the
speculative loop gives the plain loop's tokens, history and RNG stream."""
import numpy as np
import pytest

import spec_script as S
from oracle_lib import DEFAULT, GREEDY, Sampler


class OracleSampler:
    def __init__(self, seed, params):
        self.s = Sampler(seed, **params)

    def sample(self, row):
        return self.s.sample(row)

    def verify(self, rows, drafts):
        picks, _, _ = self.s.verify(rows, np.array(drafts, np.uint32))
        return picks


def truth(params, seed, n):
    out, _ = S.plain(OracleSampler(seed, params), n)
    return S.PROMPT + out


def test_the_scripted_rows_are_exact_and_depend_on_the_last_three_tokens():
    a = S.logits([3, 1, 4, 1, 5])
    assert a.dtype == np.float32 and a.shape == (S.VOCAB,)
    assert ((a >= 0) & (a < 8)).all()
    # Multiples of 2^-21: a 24-bit integer over 2^24, times 8.
    assert (a * (1 << 21) == np.round(a * (1 << 21))).all()
    assert (S.logits([9, 4, 1, 5]) == S.logits([4, 1, 5])).all()
    assert not (S.logits([4, 1, 6]) == a).all()


@pytest.mark.parametrize("params,seed", [(GREEDY, 0), (DEFAULT, 1234)])
def test_any_draft_gives_the_plain_loops_tokens(params, seed):
    # step.rs:971-1001 (the lookup drafter aside: it is an n-gram source, not part of the sampler).
    t = truth(params, seed, 64)
    want_s = OracleSampler(seed, params)
    want, want_hist = S.plain(want_s, 64)
    for name, make in [("right", S.ScriptedDrafter.right), ("wrong", S.ScriptedDrafter.wrong),
                       ("half", S.ScriptedDrafter.half), ("none", S.ScriptedDrafter.none)]:
        got_s = OracleSampler(seed, params)
        got, got_hist, calls, accepted = S.speculate(got_s, make(t), 64)
        assert got == want, name
        assert got_hist == want_hist, name
        assert got_s.s.rng_state() == want_s.s.rng_state(), name
        if name != "none":
            assert calls > 0, name
        if name == "right":
            assert accepted > 0


def test_rows_past_the_stop_never_reach_the_sampler():
    # step.rs:1003-1025: the 20-token limit falls inside a burst; the sampler must not see later rows,
    # so its next eight draws on a fixed row are the plain loop's.
    t = truth(DEFAULT, 1234, 64)
    want_s = OracleSampler(1234, DEFAULT)
    want, _ = S.plain(want_s, 20)
    got_s = OracleSampler(1234, DEFAULT)
    got, _, _, _ = S.speculate(got_s, S.ScriptedDrafter.right(t), 20)
    assert got == want
    fixed = S.logits([7, 7, 7])
    for i in range(8):
        assert got_s.sample(fixed) == want_s.sample(fixed), i


@pytest.mark.parametrize("base", [DEFAULT, GREEDY])
def test_presence_penalty_inside_a_burst_matches_the_plain_loop(base):
    # step.rs:1027-1059: `seen` holds emitted tokens only; a rejected draft's row never reaches it.
    p = dict(base, presence=0.5)
    want, want_hist = S.plain(OracleSampler(1234, p), 64)
    free, _ = S.plain(OracleSampler(1234, dict(p, presence=0.0)), 64)
    assert want != free, "the penalty should matter here"
    t = truth(p, 1234, 64)
    for make in [S.ScriptedDrafter.right, S.ScriptedDrafter.half, S.ScriptedDrafter.wrong]:
        got, got_hist, _, _ = S.speculate(OracleSampler(1234, p), make(t), 64)
        assert got == want
        assert got_hist == want_hist

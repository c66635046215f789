"""as_sample and as_verify on the reference's speculative-step tests (crates/engine/src/spec/step.rs:
971-1059), restated on its scripted rows: whatever the drafts, the GPU's speculative loop gives the
plain loop's tokens, history and RNG stream, and those are the oracle's."""
import numpy as np
import pytest
import torch

import spec_script as S
from oracle_lib import DEFAULT, GREEDY, Sampler

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=16, max_vocab=S.VOCAB)
    yield c
    c.close()


class GpuSampler:
    """One request on the GPU: its RNG state and its history (the ids it returned) on the device."""

    def __init__(self, ctx, seed, p):
        from artemis_amd import Sampling, states_tensor
        self.ctx = ctx
        self.dev = torch.device("cuda:0")
        self.p = Sampling(p["temp"], p["top_k"], p["top_p"], p["min_p"], p.get("presence", 0.0))
        self.rng = states_tensor([seed], self.dev)
        self.hist = []

    def _hist(self):
        if not self.hist:
            return None
        return torch.tensor(np.array(self.hist, np.int32), device=self.dev)

    def sample(self, row):
        lg = torch.from_numpy(np.ascontiguousarray(row[None, :], np.float32)).to(self.dev)
        ids = self._hist()
        off = torch.tensor([0, len(self.hist)], dtype=torch.int32, device=self.dev) if ids is not None else None
        tok, st, *_ = self.ctx.sample_batch(lg, [self.p], self.rng, off, ids)
        assert int(st.item()) & 0xFF == 0
        t = int(tok.item())
        self.hist.append(t)
        return t

    def verify(self, rows, drafts):
        picks, result = self.ctx.verify(torch.from_numpy(np.ascontiguousarray(rows, np.float32)).to(self.dev),
                                        torch.tensor(np.array(drafts, np.int32), device=self.dev), self.p,
                                        self.rng, self._hist(), None)
        r = result.cpu().numpy()
        read = int(r[0])
        assert int(r[1]) == read - 1 and int(r[3]) & 0xFF == 0
        got = [int(x) for x in picks.cpu().numpy()[:read]]
        assert int(r[2]) == got[-1]
        self.hist.extend(got)
        return got

    def rng_state(self):
        return [int(x) for x in self.rng.cpu().numpy().view(np.uint64)[0]]


class OracleSampler:
    def __init__(self, seed, params):
        self.s = Sampler(seed, **params)

    def sample(self, row):
        return self.s.sample(row)


def truth(params, seed, n):
    out, _ = S.plain(OracleSampler(seed, params), n)
    return S.PROMPT + out


@pytest.mark.parametrize("params,seed", [(GREEDY, 0), (DEFAULT, 1234)])
def test_any_draft_gives_the_plain_loops_tokens(ctx, params, seed):
    t = truth(params, seed, 64)
    want_o = OracleSampler(seed, params)
    want, want_hist = S.plain(want_o, 64)
    plain_gpu = GpuSampler(ctx, seed, params)
    assert S.plain(plain_gpu, 64)[0] == want
    assert plain_gpu.rng_state() == want_o.s.rng_state()
    for name, make in [("right", S.ScriptedDrafter.right), ("wrong", S.ScriptedDrafter.wrong),
                       ("half", S.ScriptedDrafter.half), ("none", S.ScriptedDrafter.none)]:
        g = GpuSampler(ctx, seed, params)
        got, got_hist, calls, accepted = S.speculate(g, make(t), 64)
        assert got == want, name
        assert got_hist == want_hist, name
        assert g.rng_state() == want_o.s.rng_state(), name
        if name == "right":
            assert accepted > 0


def test_rows_past_the_stop_never_reach_the_sampler(ctx):
    t = truth(DEFAULT, 1234, 64)
    want_o = OracleSampler(1234, DEFAULT)
    want, _ = S.plain(want_o, 20)
    g = GpuSampler(ctx, 1234, DEFAULT)
    got, _, _, _ = S.speculate(g, S.ScriptedDrafter.right(t), 20)
    assert got == want
    fixed = S.logits([7, 7, 7])
    for i in range(8):
        assert g.sample(fixed) == want_o.sample(fixed), i


@pytest.mark.parametrize("base", [DEFAULT, GREEDY])
def test_presence_penalty_inside_a_burst_matches_the_plain_loop(ctx, base):
    p = dict(base, presence=0.5)
    want, want_hist = S.plain(OracleSampler(1234, p), 64)
    t = truth(p, 1234, 64)
    for make in [S.ScriptedDrafter.right, S.ScriptedDrafter.half, S.ScriptedDrafter.wrong]:
        got, got_hist, _, _ = S.speculate(GpuSampler(ctx, 1234, p), make(t), 64)
        assert got == want
        assert got_hist == want_hist

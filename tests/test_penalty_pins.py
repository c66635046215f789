"""Pins of the history penalties (repetition, frequency, presence over a history multiset).

The reference defines only the presence penalty (crates/engine/src/sample.rs:308-323, 351-356,
378-396). Its server accepts and ignores frequency_penalty and repetition_penalty
(crates/server/src/params.rs:298-328), so this build defines them (include/artemis_sampler.h):
for an id seen c >= 1 times, in f32 with every operation rounded on its own,
    t = (rep != 1) ? (x > 0 ? x / rep : x * rep) : x,   x' = t - (c * freq + pres).

Nothing here restates that formula. Each expected value is one of these:
  - a constant worked out by hand on dyadic inputs, where every step is exact and the operation
    order cannot matter (halving, doubling, x - (c/8 + 1/2), ...);
  - the exact rational value of each step, rounded to the nearest f32 (ties to even) by a rounding
    routine written from IEEE 754's definition, for non-dyadic settings such as rep 1.05.
Invariants close the rest: presence counts once whatever the count, frequency is linear in the
count, the history's order and the placement of duplicates do not matter, and ids past the row
are ignored.

The sampler is the probe. A greedy row (temp 0) whose penalised id A sits between two copies of
the expected value, one at a lower index and one at a higher one, returns the lower copy exactly
when x' <= v and A exactly when x' >= v (ties go to the lower index, sample.rs:9-17). Both
together say x' == v. A top-k 1 row does the same in total_cmp's order (sample.rs:106-108), which
also tells -0 from +0. The CPU oracle and the HIP library run the same probes.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle_lib as O

N = 4096
A = 1000           # the penalised id
LO, HI = 500, 1500  # the copies of the expected value, below and above A's index
FILL = np.float32(-10000.0)

# (x, count, presence, frequency, repetition, expected x'), worked out by hand.
HAND = [
    (3.0, 1, 0.0, 0.0, 2.0, 1.5),        # x > 0 divides by rep
    (-3.0, 1, 0.0, 0.0, 2.0, -6.0),      # x <= 0 multiplies
    (3.0, 1, 0.0, 0.0, 0.5, 6.0),
    (-3.0, 1, 0.0, 0.0, 0.5, -1.5),
    (0.0, 1, 0.0, 0.0, 2.0, 0.0),        # +0 is not > 0: multiplied, stays +0
    (-0.0, 1, 0.0, 0.0, 2.0, -0.0),      # -0 * 2 = -0, and -0 - (+0) = -0
    (4.0, 3, 0.5, 0.25, 1.0, 2.75),      # 4 - (3/4 + 1/2)
    (4.0, 1, 0.5, 0.0, 1.0, 3.5),        # presence once ...
    (4.0, 2, 0.5, 0.0, 1.0, 3.5),        # ... whatever the count
    (4.0, 7, 0.5, 0.0, 1.0, 3.5),
    (1.0, 1, 0.0, 0.125, 1.0, 0.875),    # frequency linear in the count
    (1.0, 2, 0.0, 0.125, 1.0, 0.75),
    (1.0, 3, 0.0, 0.125, 1.0, 0.625),
    (1.0, 8, 0.0, 0.125, 1.0, 0.0),
    (5.0, 2, 0.25, 0.25, 2.0, 1.75),     # 5/2 - (2/4 + 1/4)
    (-2.0, 2, 0.25, 0.25, 2.0, -4.75),   # -2*2 - 3/4
    (6.0, 4, -0.5, 0.5, 4.0, 0.0),       # 6/4 - (2 - 1/2) = +0
    (-1.0, 3, -0.25, -0.5, 0.5, 1.25),   # -1/2 - (-3/2 - 1/4): negative penalties raise
    (2.0, 1, 0.5, 0.0, 1.0, 1.5),        # rep 1, freq 0: the reference's x - presence
]


# ---- IEEE 754 binary32 rounding of an exact rational -------------------------------------------

def _f32_neighbours(q: Fraction):
    f = np.float32(float(q))
    return [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]


def round_f32(q: Fraction) -> np.float32:
    """The f32 nearest to q, ties to the even significand (round-to-nearest-even)."""
    best = None
    for c in _f32_neighbours(q):
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - q)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    r = best[1]
    if r == 0 and q < 0:
        return np.float32(-0.0)
    return np.float32(r)


def rounded_steps(x, c, pres, freq, rep) -> np.float32:
    """Each step of the definition as an exact rational, rounded to f32 on its own."""
    x, pres, freq, rep = (np.float32(v) for v in (x, pres, freq, rep))
    t = x
    if rep != np.float32(1.0):
        if x > 0:
            t = round_f32(Fraction(float(x)) / Fraction(float(rep)))
        else:
            t = round_f32(Fraction(float(x)) * Fraction(float(rep)))
    d = round_f32(Fraction(int(c)) * Fraction(float(freq)))
    d = round_f32(Fraction(float(d)) + Fraction(float(pres)))
    diff = Fraction(float(t)) - Fraction(float(d))
    if diff == 0:
        # x - y with x == y is +0 in round-to-nearest, except (-0) - (+0) = -0.
        neg = np.signbit(t) and not np.signbit(d)
        return np.float32(-0.0) if neg else np.float32(0.0)
    return round_f32(diff)


def test_the_rounding_routine_is_ieee():
    # Halfway cases go to the even significand; exact values are exact; a double-rounding trap.
    one = Fraction(1)
    ulp = Fraction(1, 2**23)
    assert round_f32(one + ulp / 2) == np.float32(1.0)
    assert round_f32(one + ulp + ulp / 2) == np.float32(1.0) + np.float32(2.0**-22)
    assert round_f32(Fraction(3, 2)) == np.float32(1.5)
    q = one + ulp / 2 + Fraction(1, 2**60)  # just above half an ulp: rounds up
    assert round_f32(q) == np.nextafter(np.float32(1.0), np.float32(2.0))
    for a, b in [(1.0, 1.05), (7.25, 1.05), (-3.0, 1.3), (0.1, 3.0)]:
        assert round_f32(Fraction(a) / Fraction(float(np.float32(b)))) == np.float32(a) / np.float32(b)


# Non-dyadic settings: config 3's and 5's (rep 1.05, presence 0.5, frequency 0.3) and others.
ROUNDED = [(x, c, pres, freq, rep)
           for (pres, freq, rep) in [(0.5, 0.3, 1.05), (0.0, 0.0, 1.3), (0.1, 0.7, 0.9), (0.0, 0.3, 1.0)]
           for x in (7.3, 2.6, 0.37, -0.37, -4.9)
           for c in (1, 2, 5)]


def all_cases():
    cases = [(x, c, p, f, r, np.float32(v)) for (x, c, p, f, r, v) in HAND]
    cases += [(x, c, p, f, r, rounded_steps(x, c, p, f, r)) for (x, c, p, f, r) in ROUNDED]
    return cases


def probe_rows(case):
    """Four probe rows for one case: greedy with the copy below / above A's index, top-k 1 with the
    same. Returns (rows [4][N] f32, params [4], history ids of A, the expected answers)."""
    x, c, pres, freq, rep, v = case
    rows = np.full((4, N), FILL, np.float32)
    rows[:, A] = np.float32(x)
    rows[0, LO] = rows[2, LO] = v
    rows[1, HI] = rows[3, HI] = v
    s = dict(presence=pres, frequency=freq, repetition=rep)
    greedy = dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0, **s)
    top1 = dict(temp=1.0, top_k=1, top_p=1.0, min_p=0.0, **s)
    # x' == v exactly: IEEE order gives the lower copy and then A; total_cmp's order does too.
    want = [LO, A, LO, A]
    return rows, [greedy, greedy, top1, top1], [A] * c, want


def describe(case):
    x, c, pres, freq, rep, v = case
    return f"x={x} c={c} pres={pres} freq={freq} rep={rep} -> {float(v)!r} ({int(np.float32(v).view(np.uint32)):#010x})"


def oracle_pick(row, p, hist, seed=3):
    s = O.Sampler(seed, **p)
    s.add_history(hist)
    return s.sample(row)


@pytest.mark.parametrize("case", all_cases(), ids=describe)
def test_oracle_penalised_values_are_the_fixed_ones(case):
    rows, params, hist, want = probe_rows(case)
    got = [oracle_pick(rows[i], params[i], hist) for i in range(4)]
    assert got == want, describe(case)


def test_oracle_probe_catches_planted_mistakes():
    # The probe is sharp: expected values one ulp off, or with the sign of zero flipped, fail.
    x, c, pres, freq, rep, v = (3.0, 1, 0.0, 0.0, 2.0, np.float32(1.5))
    for wrong in (np.nextafter(v, np.float32(2)), np.nextafter(v, np.float32(1))):
        rows, params, hist, want = probe_rows((x, c, pres, freq, rep, wrong))
        assert [oracle_pick(rows[i], params[i], hist) for i in range(4)] != want
    rows, params, hist, want = probe_rows((-0.0, 1, 0.0, 0.0, 2.0, np.float32(0.0)))
    got = [oracle_pick(rows[i], params[i], hist) for i in range(4)]
    assert got[:2] == want[:2] and got[2:] != want[2:]  # IEEE ties the zeros; total_cmp does not


def invariance_rows(seed=21, n=N):
    rng = np.random.default_rng(seed)
    base = (rng.standard_normal(n) * 2.5).astype(np.float32)
    hist = rng.integers(0, n, size=300).astype(np.uint32)
    hist = np.concatenate([hist, np.full(6, 17, np.uint32), np.full(3, 40, np.uint32)])
    shuffled = rng.permutation(hist)
    sorted_ = np.sort(hist)
    past_end = np.concatenate([hist, np.array([n, n + 5, 2**31, 2**32 - 1], np.uint32)])
    return base, [hist, shuffled, sorted_, past_end]


SETTINGS = [dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0),
            dict(temp=0.7, top_k=40, top_p=0.9, min_p=0.05),
            dict(temp=1.0, top_k=0, top_p=0.95, min_p=0.0),
            dict(temp=0.8, top_k=0, top_p=1.0, min_p=0.02)]


@pytest.mark.parametrize("si", range(len(SETTINGS)))
def test_oracle_history_order_duplicates_and_ids_past_the_row_do_not_matter(si):
    base, hists = invariance_rows()
    s = dict(SETTINGS[si], presence=0.5, frequency=0.3, repetition=1.05)
    for seed in range(30):
        picks = [oracle_pick(base, s, h, seed) for h in hists]
        assert len(set(picks)) == 1, (seed, picks)


# ---- the same probes on the GPU, through the C ABI ------------------------------------------------

def _gpu_ctx():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    ctx = Context(max_rows=512, max_vocab=N + 8)
    return torch, ctx


def _gpu_sample(torch, ctx, rows, params, hists, seeds):
    from artemis_amd import Sampling, states_tensor
    dev = torch.device("cuda:0")
    off = np.zeros(len(params) + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.concatenate([np.asarray(h, np.uint32) for h in hists]).astype(np.uint32).view(np.int32)
    ps = [Sampling(p["temp"], p["top_k"], p["top_p"], p["min_p"], p["presence"], p["frequency"],
                   p["repetition"]) for p in params]
    lg = torch.from_numpy(np.ascontiguousarray(rows, np.float32)).to(dev)
    tok, st, *_ = ctx.sample_batch(lg, ps, states_tensor(seeds, dev), torch.from_numpy(off).to(dev),
                                   torch.from_numpy(ids.copy()).to(dev))
    torch.cuda.synchronize()
    return tok.cpu().numpy().astype(np.uint32), st.cpu().numpy()


@pytest.mark.gpu
def test_gpu_penalised_values_are_the_fixed_ones():
    torch, ctx = _gpu_ctx()
    cases = all_cases()
    rows, params, hists, want = [], [], [], []
    for case in cases:
        r, p, h, w = probe_rows(case)
        rows.append(r)
        params += p
        hists += [h] * 4
        want += w
    rows = np.concatenate(rows)
    tok, st = _gpu_sample(torch, ctx, rows, params, hists, [3] * len(params))
    bad = [describe(cases[i // 4]) + f" row {i % 4}: {tok[i]} != {want[i]}"
           for i in range(len(want)) if tok[i] != want[i]]
    assert not bad, bad[:8]
    assert ((st & 1) == 0).all()
    ctx.close()


@pytest.mark.gpu
def test_gpu_history_order_duplicates_and_ids_past_the_row_match_the_oracle():
    torch, ctx = _gpu_ctx()
    base, hists = invariance_rows()
    rows, params, hs, seeds = [], [], [], []
    for s in SETTINGS:
        s = dict(s, presence=0.5, frequency=0.3, repetition=1.05)
        for seed in range(8):
            for h in hists:
                rows.append(base)
                params.append(s)
                hs.append(h)
                seeds.append(seed)
    tok, st = _gpu_sample(torch, ctx, np.stack(rows), params, hs, seeds)
    for i in range(0, len(params), len(hists)):
        want = oracle_pick(base, params[i], hs[i], seeds[i])
        assert list(tok[i:i + len(hists)]) == [want] * len(hists), (params[i], seeds[i], tok[i:i + len(hists)], want)
    ctx.close()

"""The oracle sampler pinned by the reference's own sampler tests (crates/engine/src/sample.rs:398-1086),
restated case for case, plus brute-force checks of this build's history penalties."""
import math

import numpy as np
import pytest

from oracle_lib import (DEFAULT, GREEDY, PLAIN, Rng, Sampler, argmax_row, check, first_non_finite,
                        greedy, host_exp, host_log, logprobs, takes_one_pass)

F32 = np.float32


def logits_of(p):
    # sample.rs:424-426: (x.ln() as f32).
    return np.array([F32(math.log(x)) for x in p], dtype=np.float32)


def frequencies(s, seed, logits, n):
    smp = Sampler(seed, **s)
    count = np.zeros(len(logits))
    for _ in range(n):
        count[smp.sample(logits)] += 1
    return count / n


def drawn(s, logits, n):
    f = frequencies(s, 7, logits, n)
    return [i for i in range(len(f)) if f[i] > 0]


def near(got, want):
    for g, w in zip(got, want):
        assert abs(g - w) < 0.02, (got, want)


def with_(base, **kw):
    d = dict(base)
    d.update(kw)
    return d


def random_logits(rng, n, coarse):
    # sample.rs:635-646: rng.unit() as f32 * 12 - 6 in f32; coarse rounds x*2 half away from zero.
    out = np.empty(n, np.float32)
    for i in range(n):
        x = F32(rng.unit()) * F32(12.0) - F32(6.0)
        if coarse:
            y = x * F32(2.0)
            r = math.copysign(math.floor(abs(float(y)) + 0.5), float(y))
            x = F32(r) / F32(2.0)
        out[i] = x
    return out


def test_the_argmax_twin_equals_greedy_on_finite_rows():
    rng = Rng(40)
    for r in range(1000):
        n = 1 + rng.below(600)
        row = np.array([F32(rng.unit() * 8.0 - 4.0) for _ in range(n)], np.float32)
        if r % 3 == 0 and n > 2:
            m = row.max()
            row[n - 1] = m
            row[n // 2] = m
        assert argmax_row(row) == greedy(row), r


def test_argmax_skips_nan_and_ties_to_the_lower_id():
    # kernels/tests/twins.rs:663-680.
    nan, inf = float("nan"), float("inf")
    assert argmax_row([1.0, nan, 3.0, 3.0]) == 2
    assert argmax_row([nan, 1.0]) == 1
    assert argmax_row([nan] * 5) is None
    assert argmax_row(np.zeros(0, np.float32)) is None
    assert argmax_row([-inf] * 4) is None
    assert argmax_row([-inf, 2.0, inf, nan]) == 1
    assert argmax_row([inf, -inf]) is None
    assert argmax_row([-inf, -3.4028235e38]) == 1


def test_greedy_takes_the_lower_id_on_a_tie():
    assert greedy([0.5, 2.0, -1.0, 2.0]) == 1
    assert greedy([3.0]) == 0
    # A NaN at index 0 wins; elsewhere it never does (sample.rs:7-8).
    assert greedy([float("nan"), 1.0, 2.0]) == 0
    assert greedy([1.0, float("nan"), 2.0]) == 2


def test_default_settings_are_productions():
    assert check(**DEFAULT) is None and check(**GREEDY) is None


def test_zero_temperature_is_greedy_whatever_the_filters():
    s = dict(temp=0.0, top_k=2, top_p=0.1, min_p=0.9, presence=0.0)
    for seed in range(20):
        assert Sampler(seed, **s).sample([0.1, 3.0, 3.0, -1.0]) == 1


def test_top_k_one_always_picks_the_argmax():
    assert drawn(with_(PLAIN, temp=1.5, top_k=1), [1.0, 2.0, 1.9, 0.0], 1000) == [1]


def test_top_k_keeps_the_k_highest_with_ties_to_the_lower_id():
    assert drawn(with_(PLAIN, top_k=2), [1.0, 2.0, 2.0, 2.0, 0.5], 2000) == [1, 2]


def test_top_k_beyond_the_vocabulary_keeps_everything():
    near(frequencies(with_(PLAIN, top_k=1000), 3, logits_of([0.5, 0.25, 0.25]), 20000), [0.5, 0.25, 0.25])


def test_top_p_keeps_the_shortest_prefix_reaching_p():
    l = logits_of([0.5, 0.3, 0.15, 0.05])
    for p, want in [(0.49, [0]), (0.79, [0, 1]), (0.81, [0, 1, 2]), (1.0, [0, 1, 2, 3])]:
        assert drawn(with_(PLAIN, top_p=p), l, 4000) == want, p


def test_min_p_drops_tokens_below_its_share_of_the_top():
    l = logits_of([0.5, 0.3, 0.15, 0.05])
    assert drawn(with_(PLAIN, min_p=0.2), l, 4000) == [0, 1, 2]
    assert drawn(with_(PLAIN, min_p=0.61), l, 4000) == [0]


def test_presence_penalty_moves_a_seen_token_down():
    l = [1.0, 0.9, 0.0]

    def greedy_with(pen):
        s = Sampler(0, **with_(GREEDY, presence=pen))
        return [s.sample(l), s.sample(l), s.sample(l)]

    assert greedy_with(0.5) == [0, 1, 0]
    assert greedy_with(0.0) == [0, 0, 0]


def test_the_same_seed_gives_the_same_tokens():
    l = np.array([((i * 7919) % 1000) / 100.0 for i in range(1000)], np.float32)

    def run(seed):
        s = Sampler(seed, **DEFAULT)
        return [s.sample(l) for _ in range(200)]

    assert run(42) == run(42)
    assert run(42) != run(43)


def test_draws_follow_the_distribution():
    near(frequencies(PLAIN, 1, logits_of([0.5, 0.25, 0.25]), 20000), [0.5, 0.25, 0.25])


def test_temperature_reshapes_the_distribution():
    near(frequencies(with_(PLAIN, temp=0.5), 2, logits_of([2 / 3, 1 / 3]), 20000), [0.8, 0.2])


def test_check_refuses_settings_it_cant_honour():
    nan, inf = float("nan"), float("inf")
    bad = [
        (dict(temp=-0.1), "--temp"), (dict(temp=nan), "--temp"), (dict(temp=inf), "--temp"),
        (dict(top_p=0.0), "--top-p"), (dict(top_p=1.1), "--top-p"), (dict(top_p=nan), "--top-p"),
        (dict(min_p=-0.1), "--min-p"), (dict(min_p=1.5), "--min-p"),
        (dict(presence=nan), "--presence-penalty"), (dict(presence=-inf), "--presence-penalty"),
        # This build's two new penalties.
        (dict(frequency=nan), "--frequency-penalty"), (dict(repetition=0.0), "--repetition-penalty"),
        (dict(repetition=inf), "--repetition-penalty"),
    ]
    for kw, flag in bad:
        m = check(**with_(PLAIN, **kw))
        assert m is not None and m.startswith(flag) and "\n" not in m, (kw, m)


def candidates(l):
    return np.arange(len(l), dtype=np.uint32), np.asarray(l, np.float32)


def test_the_partial_draw_matches_the_full_sort():
    gen = Rng(99)
    cases = 0
    for n in [1, 2, 5, 63, 64, 65, 300, 5000]:
        for coarse in [False, True]:
            l = random_logits(gen, n, coarse)
            ids, vals = candidates(l)
            for temp in [0.6, 1.0, 5.0, 1e-6]:
                for top_p in [1.0, 0.95, 0.5, 0.99999]:
                    for min_p in [0.0, 0.05, 1.0]:
                        s = dict(temp=temp, top_k=0, top_p=top_p, min_p=min_p, presence=0.0)
                        for seed in range(6):
                            a, b = Sampler(seed, **s), Sampler(seed, **s)
                            for step in range(4):
                                assert b.draw_partial(ids, vals) == a.draw_full_sort(ids, vals), (
                                    n, coarse, s, seed, step)
                                cases += 1
    assert cases > 10000


def hand_penalized(l, seen, pen):
    h = np.array(l, np.float32)
    if pen != 0.0:
        for t in seen:
            if t < len(h):
                h[t] = F32(h[t]) - F32(pen)
    return h


def reference(a, l, seen):
    # sample.rs:692-702: every candidate, penalised, through draw_full_sort; the token joins `seen`.
    ids, vals = candidates(hand_penalized(l, seen, a.p.presence))
    t = a.draw_full_sort(ids, vals)
    a.add_history([t])
    seen.add(t)
    return t


def test_the_one_pass_top_k_draws_the_selections_tokens():
    gen = Rng(31)
    cases = 0
    for n in [2, 3, 50, 5000]:
        for shape in range(3):
            l = random_logits(gen, n, shape == 1)
            if shape == 2:
                for i in range(n):
                    if i % 3 == 0:
                        l[i] = 0.0 if i % 2 == 0 else -0.0
                    else:
                        l[i] = -abs(l[i]) - F32(0.5)
            ks = sorted(set(k for k in [1, 2, 9, 10, 20, 300, n - 1] if k < n), key=[1, 2, 9, 10, 20, 300, n - 1].index)
            for k in ks:
                for pen in [0.0, 1.5]:
                    s = dict(temp=0.6, top_k=k, top_p=0.95, min_p=0.0, presence=pen)
                    for seed in range(3):
                        a, b = Sampler(seed, **s), Sampler(seed, **s)
                        seen = set()
                        for step in range(6):
                            if takes_one_pass(k, n):
                                assert b.top_k(l, k) == b.selected(l, k), (n, shape, k, pen, seed, step)
                            want = reference(a, l, seen)
                            assert b.sample(l) == want, (n, shape, k, pen, seed, step)
                            cases += 1
    assert cases > 1000
    assert drawn(with_(PLAIN, top_k=5), np.ones(300, np.float32), 400) == [0, 1, 2, 3, 4]
    s = Sampler(0, **PLAIN)
    pz = np.float32(0.0).view(np.uint32).item()
    assert s.top_k([0.0, -0.0, 0.0, 1.0], 3) == [(3, np.float32(1.0).view(np.uint32).item()), (0, pz), (2, pz)]
    assert s.top_k([-0.0, 0.0], 1)[0][0] == 1
    assert takes_one_pass(1, 2) and takes_one_pass(20, 248320) and takes_one_pass(256, 248320)
    assert not takes_one_pass(0, 100) and not takes_one_pass(257, 248320) and not takes_one_pass(5, 5)
    assert not takes_one_pass(6, 5) and not takes_one_pass(1000, 248320)


def test_the_top_k_over_a_whole_vocabulary_keeps_ties_and_penalized_ids_in_low_runs():
    N = 248320
    gen = Rng(77)
    u = np.array([gen.unit() for _ in range(N)])
    base = u.astype(np.float32) * F32(4.0) - F32(8.0)
    cases = 0
    for plant in range(5):
        l = base.copy()
        if plant == 0:
            for i in range(20):
                l[i * 7] = F32(10.0) - F32(i) * F32(0.25)
            for i in [1024, 1087, 1151, 200000, N - 1]:
                l[i] = F32(10.0) - F32(19.0) * F32(0.25)
        elif plant == 1:
            for j, i in enumerate([63, 64, 127, 128, 4095, 4096, N - 2, N - 1]):
                l[i] = F32(12.0 - j)
        elif plant == 2:
            for i in range(0, N, 9973):
                l[i] = 0.0 if i % 2 == 0 else -0.0
        elif plant == 3:
            l[:] = 1.5
        else:
            for i in range(0, N, 1009):
                l[i] = F32(5.0) + F32(gen.unit())
        for k in [1, 2, 20, 256]:
            for pen in [0.0, 1.5, -6.0]:
                s = dict(temp=0.6, top_k=k, top_p=0.95, min_p=0.0, presence=pen)
                a, b = Sampler(3, **s), Sampler(3, **s)
                seen = {5, 640, 100003, N - 1}
                a.add_history(sorted(seen))
                b.add_history(sorted(seen))
                for step in range(4):
                    assert b.top_k(l, k) == b.selected(l, k), (plant, k, pen, step)
                    want = reference(a, l, seen)
                    assert b.sample(l) == want, (plant, k, pen, step)
                    cases += 1
    assert cases == 5 * 4 * 3 * 4
    s = Sampler(0, **with_(PLAIN, presence=-6.0))
    s.add_history([100003])
    assert s.top_k(base, 1)[0][0] == 100003


def test_the_top_k_reads_a_short_tail_run():
    N = 64 * 3 + 17
    for k in [1, 2, 5, 20]:
        for tail_value in [3.0, 2.0]:
            l = np.array([F32(-10.0) - F32(i % 7) * F32(0.5) for i in range(N)], np.float32)
            for j in range(k - 1):
                l[j] = F32(10.0) - F32(j) * F32(0.1)
            l[N - 5] = tail_value
            l[100] = 2.0
            s = Sampler(0, **PLAIN)
            assert s.top_k(l, k) == s.selected(l, k), (k, tail_value)
            assert s.top_k(l, k)[-1][0] == (N - 5 if tail_value == 3.0 else 100)
            p = Sampler(0, **with_(PLAIN, presence=-30.0))
            p.add_history([N - 1])
            assert p.top_k(l, k) == p.selected(l, k), (k, "penalty on the last id")
    l = np.full(N, -1.0, np.float32)
    l[N - 1] = 1.0
    assert Sampler(0, **PLAIN).top_k(l, 1) == [(N - 1, np.float32(1.0).view(np.uint32).item())]


def test_the_top_k_agrees_with_the_plain_scan_on_nan_and_infinite_logits():
    nan, inf = float("nan"), float("inf")
    n = 64 * 4 + 9
    specials = [
        [(65, nan)], [(130, inf)], [(10, -inf), (200, -inf)], [(0, inf), (1, -inf)],
        [(255, nan), (257, inf)], [(n - 1, nan)], [(i, -inf) for i in range(n)],
    ]
    for k in [1, 2, 3, 20]:
        for sp in specials:
            l = np.array([F32(-5.0) - F32(i % 11) * F32(0.25) for i in range(n)], np.float32)
            for i, v in sp:
                l[i] = v
            for pen, seen in [(0.0, []), (1.5, [3, 70, 200]), (-4.0, [3, 70, 200])]:
                s = Sampler(0, **with_(PLAIN, presence=pen))
                s.add_history(seen)
                assert s.top_k(l, k) == s.selected(l, k), (sp[:2], k, pen)


def test_the_first_non_finite_logit_is_found_wherever_it_is():
    l = np.ones(248320, np.float32)
    assert first_non_finite(l) is None
    l[0] = np.finfo(np.float32).max
    l[1] = np.finfo(np.float32).min
    assert first_non_finite(l) is None
    n = len(l)
    for at, bad in [(0, np.nan), (1023, np.inf), (1024, -np.inf), (1025, np.nan), (n - 1, -np.inf)]:
        r = l.copy()
        r[at] = bad
        i, v = first_non_finite(r)
        assert i == at and np.float32(v).view(np.uint32) == np.float32(bad).view(np.uint32)
    r = l.copy()
    r[200000] = np.nan
    r[70000] = np.inf
    assert first_non_finite(r)[0] == 70000
    assert first_non_finite([2.0, np.nan, 3.0])[0] == 1
    assert first_non_finite(np.zeros(0, np.float32)) is None


def test_an_unfiltered_draw_reaches_deep_into_the_order():
    l = np.zeros(1000, np.float32)
    smp = Sampler(5, **with_(PLAIN, temp=1.0))
    assert max(smp.sample(l) for _ in range(200)) > 500


def test_min_p_of_one_keeps_only_the_top_and_its_ties():
    s = with_(PLAIN, min_p=1.0)
    assert drawn(s, [1.0, 3.0, 2.0, 3.0], 500) == [1, 3]
    big = np.array([(i % 50) * F32(0.1) for i in range(1000)], np.float32)
    big = (np.arange(1000) % 50).astype(np.float32) * F32(0.1)
    assert all(i % 50 == 49 for i in drawn(s, big, 3000))


def test_a_tiny_temperature_is_greedy_in_effect():
    s = with_(PLAIN, temp=1e-6)
    assert drawn(s, [0.2, 1.5, 1.4, -3.0], 500) == [1]
    big = np.array([((i * 7919) % 2000) for i in range(2000)], np.float32) * F32(0.01)
    assert drawn(s, big, 200) == [greedy(big)]


def test_the_presence_penalty_acts_on_the_sampling_path_too():
    gen = Rng(4)
    base = random_logits(gen, 3000, False)
    for top_k in [0, 20]:
        pen = 0.7
        s = dict(temp=0.8, top_k=top_k, top_p=0.9, min_p=0.0, presence=pen)
        a = Sampler(3, **s)
        b = Sampler(3, **with_(s, presence=0.0))
        hand = base.copy()
        for step in range(60):
            got = a.sample(base)
            assert got == b.sample(hand), (top_k, step)
            hand[got] = base[got] - F32(pen)
    g = Sampler(0, **with_(GREEDY, presence=1.5))
    hand = base.copy()
    for _ in range(40):
        got = g.sample(base)
        assert got == greedy(hand)
        hand[got] = base[got] - F32(1.5)


# ---- logprobs.rs:54-108 ----------------------------------------------------------------------

def test_logprobs_are_a_log_softmax_of_the_raw_logits():
    l = [1.0, 3.0, 2.0, 3.0]
    lp, top = logprobs(l, 2, 3)
    lse = math.log(math.exp(1) + 2 * math.exp(3) + math.exp(2))
    assert abs(lp - (2.0 - lse)) < 1e-6
    assert [t[0] for t in top] == [1, 3, 2]
    assert abs(top[0][1] - (3.0 - lse)) < 1e-6


def test_logprobs_take_at_most_twenty_and_none_when_asked_for_none():
    l = [float(i % 37) for i in range(100)]
    top = logprobs(l, 5, 25)[1]
    assert len(top) == 20
    order = sorted(range(100), key=lambda i: (-l[i], i))
    assert [t[0] for t in top] == order[:20]
    assert logprobs(l, 5, 0)[1] == []
    assert len(logprobs([0.5, 0.25], 0, 20)[1]) == 2


def test_tied_logits_across_the_cut_off_keep_the_lower_ids():
    l = [2.0, 5.0, 9.0, 5.0, 5.0, 9.0, 5.0, 1.0, 5.0]
    assert [t[0] for t in logprobs(l, 0, 4)[1]] == [2, 5, 1, 3]
    assert [t[0] for t in logprobs(l, 0, 3)[1]] == [2, 5, 1]


def test_negative_and_positive_zero_tie_to_the_lower_id():
    assert [t[0] for t in logprobs([-1.0, -0.0, 0.0, -0.0, 0.0], 0, 4)[1]] == [1, 2, 3, 4]


def test_huge_logits_dont_overflow():
    lp, top = logprobs([1e30, 1e30 - 1.0, -1e30], 0, 2)
    assert math.isfinite(lp) and all(math.isfinite(t[1]) for t in top)


# ---- this build's history penalties ---------------------------------------------------------

def penalize_py(x, c, pres, freq, rep):
    """The penalty definition, restated independently in numpy f32 arithmetic."""
    x = F32(x)
    t = x
    if F32(rep) != F32(1.0):
        t = x / F32(rep) if x > 0 else x * F32(rep)
    d = F32(c) * F32(freq)
    d = d + F32(pres)
    return F32(t - d)


@pytest.mark.parametrize("top_k", [0, 20, 300])
def test_history_penalties_equal_a_hand_penalised_row(top_k):
    gen = Rng(12)
    base = random_logits(gen, 2000, False)
    hist = [gen.below(2000) for _ in range(300)] + [5, 5, 5, 7]
    counts = {}
    for t in hist:
        counts[t] = counts.get(t, 0) + 1
    for pres, freq, rep in [(0.5, 0.3, 1.05), (0.0, 0.0, 1.3), (0.0, 1.0, 1.0), (-2.0, 0.0, 0.9)]:
        s = dict(temp=0.7, top_k=top_k, top_p=0.9, min_p=0.05, presence=pres, frequency=freq,
                 repetition=rep)
        a = Sampler(9, **s)
        a.add_history(hist)
        b = Sampler(9, **with_(s, presence=0.0, frequency=0.0, repetition=1.0))
        c = dict(counts)
        for step in range(40):
            hand = base.copy()
            for t, n in c.items():
                hand[t] = penalize_py(base[t], n, pres, freq, rep)
            got = a.sample(base)
            assert got == b.sample(hand), (s, step)
            c[got] = c.get(got, 0) + 1


def test_history_penalties_reduce_to_the_reference_presence_penalty():
    # With repetition 1 and frequency 0 any history count gives x - presence, the reference's value.
    for x in [3.25, -1.5, 0.0, -0.0, 1e-30, 7.0]:
        for c in [1, 2, 17]:
            got = penalize_py(x, c, 0.5, 0.0, 1.0)
            assert np.float32(got).view(np.uint32) == np.float32(F32(x) - F32(0.5)).view(np.uint32)
    gen = Rng(5)
    base = random_logits(gen, 1000, False)
    a = Sampler(2, **with_(DEFAULT, presence=0.5))
    b = Sampler(2, **with_(DEFAULT, presence=0.5))
    b.add_history([3, 3, 3])  # a count of 3 for one id, 1 for the other
    a.add_history([3])
    for _ in range(50):
        assert a.sample(base) == b.sample(base)


def test_host_exp_and_log_are_the_libm_ones():
    assert host_exp(0.0) == 1.0 and host_exp(-math.inf) == 0.0
    assert host_log(1.0) == 0.0
    for x in [-1.0, -0.5, -20.0, -700.0, 0.25]:
        assert host_exp(x) == math.exp(x)

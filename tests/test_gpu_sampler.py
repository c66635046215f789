"""Parity of the HIP sampler with the CPU oracle on the GPU, through the C ABI.

Token ids, kept counts, RNG states and accepted-draft counts must be bit-exact; kept-set
probabilities within 1e-5 relative (the unfiltered fast path divides by a total that is itself
within ~1e-11 of the reference's, every other path by the same f64 value).
"""
import os

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

PROB_RTOL = 1e-5
VOCAB = 248_320


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=1024, max_vocab=VOCAB)
    yield c
    c.close()


def as_sampling(p):
    from artemis_amd import Sampling
    return Sampling(p["temp"], p["top_k"], p["top_p"], p["min_p"], p.get("presence", 0.0),
                    p.get("frequency", 0.0), p.get("repetition", 1.0))


def csr(histories, rows):
    hs = histories if histories is not None else [np.zeros(0, np.uint32)] * rows
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hs])
    ids = np.concatenate([np.asarray(h, np.uint32) for h in hs]) if off[-1] else np.zeros(0, np.uint32)
    return off, ids.astype(np.int32)


def gpu_batch(ctx, logits, params, seeds, histories=None, kept_cap=0, csr_arrays=True):
    """One as_sample call. Without histories the call still passes an (empty) CSR unless csr_arrays
    is False: a call with no history arrays at all whose rows are all greedy takes greedy_kernel."""
    from artemis_amd import states_tensor
    rows = len(params)
    dev = torch.device("cuda:0")
    lg = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).to(dev)
    if lg.dim() == 1:
        lg = lg.view(1, -1)
    stride = 0 if lg.shape[0] == 1 and rows > 1 else lg.stride(0)
    rng = states_tensor(seeds, dev)
    d_off = d_ids = None
    if csr_arrays or histories is not None:
        off, ids = csr(histories, rows)
        d_off, d_ids = torch.from_numpy(off).to(dev), torch.from_numpy(ids).to(dev)
    tok, st, kc, ki, kp = ctx.sample_batch(lg, [as_sampling(p) for p in params], rng, d_off, d_ids,
                                           kept_cap=kept_cap, row_stride=stride, n_vocab=lg.shape[1])
    torch.cuda.synchronize()
    return dict(tokens=tok.cpu().numpy().astype(np.uint32), status=st.cpu().numpy().astype(np.uint32),
                kept=kc.cpu().numpy().astype(np.uint32), kept_ids=ki.cpu().numpy().astype(np.uint32),
                kept_probs=kp.cpu().numpy(), rng=rng.cpu().numpy().view(np.uint64))


def gpu_batch_strided(ctx, padded, n, params, seeds):
    """One as_sample call without history arrays over rows of n values held in a wider row stride."""
    from artemis_amd import states_tensor
    dev = torch.device("cuda:0")
    lg = torch.from_numpy(np.ascontiguousarray(padded, np.float32)).to(dev)
    rng = states_tensor(seeds, dev)
    tok, st, kc, ki, kp = ctx.sample_batch(lg, [as_sampling(p) for p in params], rng,
                                           row_stride=lg.stride(0), n_vocab=n)
    torch.cuda.synchronize()
    return dict(tokens=tok.cpu().numpy().astype(np.uint32), status=st.cpu().numpy().astype(np.uint32),
                kept=kc.cpu().numpy().astype(np.uint32), kept_ids=ki.cpu().numpy().astype(np.uint32),
                kept_probs=kp.cpu().numpy(), rng=rng.cpu().numpy().view(np.uint64))


def oracle_rows(logits, params, seeds, histories=None, kept_cap=0):
    """Per row: a fresh oracle Sampler with the history, one draw; token, kept set, RNG state."""
    out = []
    lg = np.asarray(logits, np.float32)
    for r, p in enumerate(params):
        row = lg[0] if lg.ndim == 1 or lg.shape[0] == 1 else lg[r]
        row = lg if lg.ndim == 1 else row
        s = O.Sampler(seeds[r], **p)
        if histories is not None and len(histories[r]):
            s.add_history(histories[r])
        if O.first_non_finite(row) is not None:
            out.append(None)
            continue
        t = s.sample(row)
        ids, probs = s.last_kept(kept_cap if kept_cap else 1)
        out.append(dict(token=t, kept_ids=ids, kept_probs=probs, path=s.last_path(),
                        rng=s.rng_state(), n_kept=len(s.last_kept(1 << 30)[0])))
    return out


AS_ROW_KEPT_PARTIAL_BIT = 0x200


def check_rows(g, want, params, kept_cap=0, label=""):
    for r, w in enumerate(want):
        if w is None:
            assert g["status"][r] & 1, (label, r)
            continue
        assert g["status"][r] & 1 == 0, (label, r, g["status"][r])
        assert g["tokens"][r] == w["token"], (label, r, params[r], g["tokens"][r], w["token"], g["status"][r])
        assert list(g["rng"][r]) == w["rng"], (label, r, "rng")
        cuts = params[r]["top_p"] < 1 or params[r]["min_p"] > 0
        if params[r]["temp"] > 0 and g["status"][r] & AS_ROW_KEPT_PARTIAL_BIT:
            # Drawn past the sorted values with the kept set's size unknown: a lower bound (the header).
            assert g["kept"][r] <= w["n_kept"], (label, r, params[r], g["kept"][r], w["n_kept"])
        elif params[r]["temp"] > 0 and not (w["path"] == 4 and not cuts):
            assert g["kept"][r] == w["n_kept"], (label, r, params[r], g["kept"][r], w["n_kept"])
        if kept_cap and params[r]["temp"] > 0:
            m = min(kept_cap, len(w["kept_ids"]))
            assert (g["kept_ids"][r][:m] == w["kept_ids"][:m]).all(), (label, r)
            np.testing.assert_allclose(g["kept_probs"][r][:m], w["kept_probs"][:m], rtol=PROB_RTOL)


def test_gpu_exp_is_the_hosts(ctx):
    rng = np.random.default_rng(11)
    parts = [-rng.random(400000) * 40, -rng.random(200000) * 800, (rng.random(200000) - 0.5) * 4,
             -708 - rng.random(100000) * 40, rng.integers(0, 2**64, 100000, dtype=np.uint64).view(np.float64),
             np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 709.7, -745.2, -745.1, 1e-300, -1e-300])]
    x = np.concatenate(parts)
    want = O.exp_array(x)
    got = ctx.debug_exp(torch.from_numpy(x).cuda()).cpu().numpy()
    same = (got.view(np.uint64) == want.view(np.uint64)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), x[~same][:5]


def test_gpu_exp2f_is_within_the_sums_bound(ctx):
    # The scan's sums take 2 ulp per term for the hardware 2^x; it must stay within 1 over the
    # arguments the sums give it (x <= 0 down to the f32 normal range).
    rng = np.random.default_rng(12)
    x = np.concatenate([-(rng.random(2_000_000) * 126.0), -(rng.random(500_000) * 2.0),
                        np.array([0.0, -0.5, -1.0, -1e-30, -125.99, -126.0])]).astype(np.float32)
    y = ctx.debug_exp2f(torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    exact = np.exp2(x.astype(np.float64))
    ulp = np.spacing(exact.astype(np.float32)).astype(np.float64)
    err = np.abs(y - exact) / ulp
    assert err.max() <= 1.0, (err.max(), x[np.argmax(err)])


GRID = []
for temp in [0.0, 0.6, 1.0, 5.0, 1e-6]:
    for top_k in [0, 1, 2, 20, 300]:
        for top_p, min_p in [(1.0, 0.0), (0.95, 0.0), (0.5, 0.05), (0.99999, 0.0), (1.0, 1.0), (0.9, 0.001)]:
            GRID.append(dict(temp=temp, top_k=top_k, top_p=top_p, min_p=min_p))


def random_logits(rng, n, shape):
    x = (rng.random(n) * 12 - 6).astype(np.float32)
    if shape == 1:  # heavy ties
        x = np.round(x * 2) / 2
    elif shape == 2:  # signed zeros on top
        i = np.arange(n)
        x = np.where(i % 3 == 0, np.where(i % 2 == 0, 0.0, -0.0), -np.abs(x) - 0.5).astype(np.float32)
    return x.astype(np.float32)


@pytest.mark.parametrize("n", [1, 2, 5, 63, 64, 65, 300, 5000, 8193, 20000])
def test_small_rows_match_the_oracle(ctx, n):
    rng = np.random.default_rng(n)
    params, logits, seeds, hists = [], [], [], []
    for i, p in enumerate(GRID):
        shape = i % 3
        q = dict(p)
        if i % 4 == 1:
            q.update(presence=1.5)
        if i % 4 == 2:
            q.update(presence=0.5, frequency=0.3, repetition=1.05)
        params.append(q)
        logits.append(random_logits(rng, n, shape))
        seeds.append(i)
        hists.append(rng.integers(0, n, size=min(n, 17)).astype(np.uint32) if i % 4 else np.zeros(0, np.uint32))
    logits = np.stack(logits)
    g = gpu_batch(ctx, logits, params, seeds, hists, kept_cap=64)
    want = oracle_rows(logits, params, seeds, hists, kept_cap=64)
    check_rows(g, want, params, kept_cap=64, label=f"n={n}")
    if n >= 300:
        # Without kept lists rows past their candidates first try the histogram bins' decisions (top-k
        # 300 rows among them); in batches of 12 the idle workgroups share those passes.
        k300 = [i for i, p in enumerate(GRID) if p["top_k"] == 300 and p["temp"] in (0.6, 1.0)]
        drawn = [i for i, p in enumerate(GRID) if p["temp"] > 0]
        for sub in (k300, drawn):
            pr = [params[i] for i in sub]
            g = gpu_batch(ctx, logits[sub], pr, [seeds[i] for i in sub], [hists[i] for i in sub])
            check_rows(g, [want[i] for i in sub], pr, label=f"n={n}, no kept lists, {len(sub)} rows")


def test_nonfinite_rows_report_their_first_index_and_keep_the_stream(ctx):
    n = 20000
    rng = np.random.default_rng(3)
    rows = np.tile((rng.standard_normal(n) * 2.5).astype(np.float32), (6, 1))
    plants = [(0, np.nan), (1023, np.inf), (1024, -np.inf), (8191, np.nan), (n - 1, -np.inf)]
    for r, (i, v) in enumerate(plants):
        rows[r, i] = v
        if r == 3:
            rows[r, 15000] = np.nan  # two of them: the first is named
    params = [dict(temp=0.6, top_k=20, top_p=0.95, min_p=0.0)] * 6
    g = gpu_batch(ctx, rows, params, list(range(6)), kept_cap=0)
    for r, (i, _) in enumerate(plants):
        assert g["status"][r] == 1 and g["kept"][r] == i, (r, g["status"][r], g["kept"][r])
        assert list(g["rng"][r]) == O.Rng(r).state(), "a refused row draws nothing"
    assert g["status"][5] == 0


@pytest.mark.parametrize("n_rows", [1, 7, 300])
def test_greedy_calls_the_scan_finishes(ctx, n_rows):
    # A call whose rows are all greedy with no history arrays takes greedy_kernel and no finish kernel:
    # each row's last slice merges its slices (sample.rs:9-17, 22-34). Ties, non-finite plants, kept
    # lists, and calls of the other kind in between (their slices' shared words and the flagged-row
    # lists must stay clean); the same rows with an empty history take the scan and the finish.
    N = VOCAB
    gen = np.random.default_rng(50 + n_rows)
    rows = (np.round(gen.standard_normal((n_rows, N)) * 4) / 4).astype(np.float32)
    for r in range(n_rows):
        if r % 5 == 1:
            rows[r, gen.integers(N)] = np.nan
        if r % 5 == 2:
            rows[r, [N - 1, 3]] = [np.inf, -np.inf]
        if r % 5 == 3:
            rows[r, :] = -1.0  # all tied: the lowest index
    greedy = [dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0)] * n_rows
    mixed = [dict(temp=0.8, top_k=0, top_p=1.0, min_p=0.01)] * n_rows
    want = oracle_rows(rows, greedy, list(range(n_rows)), kept_cap=4)
    want_m = oracle_rows(rows, mixed, list(range(n_rows)))
    for rep in range(3):
        kc = 4 if rep == 1 else 0
        g = gpu_batch(ctx, rows, greedy, list(range(n_rows)), kept_cap=kc, csr_arrays=False)
        check_rows(g, want, greedy, kept_cap=kc, label=f"greedy {n_rows} rows, call {rep}")
        g = gpu_batch(ctx, rows, greedy, list(range(n_rows)), kept_cap=kc)
        check_rows(g, want, greedy, kept_cap=kc, label=f"greedy {n_rows} rows with an empty history, call {rep}")
        g = gpu_batch(ctx, rows, mixed, list(range(n_rows)), csr_arrays=rep != 0)
        check_rows(g, want_m, mixed, label=f"min-p {n_rows} rows after greedy, call {rep}")
    # Rows of one slice (the only slice is the last) and of a few, unaligned (odd widths) and aligned
    # with a ragged end (a 16-byte-aligned stride past the width).
    for n in (1, 7, 3000, 9000, 9001, 248_317):
        small = np.ascontiguousarray(rows[:, :n])
        small[0, n // 2] = small[0].max()  # a tie with an earlier maximum, or the maximum itself
        if n % 4:
            small[-1, n - 1] = small[-1].max() + 1.0  # the maximum in the ragged end
        want_s = oracle_rows(small, greedy, list(range(n_rows)))
        g = gpu_batch(ctx, small, greedy, list(range(n_rows)), csr_arrays=False)
        check_rows(g, want_s, greedy, label=f"greedy {n_rows} rows of {n}")
        if n % 4:
            pad = np.zeros((n_rows, n + 4 - n % 4), np.float32)
            pad[:, :n] = small
            g = gpu_batch_strided(ctx, pad, n, greedy, list(range(n_rows)))
            check_rows(g, want_s, greedy, label=f"greedy {n_rows} rows of {n} in a stride of {pad.shape[1]}")


def test_config1_greedy(ctx):
    from artemis_amd import workloads
    w = workloads.config1()
    for csr_arrays in (False, True):
        g = gpu_batch(ctx, w.logits, [dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0)], [0], csr_arrays=csr_arrays)
        assert g["tokens"][0] == O.greedy(w.logits[0])


def test_config2_thousand_seeds(ctx):
    from artemis_amd import workloads
    w = workloads.config2()
    params = [dict(temp=0.6, top_k=20, top_p=0.95, min_p=0.0)] * len(w.seeds)
    g = gpu_batch(ctx, w.logits, params, w.seeds, kept_cap=20)
    want = oracle_rows(w.logits, params, w.seeds, kept_cap=20)
    check_rows(g, want, params, kept_cap=20, label="config2")


def test_config3_penalised(ctx):
    from artemis_amd import workloads
    w = workloads.config3(draws=64)
    params = [dict(temp=0.7, top_k=40, top_p=0.9, min_p=0.05, presence=0.5, frequency=0.3, repetition=1.05)] * 64
    g = gpu_batch(ctx, w.logits, params, w.seeds, w.histories, kept_cap=40)
    want = oracle_rows(w.logits, params, w.seeds, w.histories, kept_cap=40)
    check_rows(g, want, params, kept_cap=40, label="config3")


def test_config5_batch(ctx):
    from artemis_amd import workloads
    w = workloads.config5()
    params = [dict(temp=p.temp, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p, presence=p.presence,
                   frequency=p.frequency, repetition=p.repetition) for p in w.params]
    g = gpu_batch(ctx, w.logits, params, w.seeds, w.histories)
    off, ids = w.hist_csr()
    want, rng = O.sample_rows(params, w.seeds, w.logits, off, ids, threads=8)
    bad = np.nonzero(g["tokens"] != want)[0]
    assert len(bad) == 0, [(int(r), params[r], int(g["tokens"][r]), int(want[r])) for r in bad[:5]]
    assert (g["rng"] == rng).all()


def test_draws_past_the_sorted_values_match_the_oracle(ctx):
    # A row whose kept set runs far past the values the finish kernel sorts (top-p keeps ~16,500
    # values, min-p's floor ~111,000), drawn under many seeds: most draws are settled from the sorted
    # values and a bound on the rest (the fast decision), some take S's sums, others the deep path;
    # every token and stream must be the oracle's. Also with only the floor cutting (no row total for
    # the fast decision: S's sums bound the tail), and with T > 1.
    from artemis_amd import AS_ROW_TAIL_PASS, workloads
    w = workloads.config5()
    r = 111
    base = w.params[r]
    row = np.ascontiguousarray(w.logits[r])
    hist = w.histories[r]
    params, seeds = [], []
    for variant in [dict(), dict(top_p=1.0), dict(temp=1.3, top_p=0.9)]:
        for s in range(48):
            p = dict(temp=base.temp, top_k=0, top_p=base.top_p, min_p=base.min_p, presence=base.presence,
                     frequency=base.frequency, repetition=base.repetition)
            p.update(variant)
            params.append(p)
            seeds.append(9000 + len(seeds))
    rows = len(params)
    g = gpu_batch(ctx, row, params, seeds, [hist] * rows)
    off, ids = csr([hist] * rows, rows)
    want, rng = O.sample_rows(params, seeds, row, off, ids, threads=8, shared=True)
    bad = np.nonzero(g["tokens"] != want)[0]
    assert len(bad) == 0, [(int(i), params[i], int(g["tokens"][i]), int(want[i]), int(g["status"][i])) for i in bad[:5]]
    assert (g["rng"] == rng).all()
    assert (g["status"][48:96] & AS_ROW_TAIL_PASS).any(), g["status"][48:96]


def test_tail_histogram_draws_match_the_oracle(ctx):
    # The finish kernel sums S for the first 16 flagged rows of a call and bins S by value;
    # the finish kernel places top-p's cut within one bin and draws past the sorted values from
    # those bounds when the fast decision (the sorted values and a bound on the rest) cannot.
    # Config 5's row 111 (top-p keeps ~16,500 values, min-p's floor ~111,000) under many seeds, 16
    # rows a call so that every row is flagged (and with T > 1, where the bins alone bound the kept
    # tail from below): tokens and streams must be the oracle's.
    from artemis_amd import AS_ROW_DEEP_PATH, AS_ROW_KEPT_PARTIAL, AS_ROW_TAIL_PASS, workloads
    w = workloads.config5()
    r = 111
    base = w.params[r]
    row = np.ascontiguousarray(w.logits[r])
    hist = w.histories[r]
    seen, deep = {}, {}
    for variant, batches in [(dict(), 8), (dict(temp=1.3), 2)]:
        key = tuple(sorted(variant.items()))
        seen[key] = deep[key] = 0
        for b in range(batches):
            params, seeds = [], []
            for s in range(16):
                p = dict(temp=base.temp, top_k=0, top_p=base.top_p, min_p=base.min_p, presence=base.presence,
                         frequency=base.frequency, repetition=base.repetition)
                p.update(variant)
                params.append(p)
                seeds.append(20000 + 16 * (b + 10 * len(variant)) + s)
            g = gpu_batch(ctx, row, params, seeds, [hist] * 16)
            off, ids = csr([hist] * 16, 16)
            want, rng = O.sample_rows(params, seeds, row, off, ids, threads=8, shared=True)
            bad = np.nonzero(g["tokens"] != want)[0]
            assert len(bad) == 0, [(int(i), params[i], int(g["tokens"][i]), int(want[i]), int(g["status"][i]))
                                   for i in bad[:5]]
            assert (g["rng"] == rng).all()
            st = g["status"]
            settled = ((st & (AS_ROW_TAIL_PASS | AS_ROW_KEPT_PARTIAL)) != 0) & ((st & AS_ROW_DEEP_PATH) == 0)
            seen[key] += int(settled.sum())
            deep[key] += int(((st & AS_ROW_DEEP_PATH) != 0).sum())
    # At the row's own T (0.36) every draw is settled past the sorted values, by the fast decision or
    # by S's sums and bins (the first bound alone once left about 1 in 20 to the deep path). At
    # T = 1.3 the draw usually lands past the sorted values, which only the deep path can take.
    assert seen[()] + deep[()] == 128, (seen, deep)
    assert deep[()] <= 3, deep


def test_more_flagged_rows_than_the_list_holds(ctx):
    # 32 rows that the scan flags for S's sums (config 5's row 111 under many seeds), no kept lists:
    # more than the 16 the list holds, so nothing is shared. Each row draws from its sorted values
    # when they settle the draw, else sums S in its own pass over the row. Tokens and streams must be
    # the oracle's, and no row may need the deep path.
    from artemis_amd import AS_ROW_DEEP_PATH, workloads
    w = workloads.config5()
    r = 111
    base = w.params[r]
    row = np.ascontiguousarray(w.logits[r])
    hist = w.histories[r]
    params = [dict(temp=base.temp, top_k=0, top_p=base.top_p, min_p=base.min_p, presence=base.presence,
                   frequency=base.frequency, repetition=base.repetition) for _ in range(32)]
    seeds = [31000 + s for s in range(32)]
    g = gpu_batch(ctx, row, params, seeds, [hist] * 32)
    off, ids = csr([hist] * 32, 32)
    want, rng = O.sample_rows(params, seeds, row, off, ids, threads=8, shared=True)
    bad = np.nonzero(g["tokens"] != want)[0]
    assert len(bad) == 0, [(int(i), int(g["tokens"][i]), int(want[i]), int(g["status"][i])) for i in bad[:5]]
    assert (g["rng"] == rng).all()
    st = g["status"]
    assert not ((st & AS_ROW_DEEP_PATH) != 0).any(), st


@pytest.mark.parametrize("n_rows", [12, 40])
def test_large_top_k_rows_match_the_oracle(ctx, n_rows):
    # Top-k rows whose k is past the slices' candidates (sample.rs:157-198 with k > 256) at the
    # model's vocabulary, without kept lists: the count cut, top-p's total over the k best, min-p's
    # floor and the draw are decided from the row's histogram bins where they can be. 12 rows share
    # the deep passes with idle workgroups, 40 take them alone. Logits: a spread like a model's,
    # heavy ties (the k-th best inside a tie run) and a narrow band with spread highs.
    from artemis_amd import AS_ROW_DEEP_PATH, AS_ROW_EXACT_PATH
    N = VOCAB
    gen = np.random.default_rng(900 + n_rows)
    ks = [257, 300, 1000, 10_000, 100_000, N - 2, N - 1]
    settings = [(1.0, 1.0, 0.0), (0.6, 0.95, 0.0), (1.0, 0.5, 0.05), (3.0, 1.0, 0.001), (0.7, 0.9, 0.02),
                (1.0, 0.99999, 0.0), (0.8, 1.0, 0.0)]
    params, logits, seeds, hists = [], [], [], []
    for r in range(n_rows):
        k = ks[r % len(ks)]
        t, tp, mp = settings[(r // len(ks) + 3 * r) % len(settings)]
        p = dict(temp=t, top_k=k, top_p=tp, min_p=mp)
        if r % 3 == 1:
            p.update(presence=1.5)
        elif r % 3 == 2:
            p.update(presence=0.5, frequency=0.3, repetition=1.05)
        shape = (r // 2) % 3
        if shape == 0:
            l = (gen.standard_normal(N) * 2.5).astype(np.float32)
        elif shape == 1:
            l = (np.round(gen.standard_normal(N) * 8) / 4).astype(np.float32)
        else:
            l = (gen.random(N) * 4 - 8).astype(np.float32)
            l[::1009] = 5.0 + gen.random(len(l[::1009])).astype(np.float32)
        params.append(p)
        logits.append(l)
        seeds.append(4100 + r)
        hists.append(gen.integers(0, N, size=40).astype(np.uint32) if r % 3 else np.zeros(0, np.uint32))
    logits = np.stack(logits)
    g = gpu_batch(ctx, logits, params, seeds, hists)
    want = oracle_rows(logits, params, seeds, hists)
    check_rows(g, want, params, label=f"large top-k, {n_rows} rows")
    # Every row is settled past the candidates; a top-p of 0.99999 over nearly the whole row may cut
    # where no bin's bounds decide, and goes on to the exact-order path.
    st = g["status"]
    assert ((st & (AS_ROW_DEEP_PATH | AS_ROW_EXACT_PATH)) != 0).all(), st
    assert all(st[r] & AS_ROW_DEEP_PATH for r in range(n_rows) if params[r]["top_p"] != 0.99999), st


def test_min_p_only_rows_past_their_candidates_match_the_oracle(ctx):
    # min-p 0.002 with no top-p and no top-k on config 5's logits (floor sets of thousands of values):
    # some draws land past every candidate, and those rows take the deep passes, which then leave
    # out every value below the floor (sample.rs:181, 237: nothing below it is kept or counted). 64
    # rows take the passes alone, 12 share them with idle workgroups.
    from artemis_amd import AS_ROW_DEEP_PATH, workloads
    w = workloads.config5()
    deep = 0
    for n_rows, base in [(64, 0), (64, 64), (12, 128)]:
        params = [dict(temp=0.7, top_k=0, top_p=1.0, min_p=0.002)] * n_rows
        rows = np.ascontiguousarray(w.logits[base:base + n_rows])
        seeds = [900 + base + r for r in range(n_rows)]
        g = gpu_batch(ctx, rows, params, seeds)
        want = oracle_rows(rows, params, seeds)
        check_rows(g, want, params, label=f"min-p only, rows {base}:{base + n_rows}")
        deep += int(((g["status"] & AS_ROW_DEEP_PATH) != 0).sum())
    assert deep > 0, "no row took the deep passes: the case is not covered"


def test_large_floor_sets_match_the_oracle(ctx):
    # min-p rows whose floor set holds thousands of values (config 5's rows 254 and 151: 4,302 and
    # 3,365 values above the floor, top-p far deeper): the scan keeps a few thousand candidates and
    # S's parts list the rest of the floor set, which the finish kernel sorts in. Tokens,
    # streams, kept counts and kept lists must be the oracle's, under many seeds.
    from artemis_amd import AS_ROW_TAIL_PASS, workloads
    w = workloads.config5()
    params, seeds, rows, hists = [], [], [], []
    for r in (254, 151):
        b = w.params[r]
        for s in range(32):
            params.append(dict(temp=b.temp, top_k=0, top_p=b.top_p, min_p=b.min_p, presence=b.presence,
                               frequency=b.frequency, repetition=b.repetition))
            seeds.append(7000 + len(seeds))
            rows.append(w.logits[r])
            hists.append(w.histories[r])
    rows = np.stack(rows)
    g = gpu_batch(ctx, rows, params, seeds, hists, kept_cap=16)
    want = oracle_rows(rows, params, seeds, hists, kept_cap=16)
    check_rows(g, want, params, kept_cap=16, label="floor sets")
    # S is summed in parts for the first 16 rows the scan flags (in the order it flags them); the finish
    # kernel settles the rest.
    assert ((g["status"] & AS_ROW_TAIL_PASS) != 0).sum() >= 16, g["status"]


def test_whole_vocabulary_plants(ctx):
    # sample.rs:807-885's plants at the model's vocabulary: ties with the k-th best in later runs,
    # penalised ids in low runs, top values on run edges, signed zeros, all equal, spread highs.
    N = VOCAB
    gen = np.random.default_rng(77)
    base = (gen.random(N).astype(np.float32) * 4 - 8).astype(np.float32)
    params, rows, hists, seeds = [], [], [], []
    for plant in range(5):
        l = base.copy()
        if plant == 0:
            for i in range(20):
                l[i * 7] = 10.0 - i * 0.25
            for i in [1024, 1087, 1151, 200000, N - 1]:
                l[i] = 10.0 - 19 * 0.25
        elif plant == 1:
            for j, i in enumerate([63, 64, 127, 128, 4095, 4096, N - 2, N - 1]):
                l[i] = 12.0 - j
        elif plant == 2:
            l[::9973] = 0.0
            l[9973::2 * 9973] = -0.0
        elif plant == 3:
            l[:] = 1.5
        else:
            l[::1009] = 5.0 + gen.random(len(l[::1009])).astype(np.float32)
        for k in [1, 2, 20, 256, 0, 1000]:
            for pen in [0.0, 1.5, -6.0]:
                params.append(dict(temp=0.6, top_k=k, top_p=0.95, min_p=0.0, presence=pen))
                rows.append(l)
                hists.append(np.array([5, 640, 100003, N - 1], np.uint32))
                seeds.append(3 + len(seeds))
    rows = np.stack(rows)
    g = gpu_batch(ctx, rows, params, seeds, hists, kept_cap=32)
    want = oracle_rows(rows, params, seeds, hists, kept_cap=32)
    check_rows(g, want, params, kept_cap=32, label="plants")


def test_argmax_rows_matches_its_twin(ctx):
    # kernels/tests/gpu_kernels.rs:1565-1618.
    gen = np.random.default_rng(41)
    embd, row_bytes = 0x3_0000_1000, 1 << 20
    for n in [512, VOCAB, 1001]:
        rows = (gen.random((6, n)) * 16 - 8).astype(np.float32)
        m = np.float32(9.0)
        for i in [n - 1, n // 2, 3, 3 + min(1024, n - 4)]:
            rows[1, i] = m
        rows[2, 0] = np.nan
        rows[2, n // 3] = np.nan
        rows[2, 7] = 8.5
        rows[3, 5] = np.inf
        rows[3, 9] = -np.inf
        rows[3, n - 2] = 8.25
        rows[4, :] = np.nan
        rows[5, :] = np.where(np.arange(n) % 2 == 0, np.inf, -np.inf)
        rows[0, n - 1] = rows[0].max()
        ids = torch.full((8,), 0x2AAAAAAA, dtype=torch.int32, device="cuda")
        out = torch.full((8,), 0x3BBBBBBB, dtype=torch.int64, device="cuda")
        ctx.argmax_rows(torch.from_numpy(rows).cuda(), ids, out, embd, row_bytes, slot=1)
        torch.cuda.synchronize()
        gi = ids.cpu().numpy().astype(np.uint32)
        go = out.cpu().numpy().view(np.uint64)
        for r in range(6):
            want = O.argmax_row(rows[r])
            assert gi[1 + r] == (0xFFFFFFFF if want is None else want), (n, r)
            assert go[1 + r] == embd + (0 if want is None else want) * row_bytes, (n, r)
        assert gi[0] == 0x2AAAAAAA and gi[7] == 0x2AAAAAAA and go[0] == 0x3BBBBBBB and go[7] == 0x3BBBBBBB


def gpu_verify(ctx, rows, drafts, p, seed, history=(), stops=()):
    from artemis_amd import states_tensor
    dev = torch.device("cuda:0")
    rng = states_tensor([seed], dev)
    picks, result = ctx.verify(torch.from_numpy(np.ascontiguousarray(rows, np.float32)).to(dev),
                               torch.tensor(np.asarray(drafts, np.int64).astype(np.int32), device=dev),
                               as_sampling(p), rng,
                               torch.tensor(np.asarray(history, np.int64).astype(np.int32), device=dev) if len(history) else None,
                               torch.tensor(np.asarray(stops, np.int64).astype(np.int32), device=dev) if len(stops) else None)
    torch.cuda.synchronize()
    return picks.cpu().numpy().astype(np.uint32), result.cpu().numpy().astype(np.uint32), rng.cpu().numpy().view(np.uint64)[0]


def test_verify_matches_the_plain_loop(ctx):
    gen = np.random.default_rng(9)
    n = 3000
    cases = 0
    for p in [dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0), dict(temp=0.6, top_k=20, top_p=0.95, min_p=0.0),
              dict(temp=0.8, top_k=0, top_p=0.9, min_p=0.02, presence=0.5),
              dict(temp=0.7, top_k=40, top_p=0.9, min_p=0.05, presence=0.5, frequency=0.3, repetition=1.05)]:
        for k in [0, 1, 3, 5, 15]:
            for mode in range(3):
                rows = (gen.standard_normal((k + 1, n)) * 2.5).astype(np.float32)
                rows[np.arange(k + 1), gen.integers(n, size=k + 1)] += 6.0
                hist = gen.integers(0, n, size=30).astype(np.uint32)
                # Drafts: all equal to the plain loop's picks, half of them, or none.
                o = O.Sampler(77, **p)
                o.add_history(hist)
                truth = []
                for i in range(k + 1):
                    truth.append(o.sample(rows[i]))
                drafts = np.array(truth[:k], np.uint32)
                if mode == 1 and k:
                    drafts[k // 2] = (drafts[k // 2] + 1) % n
                if mode == 2 and k:
                    drafts[:] = (drafts + 7) % n
                stops = [int(truth[2])] if (mode == 0 and k >= 3) else []
                want = O.Sampler(77, **p)
                want.add_history(hist)
                wpicks, wacc, wstop = want.verify(rows, drafts, stops)
                picks, result, rng = gpu_verify(ctx, rows, drafts, p, 77, hist, stops)
                read = len(wpicks)
                assert result[0] == read and result[1] == wacc, (p, k, mode, result, wpicks)
                assert (picks[:read] == np.array(wpicks, np.uint32)).all(), (p, k, mode)
                assert result[2] == wpicks[-1] and bool(result[3] & 1) == wstop
                assert list(rng) == want.rng_state(), (p, k, mode, "rng")
                cases += 1
    assert cases == 60


def test_config4_verify(ctx):
    from artemis_amd import workloads
    w = workloads.config4()
    p = dict(temp=0.6, top_k=0, top_p=0.95, min_p=0.0)
    o = O.Sampler(w.seeds[0], **p)
    wpicks, wacc, _ = o.verify(w.logits, w.drafts)
    picks, result, rng = gpu_verify(ctx, w.logits, w.drafts, p, w.seeds[0])
    assert result[0] == len(wpicks) and result[1] == wacc
    assert (picks[: len(wpicks)] == np.array(wpicks, np.uint32)).all()
    assert list(rng) == o.rng_state()


def test_sampler_object_follows_the_reference_sequence(ctx):
    from artemis_amd import Sampler, Sampling
    # sample.rs:563-578: greedy with presence 0.5 over [1.0, 0.9, 0.0] gives [0, 1, 0].
    l = torch.tensor([1.0, 0.9, 0.0], device="cuda")
    s = Sampler(Sampling(0.0, 0, 1.0, 0.0, 0.5), 0)
    assert [s.sample(l), s.sample(l), s.sample(l)] == [0, 1, 0]
    # A run of draws with the history growing, against the oracle's Sampler.
    gen = np.random.default_rng(4)
    base = (gen.random(3000) * 12 - 6).astype(np.float32)
    for top_k in [0, 20]:
        p = dict(temp=0.8, top_k=top_k, top_p=0.9, min_p=0.0, presence=0.7)
        a = Sampler(as_sampling(p), 3)
        b = O.Sampler(3, **p)
        lt = torch.from_numpy(base).cuda()
        for step in range(30):
            assert a.sample(lt) == b.sample(base), (top_k, step)


GOLDEN_PATH = os.path.join(os.path.dirname(__file__), "golden", "configs.json")


@pytest.mark.parametrize("name", ["config2", "config3", "config5"])
def test_batches_match_the_committed_goldens(ctx, name):
    import hashlib
    import json
    from artemis_amd import workloads
    g = json.load(open(GOLDEN_PATH))[name]
    w = {"config2": workloads.config2, "config3": lambda: workloads.config3(draws=64),
         "config5": workloads.config5}[name]()
    assert w.sha256() == g["sha256"]
    rows = len(w.seeds)
    params = [g["params"]] * rows if isinstance(g["params"], dict) else g["params"]
    cap = 64
    out = gpu_batch(ctx, w.logits, params, w.seeds, w.histories or None, kept_cap=cap)
    assert out["tokens"].tolist() == g["tokens"], name
    assert hashlib.sha256(out["rng"].astype("<u8").tobytes()).hexdigest() == g["rng_sha256"], name
    for r, k in enumerate(g["kept"]):
        m = min(len(k["ids"]), cap)
        # With kept lists asked for, no row takes the partial shortcut (AS_ROW_KEPT_PARTIAL): every
        # row's count, ids and probabilities are the reference's.
        assert int(out["status"][r]) & 0x200 == 0, (name, r, hex(int(out["status"][r])))
        assert int(out["kept"][r]) == k["kept_count"], (name, r)
        assert out["kept_ids"][r][:m].tolist() == k["ids"][:m], (name, r)
        np.testing.assert_allclose(out["kept_probs"][r][:m], k["probs"][:m], rtol=PROB_RTOL)


def test_verify_and_greedy_match_the_committed_goldens(ctx):
    import json
    from artemis_amd import workloads
    gold = json.load(open(GOLDEN_PATH))
    g, w = gold["config4"], workloads.config4()
    picks, result, rng = gpu_verify(ctx, w.logits, w.drafts, g["params"], g["seed"])
    read = int(result[0])
    assert read == g["read"] and int(result[1]) == g["accepted"] and int(result[2]) == g["bonus"]
    assert picks[:read].tolist() == g["picks"]
    assert ["%016x" % int(x) for x in rng] == g["rng"]
    g1, w1 = gold["config1"], workloads.config1()
    out = gpu_batch(ctx, w1.logits, [dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0)], [0])
    assert int(out["tokens"][0]) == g1["greedy"]

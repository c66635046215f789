"""Log-probabilities on the GPU (crates/engine/src/logprobs.rs:12-38) against the oracle, which
restates the same function (oracle/sampler_oracle.cc, oc_logprobs). Top ids must be bit-exact. Values
must be bit-exact on rows whose status is AS_LP_OK. On a row marked AS_LP_INEXACT (the bound on the
parallel sum's distance to the reference's left-to-right sum could move a rounding to f32) each value
must be within the library's absolute bound of the oracle's: |lp - lp_ref| <= e + one f32 ulp, with
e = gamma(n + 64) + 1.5e-12 + 2^-51 |ln total| + 2^-52 |lse| (include/artemis_sampler.h), so exp(lp) is
within about 3e-11 relative of the reference's probability, far inside the 1e-5 the probabilities
must meet. Near-certain tokens (lp close to 0) are where that is many f32 ulps."""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

VOCAB = 248_320


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=64, max_vocab=VOCAB)
    yield c
    c.close()


def run(ctx, rows, tokens, top, row_stride=None, n_vocab=None):
    dev = torch.device("cuda:0")
    lg = torch.from_numpy(np.ascontiguousarray(rows, np.float32)).to(dev)
    if lg.dim() == 1:
        lg = lg.view(1, -1)
    tok = torch.from_numpy(np.asarray(tokens, np.int32)).to(dev)
    lp, ids, lps, st = ctx.logprobs(lg, tok, top, row_stride=row_stride, n_vocab=n_vocab)
    torch.cuda.synchronize()
    return lp.cpu().numpy(), ids.cpu().numpy(), lps.cpu().numpy(), st.cpu().numpy()


U = 2.0 ** -53


def lse_bound(row, lse):
    """The library's bound e on |lse - lse_ref| for a row (include/artemis_sampler.h)."""
    n = len(row)
    g = (n + 64) * U / (1 - (n + 64) * U)
    ln_total = lse - float(np.max(row))
    return g + 1.5e-12 + 4 * U * abs(ln_total) + 2 * U * abs(lse)


def same_or_within(got, want, exact, e):
    """Bit-exact on an AS_LP_OK row; otherwise within the header's bound e + 2^-51 |lp| + one f32 ulp
    (2^-51 |lp| = 4 U |lp| covers the two f64 differences x - lse, ours and the reference's)."""
    got, want = np.float32(got), np.float32(want)
    if exact:
        return got.tobytes() == want.tobytes()
    slack = e + 4 * U * abs(float(want)) + float(np.spacing(np.abs(want)))
    return abs(float(got) - float(want)) <= slack


def check(ctx, rows, tokens, top, label=""):
    from artemis_amd import AS_LP_INEXACT
    rows = np.atleast_2d(np.asarray(rows, np.float32))
    lp, ids, lps, st = run(ctx, rows, tokens, top)
    inexact = 0
    for r in range(rows.shape[0]):
        want_lp, want_top = O.logprobs(rows[r], int(tokens[r]), top)
        exact = st[r] & AS_LP_INEXACT == 0
        inexact += 0 if exact else 1
        e = lse_bound(rows[r], float(rows[r][int(tokens[r])]) - float(want_lp))
        assert same_or_within(lp[r], want_lp, exact, e), (label, r, lp[r], want_lp, st[r])
        n = len(want_top)
        assert n == min(top, 20, rows.shape[1])
        assert ids[r][:n].tolist() == [i for i, _ in want_top], (label, r, ids[r][:n].tolist(), want_top)
        for j in range(n):
            assert same_or_within(lps[r][j], want_top[j][1], exact, e), (label, r, j, lps[r][j], want_top[j])
    return lp, ids, lps, st, inexact


# ---- logprobs.rs:54-108, the reference's own tests ------------------------------------------------

def test_logprobs_are_a_log_softmax_of_the_raw_logits(ctx):
    l = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    lp, ids, lps, st, _ = check(ctx, l, [2], 3)
    lse = np.log(np.exp(1.0) + 2 * np.exp(3.0) + np.exp(2.0))
    assert abs(float(lp[0]) - (2.0 - lse)) < 1e-6
    assert ids[0][:3].tolist() == [1, 3, 2]  # a tie goes to the lower id
    assert abs(float(lps[0][0]) - (3.0 - lse)) < 1e-6


def test_logprobs_take_at_most_twenty_and_none_when_asked_for_none(ctx):
    l = np.array([i % 37 for i in range(100)], np.float32)
    _, ids, _, _, _ = check(ctx, l, [5], 25)
    full = sorted(range(100), key=lambda i: (-l[i], i))
    assert ids[0][:20].tolist() == full[:20]
    lp, ids0, _, _, _ = check(ctx, l, [5], 0)
    check(ctx, np.array([0.5, 0.25], np.float32), [0], 20)


def test_tied_logits_across_the_cut_off_keep_the_lower_ids(ctx):
    l = np.array([2.0, 5.0, 9.0, 5.0, 5.0, 9.0, 5.0, 1.0, 5.0], np.float32)
    assert check(ctx, l, [0], 4)[1][0][:4].tolist() == [2, 5, 1, 3]
    assert check(ctx, l, [0], 3)[1][0][:3].tolist() == [2, 5, 1]


def test_negative_and_positive_zero_tie_to_the_lower_id(ctx):
    l = np.array([-1.0, -0.0, 0.0, -0.0, 0.0], np.float32)
    assert check(ctx, l, [0], 4)[1][0][:4].tolist() == [1, 2, 3, 4]


def test_huge_logits_dont_overflow(ctx):
    l = np.array([1e30, 1e30 - 1.0, -1e30], np.float32)
    lp, _, lps, _, _ = check(ctx, l, [0], 2)
    assert np.isfinite(lp[0]) and np.isfinite(lps[0][:2]).all()


# ---- the model's width ---------------------------------------------------------------------------

def test_config5_rows_match_the_oracle(ctx):
    # Config 5's rows at the model's width, each at a token from its own sampled distribution's range
    # (a top id, a middle one and the row's minimum).
    from artemis_amd import workloads
    w = workloads.config5(rows=16)
    rows = w.logits
    tokens = []
    for r in range(rows.shape[0]):
        order = np.argsort(-rows[r], kind="stable")
        tokens.append(int(order[[0, 1000, -1][r % 3]]))
    _, _, _, _, inexact = check(ctx, rows, tokens, 20, "config5")
    assert inexact <= 2, inexact


def test_batches_past_one_round_take_the_wide_parts(ctx):
    # A call whose 8,192-value parts would not fit one round of the chip's workgroups takes parts of
    # 16,384 values: 64 aligned rows at the model's width (the last part partial), and 58 rows of an
    # odd width (no 16-byte loads), each against the oracle.
    from artemis_amd import workloads
    gen = np.random.default_rng(43)
    rows = workloads.config5(rows=64).logits
    tokens = gen.integers(0, rows.shape[1], size=rows.shape[0])
    _, _, _, _, inexact = check(ctx, rows, tokens, 20, "wide parts")
    assert inexact <= 2, inexact
    rows = (gen.standard_normal((58, VOCAB - 1)) * 3.0).astype(np.float32)
    rows[7, 1000] = 40.0
    check(ctx, rows, gen.integers(0, VOCAB - 1, size=58), 20, "wide parts, odd width")


def test_both_sides_of_the_part_layout_switch():
    # 179 rows of 81,920 values make 1,790 parts of 8,192 (one round of the chip's workgroups: that
    # layout), 180 rows 1,800 (past it: parts of 16,384); the rows the two calls share must agree,
    # and every row must match the oracle.
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    gen = np.random.default_rng(47)
    n = 81_920
    rows = (gen.standard_normal((180, n)) * 2.5).astype(np.float32)
    rows[5, 100] = 30.0
    tokens = gen.integers(0, n, size=180)
    c = Context(max_rows=180, max_vocab=n)
    try:
        small = check(c, rows[:179], tokens[:179], 20, "8,192-value parts")
        wide = check(c, rows, tokens, 20, "16,384-value parts")
    finally:
        c.close()
    assert (small[1] == wide[1][:179]).all()


def test_ragged_widths_and_tops(ctx):
    gen = np.random.default_rng(11)
    for n in [1, 2, 5, 63, 8191, 8192, 8193, 20000, 100003]:
        rows = (gen.standard_normal((3, n)) * 2.5).astype(np.float32)
        tokens = gen.integers(0, n, size=3)
        for top in [0, 1, 5, 20, 25]:
            check(ctx, rows, tokens, top, f"n={n} top={top}")


def test_heavy_ties(ctx):
    # Ties across the parts' lists: every value equal (a part's list overflows and the row takes its
    # best by full passes), and 3,000 copies of the maximum spread over the row.
    n = 30000
    same = np.full(n, 1.5, np.float32)
    spread = (np.random.default_rng(5).standard_normal(n) * 2.0).astype(np.float32)
    spread[np.random.default_rng(6).choice(n, 3000, replace=False)] = 9.0
    check(ctx, np.stack([same, spread]), [7, 11], 20, "ties")


def test_wide_ranges_within_a_wave(ctx):
    # Values spanning far more than exp's range inside one wave's share of a part: a masked stretch
    # over every wave's first 16-byte groups (each wave's sum starts from those and must start again
    # from its largest value), masked values between ordinary ones, single huge values, and a masked
    # half row; at a width whose last part is partial and at the model's.
    gen = np.random.default_rng(41)
    for n in [20000, VOCAB]:
        rows = (gen.standard_normal((4, n)) * 2.5).astype(np.float32)
        rows[0, :1024] = -1e4
        rows[0, n - 1000:] = -1e4
        rows[1, ::7] = -1e30
        rows[2, 5000] = 1e4
        rows[2, n - 3] = 3e4
        rows[3, : n // 2] = -3e38
        check(ctx, rows, [1, 8, 5000, n - 1], 20, f"wide n={n}")


def test_parts_on_both_sides_of_the_fused_argument(ctx):
    # A part whose maximum m has |m| <= 256 takes each term's argument as one fused multiply-add
    # (exp_poly.h, exp_fused); a larger |m| subtracts first (exp_sat). Rows whose parts sit at and just
    # past that edge, on both signs, with values spread over exp's whole range below m.
    gen = np.random.default_rng(43)
    n = 40000
    for m in [256.0, -256.0, 256.03125, -256.03125, 300.0, -300.0, 255.5]:
        rows = np.empty((3, n), np.float32)
        rows[0] = m - np.abs(gen.standard_normal(n)) * 3.0
        rows[1] = m - gen.random(n).astype(np.float32) * 800.0
        rows[2] = m - np.abs(gen.standard_normal(n)) * 0.01
        for r in range(3):
            rows[r, gen.integers(0, n)] = m
        check(ctx, rows, [0, 17, n - 1], 20, f"m={m}")


def test_strided_and_shared_rows(ctx):
    # A padded row stride, and stride 0 (every row reads the same row).
    gen = np.random.default_rng(3)
    n, stride = 10000, 10240
    buf = (gen.standard_normal((2, stride)) * 2.5).astype(np.float32)
    lp, ids, lps, st = run(ctx, buf, [4, 9], 20, row_stride=stride, n_vocab=n)
    for r in range(2):
        want_lp, want_top = O.logprobs(buf[r, :n], [4, 9][r], 20)
        assert ids[r][:20].tolist() == [i for i, _ in want_top]
        e = lse_bound(buf[r, :n], float(buf[r, [4, 9][r]]) - float(want_lp))
        assert same_or_within(lp[r], want_lp, st[r] == 0, e)
    lp, ids, lps, st = run(ctx, buf[0], [1, 2, 3], 20, row_stride=0, n_vocab=n)
    want_top = O.logprobs(buf[0, :n], 1, 20)[1]
    for r in range(3):
        assert ids[r][:20].tolist() == [i for i, _ in want_top]


def test_near_certain_tokens_at_the_models_width(ctx):
    # One logit 30-40 above an N(0, 3) row: the reference's left-to-right sum loses every term under
    # half an ulp of 1.0 that comes after the peak, the parallel sum keeps them; the values differ by
    # many f32 ulps near lp = 0 and stay within the absolute bound.
    gen = np.random.default_rng(31)
    rows = (gen.standard_normal((6, VOCAB)) * 3.0).astype(np.float32)
    peaks = [0, 1000, 124_160, 200_000, VOCAB - 2, 77]
    for r, (p, lift) in enumerate(zip(peaks, [30.0, 32.0, 34.0, 36.0, 38.0, 40.0])):
        rows[r, p] = np.float32(rows[r].max() + lift)
    tokens = np.array(peaks, np.int32)
    lp, ids, lps, st, inexact = check(ctx, rows, tokens, 20, "peaked")
    assert (ids[:, 0] == np.array(peaks)).all()
    assert (lp <= 0).all() and (lp > -1e-6).all()

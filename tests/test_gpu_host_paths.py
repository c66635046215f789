"""Host-side paths of as_sample on the GPU, each checked against the oracle through the C ABI:

- back-to-back calls with different settings and no host synchronisation between them, which
  exercises the two pinned parameter blocks the calls alternate between (a call reuses a block only
  once the call two before it has finished reading it);
- histories with more distinct ids per slice than the scan's LDS hash counts (512), which send the
  row to the finish kernel's passes over the whole row (the deep path, then the exact-order path);
- small batches whose rows take the deep path with its passes shared among the finish kernel's
  idle workgroups, alone and alternating with larger batches on one context.
"""
import numpy as np
import pytest

from test_gpu_sampler import GRID, check_rows, csr, oracle_rows, random_logits

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

AS_ROW_EXACT_PATH = 0x100
AS_ROW_DEEP_PATH = 0x400


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=64, max_vocab=248_320, max_history=65_535)
    yield c
    c.close()


def settings(p):
    from artemis_amd import Sampling
    return Sampling(p["temp"], p["top_k"], p["top_p"], p["min_p"], p.get("presence", 0.0),
                    p.get("frequency", 0.0), p.get("repetition", 1.0))


def test_back_to_back_calls_with_different_settings(ctx):
    from artemis_amd import states_tensor
    dev = torch.device("cuda:0")
    rows, n, calls = 16, 20_000, 50
    rng = np.random.default_rng(11)
    logits = np.stack([random_logits(rng, n, i % 3) for i in range(rows)])
    hists = [rng.integers(0, n, size=40).astype(np.uint32) for _ in range(rows)]
    off, ids = csr(hists, rows)
    d_lg = torch.from_numpy(logits).to(dev)
    d_off, d_ids = torch.from_numpy(off).to(dev), torch.from_numpy(ids).to(dev)
    plan = []
    for c in range(calls):
        # Every call has its own settings (the grid rotated, penalties varied) and seeds.
        params = []
        for r in range(rows):
            q = dict(GRID[(c * 7 + r * 13) % len(GRID)])
            if (c + r) % 3 == 1:
                q.update(presence=0.5 + 0.1 * (c % 4))
            if (c + r) % 3 == 2:
                q.update(presence=0.25, frequency=0.1 * (c % 5), repetition=1.0 + 0.05 * (r % 3))
            params.append(q)
        seeds = [1000 * c + r for r in range(rows)]
        plan.append((params, seeds, states_tensor(seeds, dev), ctx.outputs(rows, 8, dev)))
    torch.cuda.synchronize()
    # Every call is issued before any result is read.
    for params, _, st, out in plan:
        ctx.sample_batch(d_lg, [settings(p) for p in params], st, d_off, d_ids, kept_cap=8, out=out)
    torch.cuda.synchronize()
    for c, (params, seeds, st, out) in enumerate(plan):
        tok, status, kept, kept_ids, kept_probs = out
        g = dict(tokens=tok.cpu().numpy().astype(np.uint32), status=status.cpu().numpy().astype(np.uint32),
                 kept=kept.cpu().numpy().astype(np.uint32), kept_ids=kept_ids.cpu().numpy().astype(np.uint32),
                 kept_probs=kept_probs.cpu().numpy(), rng=st.cpu().numpy().view(np.uint64))
        want = oracle_rows(logits, params, seeds, hists, kept_cap=8)
        check_rows(g, want, params, kept_cap=8, label=f"call {c}")


@pytest.mark.parametrize("rows", [1, 4])
def test_histories_past_the_slice_hash_take_the_exact_path(ctx, rows):
    from artemis_amd import states_tensor
    dev = torch.device("cuda:0")
    n = 248_320
    rng = np.random.default_rng(20 + rows)
    logits = (rng.standard_normal((rows, n)) * 2.5).astype(np.float32)
    # 20,000 history ids over the first 12,000 ids (about 9,700 distinct, each seen one to a few
    # times): every slice that covers that range holds more distinct ids than its 2,048-slot hash
    # (these rows' slices hold at least 4,096 values).
    hists = [rng.integers(0, 12_000, size=20_000).astype(np.uint32) for _ in range(rows)]
    for r, h in enumerate(hists):
        logits[r, int(h[0])] += 6.0  # a history id among the best
    kinds = [dict(temp=0.7, top_k=40, top_p=0.9, min_p=0.05, presence=0.5, frequency=0.3, repetition=1.05),
             dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0, presence=1.5),
             dict(temp=0.8, top_k=0, top_p=0.9, min_p=0.02, presence=0.5, frequency=0.3, repetition=1.05),
             dict(temp=1.0, top_k=20, top_p=1.0, min_p=0.0, frequency=0.4)]
    params = [kinds[r % len(kinds)] for r in range(rows)]
    seeds = [77 + r for r in range(rows)]
    off, ids = csr(hists, rows)
    st = states_tensor(seeds, dev)
    tok, status, kept, kept_ids, kept_probs = ctx.sample_batch(
        torch.from_numpy(logits).to(dev), [settings(p) for p in params], st,
        torch.from_numpy(off).to(dev), torch.from_numpy(ids).to(dev), kept_cap=16)
    torch.cuda.synchronize()
    g = dict(tokens=tok.cpu().numpy().astype(np.uint32), status=status.cpu().numpy().astype(np.uint32),
             kept=kept.cpu().numpy().astype(np.uint32), kept_ids=kept_ids.cpu().numpy().astype(np.uint32),
             kept_probs=kept_probs.cpu().numpy(), rng=st.cpu().numpy().view(np.uint64))
    want = oracle_rows(logits, params, seeds, hists, kept_cap=16)
    check_rows(g, want, params, kept_cap=16, label=f"rows={rows}")
    # The slices could not count the history: every row was settled by a pass of the finish kernel
    # over the whole row (the deep path, then the exact-order path when a bound leaves it open).
    assert all(int(s) & (AS_ROW_EXACT_PATH | AS_ROW_DEEP_PATH) for s in g["status"]), [hex(int(s)) for s in g["status"]]


@pytest.mark.parametrize("rows", [1, 3, 16])
def test_small_batches_share_the_deep_passes(ctx, rows):
    # A batch of at most 16 rows runs the finish kernel with extra workgroups, and rows whose draw or
    # cut lies past their candidates share the deep path's two passes with them (in parts taken by
    # whichever workgroup is idle). Rows without a top-k at the model's width: unfiltered at T = 1,
    # top-p 0.95 at T = 1 and 0.6, with and without a history; seeds chosen per row.
    from artemis_amd import states_tensor
    dev = torch.device("cuda:0")
    n = 248_320
    rng = np.random.default_rng(40 + rows)
    # Flat rows (sigma 1): the candidates hold a small part of the mass, so top-p's cut and most draws
    # lie far past them and every batch has deep rows.
    logits = rng.standard_normal((rows, n)).astype(np.float32)
    kinds = [dict(temp=1.0, top_k=0, top_p=0.95, min_p=0.0),
             dict(temp=1.0, top_k=0, top_p=1.0, min_p=0.0),
             dict(temp=0.6, top_k=0, top_p=0.95, min_p=0.0, presence=0.5, frequency=0.3, repetition=1.05),
             dict(temp=1.0, top_k=0, top_p=0.99, min_p=0.001)]
    params = [kinds[r % len(kinds)] for r in range(rows)]
    hists = [rng.integers(0, n, size=300).astype(np.uint32) for _ in range(rows)]
    seeds = [900 + 17 * r for r in range(rows)]
    off, ids = csr(hists, rows)
    st = states_tensor(seeds, dev)
    tok, status, kept, kept_ids, kept_probs = ctx.sample_batch(
        torch.from_numpy(logits).to(dev), [settings(p) for p in params], st,
        torch.from_numpy(off).to(dev), torch.from_numpy(ids).to(dev))
    torch.cuda.synchronize()
    g = dict(tokens=tok.cpu().numpy().astype(np.uint32), status=status.cpu().numpy().astype(np.uint32),
             kept=kept.cpu().numpy().astype(np.uint32), kept_ids=kept_ids.cpu().numpy().astype(np.uint32),
             kept_probs=kept_probs.cpu().numpy(), rng=st.cpu().numpy().view(np.uint64))
    want = oracle_rows(logits, params, seeds, hists)
    check_rows(g, want, params, label=f"rows={rows}")
    # Kept lists are not asked for (rows with them take the full deep path alone).
    assert any(int(s) & AS_ROW_DEEP_PATH for s in g["status"]), [hex(int(s)) for s in g["status"]]


def test_shared_deep_passes_between_calls(ctx):
    # Calls alternate between a small batch (deep passes shared) and a larger one (each row alone) on
    # one context, with no host synchronisation: the shared jobs are stamped with the call's number,
    # so a pass published in one call is never taken in another.
    from artemis_amd import states_tensor
    dev = torch.device("cuda:0")
    n = 248_320
    rng = np.random.default_rng(77)
    sizes = [2, 20, 1, 20, 4]
    plan = []
    for c, rows in enumerate(sizes):
        logits = (rng.standard_normal((rows, n)) * 2.5).astype(np.float32)
        params = [dict(temp=1.0, top_k=0, top_p=1.0 if r % 2 else 0.95, min_p=0.0) for r in range(rows)]
        seeds = [5000 + 31 * c + r for r in range(rows)]
        st = states_tensor(seeds, dev)
        out = ctx.outputs(rows, 0, dev)
        plan.append((logits, params, seeds, st, out, torch.from_numpy(logits).to(dev)))
    torch.cuda.synchronize()
    for logits, params, seeds, st, out, d_lg in plan:
        ctx.sample_batch(d_lg, [settings(p) for p in params], st, out=out)
    torch.cuda.synchronize()
    for c, (logits, params, seeds, st, out, _) in enumerate(plan):
        tok, status, kept, kept_ids, kept_probs = out
        g = dict(tokens=tok.cpu().numpy().astype(np.uint32), status=status.cpu().numpy().astype(np.uint32),
                 kept=kept.cpu().numpy().astype(np.uint32), kept_ids=kept_ids.cpu().numpy().astype(np.uint32),
                 kept_probs=kept_probs.cpu().numpy(), rng=st.cpu().numpy().view(np.uint64))
        want = oracle_rows(logits, params, seeds, None)
        check_rows(g, want, params, label=f"call {c}")

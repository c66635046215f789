"""Refusals on the product path, through the C ABI on the GPU.

as_sample and as_verify honour Sampling::check (crates/engine/src/sample.rs:71-94): a row whose
settings the reference refuses is refused with AS_ERR_PARAMS, a one-line message that names the
row and starts its text with the flag (the reference's test `check_refuses_settings_it_cant_honour`,
sample.rs:607-632, asserts the flag prefix and no newline), and nothing is launched: the outputs
and the RNG states keep what they held. The capacity checks (rows, history) refuse with
AS_ERR_CAPACITY on the host, or per row on the device (AS_ROW_HISTORY).
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

N = 8192
AS_ERR_PARAMS = 2
AS_ERR_CAPACITY = 3

NAN, INF = float("nan"), float("inf")
# sample.rs:607-632's refusals, then this build's two penalties.
BAD = [
    (dict(temp=-0.1), "--temp"), (dict(temp=NAN), "--temp"), (dict(temp=INF), "--temp"),
    (dict(top_p=0.0), "--top-p"), (dict(top_p=1.1), "--top-p"), (dict(top_p=NAN), "--top-p"),
    (dict(min_p=-0.1), "--min-p"), (dict(min_p=1.5), "--min-p"),
    (dict(presence=NAN), "--presence-penalty"), (dict(presence=-INF), "--presence-penalty"),
    (dict(frequency=NAN), "--frequency-penalty"), (dict(frequency=INF), "--frequency-penalty"),
    (dict(repetition=0.0), "--repetition-penalty"), (dict(repetition=-1.0), "--repetition-penalty"),
    (dict(repetition=NAN), "--repetition-penalty"),
]


@pytest.fixture(scope="module")
def env():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=8, max_vocab=N, max_history=64)
    yield c
    c.close()


def sampling(**kw):
    from artemis_amd import Sampling
    p = dict(temp=0.7, top_k=20, top_p=0.9, min_p=0.0, presence=0.0, frequency=0.0, repetition=1.0)
    p.update(kw)
    return Sampling(p["temp"], p["top_k"], p["top_p"], p["min_p"], p["presence"], p["frequency"], p["repetition"])


def call_sample(ctx, params, hist=None):
    """as_sample through ctypes; returns (rc, message, tokens, status, rng) with outputs pre-filled."""
    from artemis_amd import sampler as S
    dev = torch.device("cuda:0")
    rows = len(params)
    lg = torch.from_numpy(np.random.default_rng(1).standard_normal((rows, N)).astype(np.float32)).to(dev)
    tok = torch.full((rows,), 0x5EED, dtype=torch.int32, device=dev)
    st = torch.full((rows,), 0x77, dtype=torch.int32, device=dev)
    kc = torch.zeros(rows, dtype=torch.int32, device=dev)
    rng = S.states_tensor(list(range(rows)), dev)
    rng0 = rng.clone()
    b = S._CBatch()
    b.logits, b.row_stride, b.n_vocab, b.n_rows = lg.data_ptr(), N, N, rows
    if hist is not None:
        off = np.zeros(rows + 1, np.int32)
        off[1:] = np.cumsum([len(h) for h in hist])
        ids = np.concatenate([np.asarray(h, np.int32) for h in hist])
        toff, tids = torch.from_numpy(off).to(dev), torch.from_numpy(ids).to(dev)
        b.hist_offsets, b.hist_ids = toff.data_ptr(), tids.data_ptr()
    b.rng_state, b.tokens, b.status, b.kept_count = rng.data_ptr(), tok.data_ptr(), st.data_ptr(), kc.data_ptr()
    arr = (S._CSampling * rows)(*[p._c() for p in params])
    rc = S.lib().as_sample(ctx.h, C.byref(b), arr)
    msg = S.lib().as_last_error(ctx.h).decode()
    torch.cuda.synchronize()
    return rc, msg, tok.cpu().numpy(), st.cpu().numpy(), kc.cpu().numpy(), (rng.cpu() == rng0.cpu()).all().item()


@pytest.mark.parametrize("bad,flag", BAD, ids=[f"{f}={list(b.values())[0]}" for b, f in BAD])
def test_as_sample_refuses_a_bad_row_naming_it_and_the_flag(env, bad, flag):
    params = [sampling(), sampling(temp=0.0), sampling(**bad), sampling()]
    rc, msg, tok, st, _, rng_same = call_sample(env, params)
    assert rc == AS_ERR_PARAMS
    assert msg.startswith("row 2: ") and "\n" not in msg, msg
    text = msg[len("row 2: "):]
    assert text.startswith(flag), msg
    # The same text as the oracle's Sampling::check restatement gives.
    want = O.check(**{**O.PLAIN, **bad})
    assert text == want, (text, want)
    # Nothing ran: the outputs and the RNG states are untouched.
    assert (tok == 0x5EED).all() and (st == 0x77).all() and rng_same


@pytest.mark.parametrize("bad,flag", BAD[::3], ids=[f"{f}" for _, f in BAD[::3]])
def test_as_verify_refuses_bad_settings_naming_the_flag(env, bad, flag):
    from artemis_amd import sampler as S
    dev = torch.device("cuda:0")
    rows = torch.zeros((3, N), dtype=torch.float32, device=dev)
    drafts = torch.zeros(2, dtype=torch.int32, device=dev)
    picks = torch.full((3,), 0x5EED, dtype=torch.int32, device=dev)
    result = torch.full((4,), 0x5EED, dtype=torch.int32, device=dev)
    rng = S.states_tensor([5], dev)
    p = sampling(**bad)
    rc = S.lib().as_verify(env.h, rows.data_ptr(), N, N, drafts.data_ptr(), 2, None, 0, None, 0,
                           C.byref(p._c()), rng.data_ptr(), picks.data_ptr(), result.data_ptr())
    msg = S.lib().as_last_error(env.h).decode()
    assert rc == AS_ERR_PARAMS and msg.startswith(flag) and "\n" not in msg, msg
    torch.cuda.synchronize()
    assert (picks.cpu() == 0x5EED).all() and (result.cpu() == 0x5EED).all()


def test_as_verify_refuses_more_drafts_than_rows_without_wrapping(env):
    from artemis_amd import sampler as S
    dev = torch.device("cuda:0")
    rows = torch.zeros((2, N), dtype=torch.float32, device=dev)
    drafts = torch.zeros(2, dtype=torch.int32, device=dev)
    picks = torch.zeros(2, dtype=torch.int32, device=dev)
    result = torch.zeros(4, dtype=torch.int32, device=dev)
    rng = S.states_tensor([5], dev)
    p = sampling()
    for k in (8, 0xFFFFFFFF):  # k + 1 past max_rows, and k + 1 wrapping to 0 in 32 bits
        rc = S.lib().as_verify(env.h, rows.data_ptr(), N, N, drafts.data_ptr(), C.c_uint32(k), None, 0, None, 0,
                               C.byref(p._c()), rng.data_ptr(), picks.data_ptr(), result.data_ptr())
        assert rc == AS_ERR_CAPACITY, (k, rc)


def test_as_verify_refuses_a_history_past_max_history(env):
    from artemis_amd import sampler as S
    dev = torch.device("cuda:0")
    rows = torch.zeros((3, N), dtype=torch.float32, device=dev)
    drafts = torch.zeros(2, dtype=torch.int32, device=dev)
    hist = torch.zeros(63, dtype=torch.int32, device=dev)  # 63 + 2 drafts > 64
    picks = torch.zeros(3, dtype=torch.int32, device=dev)
    result = torch.zeros(4, dtype=torch.int32, device=dev)
    rng = S.states_tensor([5], dev)
    p = sampling()
    rc = S.lib().as_verify(env.h, rows.data_ptr(), N, N, drafts.data_ptr(), 2, hist.data_ptr(), 63, None, 0,
                           C.byref(p._c()), rng.data_ptr(), picks.data_ptr(), result.data_ptr())
    assert rc == AS_ERR_CAPACITY
    rc = S.lib().as_verify(env.h, rows.data_ptr(), N, N, drafts.data_ptr(), 2, hist.data_ptr(), 62, None, 0,
                           C.byref(p._c()), rng.data_ptr(), picks.data_ptr(), result.data_ptr())
    assert rc == 0
    torch.cuda.synchronize()


def test_as_sample_refuses_a_row_whose_history_passes_max_history_on_the_device(env):
    from artemis_amd import AS_ROW_HISTORY
    params = [sampling(presence=0.5), sampling(temp=0.0, presence=0.5), sampling(presence=0.5), sampling()]
    hist = [np.arange(64), np.arange(65), np.arange(10), np.arange(200)]
    rc, msg, tok, st, kc, _ = call_sample(env, params, hist)
    assert rc == 0, msg
    assert list(st & 0xFF) == [0, AS_ROW_HISTORY, 0, AS_ROW_HISTORY], st
    assert kc[1] == 65 and kc[3] == 200
    assert tok[1] == -1 and tok[3] == -1

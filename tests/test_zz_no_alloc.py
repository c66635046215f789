"""as_logprobs_static, the allocation-free variant of as_logprobs, through the C ABI on the GPU.

Its outputs must be as_logprobs' own, bit for bit (the same kernels over the same rows), on two
calls in a row, the second with fewer rows and a narrower vocabulary (the static scratch keeps the
first call's parts, which the second must not see); and it refuses a batch past its static scratch
with AS_ERR_CAPACITY and a message."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

AS_ERR_CAPACITY = 3


def static_call(lg, tokens, top, stride, n_vocab, stream=None):
    from artemis_amd import sampler as S
    rows = tokens.numel()
    dev = lg.device
    lp = torch.full((rows,), float("nan"), dtype=torch.float32, device=dev)
    ids = torch.full((rows, max(top, 1)), -1, dtype=torch.int32, device=dev)
    lps = torch.full((rows, max(top, 1)), float("nan"), dtype=torch.float32, device=dev)
    st = torch.full((rows,), 7, dtype=torch.int32, device=dev)
    err = C.create_string_buffer(256)
    s = stream if stream is not None else torch.cuda.current_stream()
    rc = S.lib().as_logprobs_static(C.c_void_p(s.cuda_stream), lg.data_ptr(), stride, n_vocab, rows,
                                    tokens.data_ptr(), top, lp.data_ptr(), ids.data_ptr(), lps.data_ptr(),
                                    st.data_ptr(), err, 256)
    return rc, err.value.decode(), lp, ids, lps, st


def same(a, b):
    return a.cpu().numpy().tobytes() == b.cpu().numpy().tobytes()


def test_static_logprobs_match_as_logprobs_on_two_calls_in_a_row():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    dev = torch.device("cuda:0")
    gen = np.random.default_rng(17)
    n1, r1 = 248_320, 128  # the static scratch full: 128 x 16 = 2,048 parts
    n2, r2 = 100_000, 5
    x1 = torch.from_numpy((gen.standard_normal((r1, n1)) * 2.5).astype(np.float32)).to(dev)
    x1[3, 777] = 60.0  # a near-certain token
    x2 = torch.from_numpy((gen.standard_normal((r2, n2)) * 3.0).astype(np.float32)).to(dev)
    t1 = torch.from_numpy(gen.integers(0, n1, r1).astype(np.int32)).to(dev)
    t2 = torch.from_numpy(gen.integers(0, n2, r2).astype(np.int32)).to(dev)
    ctx = Context(max_rows=r1, max_vocab=n1)
    want1 = ctx.logprobs(x1, t1, 20)
    want2 = ctx.logprobs(x2, t2, 20)
    torch.cuda.synchronize()
    rc, msg, *got1 = static_call(x1, t1, 20, n1, n1)
    assert rc == 0, msg
    rc, msg, *got2 = static_call(x2, t2, 20, n2, n2)
    assert rc == 0, msg
    torch.cuda.synchronize()
    for w, g in zip(want1, got1):
        assert same(w, g)
    for w, g in zip(want2, got2):
        assert same(w, g)
    ctx.close()


def test_static_logprobs_refuse_a_batch_past_the_scratch():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda:0")
    lg = torch.zeros((129, 248_320), dtype=torch.float32, device=dev)  # 129 x 16 = 2,064 parts
    tok = torch.zeros(129, dtype=torch.int32, device=dev)
    rc, msg, lp, *_ = static_call(lg, tok, 20, 248_320, 248_320)
    assert rc == AS_ERR_CAPACITY and "2048" in msg.replace(",", ""), (rc, msg)
    torch.cuda.synchronize()
    assert torch.isnan(lp).all()  # nothing ran


def test_static_logprobs_replay_under_graph_capture():
    # After one eager call (which looks the static scratch up), as_logprobs_static is captured into a
    # graph and replayed on new logits written into the captured input, with eager work and
    # synchronisations between the replays; every replay must give as_logprobs' outputs bit for bit.
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    dev = torch.device("cuda:0")
    gen = np.random.default_rng(23)
    n, rows, top = 248_320, 8, 20
    x = torch.from_numpy((gen.standard_normal((rows, n)) * 2.5).astype(np.float32)).to(dev)
    tok = torch.from_numpy(gen.integers(0, n, rows).astype(np.int32)).to(dev)
    rc, msg, *_ = static_call(x, tok, top, n, n)
    assert rc == 0, msg
    torch.cuda.synchronize()
    from artemis_amd import sampler as S
    lp = torch.empty(rows, dtype=torch.float32, device=dev)
    ids = torch.empty((rows, top), dtype=torch.int32, device=dev)
    lps = torch.empty((rows, top), dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    err = C.create_string_buffer(256)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream()
        rc = S.lib().as_logprobs_static(C.c_void_p(s.cuda_stream), x.data_ptr(), n, n, rows, tok.data_ptr(), top,
                                        lp.data_ptr(), ids.data_ptr(), lps.data_ptr(), st.data_ptr(), err, 256)
    assert rc == 0, err.value.decode()
    ctx = Context(max_rows=rows, max_vocab=n)
    for rep in range(3):
        fresh = torch.from_numpy((gen.standard_normal((rows, n)) * (2.0 + rep)).astype(np.float32)).to(dev)
        x.copy_(fresh)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = ctx.logprobs(fresh, tok, top)
        torch.cuda.synchronize()
        for w, got in zip(want, (lp, ids, lps, st)):
            assert same(w, got), rep
        _ = (fresh * 2.0).sum().item()  # eager work between replays
    ctx.close()

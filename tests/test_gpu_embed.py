"""The draft chain on the GPU: argmax_rows then embed_rows (crates/engine/src/mtp.rs:984-1079 calls
the pair; dispatch.rs:97-153), against the dequantization oracle (oracle/quant_oracle.cc, restating
crates/qwen36/src/quant.rs). Every value must be bit-exact: the kernel takes dequant_row's f32 steps
in its order. Tables live in HBM (the reference reads them from pinned host memory; here the same
kernel reads device addresses)."""
import os

import numpy as np
import pytest

import oracle_lib as O
from test_oracle_quant import FIXTURES, GOLD, random_table

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=16, max_vocab=4096)
    yield c
    c.close()


def embed(ctx, table_dev, picks, wtype, n):
    """embed_rows over rows `picks` of a device table, addressed as argmax_rows addresses them."""
    rb = O.row_bytes(wtype, n)
    base = table_dev.data_ptr()
    rows = torch.tensor([base + p * rb for p in picks], dtype=torch.int64, device="cuda")
    y = ctx.embed_rows(rows, wtype, n)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def same_bits(got, want):
    return np.array_equal(np.ascontiguousarray(got, np.float32).view(np.uint32),
                          np.ascontiguousarray(want, np.float32).view(np.uint32))


@pytest.mark.parametrize("name", list(FIXTURES))
def test_every_type_rows_9_2_2_0_of_a_12_row_table(ctx, name):
    # kernels/tests/gpu_prefill.rs:451-476: rows 9, 2, 2 and 0 of a 12-row table, n = 2048.
    rng = np.random.default_rng(51)
    n, picks = 2048, [9, 2, 2, 0]
    code = O.WTYPES[name]
    table = random_table(rng, name, 12, n)
    got = embed(ctx, torch.from_numpy(table).cuda(), picks, code, n)
    for t, p in enumerate(picks):
        assert same_bits(got[t], O.dequant_row(code, table[p].tobytes(), n)), (name, t)


@pytest.mark.parametrize("name", list(FIXTURES))
def test_gguf_py_rows(ctx, name):
    raw = np.fromfile(os.path.join(GOLD, FIXTURES[name] + ".bin"), dtype=np.uint8)
    want = np.fromfile(os.path.join(GOLD, FIXTURES[name] + ".f32"), dtype="<f4")
    got = embed(ctx, torch.from_numpy(raw).cuda(), [0, 0], O.WTYPES[name], len(want))
    assert same_bits(got[0], want) and same_bits(got[1], want), name


@pytest.mark.parametrize("name,n", [("F32", 1000), ("BF16", 333), ("Q8_0", 2080), ("Q8_0", 32), ("Q4_K", 256),
                                    ("Q6_K", 768)])
def test_widths_that_end_inside_a_group(ctx, name, n):
    rng = np.random.default_rng(n)
    code = O.WTYPES[name]
    table = random_table(rng, name, 5, n)
    got = embed(ctx, torch.from_numpy(table).cuda(), [4, 1, 3], code, n)
    for t, p in enumerate([4, 1, 3]):
        assert same_bits(got[t], O.dequant_row(code, table[p].tobytes(), n)), (name, n, t)


@pytest.mark.parametrize("name", ["Q6_K", "Q8_0", "BF16"])
def test_argmax_rows_then_embed_rows(ctx, name):
    # The greedy draft step: each logit row's argmax picks a table row by address, and embed_rows
    # reads the rows there, with no host round trip between them.
    rng = np.random.default_rng(7)
    vocab, n, k = 3000, 1024, 5
    code = O.WTYPES[name]
    rb = O.row_bytes(code, n)
    table = random_table(rng, name, vocab, n)
    d_table = torch.from_numpy(table).cuda()
    logits = rng.standard_normal((k, vocab)).astype(np.float32)
    logits[2, 1234] = 50.0
    ids = torch.zeros(k, dtype=torch.int32, device="cuda")
    rows = torch.zeros(k, dtype=torch.int64, device="cuda")
    ctx.argmax_rows(torch.from_numpy(logits).cuda(), ids, rows, d_table.data_ptr(), rb)
    y = ctx.embed_rows(rows, code, n)
    torch.cuda.synchronize()
    got_ids = ids.cpu().numpy()
    assert got_ids[2] == 1234
    y = y.cpu().numpy()
    for t in range(k):
        want_id = O.argmax_row(logits[t])
        assert got_ids[t] == want_id
        assert same_bits(y[t], O.dequant_row(code, table[want_id].tobytes(), n)), (name, t)


def test_refuses_bad_types_and_partial_blocks(ctx):
    from artemis_amd import SamplerError
    rows = torch.zeros(1, dtype=torch.int64, device="cuda")
    with pytest.raises(SamplerError):
        ctx.embed_rows(rows, 6, 256)
    with pytest.raises(SamplerError):
        ctx.embed_rows(rows, O.WTYPES["Q4_K"], 100)
    with pytest.raises(SamplerError):
        ctx.embed_rows(rows, O.WTYPES["Q8_0"], 48)

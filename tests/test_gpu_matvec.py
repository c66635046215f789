"""The head's matvec and the fused greedy draft step on the GPU, against the matvec twin's
restatement (oracle/quant_oracle.cc oc_matvec, restating crates/kernels/src/twin/matvec.rs) and the
argmax twin (oc_argmax_row, twin/argmax.rs). Outputs must be bit-exact, as the reference holds its
own GPU matvec to its twin (crates/kernels/tests/gpu_kernels.rs:112-140)."""
import numpy as np
import pytest

import oracle_lib as O
from test_oracle_quant import FIXTURES, random_table

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

HEAD_ROWS, HEAD_K = 248_320, 2048  # the model's output head (qwen36/src/dims.rs:38), Q6_K


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from artemis_amd import Context
    c = Context(max_rows=16, max_vocab=4096)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def gpu_matvec(ctx, name, table, rows, k, x):
    y = ctx.matvec(torch.from_numpy(table).cuda(), O.WTYPES[name], rows, k, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("name", list(FIXTURES))
def test_matvec_every_type_and_shape_bit_for_bit(ctx, name):
    # gpu_kernels.rs:80-140: decode's shapes, and the twin's bits at the model's.
    rng = np.random.default_rng(13)
    for rows, k in [(1, 2048), (37, 2048), (512, 2048), (2048, 512), (256, 256), (8192, 2048)]:
        table = random_table(rng, name, rows, k)
        x = rng.uniform(-1, 1, size=k).astype(np.float32)
        got = gpu_matvec(ctx, name, table, rows, k, x)
        want = O.matvec(O.WTYPES[name], table.tobytes(), rows, k, x)
        differ = int(np.sum(bits(got) != bits(want)))
        assert differ == 0, f"{name} {rows}x{k}: {differ} of {rows} outputs differ from the twin"


def test_matvec_order_plants_match_the_twin(ctx):
    # The oracle's order pins (test_oracle_quant.py) on the GPU: a unit's products folded in order
    # (2^24 stays 2^24), a lane's units folded in unit order (likewise) and units strided over the
    # lanes (2^24 + 2), in F32 rows.
    cases = [(1024, {0: 2.0 ** 24, 2: 1.0, 3: 1.0}, 2.0 ** 24),
             (3072, {0: 2.0 ** 24, 32 * 32: 1.0, 64 * 32: 1.0}, 2.0 ** 24),
             (3072, {16 * 32: 2.0 ** 24, 32 * 32: 1.0, 64 * 32: 1.0}, 2.0 ** 24 + 2)]
    for k, plants, want in cases:
        w = np.zeros(k, np.float32)
        for i, v in plants.items():
            w[i] = v
        x = np.ones(k, np.float32)
        table = np.frombuffer(w.tobytes(), np.uint8).copy()
        got = gpu_matvec(ctx, "F32", table, 1, k, x)
        assert float(got[0]) == want, (k, float(got[0]), want)
        assert np.array_equal(bits(got), bits(O.matvec(O.WTYPES["F32"], w.tobytes(), 1, k, x)))


def test_matvec_q8_0_rows_of_one_unit_per_lane(ctx):
    # k = 32 * 33: lane 0 sums two units, the others one; k = 64: lanes 2..31 add nothing.
    rng = np.random.default_rng(3)
    for k in (32 * 33, 64, 32):
        table = random_table(rng, "Q8_0", 40, k)
        x = rng.uniform(-1, 1, size=k).astype(np.float32)
        got = gpu_matvec(ctx, "Q8_0", table, 40, k, x)
        assert np.array_equal(bits(got), bits(O.matvec(O.WTYPES["Q8_0"], table.tobytes(), 40, k, x))), k


def head_case(ctx, name, rows, k, seed, plant=None):
    rng = np.random.default_rng(seed)
    table = random_table(rng, name, rows, k)
    if plant is not None:
        plant(table)
    x = rng.uniform(-1, 1, size=k).astype(np.float32)
    dev_w = torch.from_numpy(table).cuda()
    dev_x = torch.from_numpy(x).cuda()
    logits = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    ids = torch.full((3,), 7, dtype=torch.int32, device="cuda")
    rows_out = torch.full((3,), 9, dtype=torch.int64, device="cuda")
    embd, erb = 0x7_0000_0000, 4096
    ctx.head_argmax(dev_w, O.WTYPES[name], rows, k, dev_x, ids, rows_out, embd, erb, slot=1, logits=logits)
    # Without logits: the draft alone, into slot 2.
    ctx.head_argmax(dev_w, O.WTYPES[name], rows, k, dev_x, ids, rows_out, embd, erb, slot=2)
    torch.cuda.synchronize()
    want_y = O.matvec(O.WTYPES[name], table.tobytes(), rows, k, x)
    want = O.argmax_row(want_y)
    got_ids = ids.cpu().numpy().astype(np.uint32)
    got_rows = rows_out.cpu().numpy().view(np.uint64)
    got_y = logits.cpu().numpy()
    nan = np.isnan(want_y)  # NaN payloads differ between hosts; their places must not
    assert np.array_equal(np.isnan(got_y), nan)
    assert np.array_equal(bits(got_y[~nan]), bits(want_y[~nan]))
    wid = 0xFFFFFFFF if want is None else want
    for s in (1, 2):
        assert got_ids[s] == wid, (name, s, got_ids[s], wid)
        assert got_rows[s] == embd + (0 if want is None else want) * erb
    assert got_ids[0] == 7 and got_rows[0] == 9
    return want_y, want


def test_head_argmax_at_the_models_head(ctx):
    # 248,320 Q6_K rows of 2,048 (417 MB of weights).
    head_case(ctx, "Q6_K", HEAD_ROWS, HEAD_K, 21)


@pytest.mark.parametrize("name", ["F32", "BF16", "Q8_0", "Q4_K", "Q5_K"])
def test_head_argmax_every_type(ctx, name):
    head_case(ctx, name, 20_000, 512, 22)


def test_head_argmax_ties_go_to_the_lower_row(ctx):
    # Copies of the winning row give equal outputs: the lowest copy is the draft.
    y, _ = head_case(ctx, "F32", 200_000, 64, 23)
    top = int(np.argmax(y))

    def plant(t):
        t[top + 1] = t[top]
        t[5] = t[top]
    _, want = head_case(ctx, "F32", 200_000, 64, 23, plant=plant)
    assert want == min(5, top)


def test_head_argmax_skips_non_finite_outputs(ctx):
    # Rows with infinite weights give inf or NaN outputs, which never win; none finite: NO_DRAFT.
    k = 64
    inf = np.frombuffer(np.float32(np.inf).tobytes(), np.uint8)

    def plant(t):
        t[10, 0:4] = inf
        t[11, 0:4] = inf
        t[11, 4:8] = np.frombuffer(np.float32(-np.inf).tobytes(), np.uint8)
    y, want = head_case(ctx, "F32", 3000, k, 24, plant=plant)
    assert not np.isfinite(y[10]) and want not in (10, 11)

    def plant_all(t):
        t[:, 0:4] = inf
    head_case(ctx, "F32", 3000, k, 25, plant=plant_all)


def test_head_then_embed_is_the_greedy_draft_step(ctx):
    # decode.rs:850's head, argmax_rows and embed_rows (mtp.rs:984-1079), all on the GPU.
    rng = np.random.default_rng(26)
    rows, k, n_embd = 30_000, 2048, 2048
    head = random_table(rng, "Q6_K", rows, k)
    embd = random_table(rng, "Q6_K", rows, n_embd)
    x = rng.uniform(-1, 1, size=k).astype(np.float32)
    d_head, d_embd = torch.from_numpy(head).cuda(), torch.from_numpy(embd).cuda()
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    addr = torch.zeros(1, dtype=torch.int64, device="cuda")
    erb = O.row_bytes(O.WTYPES["Q6_K"], n_embd)
    ctx.head_argmax(d_head, O.WTYPES["Q6_K"], rows, k, torch.from_numpy(x).cuda(), ids, addr, d_embd.data_ptr(), erb)
    e = ctx.embed_rows(addr, O.WTYPES["Q6_K"], n_embd)
    torch.cuda.synchronize()
    want = O.argmax_row(O.matvec(O.WTYPES["Q6_K"], head.tobytes(), rows, k, x))
    assert int(ids.item()) == want
    assert np.array_equal(bits(e.cpu().numpy()[0]), bits(O.dequant_row(O.WTYPES["Q6_K"], embd[want].tobytes(), n_embd)))


def test_matvec_refuses_bad_shapes_and_alignment(ctx):
    from artemis_amd import SamplerError
    w = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    x = torch.zeros(2048, dtype=torch.float32, device="cuda")
    with pytest.raises(SamplerError):
        ctx.matvec(w, 6, 4, 256, x[:256])
    with pytest.raises(SamplerError):
        ctx.matvec(w, O.WTYPES["Q4_K"], 4, 160, x[:160])  # not whole 256-value blocks
    with pytest.raises(SamplerError):
        ctx.matvec(w[1:], O.WTYPES["Q6_K"], 4, 256, x[:256])  # odd address
    big = torch.zeros(8192 + 32, dtype=torch.float32, device="cuda")
    with pytest.raises(SamplerError):
        ctx.matvec(w, O.WTYPES["F32"], 1, 8192 + 32, big)  # past the staged input's room

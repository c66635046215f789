"""The dequantization oracle (oracle/quant_oracle.cc, restating crates/qwen36/src/quant.rs) against
the reference's own checks: its gguf-py rows of each weight type (crates/qwen36/tests/fixtures,
copied as data into tests/golden/quant; quant_fixtures.rs holds them to 1e-6 relative), its
hand-built blocks (quant.rs:266-409) and its row_bytes table (quant.rs:270-277). A vectorised numpy
decoding written from ggml's block layouts, and numpy's own f16 conversion, check the rest."""
import os

import numpy as np
import pytest

import oracle_lib as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant")
FIXTURES = {"F32": "f32_row", "BF16": "bf16_row", "Q8_0": "q8_0_row", "Q4_K": "q4_k_row",
            "Q5_K": "q5_k_row", "Q6_K": "q6_k_row"}


def test_row_bytes_per_type():
    # quant.rs:270-277, and a partial K-quant row (quant.rs:280-284) refused.
    W = O.WTYPES
    assert O.row_bytes(W["F32"], 4) == 16
    assert O.row_bytes(W["BF16"], 3) == 6
    assert O.row_bytes(W["Q8_0"], 2048) == 2176
    assert O.row_bytes(W["Q4_K"], 2048) == 1152
    assert O.row_bytes(W["Q5_K"], 512) == 352
    assert O.row_bytes(W["Q6_K"], 512) == 420
    assert O.row_bytes(W["Q4_K"], 100) == 0
    assert O.row_bytes(6, 256) == 0
    with pytest.raises(ValueError):
        O.dequant_row(W["Q4_K"], bytes(144), 100)


@pytest.mark.parametrize("name", list(FIXTURES))
def test_matches_gguf_py_rows(name):
    raw = open(os.path.join(GOLD, FIXTURES[name] + ".bin"), "rb").read()
    want = np.fromfile(os.path.join(GOLD, FIXTURES[name] + ".f32"), dtype="<f4")
    assert len(raw) == O.row_bytes(O.WTYPES[name], len(want))
    got = O.dequant_row(O.WTYPES[name], raw, len(want))
    # The reference's tolerance (quant_fixtures.rs:21-27) ...
    assert np.all(np.abs(got - want) <= 1e-6 * np.maximum(np.abs(want), 1.0)), name
    # ... and in fact bit for bit: gguf-py takes the same f32 steps.
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


def test_q8_0_hand_block():
    # quant.rs:287-299: d = 0.5, quants i - 16.
    b = bytearray(34)
    b[0:2] = np.float16(0.5).tobytes()
    for i in range(32):
        b[2 + i] = (i - 16) & 0xFF
    out = O.dequant_row(O.WTYPES["Q8_0"], b, 32)
    assert out.tolist() == [0.5 * (i - 16.0) for i in range(32)]


def test_q5k_hand_block():
    # quant.rs:302-320: d = 1, dmin = 0, scales 1, mins 0, low nibbles 1 and 2, high bits set.
    b = bytearray(176)
    b[0:2] = np.float16(1.0).tobytes()
    b[4:16] = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])
    b[16:48] = b"\xff" * 32
    b[48:176] = b"\x21" * 128
    out = O.dequant_row(O.WTYPES["Q5_K"], b, 256)
    for c in range(4):
        assert np.all(out[64 * c:64 * c + 32] == 17.0)
        assert np.all(out[64 * c + 32:64 * c + 64] == 18.0)


def test_q6k_hand_block_extremes():
    # quant.rs:323-334.
    b = bytearray(210)
    b[192:208] = b"\x01" * 16
    b[208:210] = np.float16(1.0).tobytes()
    assert np.all(O.dequant_row(O.WTYPES["Q6_K"], b, 256) == -32.0)
    b[0:192] = b"\xff" * 192
    assert np.all(O.dequant_row(O.WTYPES["Q6_K"], b, 256) == 31.0)


def test_bf16_and_f32_rows():
    # quant.rs:396-408.
    assert O.dequant_row(O.WTYPES["BF16"], bytes([0x80, 0x3F, 0x00, 0xC0]), 2).tolist() == [1.0, -2.0]
    raw = np.array([1.5, -0.25], "<f4").tobytes()
    assert O.dequant_row(O.WTYPES["F32"], raw, 2).tolist() == [1.5, -0.25]


def test_half_conversion_is_numpys_for_every_pattern():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.oc_half_to_float(int(h)) for h in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ggml's block layouts decoded with whole-array numpy operations (a second, independent decoding).
def _np_dequant(name, raw, n):
    a = np.frombuffer(bytes(raw), np.uint8)
    f16 = lambda x: x.copy().view("<f2").astype(np.float32)
    if name == "F32":
        return a.view("<f4").copy()
    if name == "BF16":
        return (a.view("<u2").astype(np.uint32) << 16).view(np.float32)
    if name == "Q8_0":
        b = a.reshape(-1, 34)
        return (f16(b[:, 0:2])[:, :1] * b[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)
    if name in ("Q4_K", "Q5_K"):
        bs = 144 if name == "Q4_K" else 176
        b = a.reshape(-1, bs)
        d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
        s = b[:, 4:16].astype(np.uint32)
        j = np.arange(8)
        lo = j < 4
        jj = np.where(lo, j, j - 4)
        sc = np.where(lo, s[:, jj] & 63, (s[:, jj + 8] & 0xF) | ((s[:, jj] >> 6) << 4))
        mn = np.where(lo, s[:, jj + 4] & 63, (s[:, jj + 8] >> 4) | ((s[:, jj + 4] >> 6) << 4))
        qs = b[:, bs - 128:].reshape(-1, 4, 32).astype(np.uint32)
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block 2c, 2c+1
        if name == "Q5_K":
            qh = b[:, 16:48].astype(np.uint32)
            q = q + (((qh[:, None, :] >> j[None, :, None]) & 1) << 4)
        d1 = (d * sc.astype(np.float32)).astype(np.float32)
        m1 = (dmin * mn.astype(np.float32)).astype(np.float32)
        return ((d1[:, :, None] * q.astype(np.float32)) - m1[:, :, None]).astype(np.float32).reshape(-1)
    b = a.reshape(-1, 210)
    d = f16(b[:, 208:210])
    out = np.empty((b.shape[0], 256), np.float32)
    for h in range(2):
        ql = b[:, 64 * h:64 * h + 64].astype(np.int32)
        qh = b[:, 128 + 32 * h:160 + 32 * h].astype(np.int32)
        sc = b[:, 192 + 8 * h:200 + 8 * h].view(np.int8).astype(np.float32)
        for m in range(4):
            low = (ql[:, 32 * (m & 1):32 * (m & 1) + 32] >> (4 * (m >> 1))) & 0xF
            q = (low | (((qh >> (2 * m)) & 3) << 4)) - 32
            scale = sc[:, np.arange(32) // 16 + 2 * m]
            out[:, 128 * h + 32 * m:128 * h + 32 * m + 32] = (d * scale) * q.astype(np.float32)
    return out.reshape(-1)


def random_table(rng, name, rows, n):
    """rows random rows of type `name`: random bytes with every f16 scale a finite value."""
    rb = O.row_bytes(O.WTYPES[name], n)
    t = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
    halves = {"Q8_0": (34, [0]), "Q4_K": (144, [0, 2]), "Q5_K": (176, [0, 2]), "Q6_K": (210, [208])}
    if name in halves:
        bs, offs = halves[name]
        blk = t.reshape(rows, -1, bs)
        for o in offs:
            blk[:, :, o:o + 2] = rng.uniform(-0.05, 0.05, size=blk.shape[:2]).astype("<f2").view(np.uint8).reshape(
                blk.shape[0], blk.shape[1], 2)
    elif name == "BF16":
        t[:] = (rng.standard_normal((rows, n)).astype(np.float32).view(np.uint32) >> 16).astype("<u2").view(
            np.uint8).reshape(rows, rb)
    elif name == "F32":
        t[:] = rng.standard_normal((rows, n)).astype("<f4").view(np.uint8).reshape(rows, rb)
    return t


@pytest.mark.parametrize("name", list(FIXTURES))
def test_random_blocks_match_a_vectorised_decoding(name):
    rng = np.random.default_rng(11)
    n = 2048
    t = random_table(rng, name, 4, n)
    for r in range(4):
        got = O.dequant_row(O.WTYPES[name], t[r].tobytes(), n)
        want = _np_dequant(name, t[r].tobytes(), n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, r)


# The matvec twin (oc_matvec, restating crates/kernels/src/twin/matvec.rs:21-131).

def integer_table(rng, name, rows, k):
    """Rows whose dequantized weights are small integers (scales 1, mins 0 or small), so that every
    partial sum with integer inputs is exact in f32 whatever the order."""
    t = random_table(rng, name, rows, k)
    one = np.float16(1.0).tobytes()
    if name == "F32":
        t[:] = rng.integers(-8, 9, size=(rows, k)).astype("<f4").view(np.uint8).reshape(rows, -1)
    elif name == "BF16":
        v = rng.integers(-8, 9, size=(rows, k)).astype(np.float32).view(np.uint32) >> 16
        t[:] = v.astype("<u2").view(np.uint8).reshape(rows, -1)
    elif name == "Q8_0":
        blk = t.reshape(rows, -1, 34)
        blk[:, :, 0:2] = np.frombuffer(one, np.uint8)
    elif name in ("Q4_K", "Q5_K"):
        blk = t.reshape(rows, -1, 144 if name == "Q4_K" else 176)
        blk[:, :, 0:2] = np.frombuffer(one, np.uint8)
        blk[:, :, 2:4] = np.frombuffer(one, np.uint8)
        blk[:, :, 4:16] &= 0x03  # scales and mins 0..3 (the high bits cleared)
    else:
        blk = t.reshape(rows, -1, 210)
        blk[:, :, 208:210] = np.frombuffer(one, np.uint8)
        blk[:, :, 192:208] = rng.integers(-3, 4, size=blk[:, :, 192:208].shape).astype(np.int8).view(np.uint8)
    return t


@pytest.mark.parametrize("name", list(FIXTURES))
def test_matvec_is_the_exact_dot_product_on_integer_rows(name):
    rng = np.random.default_rng(5)
    rows, k = 6, 2048
    code = O.WTYPES[name]
    t = integer_table(rng, name, rows, k)
    x = rng.integers(-4, 5, size=k).astype(np.float32)
    y = O.matvec(code, t.tobytes(), rows, k, x)
    for r in range(rows):
        w = O.dequant_row(code, t[r].tobytes(), k).astype(np.float64)
        assert np.all(w == np.round(w)), name
        assert y[r] == float(np.dot(w, x.astype(np.float64))), (name, r)


@pytest.mark.parametrize("name", list(FIXTURES))
def test_matvec_within_the_f32_bound_of_the_f64_dot(name):
    rng = np.random.default_rng(6)
    rows, k = 8, 2048
    code = O.WTYPES[name]
    t = random_table(rng, name, rows, k)
    x = rng.uniform(-1, 1, size=k).astype(np.float32)
    y = O.matvec(code, t.tobytes(), rows, k, x)
    for r in range(rows):
        w = O.dequant_row(code, t[r].tobytes(), k).astype(np.float64)
        exact = float(np.dot(w, x.astype(np.float64)))
        # Each output is at most k additions and a few scalings deep; the dequantized weights of the
        # quantized types differ from dequant_row's only by the order of the scale products.
        bound = (k + 64) * 2.0 ** -24 * float(np.sum(np.abs(w * x))) + 1e-30
        assert abs(float(y[r]) - exact) <= bound, (name, r, float(y[r]), exact, bound)


def test_matvec_adds_the_lanes_in_the_twins_tree():
    # F32 rows of k = 1024: lane l's partial is row[32 l] * x[32 l]. Partials 2^24 at lane 0 and 1 at
    # lanes 1 and 17: the tree (twin/mod.rs:15-25) adds lane 17 into lane 1 first (2, exact), then
    # 2^24 + 2; lanes added one by one would round 2^24 + 1 down twice, to 2^24.
    k = 1024
    w = np.zeros(k, np.float32)
    w[0], w[32], w[32 * 17] = 2.0 ** 24, 1.0, 1.0
    x = np.zeros(k, np.float32)
    x[::32] = 1.0
    y = O.matvec(O.WTYPES["F32"], w.tobytes(), 1, k, x)
    p = (w * x).reshape(32, 32).sum(axis=1).astype(np.float32)
    s = 16
    while s:
        p[:s] = (p[:s] + p[s:2 * s]).astype(np.float32)
        s //= 2
    assert p[0] == 2.0 ** 24 + 2 and y[0] == p[0]
    seq = np.float32(0)
    for v in (w * x).reshape(32, 32).sum(axis=1).astype(np.float32):
        seq = np.float32(seq + v)
    assert seq != y[0]


def _f32_row_dot_model(w, x, lane_of_unit, unit_order, within):
    """A model of one row's matvec in f32 for an F32 row: units of 32 products, each unit's products
    folded by `within` ("seq": left to right from 0; "pairs": pairwise), unit u to lane
    lane_of_unit(u), each lane's units folded from 0 in `unit_order`, then the 32 lanes by the twins'
    tree (twin/mod.rs:15-25). The reference is ("seq", lane = u mod 32, ascending)."""
    f = np.float32
    prods = (w.astype(f) * x.astype(f)).astype(f).reshape(-1, 32)

    def unit(u):
        v = [f(t) for t in prods[u]]
        if within == "seq":
            acc = f(0)
            for t in v:
                acc = f(acc + t)
            return acc
        while len(v) > 1:
            v = [f(v[i] + v[i + 1]) for i in range(0, len(v), 2)]
        return v[0]

    lanes = [[] for _ in range(32)]
    for u in range(prods.shape[0]):
        lanes[lane_of_unit(u)].append(u)
    p = np.zeros(32, f)
    for l in range(32):
        acc = f(0)
        for u in (lanes[l] if unit_order == "asc" else lanes[l][::-1]):
            acc = f(acc + unit(u))
        p[l] = acc
    s = 16
    while s:
        p[:s] = (p[:s] + p[s:2 * s]).astype(f)
        s //= 2
    return float(p[0])


def test_matvec_folds_a_units_products_left_to_right():
    # twin/matvec.rs:22-30: unit_dot folds its 32 products from 0 in order. 2^24, 0, 1, 1 in one
    # unit: in order each 1 rounds away (2^24 + 1 ties to 2^24); paired (or from the end), 1 + 1 = 2
    # meets 2^24 and survives.
    k = 1024
    w = np.zeros(k, np.float32)
    w[0], w[2], w[3] = 2.0 ** 24, 1.0, 1.0
    x = np.ones(k, np.float32)
    y = O.matvec(O.WTYPES["F32"], w.tobytes(), 1, k, x)
    ref = _f32_row_dot_model(w, x, lambda u: u % 32, "asc", "seq")
    assert ref == 2.0 ** 24 and y[0] == ref
    assert _f32_row_dot_model(w, x, lambda u: u % 32, "asc", "pairs") == 2.0 ** 24 + 2


def test_matvec_folds_a_lanes_units_in_unit_order():
    # twin/matvec.rs:87-98: lane l folds units l, l + 32, l + 64, ... from 0 in that order. Units 0, 32
    # and 64 (lane 0's, at k = 3,072) summing to 2^24, 1 and 1: in order the 1s round away; folded
    # from the last unit first they add to 2 before 2^24.
    k = 3072
    w = np.zeros(k, np.float32)
    w[0], w[32 * 32], w[64 * 32] = 2.0 ** 24, 1.0, 1.0
    x = np.ones(k, np.float32)
    y = O.matvec(O.WTYPES["F32"], w.tobytes(), 1, k, x)
    ref = _f32_row_dot_model(w, x, lambda u: u % 32, "asc", "seq")
    assert ref == 2.0 ** 24 and y[0] == ref
    assert _f32_row_dot_model(w, x, lambda u: u % 32, "desc", "seq") == 2.0 ** 24 + 2


def test_matvec_strides_units_over_the_lanes():
    # twin/matvec.rs:87-98: unit u belongs to lane u mod 32. Units 32 and 64 (both lane 0's) at 1 and
    # unit 16 (lane 16's) at 2^24: lane 0 holds 2 before the tree's first step adds lane 16 into it,
    # 2^24 + 2 exactly. Units given to lanes in contiguous runs (lane = u / 3 at 96 units) would meet
    # 2^24 one at a time in the tree, and each 1 would round away.
    k = 3072
    w = np.zeros(k, np.float32)
    w[16 * 32], w[32 * 32], w[64 * 32] = 2.0 ** 24, 1.0, 1.0
    x = np.ones(k, np.float32)
    y = O.matvec(O.WTYPES["F32"], w.tobytes(), 1, k, x)
    ref = _f32_row_dot_model(w, x, lambda u: u % 32, "asc", "seq")
    assert ref == 2.0 ** 24 + 2 and y[0] == ref
    assert _f32_row_dot_model(w, x, lambda u: u // 3, "asc", "seq") == 2.0 ** 24


def test_matvec_refuses_partial_units():
    with pytest.raises(ValueError):
        O.matvec(O.WTYPES["F32"], bytes(4 * 40), 1, 40, np.zeros(40, np.float32))

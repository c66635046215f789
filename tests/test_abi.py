"""The C-ABI library without a GPU: it loads, exports every entry point include/artemis_sampler.h
declares, and its host-only functions (as_check, as_rng_seed) agree with the oracle."""
import ctypes as C
import os
import re

import pytest

import oracle_lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "artemis_sampler.h")


@pytest.fixture(scope="module")
def L():
    from artemis_amd import sampler
    if not os.path.exists(sampler.LIB_PATH):
        from artemis_amd import build
        build.build()
    return sampler.lib()


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|uint64_t|const char\*)\s+(as_\w+)\(", text, re.M)))


def test_the_library_exports_every_declared_entry_point(L):
    names = declared()
    assert len(names) >= 10, names
    for name in names:
        assert hasattr(L, name), name


def test_check_matches_the_oracle(L):
    from artemis_amd import Sampling
    nan, inf = float("nan"), float("inf")
    cases = [
        dict(), dict(temp=-0.1), dict(temp=nan), dict(temp=inf), dict(top_p=0.0), dict(top_p=1.1),
        dict(top_p=nan), dict(min_p=-0.1), dict(min_p=1.5), dict(presence=nan), dict(presence=-inf),
        dict(frequency=nan), dict(repetition=0.0), dict(repetition=-1.0), dict(repetition=inf),
        dict(temp=0.0, top_k=2, top_p=0.1, min_p=0.9),
    ]
    for kw in cases:
        want = oracle_lib.check(**{**oracle_lib.PLAIN, **kw})
        s = Sampling(temp=kw.get("temp", 1.0), top_k=kw.get("top_k", 0), top_p=kw.get("top_p", 1.0),
                     min_p=kw.get("min_p", 0.0), presence_penalty=kw.get("presence", 0.0),
                     frequency_penalty=kw.get("frequency", 0.0), repetition_penalty=kw.get("repetition", 1.0))
        if want is None:
            s.check()
        else:
            with pytest.raises(ValueError) as e:
                s.check()
            assert str(e.value) == want


def test_defaults_are_productions():
    from artemis_amd import Sampling
    assert Sampling.DEFAULT == Sampling(0.6, 20, 0.95, 0.0, 0.0)
    assert Sampling.GREEDY == Sampling(0.0, 0, 1.0, 0.0, 0.0)
    Sampling.DEFAULT.check()
    Sampling.GREEDY.check()


def test_rng_seed_matches_the_oracle(L):
    from artemis_amd import rng_state
    for seed in [0, 1, 7, 1234, 2**64 - 1]:
        assert rng_state(seed) == oracle_lib.Rng(seed).state()


def test_calls_without_a_context_fail_cleanly(L):
    assert L.as_sample(None, None, None) != 0
    assert L.as_sync(None) != 0
    assert L.as_destroy(None) != 0


def test_row_bytes_matches_the_oracle(L):
    from artemis_amd import WTYPE, row_bytes
    for name, code in WTYPE.items():
        for n in (0, 1, 2, 32, 100, 256, 512, 2048, 2080, 248320):
            assert L.as_row_bytes(code, n) == oracle_lib.row_bytes(code, n), (name, n)
    assert L.as_row_bytes(6, 256) == 0
    assert row_bytes(WTYPE["Q6_K"], 2048) == 8 * 210
    with pytest.raises(Exception):
        row_bytes(WTYPE["Q4_K"], 100)


def _rust_block(text, start):
    i = text.index(start)
    return text[i:text.index("\n}", i)]


def test_integration_binding_matches_the_header(L):
    """The Rust AsSampling of the integration notes at the repository root has the header's fields in the
    header's order, its From impl passes both new penalties through, and the check messages it quotes
    are as_check's."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    header = open(HEADER).read()
    c_struct = header[:header.index("} as_sampling;")]
    c_struct = c_struct[c_struct.rindex("typedef struct {"):]
    c_fields = re.findall(r"^\s*(?:float|uint32_t)\s+(\w+);", c_struct, re.M)
    rust = _rust_block(doc, "pub struct AsSampling {")
    r_fields = re.findall(r"pub (\w+): (f32|u32),", rust)
    assert [f for f, _ in r_fields] == c_fields
    assert [t for _, t in r_fields] == ["u32" if f in ("top_k", "reserved") else "f32" for f in c_fields]
    conv = _rust_block(doc, "impl From<&engine::Sampling> for AsSampling {")
    assert "frequency: s.frequency_penalty" in conv and "repetition: s.repetition_penalty" in conv
    from artemis_amd import Sampling
    for kw, flag in ((dict(frequency_penalty=float("nan")), "--frequency-penalty"),
                     (dict(repetition_penalty=0.0), "--repetition-penalty")):
        with pytest.raises(ValueError) as e:
            Sampling(temp=1.0, top_k=0, top_p=1.0, min_p=0.0, **kw).check()
        msg = str(e.value)
        assert msg.startswith(flag)
        tail = msg.split(" ", 2)[2]  # "must be ..."
        assert f'"{flag} {{}} {tail}"' in doc, (flag, tail)

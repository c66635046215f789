"""The committed fixtures (tests/golden/configs.json, written by tests/golden/make_golden.py): the
generated inputs still hash to the recorded SHA-256, and the oracle still gives the recorded
tokens, kept sets and RNG advances."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle_lib as O
from artemis_amd import workloads

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "configs.json")))


def rows_params(g, rows):
    p = g["params"]
    return [p] * rows if isinstance(p, dict) else p


def check_batch(g, w, shared):
    assert w.sha256() == g["sha256"]
    params = rows_params(g, len(w.seeds))
    off, ids = w.hist_csr()
    has = len(ids) > 0
    toks, rng = O.sample_rows(params, w.seeds, w.logits, off if has else None, ids if has else None,
                              threads=8, shared=shared)
    assert toks.tolist() == g["tokens"]
    assert hashlib.sha256(rng.astype("<u8").tobytes()).hexdigest() == g["rng_sha256"]
    assert [["%016x" % int(x) for x in s] for s in rng[: len(g["rng_first"])]] == g["rng_first"]
    for r, k in enumerate(g["kept"]):
        s = O.Sampler(w.seeds[r], **params[r])
        if w.histories and len(w.histories[r]):
            s.add_history(w.histories[r])
        assert s.sample(w.logits[0] if shared else w.logits[r]) == k["token"]
        kid, kp = s.last_kept(len(k["ids"]))
        assert kid.tolist() == k["ids"] and kp.tolist() == k["probs"]


def test_config1_inputs_and_greedy():
    g, w = GOLDEN["config1"], workloads.config1()
    assert w.sha256() == g["sha256"]
    assert O.greedy(w.logits[0]) == g["greedy"] and O.argmax_row(w.logits[0]) == g["argmax"]


def test_config2_inputs_and_draws():
    check_batch(GOLDEN["config2"], workloads.config2(), shared=True)


def test_config3_inputs_and_draws():
    check_batch(GOLDEN["config3"], workloads.config3(draws=64), shared=True)


def test_config4_inputs_and_verify():
    g, w = GOLDEN["config4"], workloads.config4()
    assert w.sha256() == g["sha256"]
    s = O.Sampler(g["seed"], **g["params"])
    picks, acc, _ = s.verify(w.logits, w.drafts)
    assert picks == g["picks"] and acc == g["accepted"] and picks[-1] == g["bonus"]
    assert ["%016x" % x for x in s.rng_state()] == g["rng"]


def test_config5_inputs_and_draws():
    check_batch(GOLDEN["config5"], workloads.config5(), shared=False)

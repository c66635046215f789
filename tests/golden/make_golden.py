"""Writes tests/golden/configs.json: the CPU oracle's outputs on the five benchmark configurations
(artemis_amd/workloads.py) with the SHA-256 of each configuration's generated inputs.

    python tests/golden/make_golden.py

The fixture pins the inputs (a change in the generator changes the hash) and the oracle's tokens,
kept sets and RNG advances, so the GPU tests can check the library against committed data.
u64 RNG words are written as hex strings (all rows' states as the SHA-256 of their little-endian
bytes, the first rows' in full); probabilities as JSON floats (exact round trip).
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

import oracle_lib as O  # noqa: E402
from artemis_amd import workloads  # noqa: E402

KEPT_ROWS = 8  # rows whose kept sets are recorded (configs 2, 3 and 5)
KEPT_MAX = 64  # at most this many kept (id, p) pairs per row


def as_dict(p):
    return dict(temp=p.temp, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p, presence=p.presence,
                frequency=p.frequency, repetition=p.repetition)


def hexs(words):
    return ["%016x" % int(x) for x in words]


def kept_of(p, seed, row, hist=None):
    s = O.Sampler(seed, **p)
    if hist is not None and len(hist):
        s.add_history(hist)
    tok = s.sample(row)
    ids, probs = s.last_kept(KEPT_MAX)
    n = lib_kept_count(s)
    return dict(token=int(tok), kept_count=int(n), ids=[int(i) for i in ids], probs=[float(x) for x in probs])


def lib_kept_count(s):
    return O.lib().oc_sampler_last_kept(s.h, None, None, 0)


def batch(w, shared):
    params = [as_dict(p) for p in w.params]
    off, ids = w.hist_csr()
    has_hist = len(ids) > 0
    toks, rng = O.sample_rows(params, w.seeds, w.logits, off if has_hist else None, ids if has_hist else None,
                              threads=8, shared=shared)
    rows = []
    for r in range(min(KEPT_ROWS, len(params))):
        row = w.logits[0] if shared else w.logits[r]
        rows.append(kept_of(params[r], w.seeds[r], row, w.histories[r] if w.histories else None))
        assert rows[-1]["token"] == int(toks[r])
    same = all(q == params[0] for q in params)
    return dict(sha256=w.sha256(), params=params[0] if same else params, seeds=list(w.seeds),
                tokens=[int(t) for t in toks], rng_sha256=hashlib.sha256(rng.astype("<u8").tobytes()).hexdigest(),
                rng_first=[hexs(s) for s in rng[:KEPT_ROWS]], kept=rows)


def main():
    out = {"generator": "artemis_amd/workloads.py", "oracle": "oracle/sampler_oracle.cc"}
    w = workloads.config1()
    out["config1"] = dict(sha256=w.sha256(), greedy=int(O.greedy(w.logits[0])),
                          argmax=int(O.argmax_row(w.logits[0])))
    out["config2"] = batch(workloads.config2(), shared=True)
    out["config3"] = batch(workloads.config3(draws=64), shared=True)
    w = workloads.config4()
    p = as_dict(w.params[0])
    s = O.Sampler(w.seeds[0], **p)
    picks, accepted, stopped = s.verify(w.logits, w.drafts)
    out["config4"] = dict(sha256=w.sha256(), params=p, seed=w.seeds[0], drafts=[int(d) for d in w.drafts],
                          picks=[int(x) for x in picks], read=len(picks), accepted=int(accepted),
                          bonus=int(picks[-1]), rng=hexs(s.rng_state()))
    out["config5"] = batch(workloads.config5(), shared=False)
    path = os.path.join(HERE, "configs.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0, separators=(",", ":"))
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()

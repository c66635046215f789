"""ctypes binding of the CPU oracle (oracle/liboracle_sampler.so) for the tests.

The oracle is the checker: tests compare the HIP path against it and pin it against the
reference's own known-answer and property tests. Nothing in artemis_amd imports this.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle_sampler.so")

u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)
f64p = C.POINTER(C.c_double)
u64p = C.POINTER(C.c_uint64)


class Params(C.Structure):
    _fields_ = [
        ("temp", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("presence", C.c_float),
        ("frequency", C.c_float),
        ("repetition", C.c_float),
        ("pad", C.c_uint32),
    ]


def params(temp=1.0, top_k=0, top_p=1.0, min_p=0.0, presence=0.0, frequency=0.0, repetition=1.0):
    return Params(temp, top_k, top_p, min_p, presence, frequency, repetition, 0)


# The reference's presets (sample.rs:53-68) and the tests' PLAIN (sample.rs:447-453).
DEFAULT = dict(temp=0.6, top_k=20, top_p=0.95, min_p=0.0, presence=0.0)
GREEDY = dict(temp=0.0, top_k=0, top_p=1.0, min_p=0.0, presence=0.0)
PLAIN = dict(temp=1.0, top_k=0, top_p=1.0, min_p=0.0, presence=0.0)

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        L = C.CDLL(LIB_PATH)
        L.oc_rng_new.argtypes = [C.c_uint64, u64p]
        L.oc_rng_next_u64.argtypes = [u64p]
        L.oc_rng_next_u64.restype = C.c_uint64
        L.oc_rng_unit.argtypes = [u64p]
        L.oc_rng_unit.restype = C.c_double
        L.oc_rng_below.argtypes = [u64p, C.c_uint64]
        L.oc_rng_below.restype = C.c_uint64
        L.oc_greedy.argtypes = [f32p, C.c_size_t]
        L.oc_greedy.restype = C.c_uint32
        L.oc_first_non_finite.argtypes = [f32p, C.c_size_t]
        L.oc_first_non_finite.restype = C.c_int64
        L.oc_argmax_row.argtypes = [f32p, C.c_size_t]
        L.oc_argmax_row.restype = C.c_uint32
        L.oc_check.argtypes = [C.POINTER(Params), C.c_char_p, C.c_size_t]
        L.oc_check.restype = C.c_int
        L.oc_sampler_new.argtypes = [C.POINTER(Params), C.c_uint64]
        L.oc_sampler_new.restype = C.c_void_p
        L.oc_sampler_free.argtypes = [C.c_void_p]
        L.oc_sampler_add_history.argtypes = [C.c_void_p, u32p, C.c_size_t]
        L.oc_sampler_get_rng.argtypes = [C.c_void_p, u64p]
        L.oc_sampler_set_rng.argtypes = [C.c_void_p, u64p]
        L.oc_sampler_sample.argtypes = [C.c_void_p, f32p, C.c_size_t]
        L.oc_sampler_sample.restype = C.c_uint32
        L.oc_sampler_last_kept.argtypes = [C.c_void_p, u32p, f64p, C.c_size_t]
        L.oc_sampler_last_kept.restype = C.c_size_t
        L.oc_sampler_last_path.argtypes = [C.c_void_p]
        L.oc_sampler_last_path.restype = C.c_int
        for name in ("oc_sampler_draw_full_sort", "oc_sampler_draw_partial"):
            f = getattr(L, name)
            f.argtypes = [C.c_void_p, u32p, f32p, C.c_size_t]
            f.restype = C.c_uint32
        for name in ("oc_top_k", "oc_selected"):
            f = getattr(L, name)
            f.argtypes = [C.c_void_p, f32p, C.c_size_t, C.c_size_t, u32p, f32p]
            f.restype = C.c_size_t
        L.oc_takes_one_pass.argtypes = [C.c_size_t, C.c_size_t]
        L.oc_takes_one_pass.restype = C.c_int
        L.oc_verify.argtypes = [C.c_void_p, f32p, C.c_size_t, u32p, C.c_size_t, u32p, C.c_size_t,
                                u32p, u32p, u32p]
        L.oc_verify.restype = C.c_size_t
        L.oc_sampler_sample_timed.argtypes = [C.c_void_p, f32p, C.c_size_t, u32p]
        L.oc_sampler_sample_timed.restype = C.c_double
        L.oc_verify_timed.argtypes = [C.c_void_p, f32p, C.c_size_t, u32p, C.c_size_t, u32p, u32p]
        L.oc_verify_timed.restype = C.c_double
        L.oc_logprobs.argtypes = [f32p, C.c_size_t, C.c_uint32, C.c_uint32, u32p, f32p,
                                  C.POINTER(C.c_size_t)]
        L.oc_logprobs.restype = C.c_float
        L.oc_exp.argtypes = [C.c_double]
        L.oc_exp.restype = C.c_double
        L.oc_log.argtypes = [C.c_double]
        L.oc_log.restype = C.c_double
        L.oc_exp_array.argtypes = [f64p, f64p, C.c_size_t]
        L.oc_sample_rows.argtypes = [C.POINTER(Params), u64p, f32p, C.c_size_t, C.c_size_t,
                                     C.c_size_t, u32p, u32p, C.c_uint, u32p, u64p]
        L.oc_row_bytes.argtypes = [C.c_uint32, C.c_uint64]
        L.oc_row_bytes.restype = C.c_uint64
        L.oc_dequant_row.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, f32p]
        L.oc_dequant_row.restype = C.c_int
        L.oc_half_to_float.argtypes = [C.c_uint16]
        L.oc_half_to_float.restype = C.c_float
        L.oc_matvec.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, f32p, f32p]
        L.oc_matvec.restype = C.c_int
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(f32p)


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(u32p)


class Rng:
    """rng.rs's Rng."""

    def __init__(self, seed: int):
        self.s = (C.c_uint64 * 4)()
        lib().oc_rng_new(seed, self.s)

    def next_u64(self) -> int:
        return lib().oc_rng_next_u64(self.s)

    def unit(self) -> float:
        return lib().oc_rng_unit(self.s)

    def below(self, n: int) -> int:
        return lib().oc_rng_below(self.s, n)

    def state(self):
        return [int(x) for x in self.s]


def greedy(logits) -> int:
    a, p = _f32(logits)
    return lib().oc_greedy(p, len(a))


def first_non_finite(logits):
    a, p = _f32(logits)
    r = lib().oc_first_non_finite(p, len(a))
    return None if r < 0 else (r, a[r])


def argmax_row(logits):
    a, p = _f32(logits)
    r = lib().oc_argmax_row(p, len(a))
    return None if r == 0xFFFFFFFF else r


def check(**kw):
    buf = C.create_string_buffer(200)
    P = params(**kw)
    r = lib().oc_check(C.byref(P), buf, 200)
    return None if r == 0 else buf.value.decode()


class Sampler:
    """sample.rs's Sampler, with the history penalties."""

    def __init__(self, seed: int = 0, **kw):
        self.p = params(**kw)
        self.h = lib().oc_sampler_new(C.byref(self.p), seed)

    def __del__(self):
        if getattr(self, "h", None):
            lib().oc_sampler_free(self.h)
            self.h = None

    def add_history(self, ids):
        a, p = _u32(ids)
        lib().oc_sampler_add_history(self.h, p, len(a))

    def rng_state(self):
        s = (C.c_uint64 * 4)()
        lib().oc_sampler_get_rng(self.h, s)
        return [int(x) for x in s]

    def set_rng_state(self, st):
        s = (C.c_uint64 * 4)(*st)
        lib().oc_sampler_set_rng(self.h, s)

    def sample(self, logits) -> int:
        a, p = _f32(logits)
        return lib().oc_sampler_sample(self.h, p, len(a))

    def sample_timed(self, logits):
        """(token, ns): the non-finite check and one sample, timed in C."""
        a, p = _f32(logits)
        t = C.c_uint32()
        ns = lib().oc_sampler_sample_timed(self.h, p, len(a), C.byref(t))
        return t.value, ns

    def verify_timed(self, rows, drafts):
        """(picks, ns): the verify loop over k+1 rows, each checked first, timed in C."""
        r = np.ascontiguousarray(rows, dtype=np.float32)
        k = len(drafts)
        d, dp = _u32(drafts if k else [0])
        picks = np.zeros(k + 1, np.uint32)
        read = C.c_uint32()
        ns = lib().oc_verify_timed(self.h, r.ctypes.data_as(f32p), r.shape[1], dp, k,
                                   picks.ctypes.data_as(u32p), C.byref(read))
        return picks[: read.value].tolist(), ns

    def last_kept(self, cap=1 << 20):
        n = lib().oc_sampler_last_kept(self.h, None, None, 0)
        m = min(n, cap)
        ids = np.zeros(m, np.uint32)
        probs = np.zeros(m, np.float64)
        lib().oc_sampler_last_kept(self.h, ids.ctypes.data_as(u32p), probs.ctypes.data_as(f64p), m)
        return ids, probs

    def last_path(self) -> int:
        return lib().oc_sampler_last_path(self.h)

    def draw_full_sort(self, ids, vals) -> int:
        i, ip = _u32(ids)
        v, vp = _f32(vals)
        return lib().oc_sampler_draw_full_sort(self.h, ip, vp, len(i))

    def draw_partial(self, ids, vals) -> int:
        i, ip = _u32(ids)
        v, vp = _f32(vals)
        return lib().oc_sampler_draw_partial(self.h, ip, vp, len(i))

    def top_k(self, logits, k):
        a, p = _f32(logits)
        ids = np.zeros(k, np.uint32)
        vals = np.zeros(k, np.float32)
        n = lib().oc_top_k(self.h, p, len(a), k, ids.ctypes.data_as(u32p), vals.ctypes.data_as(f32p))
        return list(zip(ids[:n].tolist(), vals[:n].view(np.uint32).tolist()))

    def selected(self, logits, k):
        a, p = _f32(logits)
        ids = np.zeros(k, np.uint32)
        vals = np.zeros(k, np.float32)
        n = lib().oc_selected(self.h, p, len(a), k, ids.ctypes.data_as(u32p), vals.ctypes.data_as(f32p))
        return list(zip(ids[:n].tolist(), vals[:n].view(np.uint32).tolist()))

    def verify(self, rows, drafts, stop_ids=()):
        r = np.ascontiguousarray(rows, dtype=np.float32)
        n = r.shape[1]
        k = len(drafts)
        assert r.shape[0] == k + 1
        d, dp = _u32(drafts if k else [0])
        s, sp = _u32(list(stop_ids) if stop_ids else [0])
        picks = np.zeros(k + 1, np.uint32)
        acc = C.c_uint32()
        stopped = C.c_uint32()
        read = lib().oc_verify(self.h, r.ctypes.data_as(f32p), n, dp, k, sp, len(stop_ids),
                               picks.ctypes.data_as(u32p), C.byref(acc), C.byref(stopped))
        return picks[:read].tolist(), acc.value, bool(stopped.value)


def takes_one_pass(k, n) -> bool:
    return bool(lib().oc_takes_one_pass(k, n))


def logprobs(logits, token, top):
    a, p = _f32(logits)
    ids = np.zeros(20, np.uint32)
    lps = np.zeros(20, np.float32)
    nt = C.c_size_t()
    lp = lib().oc_logprobs(p, len(a), token, top, ids.ctypes.data_as(u32p), lps.ctypes.data_as(f32p),
                           C.byref(nt))
    return lp, list(zip(ids[: nt.value].tolist(), lps[: nt.value].tolist()))


def host_exp(x: float) -> float:
    return lib().oc_exp(x)


def host_log(x: float) -> float:
    return lib().oc_log(x)


def exp_array(x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x)
    lib().oc_exp_array(x.ctypes.data_as(f64p), y.ctypes.data_as(f64p), x.size)
    return y


def sample_rows(rows_params, seeds, logits, hist_off=None, hist_ids=None, threads=1, shared=False):
    """oc_sample_rows: one fresh-sampler draw per row. Returns (tokens u32, rng states [rows, 4])."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    n = logits.shape[-1]
    rows = len(rows_params)
    P = (Params * rows)(*[params(**p) if isinstance(p, dict) else p for p in rows_params])
    s = np.ascontiguousarray(seeds, dtype=np.uint64)
    toks = np.zeros(rows, np.uint32)
    rng = np.zeros((rows, 4), np.uint64)
    if hist_off is not None:
        ho = np.ascontiguousarray(hist_off, dtype=np.uint32)
        hi = np.ascontiguousarray(hist_ids if len(hist_ids) else [0], dtype=np.uint32)
        hop, hip = ho.ctypes.data_as(u32p), hi.ctypes.data_as(u32p)
    else:
        hop = hip = None
    lib().oc_sample_rows(P, s.ctypes.data_as(u64p), logits.ctypes.data_as(f32p), 0 if shared else n, n,
                         rows, hop, hip, threads, toks.ctypes.data_as(u32p), rng.ctypes.data_as(u64p))
    return toks, rng


# Weight types by the reference's codes (quant.glsl:2-8).
WTYPES = {"F32": 0, "BF16": 1, "Q8_0": 2, "Q4_K": 3, "Q5_K": 4, "Q6_K": 5}


def row_bytes(wtype: int, n: int) -> int:
    return lib().oc_row_bytes(wtype, n)


def dequant_row(wtype: int, row, n: int):
    """quant.rs:77-104 on one row's bytes: n f32 values."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(row), dtype=np.uint8))
    out = np.zeros(n, np.float32)
    rc = lib().oc_dequant_row(wtype, raw.ctypes.data, n, out.ctypes.data_as(f32p))
    if rc != 0:
        raise ValueError("not a whole-block row")
    return out


def matvec(wtype: int, w, rows: int, k: int, x):
    """twin/matvec.rs:126-131: y = W x, each output as the reference's 32-lane matvec row sums it."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(w), dtype=np.uint8))
    assert raw.size == rows * row_bytes(wtype, k)
    xa, xp = _f32(x)
    y = np.zeros(rows, np.float32)
    if lib().oc_matvec(wtype, raw.ctypes.data, rows, k, xp, y.ctypes.data_as(f32p)) != 0:
        raise ValueError("bad matvec shape")
    return y

"""The reference's sampler interface over the HIP library (include/artemis_sampler.h).

Mirrors crates/engine/src/sample.rs and rng.rs: `Sampling` (with `DEFAULT`, `GREEDY` and
`check`), `Sampler(s, seed).sample(logits)`, `greedy(logits)` and `Rng`; plus the batched call
the GPU path exists for (`sample_batch`), the speculative verify (`verify`) and `argmax_rows`.
Logits are torch tensors on the GPU; everything is ordered on torch's current stream. There is no
CPU fallback: without the built library or a GPU these raise.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, replace
from typing import List, Optional, Sequence

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libartemis_sampler.so")

AS_OK = 0
AS_ROW_OK = 0
AS_ROW_NONFINITE = 1
AS_ROW_HISTORY = 2
AS_ROW_EXACT_PATH = 0x100
AS_ROW_KEPT_PARTIAL = 0x200
AS_ROW_DEEP_PATH = 0x400
AS_ROW_TAIL_PASS = 0x800
NO_DRAFT = 0xFFFFFFFF
AS_LP_OK = 0
AS_LP_INEXACT = 1
LP_MAX_TOP = 20  # logprobs.rs:7


class SamplerError(RuntimeError):
    """A call into the HIP sampler failed; the message is the library's."""


class _CSampling(C.Structure):
    _fields_ = [
        ("temp", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("presence", C.c_float),
        ("frequency", C.c_float),
        ("repetition", C.c_float),
        ("reserved", C.c_uint32),
    ]


class _CBatch(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p),
        ("row_stride", C.c_uint64),
        ("n_vocab", C.c_uint32),
        ("n_rows", C.c_uint32),
        ("hist_offsets", C.c_void_p),
        ("hist_ids", C.c_void_p),
        ("rng_state", C.c_void_p),
        ("tokens", C.c_void_p),
        ("status", C.c_void_p),
        ("kept_count", C.c_void_p),
        ("kept_ids", C.c_void_p),
        ("kept_probs", C.c_void_p),
        ("kept_cap", C.c_uint32),
    ]


# Weight types of embedding rows, by the reference's codes (kernels/src/lib.rs:438-447).
WTYPE = {"F32": 0, "BF16": 1, "Q8_0": 2, "Q4_K": 3, "Q5_K": 4, "Q6_K": 5}


def row_bytes(wtype: int, n: int) -> int:
    """WType::row_bytes (quant.rs:66-74); raises for an unknown type or a partial block."""
    b = lib().as_row_bytes(wtype, n)
    if b == 0 and n != 0:
        raise SamplerError(f"weight type {wtype} has no rows of {n} values (unknown type, or not whole blocks)")
    return b


_lib = None


def lib() -> C.CDLL:
    """The built library; raises if `build()` has not produced it."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SamplerError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(LIB_PATH)
        vp, u32, u64 = C.c_void_p, C.c_uint32, C.c_uint64
        L.as_create.argtypes = [C.c_int, vp, u32, u32, u32, C.POINTER(vp)]
        L.as_destroy.argtypes = [vp]
        L.as_last_error.argtypes = [vp]
        L.as_last_error.restype = C.c_char_p
        L.as_sync.argtypes = [vp]
        L.as_check.argtypes = [C.POINTER(_CSampling), C.c_char_p, C.c_size_t]
        L.as_rng_seed.argtypes = [u64, C.POINTER(u64)]
        L.as_rng_seed.restype = None
        L.as_sample.argtypes = [vp, C.POINTER(_CBatch), C.POINTER(_CSampling)]
        L.as_verify.argtypes = [vp, vp, u64, u32, vp, u32, vp, u32, vp, u32, C.POINTER(_CSampling),
                                vp, vp, vp]
        L.as_argmax_rows.argtypes = [vp, vp, u64, u32, u32, vp, vp, u64, u32, u32]
        L.as_row_bytes.argtypes = [u32, u64]
        L.as_row_bytes.restype = u64
        L.as_embed_rows.argtypes = [vp, vp, u32, u32, vp, u32]
        L.as_matvec.argtypes = [vp, vp, u32, u32, u32, vp, vp]
        L.as_head_argmax.argtypes = [vp, vp, u32, u32, u32, vp, vp, vp, vp, u64, u32, u32]
        L.as_debug_exp.argtypes = [vp, vp, vp, u32]
        L.as_debug_exp2f.argtypes = [vp, vp, vp, u32]
        L.as_logprobs.argtypes = [vp, vp, u64, u32, u32, vp, u32, vp, vp, vp, vp]
        L.as_logprobs_static.argtypes = [vp, vp, u64, u32, u32, vp, u32, vp, vp, vp, vp, C.c_char_p, C.c_size_t]
        L.as_profile.argtypes = [vp, C.c_int]
        L.as_profile_read.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(u32)]
        _lib = L
    return _lib


@dataclass(frozen=True)
class Sampling:
    """How the sampler chooses (sample.rs:38-49), plus the frequency and repetition penalties."""

    temp: float = 0.6
    top_k: int = 20
    top_p: float = 0.95
    min_p: float = 0.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0

    def check(self) -> None:
        """Sampling::check (sample.rs:71-94): raises ValueError naming the flag."""
        buf = C.create_string_buffer(200)
        if lib().as_check(C.byref(self._c()), buf, 200) != AS_OK:
            raise ValueError(buf.value.decode())

    def _c(self) -> _CSampling:
        return _CSampling(self.temp, self.top_k, self.top_p, self.min_p, self.presence_penalty,
                          self.frequency_penalty, self.repetition_penalty, 0)


Sampling.DEFAULT = Sampling(0.6, 20, 0.95, 0.0, 0.0)  # sample.rs:53-59
Sampling.GREEDY = Sampling(0.0, 0, 1.0, 0.0, 0.0)     # sample.rs:62-68


def rng_state(seed: int) -> List[int]:
    """Rng::new (rng.rs:11-23): the xoshiro256** state for `seed`, as four u64."""
    s = (C.c_uint64 * 4)()
    lib().as_rng_seed(seed, s)
    return [int(x) for x in s]


class PackedSampling:
    """A batch's settings converted once to the C ABI's as_sampling array, for callers that sample the
    same rows' settings step after step (the engine holds such an array; building it from Python
    objects costs far more than the call)."""

    def __init__(self, params: Sequence[Sampling]):
        self.n = len(params)
        self.arr = (_CSampling * self.n)(*[p._c() for p in params])

    def __len__(self) -> int:
        return self.n


def _u64_as_i64(xs: Sequence[int]) -> List[int]:
    return [x - (1 << 64) if x >= (1 << 63) else x for x in xs]


def states_tensor(seeds: Sequence[int], device="cuda") -> torch.Tensor:
    """[n, 4] int64 (bit-cast u64) RNG states for the seeds, on the device."""
    rows = [_u64_as_i64(rng_state(s)) for s in seeds]
    return torch.tensor(rows, dtype=torch.int64, device=device)


class Context:
    """One library context on a device, ordered on torch's current stream when created."""

    def __init__(self, max_rows: int, max_vocab: int, max_history: int = 65535, device: int = 0,
                 stream: Optional[torch.cuda.Stream] = None):
        if not torch.cuda.is_available():
            raise SamplerError("no GPU: the sampler runs on the GPU only")
        L = lib()
        torch.cuda.set_device(device)
        st = stream if stream is not None else torch.cuda.current_stream(device)
        self.stream = st
        h = C.c_void_p()
        rc = L.as_create(device, C.c_void_p(st.cuda_stream), max_rows, max_vocab, max_history, C.byref(h))
        if rc != AS_OK:
            raise SamplerError(f"as_create failed ({rc})")
        self.h = h
        self.max_rows, self.max_vocab, self.device = max_rows, max_vocab, device

    def close(self):
        if getattr(self, "h", None):
            lib().as_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ok(self, rc: int):
        if rc != AS_OK:
            raise SamplerError(lib().as_last_error(self.h).decode() or f"error {rc}")

    def sync(self):
        self._ok(lib().as_sync(self.h))

    def outputs(self, n_rows: int, kept_cap: int = 0, device=None):
        """Output tensors for sample_batch's `out`: (tokens, status, kept_count, kept_ids, kept_probs)."""
        dev = device if device is not None else torch.device("cuda", self.device)
        return (torch.empty(n_rows, dtype=torch.int32, device=dev), torch.empty(n_rows, dtype=torch.int32, device=dev),
                torch.empty(n_rows, dtype=torch.int32, device=dev),
                torch.empty((n_rows, max(kept_cap, 1)), dtype=torch.int32, device=dev),
                torch.empty((n_rows, max(kept_cap, 1)), dtype=torch.float64, device=dev))

    def sample_batch(self, logits: torch.Tensor, params, rng: torch.Tensor,
                     hist_offsets: Optional[torch.Tensor] = None, hist_ids: Optional[torch.Tensor] = None,
                     kept_cap: int = 0, row_stride: Optional[int] = None, n_vocab: Optional[int] = None,
                     out=None):
        """Sampler::sample on every row at once. `params`: a sequence of Sampling, or a
        PackedSampling. Returns (tokens, status, kept_count, kept_ids, kept_probs) device tensors
        (`out` when given, from outputs()); `rng` ([n, 4] int64) is advanced in place."""
        n_rows = len(params)
        assert logits.is_cuda and logits.dtype == torch.float32
        stride = row_stride if row_stride is not None else logits.stride(0)
        nv = n_vocab if n_vocab is not None else logits.shape[-1]
        dev = logits.device
        if out is None:
            out = self.outputs(n_rows, kept_cap, dev)
        tokens, status, kept_count, kept_ids, kept_probs = out
        assert tokens.numel() >= n_rows and status.numel() >= n_rows and kept_count.numel() >= n_rows
        assert kept_ids.shape[-1] >= max(kept_cap, 1) and kept_probs.shape[-1] >= max(kept_cap, 1)
        assert rng.dtype == torch.int64 and rng.is_cuda and rng.shape[0] >= n_rows
        b = _CBatch()
        b.logits = logits.data_ptr()
        b.row_stride = stride
        b.n_vocab = nv
        b.n_rows = n_rows
        if hist_ids is not None:
            assert hist_offsets is not None and hist_offsets.dtype == torch.int32
            assert hist_ids.dtype == torch.int32
            b.hist_offsets = hist_offsets.data_ptr()
            b.hist_ids = hist_ids.data_ptr() if hist_ids.numel() else hist_offsets.data_ptr()
        b.rng_state = rng.data_ptr()
        b.tokens = tokens.data_ptr()
        b.status = status.data_ptr()
        b.kept_count = kept_count.data_ptr()
        if kept_cap:
            b.kept_ids = kept_ids.data_ptr()
            b.kept_probs = kept_probs.data_ptr()
            b.kept_cap = kept_cap
        arr = params.arr if isinstance(params, PackedSampling) else (_CSampling * n_rows)(*[p._c() for p in params])
        self._ok(lib().as_sample(self.h, C.byref(b), arr))
        return tokens, status, kept_count, kept_ids, kept_probs

    def verify(self, rows: torch.Tensor, drafts: torch.Tensor, params: Sampling, rng: torch.Tensor,
               history: Optional[torch.Tensor] = None, stop_ids: Optional[torch.Tensor] = None):
        """The speculative accept over k+1 rows; returns (picks, result) device tensors with
        result = [read, accepted, bonus, flags]."""
        k = int(drafts.numel())
        assert rows.shape[0] == k + 1
        dev = rows.device
        picks = torch.empty(k + 1, dtype=torch.int32, device=dev)
        result = torch.empty(4, dtype=torch.int32, device=dev)
        hist_len = int(history.numel()) if history is not None else 0
        n_stop = int(stop_ids.numel()) if stop_ids is not None else 0
        rc = lib().as_verify(self.h, rows.data_ptr(), rows.stride(0), rows.shape[1],
                             drafts.data_ptr() if k else None, k,
                             history.data_ptr() if hist_len else None, hist_len,
                             stop_ids.data_ptr() if n_stop else None, n_stop, C.byref(params._c()),
                             rng.data_ptr(), picks.data_ptr(), result.data_ptr())
        self._ok(rc)
        return picks, result

    def argmax_rows(self, logits: torch.Tensor, ids: torch.Tensor, rows_out: torch.Tensor, embd: int,
                    row_bytes: int, slot: int = 0, n: Optional[int] = None):
        """argmax_rows (dispatch.rs:121-153) on every row of `logits`."""
        if logits.dim() == 1:
            logits = logits.view(1, -1)
        nv = n if n is not None else logits.shape[1]
        self._ok(lib().as_argmax_rows(self.h, logits.data_ptr(), logits.stride(0), nv, logits.shape[0],
                                      ids.data_ptr(), rows_out.data_ptr(), embd, row_bytes, slot))

    def embed_rows(self, rows: torch.Tensor, wtype: int, n: int, y: Optional[torch.Tensor] = None) -> torch.Tensor:
        """embed_rows (dispatch.rs:97-120): y[t] = the embedding row at device address rows[t]
        dequantized (quant.rs:77-252). `rows`: [tokens] int64 on the device, as argmax_rows writes
        them; `wtype`: one of WTYPE's codes; returns y ([tokens, n] f32 on the device)."""
        assert rows.is_cuda and rows.dtype == torch.int64 and rows.is_contiguous()
        t = rows.numel()
        if y is None:
            y = torch.empty((t, n), dtype=torch.float32, device=rows.device)
        assert y.is_cuda and y.dtype == torch.float32 and y.is_contiguous() and y.numel() >= t * n
        self._ok(lib().as_embed_rows(self.h, rows.data_ptr(), wtype, n, y.data_ptr(), t))
        return y

    def matvec(self, w: torch.Tensor, wtype: int, rows: int, k: int, x: torch.Tensor,
               y: Optional[torch.Tensor] = None) -> torch.Tensor:
        """matvec (dispatch.rs Kernels::matvec): y = W x, bit for bit the reference's. `w`: the rows'
        bytes on the device (row r at r * row_bytes(wtype, k)); `x`: [k] f32; returns y ([rows] f32)."""
        assert w.is_cuda and x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.numel() == k
        assert w.numel() * w.element_size() >= rows * row_bytes(wtype, k)
        if y is None:
            y = torch.empty(rows, dtype=torch.float32, device=x.device)
        assert y.is_cuda and y.dtype == torch.float32 and y.numel() >= rows
        self._ok(lib().as_matvec(self.h, w.data_ptr(), wtype, rows, k, x.data_ptr(), y.data_ptr()))
        return y

    def head_argmax(self, w: torch.Tensor, wtype: int, rows: int, k: int, x: torch.Tensor, ids: torch.Tensor,
                    rows_out: torch.Tensor, embd: int, embd_row_bytes: int, slot: int = 0,
                    logits: Optional[torch.Tensor] = None) -> None:
        """The head's matvec with argmax_rows fused: ids[slot] and rows_out[slot] as argmax_rows
        (dispatch.rs:121-153) would write them from the head's logits; `logits` (optional) gets
        the logits too."""
        assert w.is_cuda and x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.numel() == k
        assert w.numel() * w.element_size() >= rows * row_bytes(wtype, k)
        assert ids.is_cuda and ids.dtype == torch.int32 and ids.numel() > slot
        assert rows_out.is_cuda and rows_out.dtype == torch.int64 and rows_out.numel() > slot
        lp = 0
        if logits is not None:
            assert logits.is_cuda and logits.dtype == torch.float32 and logits.numel() >= rows
            lp = logits.data_ptr()
        self._ok(lib().as_head_argmax(self.h, w.data_ptr(), wtype, rows, k, x.data_ptr(), lp, ids.data_ptr(),
                                      rows_out.data_ptr(), embd, embd_row_bytes, slot))

    def logprobs(self, logits: torch.Tensor, tokens: torch.Tensor, top: int, row_stride: Optional[int] = None,
                 n_vocab: Optional[int] = None):
        """logprobs (logprobs.rs:12-38) on every row: (logprob [n] f32, top_ids [n, top] int32,
        top_logprobs [n, top] f32, status [n] int32) device tensors; the first min(top, 20, n_vocab)
        columns of each row are written, any others hold -1 and NaN. `tokens`: [n] int32 on the
        device."""
        if logits.dim() == 1:
            logits = logits.view(1, -1)
        assert logits.is_cuda and logits.dtype == torch.float32
        assert tokens.is_cuda and tokens.dtype == torch.int32
        rows = tokens.numel()
        stride = row_stride if row_stride is not None else (logits.stride(0) if logits.shape[0] > 1 else logits.shape[1])
        nv = n_vocab if n_vocab is not None else logits.shape[1]
        dev = logits.device
        lp = torch.empty(rows, dtype=torch.float32, device=dev)
        cols = max(top, 1)
        if 0 < top <= min(LP_MAX_TOP, nv):
            # The library writes every column.
            ids = torch.empty((rows, cols), dtype=torch.int32, device=dev)
            lps = torch.empty((rows, cols), dtype=torch.float32, device=dev)
        else:
            ids = torch.full((rows, cols), -1, dtype=torch.int32, device=dev)
            lps = torch.full((rows, cols), float("nan"), dtype=torch.float32, device=dev)
        st = torch.empty(rows, dtype=torch.int32, device=dev)
        self._ok(lib().as_logprobs(self.h, logits.data_ptr(), stride, nv, rows, tokens.data_ptr(), top,
                                   lp.data_ptr(), ids.data_ptr() if top else None,
                                   lps.data_ptr() if top else None, st.data_ptr()))
        return lp, ids, lps, st

    def profile(self, enable: bool):
        """Start (or stop) recording HIP events around each call's scan and finish kernels."""
        self._ok(lib().as_profile(self.h, 1 if enable else 0))

    def profile_read(self):
        """(scan_ms, finish_ms, calls) summed since profile(True); waits for the stream."""
        a, b, k = C.c_double(), C.c_double(), C.c_uint32()
        self._ok(lib().as_profile_read(self.h, C.byref(a), C.byref(b), C.byref(k)))
        return a.value, b.value, k.value

    def debug_exp(self, x: torch.Tensor) -> torch.Tensor:
        y = torch.empty_like(x)
        self._ok(lib().as_debug_exp(self.h, x.data_ptr(), y.data_ptr(), x.numel()))
        return y

    def debug_exp2f(self, x: torch.Tensor) -> torch.Tensor:
        """2^x by the GPU instruction behind the scan's sums (diagnostics)."""
        assert x.is_cuda and x.dtype == torch.float32
        y = torch.empty_like(x)
        self._ok(lib().as_debug_exp2f(self.h, x.data_ptr(), y.data_ptr(), x.numel()))
        torch.cuda.synchronize()
        return y


_contexts = {}


def _context_for(n_vocab: int, device: int) -> Context:
    key = device
    c = _contexts.get(key)
    if c is None or c.max_vocab < n_vocab:
        c = Context(max_rows=64, max_vocab=max(n_vocab, 262144), device=device)
        _contexts[key] = c
    return c


class Sampler:
    """Sampler (sample.rs:97-153): draws tokens from device logits with a seeded stream. The
    history penalties act on the tokens this sampler returned, as the reference's `seen`."""

    def __init__(self, s: Sampling, seed: int):
        self.s = s
        self.seed = seed
        self.history: List[int] = []
        self._rng = None
        self._rng_host = rng_state(seed)

    def _state(self, device):
        if self._rng is None:
            self._rng = torch.tensor([_u64_as_i64(self._rng_host)], dtype=torch.int64, device=device)
        return self._rng

    def sample(self, logits: torch.Tensor) -> int:
        """The next token; raises on a row holding NaN or an infinity (Error::NonFinite)."""
        if logits.numel() == 0:
            raise ValueError("sampling from no logits")
        row = logits.reshape(1, -1)
        ctx = _context_for(row.shape[1], row.device.index or 0)
        if self.history:
            ids = torch.tensor(self.history, dtype=torch.int32, device=row.device)
            off = torch.tensor([0, len(self.history)], dtype=torch.int32, device=row.device)
        else:
            ids = off = None
        tok, st, *_ = ctx.sample_batch(row, [self.s], self._state(row.device), off, ids)
        t, s = int(tok.item()), int(st.item())
        if s & AS_ROW_NONFINITE:
            raise SamplerError(f"non-finite logit at {int(_[0].item())}")
        self.history.append(t)
        return t


def logprobs(logits: torch.Tensor, token: int, top: int):
    """logprobs (logprobs.rs:12-38) of one finite row on the GPU: (token's log-probability,
    [(id, log-probability)] for the min(top, 20, n) highest logits, by logit descending then id)."""
    row = logits.reshape(1, -1)
    ctx = _context_for(row.shape[1], row.device.index or 0)
    tok = torch.tensor([token], dtype=torch.int32, device=row.device)
    lp, ids, lps, _ = ctx.logprobs(row, tok, top)
    n = min(top, LP_MAX_TOP, row.shape[1])
    ids_h, lps_h = ids.cpu().numpy()[0], lps.cpu().numpy()[0]
    return float(lp.item()), [(int(ids_h[i]), float(lps_h[i])) for i in range(n)]


def greedy(logits: torch.Tensor) -> int:
    """greedy (sample.rs:9-17) of a finite row."""
    return Sampler(Sampling.GREEDY, 0).sample(logits)

"""MI355X (gfx950) token sampler and speculative verify: HIP kernels behind a C ABI
(include/artemis_sampler.h), with the reference's sampler interface in `artemis_amd.sampler`."""
from .sampler import (AS_LP_INEXACT, AS_LP_OK, AS_ROW_DEEP_PATH, AS_ROW_EXACT_PATH, AS_ROW_HISTORY,
                      AS_ROW_KEPT_PARTIAL, AS_ROW_NONFINITE, AS_ROW_OK, AS_ROW_TAIL_PASS, LP_MAX_TOP, NO_DRAFT, WTYPE, Context,
                      PackedSampling, Sampler, SamplerError, Sampling, greedy, logprobs, rng_state, row_bytes,
                      states_tensor)

__all__ = ["AS_LP_INEXACT", "AS_LP_OK", "AS_ROW_DEEP_PATH", "AS_ROW_EXACT_PATH", "AS_ROW_HISTORY", "AS_ROW_KEPT_PARTIAL",
           "AS_ROW_NONFINITE", "AS_ROW_OK", "AS_ROW_TAIL_PASS", "LP_MAX_TOP", "NO_DRAFT", "Context",
           "PackedSampling", "Sampler", "SamplerError", "Sampling", "WTYPE", "greedy", "logprobs", "rng_state",
           "row_bytes", "states_tensor"]

// Host-side launchers of the sampler kernels (each defined beside its kernel).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sampler_device.h"

namespace as_launch {

// Values one scan workgroup covers (256 threads x 32 values).
constexpr int kSegment = 8192;
// Candidates the finish kernel sorts in LDS: segments x per-segment candidates must fit.
constexpr int kCandCap = 8192;
// Per-segment candidate budget (the finish kernel takes segments x budget <= kCandCap).
constexpr int kPartialCand = 256;
// Rows without a top-k keep each segment's values at or above the 192nd largest of its threads'
// two largest values (about 200 values of a segment of normally spread logits).
constexpr int kPartialRank = 192;

struct FinishArgs {
  const float* logits;
  uint64_t row_stride;
  uint32_t n;
  uint32_t n_seg;
  const as_dev::RowParams* params;
  const uint32_t* hist_off;
  const uint32_t* hist_ids;
  const uint32_t* extra_ids;
  const as_dev::SegStats* stats;
  const uint64_t* cands;
  uint32_t cand_stride;
  uint32_t kept_cap;
  uint64_t* rng_state;
  uint32_t* tokens;
  uint32_t* status;
  uint32_t* kept_count;
  uint32_t* kept_ids;
  double* kept_probs;
  uint32_t vec;             // the rows are 16-byte aligned (float4 loads)
  uint32_t* scratch;        // deep and exact paths: 5 x n u32 (+ alignment) per row
  uint64_t scratch_stride;  // u32 per row
};

hipError_t scan(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride, uint32_t n,
                uint32_t n_rows, uint32_t n_seg, const as_dev::RowParams* params,
                const uint32_t* hist_off, const uint32_t* hist_ids, const uint32_t* extra_ids,
                as_dev::SegStats* stats, uint64_t* cands, uint32_t cand_stride);

hipError_t finish(hipStream_t stream, uint32_t n_rows, const FinishArgs* a);

hipError_t accept(hipStream_t stream, const uint32_t* picks, const uint32_t* status,
                  const uint32_t* drafts, uint32_t k, const uint32_t* stop_ids, uint32_t n_stop,
                  uint64_t* rng_state, uint32_t draws_per_row, uint32_t* result);

hipError_t argmax_rows(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride,
                       uint32_t n, uint32_t n_rows, uint32_t* ids, uint64_t* rows_out,
                       uint64_t embd, uint32_t row_bytes, uint32_t slot);

hipError_t debug_exp(hipStream_t stream, const double* x, double* y, uint32_t n);

}  // namespace as_launch

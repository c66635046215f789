// Pass 2, one 1024-thread workgroup per row: merges the slices' results and chooses the token.
//
// The scan leaves, per slice, its statistics (non-finite index, greedy pick, largest key, sums) and
// the values ranking at or above its bound; R, the largest bound of a truncated slice (raised to
// min-p's floor), makes every value of the row ranking >= R a candidate. The candidates >= R are
// loaded into LDS and bucket-sorted by rank.
//
// Top-k rows: when at least k candidates rank >= R they hold the row's k best, and one thread runs
// draw_full_sort's f64 tail (sample.rs:157-198) in the reference's own order, so every sum and
// comparison is bit-exact.
//
// Rows without a top-k (draw_partial, sample.rs:208-293): the sorted candidates are a complete rank
// prefix down to R. The min-p cut is an exact comparison. The top-p cut and the unfiltered draw
// depend on a sum over the whole row in index order; that sum comes from the slices' partial sums
// with a rigorous error bound that covers the reference's own left-to-right rounding, and a
// decision is taken only when the bound cannot change it. The kept set's draw is then exact.
// A row whose cut or draw lies past the candidates takes the deep path (a histogram of the row,
// then every value down to the deciding bin, sorted in HBM scratch); one whose decision a bound
// still cannot settle takes the exact-order path: a stable radix sort of the whole row and the
// reference's sequential folds, so its token is the reference's in every case.
#include "sampler_device.h"
#include "launch.h"
#include "fold.h"
#include "../../include/artemis_sampler.h"

#define AS_FIN_NS as_fin_sliced
#define AS_FIN_THREADS 1024
#define AS_FIN_MAX_SEG 256
#include "finish_body.h"

using namespace as_dev;
using as_launch::FinishArgs;

namespace {

// The arguments are read from device memory (the scan's copy of its kernel argument), which costs
// each workgroup less than a large kernel-argument block. Workgroup b finishes row b; those past the
// call's rows only take parts of S's sums (tail_help), which every workgroup whose row is not
// flagged does first.
__global__ __launch_bounds__(1024) void finish_kernel(const FinishArgs* __restrict__ ap) {
  const FinishArgs& a = *ap;
  const uint32_t row = blockIdx.x;
  // The host learns that the call's parameter upload (which ran before its scan) no longer reads its
  // staging block; the next call's list of flagged rows empties (this call's scan and the call
  // before it have ended).
  if (row == 0 && threadIdx.x == 0) {
    __hip_atomic_store(a.done, a.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    a.tail_next->count = 0u;
  }
  as_fin_sliced::tail_list_load(a, row);
  as_fin_sliced::row_prefetch(a, row);
  __syncthreads();
  as_fin_sliced::tail_help(a, row, gridDim.x);
  if (row < a.n_rows) {
    as_fin_sliced::finish_row(a, row);
    // A flagged row's S sums and histogram go back to zero for the next call once every part has
    // ended and every path above is done with them.
    __syncthreads();
    if (as_fin_sliced::shm().tail_slot != kNone) as_fin_sliced::tail_end(a, row);
  }
  // A small batch: the row is finished (it publishes no more deep passes); then this workgroup takes
  // parts of the other rows' passes until every row is finished.
  if (a.deep_help) {
    if (row < a.n_rows && threadIdx.x == 0)
      __hip_atomic_fetch_add(a.deep_done, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    as_fin_sliced::deep_help(a, row);
  }
}

}  // namespace

namespace as_launch {

hipError_t finish(hipStream_t stream, uint32_t groups, const FinishArgs* a) {
  hipLaunchKernelGGL(finish_kernel, dim3(groups), dim3(1024), 0, stream, a);
  return hipGetLastError();
}

}  // namespace as_launch

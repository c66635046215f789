// Pass 1 over the logits, the only kernel that streams the rows from HBM: one 256-thread workgroup
// per slice of a row (about a quarter of a 248,320-value row at batch 256, smaller slices for small
// batches). Each wave walks its own 1,024-value chunks of the slice (chunks w, w+4, w+8, ...) with
// the loads of the next chunk in flight while it works on the current one, and with no barrier until
// the slice ends. Per value it does only what every value needs; what few values need is done when
// they occur:
//   - the first non-finite index (sample.rs:22-34): fma(x, 0, acc) turns NaN once any raw value is
//     NaN or infinite; only then is the slice searched for the index;
//   - rows with penalties: the history's ids in this slice are marked in an LDS bitmap and counted
//     in an LDS hash; the stream leaves them out, and at the end of the slice each one's penalised
//     value (sample.rs:308-323, extended to a count) joins the candidates, the maximum and the sums;
//   - greedy rows: each lane's running argmax by IEEE `>`, lowest index (sample.rs:9-17, 378-396),
//     updated value by value only in the chunks whose maximum beats it;
//   - rows that draw: each wave keeps, in an LDS buffer, every value of its stream that ranks at or
//     above its threshold tau; values are tested four at a time by their maximum. tau rises when the
//     buffer holds a few times C values (C = top_k, or a fixed depth for rows without a top-k) to the
//     C-th best it holds, and the wave publishes that key to the row's shared word with a
//     device-wide atomic max. Every wave of the row reads the word once per kShareEvery chunks and raises its
//     own tau to it: for a top-k row a wave holding k values at or above a key proves that no value
//     below it is among the row's k best (sample.rs:157-166), so all slices filter with the best
//     bound any of them has found. Rows with min-p also share the largest value seen, and no wave
//     keeps a value below that value plus ln(min_p) (sample.rs:181, 237);
//   - rows without a top-k whose cut or draw needs the row's total (sample.rs:218-222, 274-282):
//     sums of exp(l - ref) or exp((l - ref) / T), ref each lane's running maximum of the raw values
//     (moved once per chunk), each term from the hardware's f32 exp2, a chunk's 16 terms added in a
//     tree in f32 and then into f64, with a per-slice bound on their error and sums of exp(d) * |d|
//     for the finish kernel's error bound.
// At the end of the slice every kept value ranking at or above the slice's bound (the highest wave
// threshold and the row's shared one) goes to HBM.
#include "sampler_device.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

#define AS_SCAN_NS as_scan_sliced
#define AS_SCAN_THREADS 256
#define AS_SCAN_HASH as_launch::kHistSlots
#define AS_SCAN_SLICE_MAX as_launch::kSliceMax
#define AS_SCAN_DEPTH 2
#include "scan_body.h"

using namespace as_dev;

namespace {

// A call whose rows are all greedy with no history (no penalty acts, no row can be refused for its
// history) needs no finish kernel: the last slice of each row to end merges the row's slices as the
// finish kernel would, the first non-finite index (sample.rs:22-34) and else the greedy pick by its
// total order (sample.rs:9-17), and writes the row's outputs. Each slice stores the three words the
// merge reads with device-coherent stores, waits for them, and counts itself ended in the row's
// RowShare::arrived; the slice that brings the count to n_seg reads every slice's words with
// device-coherent loads and sets the count back to zero. (Release and acquire fences at device
// scope would write back and invalidate the XCD's whole L2 instead.)
__device__ __forceinline__ void finish_greedy_row(const as_launch::FinishArgs& a, const SegStats& mine, SegStats* stats,
                                  RowShare* share, uint32_t row, uint32_t seg, uint32_t n_seg) {
  uint32_t& last = as_scan_sliced::shm().red_u[0];
  __syncthreads();  // the slice's LDS is no longer read
  if (threadIdx.x == 0) {
    SegStats* t = stats + (uint64_t)row * n_seg + seg;
    auto st = [](uint32_t* w, uint32_t v) { __hip_atomic_store(w, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    st(&t->nonfinite, mine.nonfinite);
    st(&t->greedy_idx, mine.greedy_idx);
    st(reinterpret_cast<uint32_t*>(&t->greedy_val), __builtin_bit_cast(uint32_t, mine.greedy_val));
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t old = __hip_atomic_fetch_add(&share[row].arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old + 1 == n_seg ? 1u : 0u;
  }
  __syncthreads();
  if (!last || threadIdx.x >= kWave) return;
  const uint32_t lane = threadIdx.x;
  uint32_t bad = kNone, gi = kNone;
  float gv = 0.0f;
  for (uint32_t b0 = 0; b0 < n_seg; b0 += kWave) {
    const uint32_t s = b0 + lane;
    if (s < n_seg) {
      const SegStats* t = stats + (uint64_t)row * n_seg + s;
      auto ld = [](const uint32_t* w) { return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
      bad = min(bad, ld(&t->nonfinite));
      const uint32_t idx = ld(&t->greedy_idx);
      const float val = __builtin_bit_cast(float, ld(reinterpret_cast<const uint32_t*>(&t->greedy_val)));
      greedy_merge(gv, gi, val, idx);
    }
  }
  bad = wave_min_u32(bad);
  wave_greedy(gv, gi);
  if (lane == 0) {
    if (bad != kNone) {
      a.tokens[row] = kNone;
      a.status[row] = AS_ROW_NONFINITE;
      if (a.kept_count) a.kept_count[row] = bad;
    } else {
      a.tokens[row] = gi;
      a.status[row] = AS_ROW_OK;
      if (a.kept_count) a.kept_count[row] = 1;
      if (a.kept_ids && a.kept_cap > 0) {
        a.kept_ids[(uint64_t)row * a.kept_cap] = gi;
        if (a.kept_probs) a.kept_probs[(uint64_t)row * a.kept_cap] = 1.0;
      }
    }
    __hip_atomic_store(&share[row].arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The sliced scan: workgroup (x, y) scans slice x of row r[y] (rows in the host's order). The
// finish kernel's arguments arrive here by value and the first workgroup stores them where the
// finish kernel reads them; a call the scan finishes (kFinish: every row greedy, no history) takes
// its own instantiation, so that the others' code holds none of its argument reads.
template <bool kVec, bool kFinish>
__global__ __launch_bounds__(256, 3) void scan_kernel(
    const float* __restrict__ logits, const float* __restrict__ zero, uint64_t row_stride, uint32_t n,
    uint32_t n_seg, uint32_t slice_len, const RowParams* __restrict__ params, RowShare* share,
    const uint32_t* __restrict__ hist_off, const uint32_t* __restrict__ hist_ids,
    const uint32_t* __restrict__ extra_ids, SegStats* __restrict__ stats, uint64_t* __restrict__ cands,
    uint32_t cand_stride, TailList* tail_list, as_launch::FinishArgs* __restrict__ args_out,
    const as_launch::FinishArgs args, const as_launch::RowOrder order) {
  const uint32_t row = order.on ? (uint32_t)order.r[blockIdx.y] : blockIdx.y;
  const SegStats st = as_scan_sliced::scan_slice<kVec>(logits, zero, row_stride, n, n_seg, slice_len, params, share,
                                                       hist_off, hist_ids, extra_ids, stats, cands, cand_stride,
                                                       tail_list, row, blockIdx.x);
  // After the slice, so that reading the argument delays none of the slice's loads.
  if (kFinish) {
    finish_greedy_row(args, st, stats, share, row, blockIdx.x, n_seg);
    // What the finish kernel does once per call: the host learns that the call's parameter upload
    // (which ran before this kernel) is over, and the next call's list of flagged rows empties.
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
      __hip_atomic_store(args.done, args.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      args.tail_next->count = 0u;
    }
  } else if (blockIdx.x == 0 && blockIdx.y == 0) {
    constexpr uint32_t kWords = sizeof(as_launch::FinishArgs) / 4;
    static_assert(kWords <= 256, "one word per thread");
    if (threadIdx.x < kWords)
      reinterpret_cast<uint32_t*>(args_out)[threadIdx.x] = reinterpret_cast<const uint32_t*>(&args)[threadIdx.x];
  }
}

}  // namespace

namespace as_launch {

hipError_t scan(hipStream_t stream, bool vec, const float* logits, const float* zero, uint64_t row_stride,
                uint32_t n, uint32_t n_rows, uint32_t n_seg, uint32_t slice_len, const RowParams* params,
                const FinishArgs& args, FinishArgs* args_out, RowShare* share, const uint32_t* hist_off,
                const uint32_t* hist_ids, const uint32_t* extra_ids, SegStats* stats, uint64_t* cands,
                uint32_t cand_stride, TailList* tail_list, const RowOrder& order) {
  dim3 grid(n_seg, n_rows);
  auto k = vec ? (args.scan_finishes ? scan_kernel<true, true> : scan_kernel<true, false>)
               : (args.scan_finishes ? scan_kernel<false, true> : scan_kernel<false, false>);
  hipLaunchKernelGGL(k, grid, dim3(256), 0, stream, logits, zero, row_stride, n, n_seg, slice_len, params, share,
                     hist_off, hist_ids, extra_ids, stats, cands, cand_stride, tail_list, args_out, args, order);
  return hipGetLastError();
}

}  // namespace as_launch

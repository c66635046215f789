// Pass 1 over the logits, the kernel that streams the rows from HBM (greedy_kernel below takes calls
// of greedy rows without history instead): one 256-thread workgroup per slice of a row (about a
// third of a 248,320-value row at batch 256, smaller slices for small batches). Each wave walks its own 1,024-value chunks of the slice (chunks w, w+4, w+8, ...) with
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
// history) needs none of the scan's candidates, thresholds and sums, and no finish kernel:
// greedy_kernel streams each slice for the first non-finite index (sample.rs:22-34) and the greedy
// pick by IEEE `>`, lowest index (sample.rs:9-17), and the last slice of each row to end merges the
// row's slices and writes its outputs. Each slice stores the three words the merge reads with
// device-coherent stores, waits for them, and counts itself ended in the row's RowShare::arrived; the
// slice that brings the count to n_seg reads every slice's words with device-coherent loads and sets
// the count back to zero. (Release and acquire fences at device scope would write back and invalidate
// the XCD's whole L2 instead.) Its code is a small part of the scan's, which a call of one row starts
// on a few dozen CUs at once.
constexpr uint32_t kGreedyLoads = 8;  // 16-byte loads in flight per thread

template <bool kVec>
__global__ __launch_bounds__(256) void greedy_kernel(const float* __restrict__ logits, uint64_t row_stride,
                                                     uint32_t n, uint32_t n_seg, uint32_t slice_len,
                                                     RowShare* share, SegStats* stats,
                                                     const as_launch::FinishArgs args,
                                                     const as_launch::RowOrder order) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr uint32_t kThreads = 256, kWaves = kThreads / kWave;
  __shared__ uint32_t red_bad[kWaves], red_idx[kWaves], last;
  __shared__ float red_val[kWaves];
  const uint32_t row = order.on ? (uint32_t)order.r[blockIdx.y] : blockIdx.y;
  const uint32_t seg = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const uint32_t b0 = seg * slice_len, b1 = min(b0 + slice_len, n);
  const float* x = logits + (uint64_t)row * row_stride;
  uint32_t bad = kNone, gi = kNone;
  float gv = -__builtin_inff();
  // Each thread sees its values in index order, so a strict `>` keeps the lowest index of a tie; the
  // merges below take the lower index too.
  auto see = [&](float v, uint32_t i) {
    if (!(__builtin_fabsf(v) <= __FLT_MAX__)) bad = min(bad, i);
    if (v > gv) {
      gv = v;
      gi = i;
    }
  };
  uint32_t tail = b0;  // the first value the 16-byte groups leave
  if (kVec) {
    // Whole 16-byte groups (the slice starts on a multiple of 1,024 values and the rows are
    // 16-byte aligned), kGreedyLoads per thread in flight.
    const uint32_t groups = (b1 - b0) / 4;
    for (uint32_t g0 = tid; g0 < groups; g0 += kGreedyLoads * kThreads) {
      f32x4 q[kGreedyLoads];
#pragma unroll
      for (uint32_t u = 0; u < kGreedyLoads; ++u) {
        const uint32_t g = g0 + u * kThreads;
        if (g < groups) q[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + b0 + 4 * g));
      }
#pragma unroll
      for (uint32_t u = 0; u < kGreedyLoads; ++u) {
        const uint32_t g = g0 + u * kThreads;
        if (g < groups)
#pragma unroll
          for (int c = 0; c < 4; ++c) see(q[u][c], b0 + 4 * g + c);
      }
    }
    tail = b0 + 4 * groups;
  }
  for (uint32_t i0 = tail + tid; i0 < b1; i0 += kGreedyLoads * kThreads) {
    float q[kGreedyLoads];
#pragma unroll
    for (uint32_t u = 0; u < kGreedyLoads; ++u) {
      const uint32_t i = i0 + u * kThreads;
      if (i < b1) q[u] = x[i];
    }
#pragma unroll
    for (uint32_t u = 0; u < kGreedyLoads; ++u) {
      const uint32_t i = i0 + u * kThreads;
      if (i < b1) see(q[u], i);
    }
  }
  bad = wave_min_u32(bad);
  wave_greedy(gv, gi);
  if (lane == 0) {
    red_bad[w] = bad;
    red_val[w] = gv;
    red_idx[w] = gi;
  }
  __syncthreads();
  if (tid == 0) {
    for (uint32_t k = 1; k < kWaves; ++k) {
      bad = min(bad, red_bad[k]);
      greedy_merge(gv, gi, red_val[k], red_idx[k]);
    }
    SegStats* t = stats + (uint64_t)row * n_seg + seg;
    auto st = [](uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    st(&t->nonfinite, bad);
    st(&t->greedy_idx, gi);
    st(reinterpret_cast<uint32_t*>(&t->greedy_val), __builtin_bit_cast(uint32_t, gv));
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t old = __hip_atomic_fetch_add(&share[row].arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old + 1 == n_seg ? 1u : 0u;
    // What the finish kernel does once per call: the host learns that the call's parameter upload
    // (which ran before this kernel) is over, and the next call's list of flagged rows empties.
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      __hip_atomic_store(args.done, args.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      args.tail_next->count = 0u;
    }
  }
  __syncthreads();
  if (!last || tid >= kWave) return;
  const as_launch::FinishArgs& a = args;
  bad = kNone;
  gi = kNone;
  gv = 0.0f;
  for (uint32_t s0 = 0; s0 < n_seg; s0 += kWave) {
    const uint32_t s = s0 + lane;
    if (s < n_seg) {
      const SegStats* t = stats + (uint64_t)row * n_seg + s;
      auto ld = [](const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
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
// finish kernel reads them.
template <bool kVec>
__global__ __launch_bounds__(256, 3) void scan_kernel(
    const float* __restrict__ logits, const float* __restrict__ zero, uint64_t row_stride, uint32_t n,
    uint32_t n_seg, uint32_t slice_len, const RowParams* __restrict__ params, RowShare* share,
    const uint32_t* __restrict__ hist_off, const uint32_t* __restrict__ hist_ids,
    const uint32_t* __restrict__ extra_ids, SegStats* __restrict__ stats, uint64_t* __restrict__ cands,
    uint32_t cand_stride, TailList* tail_list, as_launch::FinishArgs* __restrict__ args_out,
    const as_launch::FinishArgs args, const as_launch::RowOrder order) {
  const uint32_t row = order.on ? (uint32_t)order.r[blockIdx.y] : blockIdx.y;
  (void)as_scan_sliced::scan_slice<kVec>(logits, zero, row_stride, n, n_seg, slice_len, params, share, hist_off,
                                         hist_ids, extra_ids, stats, cands, cand_stride, tail_list, row,
                                         blockIdx.x);
  // After the slice, so that reading the argument delays none of the slice's loads.
  if (blockIdx.x == 0 && blockIdx.y == 0) {
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
  if (args.scan_finishes) {
    hipLaunchKernelGGL(vec ? greedy_kernel<true> : greedy_kernel<false>, grid, dim3(256), 0, stream, logits,
                       row_stride, n, n_seg, slice_len, share, stats, args, order);
  } else {
    hipLaunchKernelGGL(vec ? scan_kernel<true> : scan_kernel<false>, grid, dim3(256), 0, stream, logits, zero,
                       row_stride, n, n_seg, slice_len, params, share, hist_off, hist_ids, extra_ids, stats, cands,
                       cand_stride, tail_list, args_out, args, order);
  }
  return hipGetLastError();
}

}  // namespace as_launch

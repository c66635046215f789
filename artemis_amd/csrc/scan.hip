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

#define AS_SCAN_NS as_scan_sliced
#define AS_SCAN_THREADS 256
#define AS_SCAN_HASH as_launch::kHistSlots
#define AS_SCAN_SLICE_MAX as_launch::kSliceMax
#define AS_SCAN_DEPTH 2
#include "scan_body.h"

using namespace as_dev;

namespace {

// The sliced scan: workgroup (x, y) scans slice x of row r[y] (rows in the host's order). The
// finish kernel's arguments arrive here by value (the scan reads none of them) and the first
// workgroup stores them where the finish kernel reads them.
template <bool kVec>
__global__ __launch_bounds__(256, 3) void scan_kernel(
    const float* __restrict__ logits, const float* __restrict__ zero, uint64_t row_stride, uint32_t n,
    uint32_t n_seg, uint32_t slice_len, const RowParams* __restrict__ params, RowShare* share,
    const uint32_t* __restrict__ hist_off, const uint32_t* __restrict__ hist_ids,
    const uint32_t* __restrict__ extra_ids, SegStats* __restrict__ stats, uint64_t* __restrict__ cands,
    uint32_t cand_stride, TailList* tail_list, as_launch::FinishArgs* __restrict__ args_out,
    const as_launch::FinishArgs args, const as_launch::RowOrder order) {
  const uint32_t row = order.on ? (uint32_t)order.r[blockIdx.y] : blockIdx.y;
  as_scan_sliced::scan_slice<kVec>(logits, zero, row_stride, n, n_seg, slice_len, params, share, hist_off, hist_ids,
                                   extra_ids, stats, cands, cand_stride, tail_list, row, blockIdx.x);
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
  if (vec)
    hipLaunchKernelGGL(scan_kernel<true>, grid, dim3(256), 0, stream, logits, zero, row_stride, n, n_seg, slice_len,
                       params, share, hist_off, hist_ids, extra_ids, stats, cands, cand_stride, tail_list, args_out,
                       args, order);
  else
    hipLaunchKernelGGL(scan_kernel<false>, grid, dim3(256), 0, stream, logits, zero, row_stride, n, n_seg, slice_len,
                       params, share, hist_off, hist_ids, extra_ids, stats, cands, cand_stride, tail_list, args_out,
                       args, order);
  return hipGetLastError();
}

}  // namespace as_launch

// The row kernel: one 512-thread workgroup per row scans the whole row and then chooses its token,
// in one launch. It is the sliced scan's body (scan_body.h) with eight waves and one slice per row,
// followed in the same workgroup by the finish's body (finish_body.h): the candidates and
// statistics the scan leaves are this workgroup's own, still in its CU's cache, and the threshold the
// waves share lives in LDS and is read every other chunk. The two bodies share the workgroup's LDS
// (dynamic LDS, the larger of the two). Eight waves (two per SIMD) leave each wave the registers the
// stream needs without spilling; sixteen would spill inside the stream loop, and every reload's wait
// on the vector-memory counter would also wait for the chunk loads in flight. S is not summed in parts and there is no separate finish launch: a min-p row whose floor set
// overflows its waves' buffers bounds its unsorted tail with the finish's own pass over the row.
//
// Used for batches large enough to occupy the GPU with one workgroup per row (a CU each: the LDS
// holds one); smaller batches take the sliced scan, which spreads each row over several workgroups.
#include <mutex>

#include "sampler_device.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

extern __shared__ __attribute__((aligned(16))) unsigned char as_dyn_lds[];

#define AS_DYNAMIC_LDS 1
#define AS_SCAN_NS as_scan_row
#define AS_SCAN_THREADS 512
#define AS_SCAN_HASH 2048u
#define AS_SCAN_SLICE_MAX as_launch::kRowMaxVocab
#define AS_SCAN_DEPTH 2
#define AS_SCAN_SHARE_LDS 1
#define AS_SCAN_SHARE_EVERY 2
#include "scan_body.h"
#define AS_FIN_NS as_fin_row
#define AS_FIN_THREADS 512
#define AS_FIN_MAX_SEG 16
#include "finish_body.h"

using namespace as_dev;
using as_launch::FinishArgs;

namespace {

constexpr uint32_t kRowThreads = 512;
static_assert(kRowThreads == AS_SCAN_THREADS && kRowThreads == AS_FIN_THREADS, "one workgroup size");
constexpr size_t kLds = sizeof(as_scan_row::Shared) > sizeof(as_fin_row::Shared) ? sizeof(as_scan_row::Shared)
                                                                                   : sizeof(as_fin_row::Shared);
static_assert(kLds <= 160 * 1024, "one workgroup's LDS on a CDNA4 CU");

template <bool kVec>
__global__ __launch_bounds__(512, 1) void row_kernel(
    const float* __restrict__ logits, const float* __restrict__ zero, uint64_t row_stride, uint32_t n,
    const uint32_t* block_in, uint32_t* __restrict__ block_out, RowShare* share,
    const uint32_t* __restrict__ hist_off, const uint32_t* __restrict__ hist_ids,
    const uint32_t* __restrict__ extra_ids, SegStats* __restrict__ stats, uint64_t* __restrict__ cands,
    uint32_t cand_stride, const FinishArgs a) {
  const uint32_t row = blockIdx.x;
  as_scan_row::scan_slice<kVec>(logits, zero, row_stride, n, 1u, n, block_in, block_out, share, hist_off,
                                hist_ids, extra_ids, stats, cands, cand_stride, nullptr, row, 0u);
  // The scan's writes (its statistics, candidates and the row's parameter block) are the finish's
  // inputs, read by this same workgroup.
  __syncthreads();
  as_fin_row::finish_row(a, row);
  __syncthreads();
  // Every workgroup read its row's parameters from the call's pinned block at its start; the last one
  // to end tells the host the block is free for reuse.
  if (threadIdx.x == 0) {
    const uint32_t ended = __hip_atomic_fetch_add(a.fused_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (ended + 1 == gridDim.x) {
      __hip_atomic_store(a.fused_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.done, a.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

std::once_flag g_lds_once;
hipError_t g_lds_err = hipSuccess;

}  // namespace

namespace as_launch {

size_t row_kernel_lds() { return kLds; }

hipError_t sample_rows(hipStream_t stream, bool vec, const float* logits, const float* zero, uint64_t row_stride,
                       uint32_t n, uint32_t n_rows, const void* block_in, void* block_out, RowShare* share,
                       const uint32_t* hist_off, const uint32_t* hist_ids, const uint32_t* extra_ids,
                       SegStats* stats, uint64_t* cands, uint32_t cand_stride, const FinishArgs& a) {
  // More than 64 KiB of dynamic LDS needs the kernel's permission, given once per process.
  std::call_once(g_lds_once, [] {
    g_lds_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&row_kernel<true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
    if (g_lds_err == hipSuccess)
      g_lds_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&row_kernel<false>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
  });
  if (g_lds_err != hipSuccess) return g_lds_err;
  const uint32_t* in = static_cast<const uint32_t*>(block_in);
  uint32_t* out = static_cast<uint32_t*>(block_out);
  if (vec)
    hipLaunchKernelGGL(row_kernel<true>, dim3(n_rows), dim3(kRowThreads), kLds, stream, logits, zero, row_stride, n, in, out,
                       share, hist_off, hist_ids, extra_ids, stats, cands, cand_stride, a);
  else
    hipLaunchKernelGGL(row_kernel<false>, dim3(n_rows), dim3(kRowThreads), kLds, stream, logits, zero, row_stride, n, in,
                       out, share, hist_off, hist_ids, extra_ids, stats, cands, cand_stride, a);
  return hipGetLastError();
}

}  // namespace as_launch

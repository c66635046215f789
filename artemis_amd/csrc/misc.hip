// The verify accept step, the greedy draft pick (argmax_rows) and the exp check kernel.
#include "sampler_device.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

using namespace as_dev;

namespace {

// spec/step.rs:347-379 over picks that all k+1 rows already made: the first pick that is a stop id
// (turn.rs:350-352) or differs from the draft after it ends the burst. One thread: k <= 15.
__global__ void accept_kernel(const uint32_t* __restrict__ picks, const uint32_t* __restrict__ status,
                              const uint32_t* __restrict__ drafts, uint32_t k,
                              const uint32_t* __restrict__ stop_ids, uint32_t n_stop,
                              uint64_t* __restrict__ rng_state, uint32_t draws_per_row,
                              uint32_t* __restrict__ result) {
  if (threadIdx.x != 0) return;
  uint32_t read = 0, flags = 0;
  for (uint32_t i = 0; i <= k; ++i) {
    if (status[i] & AS_ROW_NONFINITE) {
      flags |= 2u;
      break;
    }
    const uint32_t y = picks[i];
    read = i + 1;
    if (status[i] & AS_ROW_EXACT_PATH) flags |= 0x100u;
    bool stop = false;
    for (uint32_t j = 0; j < n_stop; ++j) stop = stop || stop_ids[j] == y;
    if (stop) {
      flags |= 1u;
      break;
    }
    if (i < k && drafts[i] != y) break;
  }
  // The stream advances by one draw per row the sampler read.
  if (draws_per_row) {
    uint64_t s[4] = {rng_state[0], rng_state[1], rng_state[2], rng_state[3]};
    for (uint32_t i = 0; i < read; ++i) rng_next(s);
    for (int j = 0; j < 4; ++j) rng_state[j] = s[j];
  }
  result[0] = read;
  result[1] = read > 0 ? read - 1 : 0;
  result[2] = read > 0 ? picks[read - 1] : AS_NO_DRAFT;
  result[3] = flags;
}

constexpr int kArgThreads = 256;

// argmax_rows.comp: the largest finite value, ties to the lower index, NO_DRAFT for none; the
// embedding-row address of the pick. One workgroup per row, 16-byte loads.
template <bool kVec>
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float* __restrict__ logits,
                                                             uint64_t row_stride, uint32_t n,
                                                             uint32_t* __restrict__ ids,
                                                             uint64_t* __restrict__ rows_out,
                                                             uint64_t embd, uint32_t row_bytes,
                                                             uint32_t slot) {
  __shared__ float rv[kArgThreads / kWave];
  __shared__ uint32_t ri[kArgThreads / kWave];
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const float* src = logits + (uint64_t)row * row_stride;
  float bv = 0.0f;
  uint32_t bi = kNone;
  if (kVec) {
    const uint32_t n4 = n / 4;
    for (uint32_t q = tid; q < n4; q += kArgThreads) {
      const float4 f = reinterpret_cast<const float4*>(src)[q];
      const float e[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (is_finite_bits(e[c])) greedy_merge(bv, bi, e[c], 4 * q + c);
    }
    for (uint32_t i = 4 * n4 + tid; i < n; i += kArgThreads)
      if (is_finite_bits(src[i])) greedy_merge(bv, bi, src[i], i);
  } else {
    for (uint32_t i = tid; i < n; i += kArgThreads)
      if (is_finite_bits(src[i])) greedy_merge(bv, bi, src[i], i);
  }
  wave_greedy(bv, bi);
  if ((tid & (kWave - 1)) == 0) {
    rv[tid / kWave] = bv;
    ri[tid / kWave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgThreads / kWave; ++w) greedy_merge(bv, bi, rv[w], ri[w]);
    ids[slot + row] = bi;
    rows_out[slot + row] = embd + (uint64_t)(bi == kNone ? 0u : bi) * (uint64_t)row_bytes;
  }
}

__global__ void exp_kernel(const double* __restrict__ x, double* __restrict__ y, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = as_exp::exp(x[i]);
}

// The hardware 2^x (V_EXP_F32) the scan's sums are built on.
__global__ void exp2f_kernel(const float* __restrict__ x, float* __restrict__ y, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = __builtin_amdgcn_exp2f(x[i]);
}

}  // namespace

namespace as_launch {

hipError_t accept(hipStream_t stream, const uint32_t* picks, const uint32_t* status,
                  const uint32_t* drafts, uint32_t k, const uint32_t* stop_ids, uint32_t n_stop,
                  uint64_t* rng_state, uint32_t draws_per_row, uint32_t* result) {
  hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, stream, picks, status, drafts, k, stop_ids,
                     n_stop, rng_state, draws_per_row, result);
  return hipGetLastError();
}

hipError_t argmax_rows(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride,
                       uint32_t n, uint32_t n_rows, uint32_t* ids, uint64_t* rows_out,
                       uint64_t embd, uint32_t row_bytes, uint32_t slot) {
  if (vec)
    hipLaunchKernelGGL(argmax_kernel<true>, dim3(n_rows), dim3(kArgThreads), 0, stream, logits,
                       row_stride, n, ids, rows_out, embd, row_bytes, slot);
  else
    hipLaunchKernelGGL(argmax_kernel<false>, dim3(n_rows), dim3(kArgThreads), 0, stream, logits,
                       row_stride, n, ids, rows_out, embd, row_bytes, slot);
  return hipGetLastError();
}

hipError_t debug_exp(hipStream_t stream, const double* x, double* y, uint32_t n) {
  hipLaunchKernelGGL(exp_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, y, n);
  return hipGetLastError();
}

hipError_t debug_exp2f(hipStream_t stream, const float* x, float* y, uint32_t n) {
  hipLaunchKernelGGL(exp2f_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, y, n);
  return hipGetLastError();
}

}  // namespace as_launch

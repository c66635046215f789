// Between the scan and the finish kernel: for a min-p row without a top-k whose scan did not keep
// every value above the floor (RowShare::gave_up; its floor set is thousands of values), the
// weights of S, the values that rank below the finish kernel's bound R and lie at or above the
// floor: W = sum of exp((l - top) / T) and M = sum of exp(l - top), and |S|; when S has at most
// kTailKeep values they also go to the row's scratch (packed rank keys, in any order), so that the
// finish kernel can sort the whole floor set; and S's histogram by value (TailBins), which places
// top-p's cut within one bin. The finish kernel's
// draw needs them when the kept set (sample.rs:230-272) runs past its sorted candidates: the kept
// values past them are S's first in rank order (all of S when the floor cuts first). The scan lists
// the rows it flags (TailList: the first kTailRows; a row past them is left to the finish kernel);
// each row is covered in parts of kTailLen values, which up to kTailGroups 256-thread workgroups
// take in turn, and the parts' sums add with device atomics.
#include "sampler_device.h"
#include "launch.h"

using namespace as_dev;
using as_launch::FinishArgs;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr uint32_t kLen = as_launch::kTailLen;
constexpr uint32_t kHash = 512;  // distinct history ids in a part
constexpr uint32_t kStage = 2048;  // values of S a part stages in LDS before they go to scratch
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
typedef float f32x4 __attribute__((ext_vector_type(4)));
static_assert(kLen % (16 * kThreads) == 0, "whole steps");

constexpr uint32_t kBins = as_dev::kTailBins;

struct Shared {
  double bin_m[kBins];  // the part's histogram of S (TailBins)
  double bin_w[kBins];
  float vals[kLen];     // the part's raw values (the history's are read here)
  uint32_t bitmap[kLen / 32];
  uint32_t hid[kHash];
  uint32_t hcnt[kHash];
  uint64_t stage[kStage];
  double red[kWaves];
  uint32_t red_u[kWaves];
  uint32_t overflow;
  uint32_t staged;
  uint32_t base;
};
__shared__ Shared g_tsh;

// Whether the finish kernel can need S for the row: a min-p row without a top-k that a slice flagged
// (its bound lay above its floor), whose finish takes its fast path (no slice with unfinished statistics
// or non-finite values), and whose candidates' bound R lies above the floor. Fills R, the row's
// largest value and the floor (as an f32).
__device__ bool needs_tail(const FinishArgs& a, uint32_t row, uint64_t* R_out, float* top_out, float* fl_out) {
  if (a.share[row].gave_up == 0u) return false;
  const RowParams& p = a.params[row];
  if (p.mode != kModePartial || !(p.min_p > 0.0f)) return false;
  uint32_t top = 0;
  uint64_t R = 0;
  for (uint32_t s = 0; s < a.n_seg; ++s) {
    const SegStats& t = a.stats[(uint64_t)row * a.n_seg + s];
    top = max(top, t.max_key);
    if (t.truncated & 1u) R = max(R, t.bound);
    if ((t.truncated & 2u) || t.nonfinite != kNone) return false;
  }
  const float topf = key_value(top);
  const float fl = floor_f32(__dadd_rn((double)topf, p.ln_min_p));
  if (((uint64_t)total_key(fl) << 32) >= R) return false;
  *R_out = R;
  *top_out = topf;
  *fl_out = fl;
  return true;
}

// One part of one flagged row: its share of S's sums, bins and list. Every load that needs only the
// row is issued at once (the part's values, the history's bounds, the row's parameters and slice
// statistics), then the history's ids; the history's raw values are read from the part's values,
// staged in LDS.
__device__ __forceinline__ void tail_part(const FinishArgs& a, uint32_t row, uint32_t part) {
  Shared& sh = g_tsh;
  const uint32_t tid = threadIdx.x;
  const uint32_t n = a.n, b0 = part * kLen, b1 = min(b0 + kLen, n), len = b1 - b0;
  const float* x = a.logits + (uint64_t)row * a.row_stride;
  const bool vec = a.vec && a.row_stride % 4 == 0 && len == kLen;
  float v[16];
  if (vec) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 q = *reinterpret_cast<const f32x4*>(x + b0 + (j * kThreads + tid) * 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * j + c] = q[c];
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t off = k * kThreads + tid;
      v[k] = off < len ? x[b0 + off] : 0.0f;
    }
  }
  const RowParams& p = a.params[row];
  uint32_t hb;
  const uint32_t he = as_launch::history_bounds(a, p, row, &hb);
  uint64_t R = 0;
  float topf = 0.0f, fl = 0.0f;
  if (!needs_tail(a, row, &R, &topf, &fl)) return;
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  constexpr int kHistRegs = 8;
  uint32_t hreg[kHistRegs];
#pragma unroll
  for (int k = 0; k < kHistRegs; ++k) {
    const uint32_t h = hb + tid + k * kThreads;
    hreg[k] = (pen && h < he) ? a.hist_ids[h] : kEmpty;
  }
  // The part's values into LDS (position off = value b0 + off).
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t off = vec ? ((k / 4) * kThreads + tid) * 4 + (k % 4) : k * kThreads + tid;
    if (off < kLen) sh.vals[off] = v[k];
  }
  if (pen) {
    for (uint32_t i = tid; i < kLen / 32; i += kThreads) sh.bitmap[i] = 0;
    for (uint32_t i = tid; i < kHash; i += kThreads) {
      sh.hid[i] = kEmpty;
      sh.hcnt[i] = 0;
    }
  }
  if (tid == 0) {
    sh.overflow = 0;
    sh.staged = 0;
  }
  for (uint32_t b = tid; b < kBins; b += kThreads) {
    sh.bin_m[b] = 0.0;
    sh.bin_w[b] = 0.0;
  }
  __syncthreads();
  if (pen) {
    auto mark = [&](uint32_t id) {
      const uint32_t off = id - b0;
      if (off >= len) return;
      atomicOr(&sh.bitmap[off >> 5], 1u << (off & 31u));
      uint32_t h = (id * 0x9E3779B1u) >> (32 - 9);
      static_assert(kHash == 1u << 9, "the hash's top bits");
      for (uint32_t probe = 0; probe < kHash; ++probe) {
        const uint32_t prev = atomicCAS(&sh.hid[h], kEmpty, id);
        if (prev == kEmpty || prev == id) {
          atomicAdd(&sh.hcnt[h], 1u);
          return;
        }
        h = (h + 1) & (kHash - 1);
      }
      sh.overflow = 1;
    };
#pragma unroll
    for (int k = 0; k < kHistRegs; ++k)
      if (hreg[k] != kEmpty) mark(hreg[k]);
    for (uint32_t h = hb + tid + kHistRegs * kThreads; h < he; h += kThreads) mark(a.hist_ids[h]);
    for (uint32_t h = tid; h < extra; h += kThreads) mark(a.extra_ids[h]);
    __syncthreads();
  }
  if (sh.overflow) {
    if (tid == 0) __hip_atomic_fetch_or(&a.tail[row].failed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // In S: v >= fl, and v ranks below R: v < R's value, or (rarely) equal to it and below in the
  // packed order (which also orders -0 below +0).
  const float rv = key_value((uint32_t)(R >> 32));
  const float s1 = 1.44269502f, sw = (1.0f / p.temp) * s1;
  // The histogram's scale: (rv - v) * bscale is monotone in v, so bins follow the rank order.
  const float span = rv - fl;
  const float bscale = (span > 0.0f && span < __builtin_inff()) ? (float)kBins / span : 0.0f;
  float gw = 0.0f, gm = 0.0f;
  uint32_t cnt = 0;
  auto in_s = [&](float val, uint32_t id) {
    bool in = val >= fl && val < rv;
    if (__builtin_expect(val == rv, 0)) in = val >= fl && pack(total_key(val), id) < R;
    return in;
  };
  // Called by every lane of the wave at once: the values in S add their terms and bins, and are
  // staged with one LDS atomic per wave.
  auto add = [&](bool in, float val, uint32_t id) {
    if (in) {
      const float d = val - topf;
      const float tw = __builtin_amdgcn_exp2f(d * sw), tm = __builtin_amdgcn_exp2f(d * s1);
      gw += tw;
      gm += tm;
      const uint32_t b = (uint32_t)fminf((rv - val) * bscale, (float)(kBins - 1));
      atomicAdd(&sh.bin_w[b], (double)tw);
      atomicAdd(&sh.bin_m[b], (double)tm);
      ++cnt;
    }
    const uint64_t mk = __ballot(in);
    if (mk) {
      uint32_t base = 0;
      if ((tid & (kWave - 1)) == 0) base = atomicAdd(&sh.staged, (uint32_t)__popcll(mk));
      base = __builtin_amdgcn_readfirstlane(base);
      const uint32_t i = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
      if (in && i < kStage) sh.stage[i] = pack(total_key(val), id);
    }
  };
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t off = vec ? ((k / 4) * kThreads + tid) * 4 + (k % 4) : k * kThreads + tid;
    const bool valid = off < len && !(pen && ((sh.bitmap[off >> 5] >> (off & 31u)) & 1u));
    add(valid && in_s(v[k], b0 + off), v[k], b0 + off);
  }
  double w = (double)gw, m = (double)gm;
  if (pen) {
    static_assert(kHash % kThreads == 0, "every thread takes the same number of slots");
    for (uint32_t s = tid; s < kHash; s += kThreads) {
      const uint32_t id = sh.hid[s];
      const bool has = id != kEmpty;
      const float val = has ? penalize(sh.vals[id - b0], sh.hcnt[s], p) : 0.0f;
      gw = 0.0f;
      gm = 0.0f;
      add(has && in_s(val, id), val, id);
      w += (double)gw;
      m += (double)gm;
    }
  }
  w = block_sum_f64<kWaves>(w, sh.red);
  m = block_sum_f64<kWaves>(m, sh.red);
  cnt = block_sum_u32<kWaves>(cnt, sh.red_u);
  RowTail& t = a.tail[row];
  // The part's bins into the row's (block_sum_f64 above ended with a barrier: the LDS bins are whole).
  as_dev::TailBins& tb = a.tail_bins[row];
  for (uint32_t b = tid; b < kBins; b += kThreads) {
    if (sh.bin_w[b] != 0.0) __hip_atomic_fetch_add(&tb.w[b], sh.bin_w[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (sh.bin_m[b] != 0.0) __hip_atomic_fetch_add(&tb.m[b], sh.bin_m[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) {
    __hip_atomic_fetch_add(&t.w, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(&t.m, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.base = __hip_atomic_fetch_add(&t.count, cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (cnt > kStage) __hip_atomic_fetch_or(&t.lost, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // The staged values to scratch, at the part's place in the row's list, when the list can hold them.
  const uint32_t base = sh.base, staged = min(cnt, kStage);
  uint64_t* list = reinterpret_cast<uint64_t*>(a.scratch + (uint64_t)row * a.scratch_stride);
  if (base + staged <= kTailKeep)
    for (uint32_t i = tid; i < staged; i += kThreads) list[base + i] = sh.stage[i];
  __syncthreads();
  if (tid == 0) __hip_atomic_fetch_add(&t.parts, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// The workgroups take the (flagged row, part) items in turn. The arguments are the scan's device copy
// of the call's block: a large kernel-argument block costs every workgroup more than that load.
__global__ __launch_bounds__(kThreads) void tail_kernel(const FinishArgs* __restrict__ ap) {
  const FinishArgs& a = *ap;
  const uint32_t parts = (a.n + kLen - 1) / kLen;
  for (uint32_t item = blockIdx.x; item < as_launch::kTailRows * parts; item += gridDim.x) {
    // The list's count and this item's entry, loaded together (an entry past the count is unused).
    const uint32_t r = a.tail_list->rows[item / parts];
    const uint32_t flagged = min(a.tail_list->count, as_launch::kTailRows);
    if (item >= flagged * parts) break;
    __syncthreads();  // the previous item's tables are no longer read
    tail_part(a, r, item % parts);
  }
}

}  // namespace

namespace as_launch {

hipError_t tail(hipStream_t stream, uint32_t n_rows, uint32_t n, const FinishArgs* a) {
  const uint32_t items = min(n_rows, kTailRows) * ((n + kTailLen - 1) / kTailLen);
  hipLaunchKernelGGL(tail_kernel, dim3(min(items, kTailGroups)), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace as_launch

// Log-probabilities of the model's own distribution (crates/engine/src/logprobs.rs:12-38): the
// log-softmax of a row's raw logits (before penalties, temperature and filters) at the sampled token,
// and the `top` highest logits' (at most 20), sorted by logit descending with -0 and +0 tied, then by
// the lower id (logprobs.rs:40-48). Rows must be finite (the reference's run_step guarantees it).
//
// Two kernels over the rows in HBM:
//   - lp_part_kernel: one 256-thread workgroup per kLpPart values of a row. Its largest value m_p,
//     S_p = sum of exp(x - m_p) in f64 (each term within 3 ulps of the reference's exp, from a
//     table-free polynomial: exp_neg), and its 20 best by the reference's order: a threshold T from the
//     waves (each wave's 20th best lane maximum: at least 20 values of the part rank at or above
//     the largest of them) collects the few values at or above it into LDS, which a rank count sorts.
//   - lp_row_kernel: one workgroup per row. M = max m_p; total = sum of S_p * exp(m_p - M);
//     lse = M + ln(total) (logprobs.rs:14-16); the parts' lists merge into the row's `top` best; each
//     output is (x - lse) rounded to f32 (logprobs.rs:18, 34).
//
// The reference sums exp(x - M) left to right over the row; this sum is parallel, with a bound on
// the distance between the two: gamma(n + 64) relative (both orders' rounding, at most 4 ulps per
// term between the two exps, and the rescale of each part), plus the logarithm's own ulp. An output is exact when that
// bound cannot change its rounding to f32; otherwise the row's status says AS_LP_INEXACT and the
// value is within one f32 ulp of the reference's.
#include "sampler_device.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

using namespace as_dev;
using as_launch::LpPart;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr uint32_t kPart = as_launch::kLpPart;
constexpr uint32_t kPer = kPart / kThreads;  // values per thread
constexpr uint32_t kTop = as_launch::kLpTop;
constexpr uint32_t kList = 1024;             // a part's values at or above its threshold
constexpr uint32_t kMerge = as_launch::kLpMerge;
constexpr double kU = 1.1102230246251565e-16;  // 2^-53
typedef float f32x4 __attribute__((ext_vector_type(4)));
static_assert(kPer % 4 == 0, "whole 16-byte groups per thread");

// The reference's order as one descending u64: the logit's rank key with -0 mapped to +0 (they tie),
// then the lower id.
__device__ __forceinline__ uint64_t lp_key(float x, uint32_t id) { return pack(total_key(x == 0.0f ? 0.0f : x), id); }

// The q-th largest of the lanes' keys (distinct; 0 for an empty lane), or 0 when fewer than q
// lanes hold one.
__device__ __forceinline__ uint64_t wave_qth_u64(uint64_t x, uint32_t q) {
  uint64_t m = 0;
  for (uint32_t it = 0; it < q; ++it) {
    m = wave_max_u64(x);
    if (m == 0) return 0;
    if (x == m) x = 0;
  }
  return m;
}

__device__ __forceinline__ double gamma_n(double n) { return n * kU / (1.0 - n * kU); }

// exp(d) for d <= 0 without a table (the table's gathers from LDS conflict across lanes): d = k ln2 + r
// with |r| <= ln2/2 (ln2 split in two, the product by k exact in the high part), then e^r by its Taylor
// series to degree 12 (truncation below 2e-16 relative) in Horner form, and 2^k by the exponent
// field. Within a few ulps of exp(d), which the sum's bound allows per term; d below -700 gives 0
// (such a term is under 2^-1000 of the row's largest, which is 1).
__device__ __forceinline__ double exp_neg(double d) {
  const double kLog2e = 1.4426950408889634;
  const double kLn2Hi = 6.93147180369123816490e-01, kLn2Lo = 1.90821492927058770002e-10;
  const double dc = fmax(d, -708.0);  // 2^k stays a normal number; below -700 the result is 0 anyway
  const double k = __builtin_rint(dc * kLog2e);
  const double r = __builtin_fma(-k, kLn2Lo, __builtin_fma(-k, kLn2Hi, dc));
  double p = 1.0 / 479001600.0;  // 1/12!
  p = __builtin_fma(p, r, 1.0 / 39916800.0);
  p = __builtin_fma(p, r, 1.0 / 3628800.0);
  p = __builtin_fma(p, r, 1.0 / 362880.0);
  p = __builtin_fma(p, r, 1.0 / 40320.0);
  p = __builtin_fma(p, r, 1.0 / 5040.0);
  p = __builtin_fma(p, r, 1.0 / 720.0);
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const int64_t ki = (int64_t)k;
  const double scale = __builtin_bit_cast(double, (uint64_t)(ki + 1023) << 52);
  return d < -700.0 ? 0.0 : p * scale;
}

struct PartShared {
  uint64_t list[kList];
  uint32_t n_list;
  uint32_t red_u[kWaves];
  double red_d[kWaves];
  uint64_t red_k[kWaves];
};

__global__ __launch_bounds__(kThreads) void lp_part_kernel(const float* __restrict__ logits, uint64_t row_stride,
                                                           uint32_t n, uint32_t vec, LpPart* __restrict__ parts,
                                                           uint32_t n_parts) {
  __shared__ PartShared sh;
  const uint32_t part = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const uint32_t lane = tid & (kWave - 1), w = tid / kWave;
  const float* x = logits + (uint64_t)row * row_stride;
  const uint32_t b0 = part * kPart, b1 = min(b0 + kPart, n);
  if (tid == 0) sh.n_list = 0;

  // Value q of this thread is at b0 + off(q): 16-byte groups when the row allows them.
  const bool v4 = vec && b1 - b0 == kPart;
  auto off = [&](uint32_t q) { return v4 ? ((q / 4) * kThreads + tid) * 4 + (q % 4) : q * kThreads + tid; };
  float v[kPer];
  if (v4) {
#pragma unroll
    for (uint32_t g = 0; g < kPer / 4; ++g) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(x + b0 + (g * kThreads + tid) * 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * g + c] = t[c];
    }
  } else {
#pragma unroll
    for (uint32_t q = 0; q < kPer; ++q) v[q] = (b0 + off(q) < b1) ? x[b0 + off(q)] : 0.0f;
  }

  // The part's largest value (by rank key: the largest of finite values).
  uint32_t kmax = 0;
  uint64_t best = 0;
#pragma unroll
  for (uint32_t q = 0; q < kPer; ++q) {
    if (b0 + off(q) >= b1) continue;
    kmax = max(kmax, total_key(v[q]));
    best = max(best, lp_key(v[q], b0 + off(q)));
  }
  kmax = block_max_u32<kWaves>(kmax, sh.red_u);
  const float m = key_value(kmax);
  const double md = (double)m;

  // S_p, each term the reference's exp(f64(x) - m).
  double s = 0.0;
#pragma unroll
  for (uint32_t q = 0; q < kPer; ++q)
    if (b0 + off(q) < b1) s += exp_neg((double)v[q] - md);
  s = block_sum_f64<kWaves>(s, sh.red_d);

  // The threshold: each wave's kTop-th best lane maximum, the largest of them.
  const uint64_t tw = wave_qth_u64(best, kTop);
  if (lane == 0) sh.red_k[w] = tw;
  __syncthreads();
  uint64_t T = sh.red_k[0];
  for (int k = 1; k < kWaves; ++k) T = max(T, sh.red_k[k]);
  // Every value at or above it, into the list.
#pragma unroll
  for (uint32_t q = 0; q < kPer; ++q) {
    if (b0 + off(q) >= b1) continue;
    const uint64_t key = lp_key(v[q], b0 + off(q));
    if (key >= T) {
      const uint32_t i = atomicAdd(&sh.n_list, 1u);
      if (i < kList) sh.list[i] = key;
    }
  }
  __syncthreads();
  const uint32_t n_list = sh.n_list;
  LpPart& out = parts[(uint64_t)row * n_parts + part];
  // The list's kTop best, in order: each entry's place is the number of entries above it.
  if (n_list <= kList) {
    for (uint32_t i = tid; i < n_list; i += kThreads) {
      const uint64_t key = sh.list[i];
      uint32_t r = 0;
      for (uint32_t j = 0; j < n_list; ++j) r += sh.list[j] > key ? 1u : 0u;
      if (r < kTop) out.top[r] = key;
    }
  }
  if (tid == 0) {
    out.sum = s;
    out.max = m;
    out.n_top = min(n_list, kTop);
    out.overflow = n_list > kList ? 1u : 0u;
  }
}

struct RowShared {
  uint64_t tab[256];
  uint64_t merged[kMerge];
  uint64_t top[kTop];
  uint32_t overflow;
  uint32_t inexact;
  uint32_t red_u[kWaves];
  double red_d[kWaves];
  uint64_t red_k[kWaves];
};

// f32(xd - lse) and whether every lse within e of the computed one rounds the same way.
__device__ __forceinline__ float lp_round(double xd, double lse, double e, bool* exact) {
  const double d = xd - lse;
  const float r = (float)d;
  const double slack = e + fabs(d) * kU;  // the subtraction's own rounding
  *exact = (float)(d - slack) == r && (float)(d + slack) == r;
  return r;
}

__global__ __launch_bounds__(kThreads) void lp_row_kernel(const float* __restrict__ logits, uint64_t row_stride,
                                                          uint32_t n, const LpPart* __restrict__ parts,
                                                          uint32_t n_parts, const uint32_t* __restrict__ tokens,
                                                          uint32_t top, float* __restrict__ logprob,
                                                          uint32_t* __restrict__ top_ids, float* __restrict__ top_lps,
                                                          uint32_t* __restrict__ status) {
  __shared__ RowShared sh;
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const float* x = logits + (uint64_t)row * row_stride;
  const LpPart* pp = parts + (uint64_t)row * n_parts;
  sh.tab[tid] = as_exp::kTable[tid];
  if (tid == 0) {
    sh.overflow = 0;
    sh.inexact = 0;
  }
  // M: the largest part maximum.
  uint32_t kmax = 0;
  for (uint32_t p = tid; p < n_parts; p += kThreads) kmax = max(kmax, total_key(pp[p].max));
  kmax = block_max_u32<kWaves>(kmax, sh.red_u);
  const double M = (double)key_value(kmax);
  // total = sum of S_p * exp(m_p - M); the parts' lists into one.
  double t = 0.0;
  for (uint32_t p = tid; p < n_parts; p += kThreads) {
    const LpPart& q = pp[p];
    t += q.sum * as_exp::exp_with(sh.tab, (double)q.max - M);
    if (q.overflow) sh.overflow = 1;
    // Part p's list at merged[p * kTop ...), padded with zeros (below every key).
    for (uint32_t i = 0; i < kTop; ++i) sh.merged[p * kTop + i] = i < q.n_top ? q.top[i] : 0ull;
  }
  const double total = block_sum_f64<kWaves>(t, sh.red_d);
  const double lnt = log(total);
  const double lse = M + lnt;
  // The distance to the reference's lse: both sums' roundings (n terms each, the parts' rescales),
  // the logarithm's ulp and the final addition.
  const double e = gamma_n((double)n + 64.0) + 4.0 * kU * fabs(lnt) + 2.0 * kU * fabs(lse);

  const uint32_t nt = min(min(top, kTop), n);
  if (nt > 0) {
    if (!sh.overflow) {
      // The parts' lists hold the row's nt best (each part's list holds its own best kTop). An
      // entry's rank is the count of larger keys, found in each part's descending list by bisection;
      // only an entry at place i < nt of its own list can rank below nt.
      const uint32_t nm = n_parts * kTop;
      for (uint32_t e = tid; e < nm; e += kThreads) {
        const uint32_t i = e % kTop;
        const uint64_t key = sh.merged[e];
        if (i >= nt || key == 0ull) continue;
        uint32_t r = 0;
        for (uint32_t p = 0; p < n_parts; ++p) {
          const uint64_t* l = sh.merged + p * kTop;
          uint32_t lo = 0, hi = kTop;  // l[0..lo) > key >= l[hi..kTop)
          while (lo < hi) {
            const uint32_t mid = (lo + hi) / 2;
            if (l[mid] > key) lo = mid + 1;
            else hi = mid;
          }
          r += lo;
        }
        if (r < nt) sh.top[r] = key;
      }
    } else {
      // Heavy ties overflowed a part's list: the row's best, one full pass each (the largest key
      // below the one before).
      uint64_t prev = ~0ull;
      for (uint32_t r = 0; r < nt; ++r) {
        uint64_t b = 0;
        for (uint32_t i = tid; i < n; i += kThreads) {
          const uint64_t key = lp_key(x[i], i);
          if (key < prev && key > b) b = key;
        }
        b = wave_max_u64(b);
        if ((tid & (kWave - 1)) == 0) sh.red_k[tid / kWave] = b;
        __syncthreads();
        b = sh.red_k[0];
        for (int k = 1; k < kWaves; ++k) b = max(b, sh.red_k[k]);
        __syncthreads();
        if (tid == 0) sh.top[r] = b;
        prev = b;
      }
    }
    __syncthreads();
    for (uint32_t r = tid; r < nt; r += kThreads) {
      const uint32_t id = packed_id(sh.top[r]);
      bool exact;
      const float lp = lp_round((double)x[id], lse, e, &exact);
      top_ids[(uint64_t)row * top + r] = id;
      top_lps[(uint64_t)row * top + r] = lp;
      if (!exact) sh.inexact = 1;
    }
  }
  if (tid == 0) {
    const uint32_t tok = tokens[row];
    bool exact = true;
    float lp = __builtin_nanf("");
    if (tok < n) lp = lp_round((double)x[tok], lse, e, &exact);
    logprob[row] = lp;
    if (!exact) sh.inexact = 1;
    if (tok >= n) sh.inexact = 1;
  }
  __syncthreads();
  if (tid == 0 && status) status[row] = sh.inexact ? AS_LP_INEXACT : AS_LP_OK;
}

}  // namespace

namespace as_launch {

hipError_t logprobs(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride, uint32_t n,
                    uint32_t n_rows, LpPart* parts, const uint32_t* tokens, uint32_t top, float* logprob,
                    uint32_t* top_ids, float* top_lps, uint32_t* status) {
  const uint32_t n_parts = lp_parts(n);
  hipLaunchKernelGGL(lp_part_kernel, dim3(n_parts, n_rows), dim3(kThreads), 0, stream, logits, row_stride, n,
                     vec ? 1u : 0u, parts, n_parts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lp_row_kernel, dim3(n_rows), dim3(kThreads), 0, stream, logits, row_stride, n, parts, n_parts,
                     tokens, top, logprob, top_ids, top_lps, status);
  return hipGetLastError();
}

}  // namespace as_launch

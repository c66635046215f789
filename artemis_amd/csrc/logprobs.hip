// Log-probabilities of the model's own distribution (crates/engine/src/logprobs.rs:12-38): the
// log-softmax of a row's raw logits (before penalties, temperature and filters) at the sampled token,
// and the `top` highest logits' (at most 20), sorted by logit descending with -0 and +0 tied, then by
// the lower id (logprobs.rs:40-48). Rows must be finite (the reference's run_step guarantees it).
//
// Two kernels over the rows in HBM:
//   - lp_part_kernel: one 256-thread workgroup per part of a row (kLpPart values, or kLpPartSmall
//     for a call whose grid of those fills at most one round of the chip: lp_part_len). Its largest value m_p,
//     S_p = sum of exp(x - m_p) in f64 (each term within kExpRel of the reference's exp, from a
//     table-free polynomial: exp_fused), and its 20 best by the reference's order: each wave's 5th
//     largest lane maximum (by value), the smallest of the four, is a threshold with at least 20
//     values of the part at or above it; the few values there go into LDS (each wave's into a
//     segment of its own, at places a ballot per value gives), where a rank count of their (value,
//     id) keys sorts them.
//   - lp_row_kernel: one workgroup per row. M = max m_p; total = sum of S_p * exp(m_p - M);
//     lse = M + ln(total) (logprobs.rs:14-16); the row's nt best come from a merge of the parts'
//     sorted lists (a tournament on one wave); each output is (x - lse) rounded to f32
//     (logprobs.rs:18, 34).
//
// The reference sums exp(x - M) left to right over the row; this sum is parallel, with a bound on
// the distance between the two: gamma(n + 64) relative (both orders' rounding and the rescale of
// each part), kExpRel for the terms' exp, plus the logarithm's own ulp. An output is exact when that
// bound cannot change its rounding to f32; otherwise the row's status says AS_LP_INEXACT, and the
// value is within the bound plus one f32 ulp of the reference's, absolute (near lp = 0 that is many
// ulps: the reference's left-to-right sum drops the terms under half an ulp of its running total).
#include <cstdio>
#include <mutex>

#include "sampler_device.h"
#include "exp_poly.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

using namespace as_dev;
using as_launch::LpPart;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr uint32_t kTop = as_launch::kLpTop;
constexpr uint32_t kList = 1024;             // a part's values at or above its threshold
constexpr uint32_t kMerge = as_launch::kLpMerge;
constexpr uint32_t kEntries = kMerge / kThreads;  // list slots per thread in a row's merge
constexpr double kU = 1.1102230246251565e-16;  // 2^-53
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The reference's order as one descending u64: the logit's rank key with -0 mapped to +0 (they tie),
// then the lower id.
__device__ __forceinline__ uint64_t lp_key(float x, uint32_t id) { return pack(total_key(x == 0.0f ? 0.0f : x), id); }

// A key m such that at least q lanes hold a key at or above it (the q-th largest distinct key, or
// lower when lanes tie), or 0 when fewer than q lanes hold one (0: an empty lane). m0: the wave's
// largest x.
__device__ __forceinline__ uint32_t wave_qth_u32(uint32_t x, uint32_t m0, uint32_t q) {
  uint32_t m = m0;
  for (uint32_t it = 1; it < q; ++it) {
    if (m == 0) return 0;
    if (x == m) x = 0;
    m = wave_max_u32(x);
  }
  return m;
}

__device__ __forceinline__ double gamma_n(double n) { return n * kU / (1.0 - n * kU); }

// Each term's relative error against the reference's exp (ExpPoly::exp_fused and exp_sat, exp_poly.h).
constexpr double kExpRel = kExpPolyRel;

// The value part of lp_key.
__device__ __forceinline__ uint32_t lp_vkey(float x) { return total_key(x == 0.0f ? 0.0f : x); }

// Each wave's kLaneQ-th best lane maximum; the smallest of them has kWaves * kLaneQ values of the part
// at or above it.
constexpr uint32_t kLaneQ = (kTop + kWaves - 1) / kWaves;
static_assert(kLaneQ * kWaves >= kTop, "the waves' thresholds cover the part's best kTop");

// Each wave lists its values at or above the part's threshold in a segment of its own.
constexpr uint32_t kSeg = kList / kWaves;

struct PartShared {
  uint64_t list[kList];
  uint32_t n_seg[kWaves];
  uint32_t red_t[kWaves];
  uint32_t red_u[kWaves];
  double red_d[kWaves];
};

// One part, b0 .. b1 of row x, kPer values per thread. kV4: the part is whole and 16-byte aligned,
// each thread's values in 16-byte groups.
template <bool kV4, uint32_t kPer>
__device__ __forceinline__ void lp_part(PartShared& sh, const float* __restrict__ x, uint32_t b0, uint32_t b1,
                                        LpPart& out) {
  static_assert(kPer % 8 == 0, "whole 16-byte groups per thread, in two halves");
  static_assert(kPer / 2 <= 32, "a thread's running sums stay 32 roundings deep");
  const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  auto off = [&](uint32_t q) { return kV4 ? ((q / 4) * kThreads + tid) * 4 + (q % 4) : q * kThreads + tid; };
  auto valid = [&](uint32_t q) { return kV4 || b0 + off(q) < b1; };
  float v[kPer];
  if (kV4) {
#pragma unroll
    for (uint32_t g = 0; g < kPer / 4; ++g) {
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + b0 + (g * kThreads + tid) * 4));
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * g + c] = t[c];
    }
  } else {
#pragma unroll
    for (uint32_t q = 0; q < kPer; ++q) v[q] = valid(q) ? x[b0 + off(q)] : 0.0f;
  }

  // The thread's largest value (rows are finite; -0 and +0 have one key). A thread holds values when
  // its first one is in the part.
  float bv = v[0];
#pragma unroll
  for (uint32_t q = 1; q < kPer; ++q)
    if (valid(q)) bv = fmaxf(bv, v[q]);
  const bool has = valid(0);
  const uint32_t bk = has ? lp_vkey(bv) : 0u;

  // The part's largest value (-0 and +0 alike: both give the same differences).
  const uint32_t wk = wave_max_u32(bk);
  if (lane == 0) sh.red_u[w] = wk;
  __syncthreads();
  uint32_t kmax = sh.red_u[0];
  for (int k = 1; k < kWaves; ++k) kmax = max(kmax, sh.red_u[k]);
  const float m = key_value(kmax);
  const double md = (double)m;

  // S_p, each term within kExpRel of the reference's exp(f64(x) - m). Each half of the thread's
  // values has its own running sum (at most 32 roundings deep, as the bound on the row's sum counts).
  // A part whose maximum is at most kFusedMax in size takes each term's argument in one fused
  // multiply-add (exp_fused); others subtract m first (exp_sat). Both are within kExpPolyRel.
  ExpPoly ep;
  ep.load();
  double s = 0.0, s2 = 0.0;
  if (fabs(md) <= kFusedMax) {
    const double cm = ExpPoly::fused_offset(md);
#pragma unroll
    for (uint32_t q = 0; q < kPer / 2; ++q) {
      if (valid(q)) s += ep.exp_fused((double)v[q], cm);
      if (valid(q + kPer / 2)) s2 += ep.exp_fused((double)v[q + kPer / 2], cm);
    }
  } else {
    // (Each value passes through an empty asm here, so that the compiler does not convert every value
    // to f64 ahead of the branch, for both loops at once, and hold them all in registers.)
#pragma unroll
    for (uint32_t q = 0; q < kPer / 2; ++q) {
      float a0 = v[q], a1 = v[q + kPer / 2];
      __asm__("" : "+v"(a0), "+v"(a1));
      if (valid(q)) s += ep.exp_sat((double)a0 - md);
      if (valid(q + kPer / 2)) s2 += ep.exp_sat((double)a1 - md);
    }
  }
  s += s2;

  // The threshold: the smallest of the waves' kLaneQ-th largest lane maxima (0 when a wave holds
  // fewer). Each wave has kLaneQ lanes whose maximum is at or above it, so at least kTop values of the
  // part are, and every value among the part's kTop best is.
  const uint32_t tw = wave_qth_u32(bk, wk, kLaneQ);
  s = wave_sum_f64(s);
  if (lane == 0) {
    sh.red_t[w] = tw;
    sh.red_d[w] = s;
  }
  __syncthreads();
  uint32_t T = sh.red_t[0];
  for (int k = 1; k < kWaves; ++k) T = min(T, sh.red_t[k]);
  // Every value at or above the threshold's value (all of them for T = 0), into the wave's segment:
  // each lane's place is the number of lanes below it that list a value at the same step.
  const float t_val = T ? key_value(T) : -__builtin_inff();
  uint64_t* seg = sh.list + w * kSeg;
  uint32_t nw = 0;
#pragma unroll
  for (uint32_t q = 0; q < kPer; ++q) {
    const bool c = valid(q) && v[q] >= t_val;
    const uint64_t b = __ballot(c);
    if (b) {
      const uint32_t i = nw + __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
      if (c && i < kSeg) seg[i] = pack(lp_vkey(v[q]), b0 + off(q));
      nw += (uint32_t)__popcll(b);
    }
  }
  if (lane == 0) sh.n_seg[w] = nw;
  __syncthreads();
  uint32_t n_list = 0;
  bool overflow = false;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    n_list += sh.n_seg[k];
    overflow |= sh.n_seg[k] > kSeg;
  }
  // The list's kTop best, in order: each entry's place is the number of entries above it.
  if (!overflow) {
    for (uint32_t i = tid; i < n_list; i += kThreads) {
      uint32_t k = 0, j = i;
      while (j >= sh.n_seg[k]) j -= sh.n_seg[k++];
      const uint64_t key = sh.list[k * kSeg + j];
      uint32_t r = 0;
      for (uint32_t k2 = 0; k2 < kWaves; ++k2)
        for (uint32_t j2 = 0; j2 < sh.n_seg[k2]; ++j2) r += sh.list[k2 * kSeg + j2] > key ? 1u : 0u;
      if (r < kTop) out.top[r] = key;
    }
  }
  if (tid == 0) {
    double S = sh.red_d[0];
    for (int k = 1; k < kWaves; ++k) S = __dadd_rn(S, sh.red_d[k]);
    out.sum = S;
    out.max = m;
    out.n_top = min(n_list, kTop);
    out.overflow = overflow ? 1u : 0u;
  }
}

template <uint32_t kPart>
__global__ __launch_bounds__(kThreads) void lp_part_kernel(const float* __restrict__ logits, uint64_t row_stride,
                                                           uint32_t n, uint32_t vec, LpPart* __restrict__ parts,
                                                           uint32_t n_parts) {
  __shared__ PartShared sh;
  const uint32_t part = blockIdx.x, row = blockIdx.y;
  const float* x = logits + (uint64_t)row * row_stride;
  const uint32_t b0 = part * kPart, b1 = min(b0 + kPart, n);
  LpPart& out = parts[(uint64_t)row * n_parts + part];
  if (vec && b1 - b0 == kPart) lp_part<true, kPart / kThreads>(sh, x, b0, b1, out);
  else lp_part<false, kPart / kThreads>(sh, x, b0, b1, out);
}

struct RowShared {
  uint64_t tab[256];
  uint64_t lists[kMerge];         // the parts' lists end to end, kTop slots each
  uint64_t top[kTop];
  uint32_t n_top[kMerge / kTop];  // per part: its list's length
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

// One workgroup per row. Every load it needs (the parts' fields and lists, the token's logit) is
// issued at once, before any is used: one round trip to HBM.
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
  const uint32_t tok = tokens[row];
  const uint32_t nt = min(min(top, kTop), n);
  // One part per thread (n_parts <= kMerge / kTop < kThreads), and list slots i = tid + k kThreads of
  // the parts' lists laid end to end (those past a part's n_top are never read below). The
  // addresses are clamped into the row's parts, so that every load is issued unconditionally.
  const bool mine = tid < n_parts;
  const LpPart& q = pp[min(tid, n_parts - 1)];
  const float mx = q.max;
  const double sum = q.sum;
  const uint32_t nq = q.n_top, ovf = q.overflow;
  const uint32_t nm = n_parts * kTop;
  uint64_t ent[kEntries];
  if (nt > 0) {
#pragma unroll
    for (uint32_t k = 0; k < kEntries; ++k) {
      const uint32_t i = min(tid + k * kThreads, nm - 1);
      ent[k] = pp[i / kTop].top[i % kTop];
    }
  }
  const float xt = x[min(tok, n - 1)];

  sh.tab[tid] = as_exp::kTable[tid];
  if (tid == 0) {
    sh.overflow = 0;
    sh.inexact = 0;
  }
  if (mine) sh.n_top[tid] = nq;
  if (nt > 0) {
#pragma unroll
    for (uint32_t k = 0; k < kEntries; ++k)
      if (tid + k * kThreads < nm) sh.lists[tid + k * kThreads] = ent[k];
  }
  // M: the largest part maximum.
  const uint32_t kmax = block_max_u32<kWaves>(mine ? total_key(mx) : 0u, sh.red_u);
  if (mine && ovf) sh.overflow = 1;  // after the block's barriers: thread 0 has cleared it
  const double M = (double)key_value(kmax);
  // total = sum of S_p * exp(m_p - M).
  const double t = mine ? sum * as_exp::exp_with(sh.tab, (double)mx - M) : 0.0;
  const double total = block_sum_f64<kWaves>(t, sh.red_d);  // its barriers publish overflow and the lists
  const double lnt = log(total);
  const double lse = M + lnt;
  // The distance to the reference's lse: both sums' roundings (the reference's n in order; ours at
  // most 55 deep: 33 in a thread, 6 in its wave, 3 across the part's waves, 3 in the part's rescale,
  // 10 in the row's sum), each term's exp, the logarithm's ulp and the final addition.
  const double e = gamma_n((double)n + 64.0) + kExpRel + 4.0 * kU * fabs(lnt) + 2.0 * kU * fabs(lse);

  if (nt > 0) {
    if (!sh.overflow) {
      // The row's nt best, in order, from the parts' sorted lists: a tournament on wave 0, where lane
      // l holds the heads of parts l and l + 64; the largest head is the next best (keys are
      // distinct: they hold the ids), and its part's list moves on. The lists hold at least nt
      // entries together (a part lists min(its values, kTop) or more).
      static_assert(kMerge / kTop <= 2 * kWave, "two parts per lane");
      if (tid < kWave) {
        const uint32_t p0 = tid, p1 = tid + kWave;
        const uint32_t n0 = p0 < n_parts ? sh.n_top[p0] : 0u, n1 = p1 < n_parts ? sh.n_top[p1] : 0u;
        uint32_t h0 = 0, h1 = 0;
        uint64_t k0 = n0 > 0 ? sh.lists[p0 * kTop] : 0ull, k1 = n1 > 0 ? sh.lists[p1 * kTop] : 0ull;
        for (uint32_t r = 0; r < nt; ++r) {
          const uint64_t m = wave_max_u64(max(k0, k1));
          if (tid == 0) sh.top[r] = m;
          if (m == k0) {
            ++h0;
            k0 = h0 < n0 ? sh.lists[p0 * kTop + h0] : 0ull;
          } else if (m == k1) {
            ++h1;
            k1 = h1 < n1 ? sh.lists[p1 * kTop + h1] : 0ull;
          }
        }
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
      // The key holds the logit (-0 as +0, which gives the same difference).
      bool exact;
      const float lp = lp_round((double)packed_value(sh.top[r]), lse, e, &exact);
      top_ids[(uint64_t)row * top + r] = packed_id(sh.top[r]);
      top_lps[(uint64_t)row * top + r] = lp;
      if (!exact) sh.inexact = 1;
    }
  }
  if (tid == 0) {
    bool exact = true;
    float lp = __builtin_nanf("");
    if (tok < n) lp = lp_round((double)xt, lse, e, &exact);
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
  const uint32_t len = lp_part_len(n, n_rows), n_parts = (n + len - 1) / len;
  if (len == kLpPartSmall)
    hipLaunchKernelGGL(lp_part_kernel<kLpPartSmall>, dim3(n_parts, n_rows), dim3(kThreads), 0, stream, logits,
                       row_stride, n, vec ? 1u : 0u, parts, n_parts);
  else
    hipLaunchKernelGGL(lp_part_kernel<kLpPart>, dim3(n_parts, n_rows), dim3(kThreads), 0, stream, logits,
                       row_stride, n, vec ? 1u : 0u, parts, n_parts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lp_row_kernel, dim3(n_rows), dim3(kThreads), 0, stream, logits, row_stride, n, parts, n_parts,
                     tokens, top, logprob, top_ids, top_lps, status);
  return hipGetLastError();
}

}  // namespace as_launch

// ---- as_logprobs_static: the same two kernels with no allocation ---------------------------------
//
// The parts' results live in `scratch`, a file-scope device array each GPU holds once, for the life
// of the process. On the host the array's name is only a stand-in for the device symbol: its device
// address comes from hipGetSymbolAddress, once per device, and only that address is ever handed to a
// kernel. Every call on a GPU shares the array, so calls that overlap on one GPU race; each call's
// part kernel writes every field its row kernel reads, so nothing needs clearing between calls.

namespace {

constexpr uint32_t kStaticParts = 2048;  // 128 rows of the model's 248,320 values (16 parts each)
static __device__ __align__(256) as_launch::LpPart scratch[kStaticParts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
as_launch::LpPart* g_scratch[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up on a device's first call).
hipError_t static_scratch(int dev, as_launch::LpPart** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch[dev] = static_cast<as_launch::LpPart*>(p);
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

int static_fail(char* err, size_t cap, int code, const char* msg) {
  if (err && cap) std::snprintf(err, cap, "%s", msg);
  return code;
}

}  // namespace

extern "C" int as_logprobs_static(void* hip_stream, const float* logits, uint64_t row_stride, uint32_t n_vocab,
                                  uint32_t n_rows, const uint32_t* tokens, uint32_t top, float* logprob,
                                  uint32_t* top_ids, float* top_logprobs, uint32_t* status, char* err,
                                  size_t err_cap) {
  if (err && err_cap) err[0] = 0;
  if (!logits || !tokens || !logprob || n_vocab == 0 || n_rows == 0)
    return static_fail(err, err_cap, AS_ERR_INVALID, "as_logprobs_static: null array or zero size");
  if (top > 0 && (!top_ids || !top_logprobs))
    return static_fail(err, err_cap, AS_ERR_INVALID, "as_logprobs_static: top > 0 needs top_ids and top_logprobs");
  if (row_stride != 0 && row_stride < n_vocab)
    return static_fail(err, err_cap, AS_ERR_INVALID, "as_logprobs_static: row_stride below n_vocab");
  const uint32_t parts = as_launch::lp_parts_of(n_vocab, n_rows);
  if (parts * as_launch::kLpTop > as_launch::kLpMerge)
    return static_fail(err, err_cap, AS_ERR_CAPACITY, "as_logprobs_static: vocabulary wider than the merge holds");
  if ((uint64_t)n_rows * parts > kStaticParts) {
    char msg[200];
    std::snprintf(msg, sizeof msg,
                  "as_logprobs_static: %u rows of %u values need %llu parts of %u values; the static scratch "
                  "holds %u (n_rows x parts per row <= %u)",
                  n_rows, n_vocab, (unsigned long long)n_rows * parts, as_launch::lp_part_len(n_vocab, n_rows),
                  kStaticParts, kStaticParts);
    return static_fail(err, err_cap, AS_ERR_CAPACITY, msg);
  }
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e = hipErrorInvalidDevice;
  as_launch::LpPart* parts_buf = nullptr;
  if (e == hipSuccess) e = static_scratch(dev, &parts_buf);
  if (e == hipSuccess) {
    const bool vec = ((uintptr_t)logits & 15u) == 0 && row_stride % 4 == 0;
    e = as_launch::logprobs((hipStream_t)hip_stream, vec, logits, row_stride, n_vocab, n_rows, parts_buf, tokens,
                            top, logprob, top_ids, top_logprobs, status);
  }
  if (e != hipSuccess) {
    char msg[200];
    std::snprintf(msg, sizeof msg, "as_logprobs_static: %s", hipGetErrorString(e));
    return static_fail(err, err_cap, AS_ERR_HIP, msg);
  }
  return AS_OK;
}

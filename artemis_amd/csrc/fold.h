// Helpers both sampler kernels share: device-coherent accesses between workgroups, the rounding
// bounds of f64 sums, and draw_full_sort's folds (top-p's cut and the draw, sample.rs:157-198) on
// one wave, certified by bounds where they can and in the reference's own order where they cannot.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sampler_device.h"

namespace as_dev {

constexpr double kU = 1.1102230246251565e-16;  // 2^-53, the unit roundoff

__device__ __forceinline__ double gamma_n(double n) { return n * kU / (1.0 - n * kU); }
// An upper bound of gamma_n with no division, for n * kU below 2^-30 (n below 2^22 here):
// gamma_n = n u (1 + n u + ...) <= n u (1 + 2 n u), and the margin 1e-9 also covers the products'
// own roundings.
__device__ __forceinline__ double gamma_ub(double n) { return n * (kU * (1.0 + 1e-9)); }

// A pointer to global memory as such (gload explains why: flat instructions would share the LDS wait
// counter). Every atomic and device-coherent access of the kernel's HBM goes through one.
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gp(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

// Device-coherent loads and stores (relaxed, agent scope): what other workgroups of the kernel write
// with device atomics or such stores, whatever this XCD's L2 holds.
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_agent(const double* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// --- sequential folds on one wave --------------------------------------------------------------
//
// The reference folds a few hundred f64 terms left to right (draw_full_sort's totals and
// cumulatives, sample.rs:169-197; draw_partial's draw, 260-272). One wave does it from registers, 64
// terms a step: every lane adds lane 0's term, then lane 1's, and so on (through readlane), which
// are the reference's roundings in the reference's order, and lane j keeps the running sum once its
// own term is in. The terms' divisions (cum += w / total) do not depend on the running sum, so the
// lanes compute them at once beforehand. Only wave 0 (tid < 64) calls these.

// Lane j of the wave: carry + x_0 + ... + x_j, added left to right.
__device__ __forceinline__ double wave_seq_prefix(double x, double carry) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
  double s = carry, mine = carry;
#pragma unroll
  for (int j = 0; j < kWave; ++j) {
    const uint32_t l = (uint32_t)__builtin_amdgcn_readlane(lo, j), h = (uint32_t)__builtin_amdgcn_readlane(hi, j);
    s = __dadd_rn(s, __longlong_as_double((long long)(((uint64_t)h << 32) | l)));
    if (lane == (uint32_t)j) mine = s;
  }
  return mine;
}
__device__ __forceinline__ double wave_lane63(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t l = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, kWave - 1);
  const uint32_t h = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), kWave - 1);
  return __longlong_as_double((long long)(((uint64_t)h << 32) | l));
}
// The left fold of w[0..m) (zeros past m change no sum of positive terms).
__device__ __forceinline__ double wave_seq_total(const double* w, uint32_t m) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  double carry = 0.0;
  for (uint32_t b0 = 0; b0 < m; b0 += kWave) {
    const double x = (b0 + lane < m) ? w[b0 + lane] : 0.0;
    carry = wave_lane63(wave_seq_prefix(x, carry));
  }
  return carry;
}

// draw_full_sort's top-p cut (sample.rs:166-179) over w[0..m) in the reference's order: the total,
// then cum += w_i / total until cum reaches top_p; returns the kept count (m when it never does).
__device__ __forceinline__ uint32_t wave_seq_cut(const double* w, uint32_t m, double top_p) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const double tot = wave_seq_total(w, m);
  double carry = 0.0;
  for (uint32_t b0 = 0; b0 < m; b0 += kWave) {
    const uint32_t i = b0 + lane;
    const double q = (i < m) ? __ddiv_rn(w[i], tot) : 0.0;
    const double cum = wave_seq_prefix(q, carry);
    const uint64_t hit = __ballot(i < m && cum >= top_p);
    if (hit) return b0 + (uint32_t)__builtin_ctzll(hit) + 1;
    carry = wave_lane63(cum);
  }
  return m;
}
// The draw over w[0..m) in the reference's order (sample.rs:184-197, 260-272): u = u01 * total,
// then the first rank whose cumulative weight passes u (the last when none does). *tot gets the total.
__device__ __forceinline__ uint32_t wave_seq_draw(const double* w, uint32_t m, double u01, double* tot) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const double t = wave_seq_total(w, m);
  const double u = __dmul_rn(u01, t);
  *tot = t;
  double carry = 0.0;
  for (uint32_t b0 = 0; b0 < m; b0 += kWave) {
    const uint32_t i = b0 + lane;
    const double cum = wave_seq_prefix((i < m) ? w[i] : 0.0, carry);
    const uint64_t hit = __ballot(i < m && u < cum);
    if (hit) return b0 + (uint32_t)__builtin_ctzll(hit);
    carry = wave_lane63(cum);
  }
  return m - 1;
}

// --- certified decisions on one wave ----------------------------------------------------------
//
// Up to kWPer * 64 sorted values, lane l holding ranks kWPer*l .. kWPer*l + kWPer-1 in registers.
// Their prefix sums come from a fold of kWPer in the lane and a scan over the lanes: each is a sum
// of positive terms through at most kWPer + 7 roundings, within gamma(kWPer + 7) of its exact value,
// as the reference's left fold of j + 1 terms is within gamma(j) of it. A decision the two bounds
// agree on is the reference's; otherwise the caller takes the sequential fold above.
constexpr int kWPer = 4;
constexpr uint32_t kWaveMax = kWPer * kWave;

// Inclusive prefix sums pre[] of the values w[] in rank order; returns the total to every lane.
__device__ __forceinline__ double wave_prefix(const double (&w)[kWPer], double (&pre)[kWPer]) {
  double run = 0.0;
#pragma unroll
  for (int q = 0; q < kWPer; ++q) {
    run = __dadd_rn(run, w[q]);
    pre[q] = run;
  }
  const double incl = wave_scan_f64(run);
  const double excl = wave_prev_f64(incl);
#pragma unroll
  for (int q = 0; q < kWPer; ++q) pre[q] = __dadd_rn(excl, pre[q]);
  return wave_lane_f64(incl, kWave - 1);
}
// The first rank below m whose flag is set (m when none).
__device__ __forceinline__ uint32_t wave_first(const bool (&f)[kWPer], uint32_t m) {
  const uint32_t i0 = (threadIdx.x & (kWave - 1)) * kWPer;
  uint32_t first = m;
#pragma unroll
  for (int q = kWPer - 1; q >= 0; --q)
    if (f[q] && i0 + q < m) first = i0 + q;
  return wave_min_u32(first);
}
// draw_full_sort's top-p cut over the m values' weights w (zero past m): the kept count, or kNone
// when the bounds cannot decide. The reference's cumulative at rank j, its left fold of
// fl(w_i / total), lies within gamma(j + 1) of exact / its total, which is within gamma(m) of exact;
// ours (prefix / total) within gamma(kWPer + 8) of exact.
__device__ __forceinline__ uint32_t wave_topp_cut(const double (&w)[kWPer], uint32_t m, double top_p) {
  double pre[kWPer];
  const double S = wave_prefix(w, pre);
  const uint32_t i0 = (threadIdx.x & (kWave - 1)) * kWPer;
  const double base = 2.0 * gamma_ub(2.0 * kWPer + 16.0) + gamma_ub(2.0 * (double)m + 4.0) + 10.0 * kU;
  // pre / S against top_p as pre against top_p * S (S > 0): the products' roundings are within the
  // 10 u of base.
  const double t = top_p * S;
  bool lo[kWPer], hi[kWPer];
#pragma unroll
  for (int q = 0; q < kWPer; ++q) {
    const double rel = base + gamma_ub(2.0 * (double)(i0 + q) + 4.0);
    lo[q] = pre[q] * (1.0 + rel) >= t;  // the reference's cumulative may have reached top_p
    hi[q] = pre[q] * (1.0 - rel) >= t;  // it certainly has
  }
  const uint32_t jl = wave_first(lo, m), jh = wave_first(hi, m);
  if (jl != jh) return kNone;
  return jh < m ? jh + 1 : m;
}
// The draw over the m values' weights w (zero past m) with u = u01 * total (sample.rs:184-197,
// 260-272): the first rank whose cumulative passes u (m - 1 when none does), or kNone when the
// bounds cannot decide. *tot gets our total (within gamma(m) + gamma(kWPer + 8) of the reference's).
__device__ __forceinline__ uint32_t wave_draw(const double (&w)[kWPer], uint32_t m, double u01, double* tot) {
  double pre[kWPer];
  const double S = wave_prefix(w, pre);
  *tot = S;
  const uint32_t i0 = (threadIdx.x & (kWave - 1)) * kWPer;
  const double g = gamma_ub(2.0 * kWPer + 16.0);
  const double d = gamma_ub((double)m + 1.0) + g + 4.0 * kU;
  const double ulo = u01 * S * (1.0 - d) * (1.0 - 3.0 * kU), uhi = u01 * S * (1.0 + d) * (1.0 + 3.0 * kU);
  bool may[kWPer], sure[kWPer];
#pragma unroll
  for (int q = 0; q < kWPer; ++q) {
    const double rel = gamma_ub((double)(i0 + q) + 1.0) + g + 4.0 * kU;
    may[q] = pre[q] * (1.0 + rel) > ulo;
    sure[q] = pre[q] * (1.0 - rel) > uhi;
  }
  const uint32_t jp = wave_first(may, m), jc = wave_first(sure, m);
  if (jp != jc) return kNone;
  return jc < m ? jc : m - 1;
}

// draw_full_sort's tail (sample.rs:164-197) over the k best values of a row, sorted in rank order in
// sk[0..k) (packed keys, k <= kWaveMax): the weights first, by the threads below k (every thread of
// the block calls it; a barrier must follow): w[i] = exp((l_i - top) / T) at wd[i] and, with top-p,
// exp(l_i - top) at wd[kWaveMax + i], from the host-exact exp (tab: its table in LDS).
__device__ __forceinline__ void topk_weights(const uint64_t* sk, uint32_t k, double top, double temp, bool topp,
                                             const uint64_t* tab, double* wd) {
  const uint32_t tid = threadIdx.x;
  if (tid < k) {
    const double v = (double)packed_value(sk[tid]);
    wd[tid] = as_exp::exp_with(tab, __ddiv_rn(__dsub_rn(v, top), temp));
    if (topp) wd[kWaveMax + tid] = as_exp::exp_with(tab, __dsub_rn(v, top));
  }
}
// Then wave 0 (threads below 64 only): top-p's cut at T = 1, min-p's floor (the ranks are sorted, so
// it keeps a prefix) and the draw, each decided by bounds and by the reference's sequential folds
// only when the bounds cannot. *keep gets the kept count, *pick the rank drawn, *tot the kept total.
__device__ __forceinline__ void topk_decide(const uint64_t* sk, uint32_t k, double top_p, bool topp, bool has_floor,
                                            double floor, double u01, const double* wd, uint32_t* keep,
                                            uint32_t* pick, double* tot) {
  const uint32_t i0 = (threadIdx.x & (kWave - 1)) * kWPer;
  const double* w1s = wd + kWaveMax;
  uint32_t kk = k;
  if (topp) {
    double w[kWPer];
#pragma unroll
    for (int q = 0; q < kWPer; ++q) w[q] = (i0 + q < k) ? w1s[i0 + q] : 0.0;
    kk = wave_topp_cut(w, k, top_p);
    if (kk == kNone) kk = wave_seq_cut(w1s, k, top_p);
  }
  if (has_floor) {
    bool below[kWPer];
#pragma unroll
    for (int q = 0; q < kWPer; ++q) below[q] = (i0 + q < kk) && !((double)packed_value(sk[i0 + q]) >= floor);
    kk = wave_first(below, kk);
  }
  double w[kWPer], t = 0.0;
#pragma unroll
  for (int q = 0; q < kWPer; ++q) w[q] = (i0 + q < kk) ? wd[i0 + q] : 0.0;
  uint32_t pk = wave_draw(w, kk, u01, &t);
  if (pk == kNone) pk = wave_seq_draw(wd, kk, u01, &t);
  *keep = kk;
  *pick = pk;
  *tot = t;
}

}  // namespace as_dev

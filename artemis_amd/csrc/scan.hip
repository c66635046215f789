// Pass 1 over the logits: one workgroup per 8,192-value segment of a row, the only kernel that
// reads the rows from HBM. Each thread holds 32 values in registers (eight 16-byte loads, all in
// flight at once), applies the history penalties from an LDS count table, and produces the
// segment's share of everything the finish kernel decides from:
//   - the first non-finite index (sample.rs:22-34),
//   - greedy's argmax (sample.rs:9-17, 378-396),
//   - the largest rank key (the `top` of sample.rs:164, 212-216),
//   - the segment's best candidates in rank order (its top k, or a fixed budget for rows without a
//     top-k), found by a binary search on the key threshold and compacted to HBM,
//   - for rows without a top-k, f64 sums of exp(l - m) or exp((l - m) / T) with m the segment's
//     max, each term with the host-exact exp, and sums of exp(d) * |d| for the error bound.
#include "sampler_device.h"
#include "launch.h"

using namespace as_dev;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kPer = 32;
constexpr int kVec = kPer / 4;
typedef float f32x4 __attribute__((ext_vector_type(4)));
static_assert(kThreads * kPer == as_launch::kSegment, "segment size");

// Exclusive prefix sum over the block (in thread order) of one u32 per thread; *total gets the sum.
__device__ uint32_t block_exclusive_scan(uint32_t x, uint32_t* wave_tot, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  uint32_t incl = x;
  for (int o = 1; o < kWave; o <<= 1) {
    uint32_t y = (uint32_t)__shfl_up((int)incl, o, kWave);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == kWave - 1) wave_tot[w] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int k = 0; k < kWaves; ++k) {
    if (k < w) before += wave_tot[k];
    all += wave_tot[k];
  }
  *total = all;
  return before + incl - x;
}

template <bool kVecLoad>
__global__ __launch_bounds__(kThreads) void scan_kernel(
    const float* __restrict__ logits, uint64_t row_stride, uint32_t n, uint32_t n_seg,
    const RowParams* __restrict__ params, const uint32_t* __restrict__ hist_off,
    const uint32_t* __restrict__ hist_ids, const uint32_t* __restrict__ extra_ids,
    SegStats* __restrict__ stats, uint64_t* __restrict__ cands, uint32_t cand_stride) {
  __shared__ uint32_t cnt[as_launch::kSegment / 2];  // u16 history counts, two per word
  __shared__ uint64_t tab[256];
  __shared__ uint32_t red_u[kWaves];
  __shared__ uint32_t red_u2[kWaves];
  __shared__ double red_d[kWaves];
  __shared__ uint32_t tm[2 * kThreads];
  __shared__ uint32_t slot;

  const uint32_t row = blockIdx.y, seg = blockIdx.x, tid = threadIdx.x;
  const RowParams p = params[row];
  const uint32_t base = seg * (uint32_t)as_launch::kSegment;
  const uint32_t len = min((uint32_t)as_launch::kSegment, n - base);
  const float* src = logits + (uint64_t)row * row_stride + base;

  float v[kPer];
  if (kVecLoad && len == (uint32_t)as_launch::kSegment) {
    // A full segment: eight unconditional 16-byte loads, all in flight before the first use.
    f32x4 q[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j)
      q[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + (j * kThreads + tid) * 4));
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      v[4 * j + 0] = q[j][0];
      v[4 * j + 1] = q[j][1];
      v[4 * j + 2] = q[j][2];
      v[4 * j + 3] = q[j][3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const uint32_t e = (j * kThreads + tid) * 4;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * j + c] = (e + c < len) ? src[e + c] : 0.0f;
    }
  }
  // History ids are loaded now, while the logits are in flight: the first 8 per thread (a
  // 2,048-id history in one go), the rest later.
  uint32_t hb = 0, he = 0;
  if (hist_ids) {
    if (hist_off) {
      hb = hist_off[row];
      he = hist_off[row + 1];
    } else {
      hb = p.hist_begin;
      he = p.hist_begin + p.hist_len;
    }
  }
  const uint32_t extra = extra_ids ? p.extra : 0;
  // Counts are u16 here; a longer history is left to the exact path's u32 counts.
  const bool long_history = (uint64_t)(he - hb) + extra > 0xFFFFu;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0) && !long_history;
  constexpr int kHistRegs = 8;
  uint32_t hreg[kHistRegs];
  if (pen && he > hb) {
#pragma unroll
    for (int q = 0; q < kHistRegs; ++q) hreg[q] = hist_ids[min(hb + tid + q * kThreads, he - 1)];
  }
  tab[tid] = as_exp::kTable[tid];

  // The raw row's first non-finite value.
  uint32_t bad = kNone;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const uint32_t e = ((q / 4) * kThreads + tid) * 4 + (q & 3);
    if (e < len && !is_finite_bits(v[q])) bad = min(bad, base + e);
  }
  bad = block_min_u32<kWaves>(bad, red_u);

  // Penalties from the history (and, for verify rows, the drafts before the row).
  if (pen && bad == kNone) {
    for (int i = tid; i < as_launch::kSegment / 2; i += kThreads) cnt[i] = 0;
    __syncthreads();
    if (he > hb) {
#pragma unroll
      for (int q = 0; q < kHistRegs; ++q) {
        const uint32_t off = hreg[q] - base;
        if (hb + tid + q * kThreads < he && off < len) atomicAdd(&cnt[off >> 1], 1u << ((off & 1) * 16));
      }
    }
    for (uint32_t h = hb + tid + kHistRegs * kThreads; h < he; h += kThreads) {
      const uint32_t off = hist_ids[h] - base;
      if (off < len) atomicAdd(&cnt[off >> 1], 1u << ((off & 1) * 16));
    }
    for (uint32_t h = tid; h < extra; h += kThreads) {
      const uint32_t off = extra_ids[h] - base;
      if (off < len) atomicAdd(&cnt[off >> 1], 1u << ((off & 1) * 16));
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const uint32_t e = (j * kThreads + tid) * 4;
      const uint32_t w0 = cnt[e >> 1], w1 = cnt[(e >> 1) + 1];
      const uint32_t c4[4] = {w0 & 0xFFFFu, w0 >> 16, w1 & 0xFFFFu, w1 >> 16};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (c4[c] != 0 && e + c < len) v[4 * j + c] = penalize(v[4 * j + c], c4[c], p);
    }
  }

  // Rank keys from here on; 0 marks a slot past the segment's end (no finite value has key 0).
  uint32_t k[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const uint32_t e = ((q / 4) * kThreads + tid) * 4 + (q & 3);
    k[q] = (e < len) ? total_key(v[q]) : 0u;
  }

  // The two largest keys of each thread, and the segment's largest.
  uint32_t tmax = 0, tmax2 = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    tmax2 = max(tmax2, min(tmax, k[q]));
    tmax = max(tmax, k[q]);
  }
  const uint32_t mk = block_max_u32<kWaves>(tmax, red_u);

  // Greedy (sample.rs:9-17, 378-396): the lowest index holding the largest value by IEEE `>`,
  // so +0 and -0 tie. Only greedy rows need it.
  uint32_t gi = kNone;
  float gv = 0.0f;
  if (p.mode == kModeGreedy && bad == kNone) {
    gv = key_value(mk);
    uint32_t first = kNone;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const uint32_t e = ((q / 4) * kThreads + tid) * 4 + (q & 3);
      if (k[q] != 0u && key_value(k[q]) == gv) first = min(first, base + e);
    }
    gi = block_min_u32<kWaves>(first, red_u);
  }

  SegStats st;
  st.nonfinite = bad;
  st.greedy_idx = gi;
  st.greedy_val = gv;
  st.max_key = mk;
  st.n_cand = 0;
  st.truncated = ((p.flags & kFlagPenalties) && long_history) ? 2u : 0u;
  st.bound = 0;
  st.sum = 0.0;
  st.sum_abs = 0.0;

  const uint32_t C = p.cand;
  if (bad == kNone && C > 0) {
    uint64_t* out = cands + ((uint64_t)row * n_seg + seg) * cand_stride;
    const int lane = tid & (kWave - 1), w = tid / kWave;
    if (len <= C) {
      // The whole segment, in index order.
      uint32_t wc = 0;
#pragma unroll
      for (int q = 0; q < kPer; ++q) wc += (uint32_t)__popcll(__ballot(k[q] != 0u));
      if (lane == 0) red_u2[w] = wc;
      __syncthreads();
      uint32_t run = 0;
      for (int x = 0; x < w; ++x) run += red_u2[x];
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const uint64_t m = __ballot(k[q] != 0u);
        const uint32_t e = ((q / 4) * kThreads + tid) * 4 + (q & 3);
        if (k[q] != 0u) out[run + __popcll(m & ((1ull << lane) - 1))] = pack(k[q], base + e);
        run += (uint32_t)__popcll(m);
      }
      st.n_cand = len;
    } else {
      // tau = the C-th largest of the 512 values that are some thread's largest or second largest:
      // they are distinct values, so at least C values are >= tau and the segment's C best are
      // among the values >= tau. Each wave finds tau on its own from the 512 in LDS (eight per
      // lane, counted by ballots).
      tm[tid] = tmax;
      tm[tid + kThreads] = tmax2;
      __syncthreads();
      uint32_t a[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) a[x] = tm[lane + 64 * x];
      uint64_t lo = 0, hi = (uint64_t)mk + 1;
      while (hi - lo > 1) {
        const uint32_t mid = (uint32_t)(lo + ((hi - lo) >> 1));
        uint32_t c = 0;
#pragma unroll
        for (int x = 0; x < 8; ++x) c += (uint32_t)__popcll(__ballot(a[x] >= mid));
        if (c >= C) lo = mid; else hi = mid;
      }
      const uint32_t tau = (uint32_t)lo;
      uint32_t wc = 0;
#pragma unroll
      for (int q = 0; q < kPer; ++q) wc += (uint32_t)__popcll(__ballot(k[q] >= tau));
      if (lane == 0) red_u2[w] = wc;
      __syncthreads();
      uint32_t M = 0, run = 0;
      for (int x = 0; x < kWaves; ++x) {
        if (x < w) run += red_u2[x];
        M += red_u2[x];
      }
      if (M <= p.cap) {
        // Every value >= tau, compacted by ballots in (load, lane) order.
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
          const uint64_t m = __ballot(k[q] >= tau);
          const uint32_t e = ((q / 4) * kThreads + tid) * 4 + (q & 3);
          if (k[q] >= tau) out[run + __popcll(m & ((1ull << lane) - 1))] = pack(k[q], base + e);
          run += (uint32_t)__popcll(m);
        }
        st.n_cand = M;
        st.truncated |= (M < len) ? 1u : 0u;
        st.bound = (uint64_t)tau << 32;
      } else {
        // Too many values tie near tau (a flat or coarse row): the exact C best instead. Largest t
        // with at least C keys >= t, by ballot counts; the keys > t, then the lowest ids equal to t.
        if (tid == 0) slot = 0;
        uint64_t lo2 = 0, hi2 = (uint64_t)mk + 1;
        uint32_t cnt_lo = len, cnt_hi = 0;
        int parity = 0;
        while (hi2 - lo2 > 1 && cnt_lo != C) {
          const uint32_t mid = (uint32_t)(lo2 + ((hi2 - lo2) >> 1));
          uint32_t c = 0;
#pragma unroll
          for (int q = 0; q < kPer; ++q) c += (uint32_t)__popcll(__ballot(k[q] >= mid));
          uint32_t* buf = parity ? red_u2 : red_u;
          __syncthreads();
          if (lane == 0) buf[w] = c;
          __syncthreads();
          c = 0;
#pragma unroll
          for (int x = 0; x < kWaves; ++x) c += buf[x];
          parity ^= 1;
          if (c >= C) {
            lo2 = mid;
            cnt_lo = c;
          } else {
            hi2 = mid;
            cnt_hi = c;
          }
        }
        __syncthreads();
        const uint32_t t = (uint32_t)lo2;
        uint32_t tie_max = 0;
        if (cnt_lo == C) {
#pragma unroll
          for (int q = 0; q < kPer; ++q) {
            const uint32_t e = ((q / 4) * kThreads + tid) * 4 + (q & 3);
            if (k[q] >= t) {
              out[atomicAdd(&slot, 1u)] = pack(k[q], base + e);
              if (k[q] == t) tie_max = max(tie_max, base + e);
            }
          }
        } else {
          const uint32_t need = C - cnt_hi;
          // Ties in index order: the index of value q is ((q/4)*kThreads + tid)*4 + q%4, so the
          // order is (load j, thread, lane of the float4).
          uint32_t running = 0;
          for (int j = 0; j < kVec; ++j) {
            uint32_t mine = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) mine += (k[4 * j + c] == t) ? 1u : 0u;
            uint32_t total;
            uint32_t r = running + block_exclusive_scan(mine, red_u2, &total);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const uint32_t e = (j * kThreads + tid) * 4 + c;
              const uint32_t kk = k[4 * j + c];
              if (kk > t) {
                out[atomicAdd(&slot, 1u)] = pack(kk, base + e);
              } else if (kk == t) {
                if (r < need) {
                  out[atomicAdd(&slot, 1u)] = pack(kk, base + e);
                  tie_max = max(tie_max, base + e);
                }
                ++r;
              }
            }
            running += total;
          }
        }
        tie_max = block_max_u32<kWaves>(tie_max, red_u);
        st.n_cand = C;
        st.truncated |= 1u;
        st.bound = pack(t, tie_max);
      }
    }
  }

  if (bad == kNone && (p.flags & (kFlagSumTop | kFlagSumTemp))) {
    const double m = (double)key_value(mk);
    const bool by_temp = (p.flags & kFlagSumTemp) != 0;
    const double temp = (double)p.temp;
    double s = 0.0, sa = 0.0;
    __syncthreads();  // tab[] is written
#pragma unroll 4
    for (int q = 0; q < kPer; ++q) {
      if (k[q] != 0u) {
        double d = __dsub_rn((double)key_value(k[q]), m);
        if (by_temp) d = __ddiv_rn(d, temp);
        const double x = as_exp::exp_with(tab, d);
        s = __dadd_rn(s, x);
        if (x != 0.0) sa = __dadd_rn(sa, __dmul_rn(x, fabs(d)));
      }
    }
    st.sum = block_sum_f64<kWaves>(s, red_d);
    st.sum_abs = block_sum_f64<kWaves>(sa, red_d);
  }

  if (tid == 0) stats[(uint64_t)row * n_seg + seg] = st;
}

}  // namespace

namespace as_launch {

hipError_t scan(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride, uint32_t n,
                uint32_t n_rows, uint32_t n_seg, const as_dev::RowParams* params,
                const uint32_t* hist_off, const uint32_t* hist_ids, const uint32_t* extra_ids,
                as_dev::SegStats* stats, uint64_t* cands, uint32_t cand_stride) {
  dim3 grid(n_seg, n_rows);
  if (vec)
    hipLaunchKernelGGL(scan_kernel<true>, grid, dim3(kThreads), 0, stream, logits, row_stride, n,
                       n_seg, params, hist_off, hist_ids, extra_ids, stats, cands, cand_stride);
  else
    hipLaunchKernelGGL(scan_kernel<false>, grid, dim3(kThreads), 0, stream, logits, row_stride, n,
                       n_seg, params, hist_off, hist_ids, extra_ids, stats, cands, cand_stride);
  return hipGetLastError();
}

}  // namespace as_launch

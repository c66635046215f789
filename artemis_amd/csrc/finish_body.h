// The finish's body: one workgroup merges one row's scan results and chooses its token (see
// finish.hip for the algorithm). Included by a kernel file after it defines
//   AS_FIN_NS       the namespace of this copy,
//   AS_FIN_THREADS  threads per workgroup (a power of two, 256 to 1024),
//   AS_FIN_MAX_SEG  the most slices a row may have,
// The entry point is AS_FIN_NS::finish_row.
namespace {
namespace AS_FIN_NS {

using namespace as_dev;
using as_launch::FinishArgs;

constexpr int kThreads = AS_FIN_THREADS;
constexpr int kWaves = kThreads / kWave;
constexpr int kCap = as_launch::kFinishCap;
// Prefix scans hold kScanPer consecutive values per thread (kCap in all).
constexpr int kScanPer = kCap / kThreads;
static_assert(kCap % kThreads == 0 && kThreads >= 256 && (kThreads & (kThreads - 1)) == 0, "a power of two");
constexpr int kMaxSeg = AS_FIN_MAX_SEG;
constexpr int kStage = 4096;
struct Shared {
  uint64_t sk[kCap];  // candidates (exact path: per-wave digit counts)
  double wd[kCap];    // weights and prefix sums (exact path: staging for sequential folds)
  uint64_t tab[256];
  uint32_t hist[256];
  uint32_t base[256];
  uint32_t tot[256];
  uint32_t seg_off[kMaxSeg + 1];
  SegStats seg[kMaxSeg];
  uint32_t bcnt[1024];
  uint32_t bstart[1024];
  uint32_t red_u[kWaves];
  double red_d[kWaves];
  double red_d2[kWaves];
  // Row scalars.
  uint32_t hist_over;
  uint32_t bad, gi, mk, total, trunc, keep, pick, done, exact, prefix, stats_bad, nsk, tail_over, have_tail, tail_count,
      tail_listed, tail_parts;
  uint64_t bound_key;
  double u01, sum, x, eps, x1, eps1, r_prefix, w_lo, w_hi, m_lo, m_hi, dp_lo, dp_hi;
  uint32_t draw_rng;  // the row draws: its stream advances once the candidates are in flight
  // S's sums (tail_list_load, tail_help, tail_wait): this call's flagged rows, this row's place among them.
  uint32_t tl_n, tl_rows[kTailListMax], tl_help[kTailListMax], tl_me, tail_slot, tail_waited, tail_won;
  // The shared deep passes (deep_run, deep_help, deep_part).
  uint32_t dp_pick, dp_stop, dp_q, dp_base, dp_staged, dp_mk, dp_r[2 * 3];
  uint32_t dp_pub;  // this row published its histogram pass early (deep_publish_hist)
  // The fast decision's hand-over from wave 0 to the block: how many weights to scan (0: none),
  // whether the kept set runs past them, and the bounds on u.
  uint32_t fp_m, fp_past;
  uint32_t vast;  // a slice found min-p's floor set vast
  // The row's parameters, RNG state and history bounds, loaded with the list of flagged rows at the
  // kernel's start (row_prefetch), so that a row that first takes parts of S finds them in LDS.
  RowParams prm;
  uint64_t rng4[4];
  uint32_t pf_hb, pf_he;
  double fp_lo, fp_hi;
};
// The workgroup's LDS, at file scope so that the out-of-line paths below address it as LDS.
__shared__ Shared g_sh_static;
__device__ __forceinline__ Shared& shm() { return g_sh_static; }

// --- block helpers ------------------------------------------------------------------------------

// Exclusive prefix sum of one f64 per thread over the block: a wave scan, then every wave scans the
// waves' totals (depth 6 + 4 + 1 over any thread's terms).
__device__ double block_exclusive_scan_f64(double x, double* wave_tot) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const double incl = wave_scan_f64(x);
  __syncthreads();
  if (lane == kWave - 1) wave_tot[w] = incl;
  __syncthreads();
  const double waves = wave_scan_f64(lane < kWaves ? wave_tot[lane] : 0.0);
  const double before = w == 0 ? 0.0 : wave_lane_f64(waves, (uint32_t)(w - 1));
  // incl - x is not exact; the exclusive value is the wave's inclusive scan shifted by a lane.
  return __dadd_rn(before, wave_prev_f64(incl));
}

// --- the exact-order path ---------------------------------------------------------------------

// Thread 0's left-to-right f64 fold of term(i), i in [0, m), staged through LDS in tiles that all
// threads fill. Returns the sum to every thread.
template <class Term>
__device__ __forceinline__ double seq_fold(Shared& sh, uint32_t m, Term term) {
  double* stage = sh.wd;
  double acc = 0.0;
  for (uint32_t t0 = 0; t0 < m; t0 += kStage) {
    const uint32_t c = min((uint32_t)kStage, m - t0);
    for (uint32_t i = threadIdx.x; i < c; i += kThreads) stage[i] = term(t0 + i);
    __syncthreads();
    if (threadIdx.x == 0)
      for (uint32_t i = 0; i < c; ++i) acc = __dadd_rn(acc, stage[i]);
    __syncthreads();
  }
  if (threadIdx.x == 0) sh.sum = acc;
  __syncthreads();
  const double r = sh.sum;
  __syncthreads();
  return r;
}

// One stable pass of an LSD radix sort on 8 bits: (src_key, src_id) -> (dst_key, dst_id).
__device__ __forceinline__ void radix_pass(Shared& sh, uint32_t n, int shift, const uint32_t* src_key,
                           const uint32_t* src_id, uint32_t* dst_key, uint32_t* dst_id) {
  uint32_t* wcnt = reinterpret_cast<uint32_t*>(sh.sk);  // [kWaves][256]
  const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  if (tid < 256) sh.hist[tid] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kThreads) atomicAdd(&sh.hist[(src_key[i] >> shift) & 255u], 1u);
  __syncthreads();
  if (tid == 0) {
    uint32_t run = 0;
    for (int d = 0; d < 256; ++d) {
      sh.base[d] = run;
      run += sh.hist[d];
    }
  }
  for (uint32_t i = tid; i < kWaves * 256; i += kThreads) wcnt[i] = 0;
  __syncthreads();
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (uint32_t t0 = 0; t0 < n; t0 += kThreads) {
    const uint32_t i = t0 + tid;
    const bool valid = i < n;
    const uint32_t k = valid ? src_key[i] : 0u, id = valid ? src_id[i] : 0u;
    const uint32_t d = (k >> shift) & 255u;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t bb = __ballot(valid && ((d >> b) & 1u));
      peers &= ((d >> b) & 1u) ? bb : ~bb;
    }
    const uint32_t rank = __popcll(peers & below), count = __popcll(peers);
    if (valid && rank == count - 1) wcnt[w * 256 + d] = count;
    __syncthreads();
    if (tid < 256) {
      uint32_t run = 0;
      for (int ww = 0; ww < kWaves; ++ww) {
        const uint32_t c = wcnt[ww * 256 + tid];
        wcnt[ww * 256 + tid] = run;
        run += c;
      }
      sh.tot[tid] = run;
    }
    __syncthreads();
    if (valid) {
      const uint32_t pos = sh.base[d] + wcnt[w * 256 + d] + rank;
      dst_key[pos] = k;
      dst_id[pos] = id;
    }
    __syncthreads();
    if (tid < 256) sh.base[tid] += sh.tot[tid];
    for (uint32_t j = tid; j < kWaves * 256; j += kThreads) wcnt[j] = 0;
    __syncthreads();
  }
}

// The reference's algorithm in its own order: Sampler::sample's dispatch (sample.rs:136-149),
// draw_full_sort (157-198) for top-k rows and draw_partial (208-293) otherwise.
__device__ __noinline__ void exact_row(const FinishArgs& a, const RowParams& p, uint32_t row) {
  Shared& sh = shm();
  const uint32_t n = a.n, tid = threadIdx.x;
  uint32_t* S = a.scratch + (uint64_t)row * a.scratch_stride;
  uint32_t* cnt = S;
  uint32_t* keyA = S + n;
  uint32_t* idA = S + 2 * (uint64_t)n;
  uint32_t* keyB = S + 3 * (uint64_t)n;
  uint32_t* idB = S + 4 * (uint64_t)n;
  const float* x = a.logits + (uint64_t)row * a.row_stride;

  uint32_t hb;
  const uint32_t he = history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  if (pen) {
    for (uint32_t i = tid; i < n; i += kThreads) cnt[i] = 0;
    __syncthreads();
    for (uint32_t h = hb + tid; h < he; h += kThreads) {
      const uint32_t id = gload(a.hist_ids + h);
      if (id < n) atomicAdd(&cnt[id], 1u);
    }
    for (uint32_t h = tid; h < extra; h += kThreads) {
      const uint32_t id = gload(a.extra_ids + h);
      if (id < n) atomicAdd(&cnt[id], 1u);
    }
    __syncthreads();
  }
  auto value = [&](uint32_t i) -> float {
    float v = x[i];
    if (pen) {
      const uint32_t c = cnt[i];
      if (c) v = penalize(v, c, p);
    }
    return v;
  };
  for (uint32_t i = tid; i < n; i += kThreads) {
    keyA[i] = ~total_key(value(i));
    idA[i] = i;
  }
  __syncthreads();
  radix_pass(sh, n, 0, keyA, idA, keyB, idB);
  radix_pass(sh, n, 8, keyB, idB, keyA, idA);
  radix_pass(sh, n, 16, keyA, idA, keyB, idB);
  radix_pass(sh, n, 24, keyB, idB, keyA, idA);
  // Rank j: id idA[j], value key_value(~keyA[j]).
  auto rv = [&](uint32_t j) -> double { return (double)key_value(~keyA[j]); };
  const double top = rv(0);
  const double temp = (double)p.temp;
  const bool has_floor = p.min_p > 0.0f;
  const double floor = __dadd_rn(top, p.ln_min_p);
  const double top_p = (double)p.top_p;
  const uint64_t* tab = sh.tab;
  auto w_temp = [&](double v) { return as_exp::exp_with(tab, __ddiv_rn(__dsub_rn(v, top), temp)); };
  auto w_one = [&](double v) { return as_exp::exp_with(tab, __dsub_rn(v, top)); };

  uint32_t keep = 0;
  bool unfiltered = false;
  if (p.mode == kModeExactTopK || p.mode == kModeTopK) {
    const uint32_t k = p.top_k;
    keep = k;
    if (p.top_p < 1.0f) {
      const double total = seq_fold(sh, k, [&](uint32_t j) { return w_one(rv(j)); });
      // The cumulative walk, thread 0 over staged weights.
      if (tid == 0) sh.done = 0;
      for (uint32_t t0 = 0; t0 < k; t0 += kStage) {
        const uint32_t c = min((uint32_t)kStage, k - t0);
        for (uint32_t i = tid; i < c; i += kThreads) sh.wd[i] = w_one(rv(t0 + i));
        __syncthreads();
        if (tid == 0) {
          double cum = sh.sum;  // carried between tiles
          if (t0 == 0) cum = 0.0;
          for (uint32_t i = 0; i < c; ++i) {
            cum = __dadd_rn(cum, __ddiv_rn(sh.wd[i], total));
            if (cum >= top_p) {
              sh.keep = t0 + i + 1;
              sh.done = 1;
              break;
            }
          }
          sh.sum = cum;
        }
        __syncthreads();
        if (sh.done) break;
      }
      if (sh.done) keep = sh.keep;
      __syncthreads();
    }
    if (has_floor) {
      uint32_t first = keep;
      for (uint32_t j = tid; j < keep; j += kThreads)
        if (!(rv(j) >= floor)) first = min(first, j);
      keep = block_min_u32<kWaves>(first, sh.red_u);
    }
  } else if (p.top_p < 1.0f || has_floor) {
    double total1 = 0.0;
    if (p.top_p < 1.0f) total1 = seq_fold(sh, n, [&](uint32_t i) { return w_one((double)value(i)); });
    keep = n;
    if (tid == 0) {
      sh.done = 0;
      sh.sum = 0.0;
    }
    __syncthreads();
    for (uint32_t t0 = 0; t0 < n; t0 += kStage) {
      const uint32_t c = min((uint32_t)kStage, n - t0);
      for (uint32_t i = tid; i < c; i += kThreads) {
        const double v = rv(t0 + i);
        // -1 marks the first token min-p drops (tested before top-p, sample.rs:237-251).
        sh.wd[i] = (has_floor && v < floor) ? -1.0 : (p.top_p < 1.0f ? w_one(v) : 0.0);
      }
      __syncthreads();
      if (tid == 0) {
        double cum = sh.sum;
        for (uint32_t i = 0; i < c; ++i) {
          if (sh.wd[i] < 0.0) {
            sh.keep = t0 + i;
            sh.done = 1;
            break;
          }
          if (p.top_p < 1.0f) {
            cum = __dadd_rn(cum, __ddiv_rn(sh.wd[i], total1));
            if (cum >= top_p) {
              sh.keep = t0 + i + 1;
              sh.done = 1;
              break;
            }
          }
        }
        sh.sum = cum;
      }
      __syncthreads();
      if (sh.done) break;
    }
    if (sh.done) keep = sh.keep;
    __syncthreads();
  } else {
    unfiltered = true;
    keep = n;
  }

  // The draw: u = unit() * total, then the first rank whose cumulative weight exceeds u.
  double total;
  if (unfiltered)
    total = seq_fold(sh, n, [&](uint32_t i) { return w_temp((double)value(i)); });
  else
    total = seq_fold(sh, keep, [&](uint32_t j) { return w_temp(rv(j)); });
  const double u = __dmul_rn(sh.u01, total);
  if (tid == 0) {
    sh.done = 0;
    sh.sum = 0.0;
    sh.pick = keep - 1;  // sample.rs:197, 272, 288: the last kept when u is never passed
  }
  __syncthreads();
  for (uint32_t t0 = 0; t0 < keep; t0 += kStage) {
    const uint32_t c = min((uint32_t)kStage, keep - t0);
    for (uint32_t i = tid; i < c; i += kThreads) sh.wd[i] = w_temp(rv(t0 + i));
    __syncthreads();
    if (tid == 0) {
      double cum = sh.sum;
      for (uint32_t i = 0; i < c; ++i) {
        cum = __dadd_rn(cum, sh.wd[i]);
        if (u < cum) {
          sh.pick = t0 + i;
          sh.done = 1;
          break;
        }
      }
      sh.sum = cum;
    }
    __syncthreads();
    if (sh.done) break;
  }
  const uint32_t pick = sh.pick;
  if (tid == 0) {
    a.tokens[row] = idA[pick];
    a.status[row] = AS_ROW_OK | AS_ROW_EXACT_PATH;
    if (a.kept_count) a.kept_count[row] = keep;
  }
  if (a.kept_ids) {
    const uint32_t m = min(keep, a.kept_cap);
    for (uint32_t j = tid; j < m; j += kThreads) {
      a.kept_ids[(uint64_t)row * a.kept_cap + j] = idA[j];
      if (a.kept_probs) a.kept_probs[(uint64_t)row * a.kept_cap + j] = __ddiv_rn(w_temp(rv(j)), total);
    }
  }
}

// --- the fast path's sort and certified draw --------------------------------------------------

constexpr uint32_t kBuckets = 1024;
static_assert(kBuckets % kThreads == 0 && kBuckets <= sizeof(Shared::bcnt) / 4, "buckets per thread");

// Exclusive prefix sum of one u32 per thread over the block; *total gets the sum.
__device__ uint32_t block_exclusive_scan_u32(uint32_t x, uint32_t* wave_tot, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint32_t incl = wave_scan_u32(x);
  __syncthreads();
  if (lane == kWave - 1) wave_tot[w] = incl;
  __syncthreads();
  const uint32_t waves = wave_scan_u32(lane < kWaves ? wave_tot[lane] : 0u);
  *total = wave_lane_u32(waves, kWaves - 1);
  return (w == 0 ? 0u : wave_lane_u32(waves, (uint32_t)(w - 1))) + incl - x;
}

// The row's total from the slices' sums: total1 (by_temp false: sum of exp(l - top)) or the
// unfiltered total (sum of exp((l - top) / T)), with a bound eps on its distance to the reference's
// left fold in index order (sample.rs:218-222, 274-282). Each slice's sum is rescaled from its own
// reference (sum_ref) to the row's largest value (a host-exact exp and a product). The bound adds up:
//   - the reference's own fold of n terms and its exp: (n + 1) * 2^-53 per unit of X, with the
//     fold of the slices (n_seg) and 64 to spare;
//   - each slice's own evaluation, at most err_rel * sum + err_abs * sum_abs (sum_abs moved to the
//     row's largest value by adding |dm| * sum), and 4 * 2^-53 per unit for its rescale;
//   - the reference's argument roundings, 2^-53 * |d| per term and per rounding (babs);
//   - terms the scan's exp flushed to 0: below 2^-126 each.
// Wave 0 adds the slices' parts, one slice per lane, in a wave reduction: any order of adding n_seg
// positive parts is within n_seg * 2^-53 of their left fold, which the bound's n_seg term covers.
__device__ __forceinline__ void slices_total(const FinishArgs& a, Shared& sh, double top, double temp,
                                             bool by_temp, double* X, double* eps) {
  if (threadIdx.x < kWave) {
    double x = 0.0, babs = 0.0, own = 0.0;
    for (uint32_t s = threadIdx.x; s < a.n_seg; s += kWave) {
      const SegStats& t = sh.seg[s];
      if (t.sum == 0.0) continue;
      const double ms = (double)t.sum_ref;
      double dm = fabs(__dsub_rn(top, ms)), dd = __dsub_rn(ms, top);
      if (by_temp) {
        dm = __ddiv_rn(dm, temp);
        dd = __ddiv_rn(dd, temp);
      }
      const double sc = as_exp::exp_with(sh.tab, dd);
      const double part = __dmul_rn(t.sum, sc);
      const double pabs = __dmul_rn(sc, __dadd_rn(t.sum_abs, __dmul_rn(dm, t.sum)));
      x = __dadd_rn(x, part);
      babs = __dadd_rn(babs, pabs);
      own = __dadd_rn(own, __dadd_rn(__dmul_rn(part, (double)t.err_rel + 4.0 * kU), __dmul_rn(pabs, (double)t.err_abs)));
    }
    x = wave_sum_f64(x);
    babs = wave_sum_f64(babs);
    own = wave_sum_f64(own);
    if (threadIdx.x == 0) {
      const double terms = (double)a.n + (double)a.n_seg + 64.0;
      sh.x = x;
      sh.eps = 1.02 * (kU * ((by_temp ? 2.1 : 1.1) * babs + terms * x) + own) + (double)a.n * 0x1p-126;
    }
  }
  __syncthreads();
  *X = sh.x;
  *eps = sh.eps;
  __syncthreads();
}


// Sorts the candidates sh.sk[off..off + total) whose packed rank is >= R into rank order (packed
// descending), in place from sh.sk[off], and returns how many there are, P (off + total <= kCap).
// Only the first `need` ranks are guaranteed placed: a bucket that starts at or past `need` is left
// unsorted. A bucket sort: buckets by distance from kmax (at least every key sorted: the row's
// largest), then each value's place inside its bucket by counting the bucket's values above it
// (quadratic in a bucket's size, which heavy ties make large).
// At most kRankSort values are sorted by counting: thread i takes value i's rank, the number of
// values above it (the packed keys are distinct), in one pass over the LDS copy.
constexpr uint32_t kRankSort = 256;
static_assert(kRankSort <= (uint32_t)kThreads, "one value per thread");
__device__ __forceinline__ uint32_t sort_candidates(Shared& sh, uint32_t total, uint64_t R,
                                                    uint32_t kmax, uint32_t need, uint32_t off = 0) {
  const uint32_t tid = threadIdx.x;
  uint64_t* sk = sh.sk + off;
  if (total <= kRankSort) {
    // kThreads / kRankSort threads per value, each counting the values above it in its share of
    // the list (eight LDS reads in flight per step; every lane of a wave reads the same words),
    // their counts added in sh.hist.
    constexpr uint32_t kWays = (uint32_t)kThreads / kRankSort;
    static_assert(kRankSort <= 256 && kWays >= 1, "a counter per value in sh.hist");
    const uint32_t v = tid % kRankSort, way = tid / kRankSort;
    const uint64_t x = (v < total) ? sk[v] : 0ull;
    const bool mine = v < total && x >= R;
    if (tid < kRankSort) sh.hist[tid] = 0;
    const uint32_t share = (total + kWays - 1) / kWays, j0 = way * share, j1 = min(total, j0 + share);
    uint32_t c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (mine) {
      uint32_t j = j0;
      for (; j + 8 <= j1; j += 8)
#pragma unroll
        for (int u = 0; u < 8; ++u) c[u] += (sk[j + u] > x) ? 1u : 0u;  // every y > x >= R is kept
      for (; j < j1; ++j) c[0] += (sk[j] > x) ? 1u : 0u;
    }
    uint32_t r = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) r += c[u];
    const uint32_t P = (uint32_t)__syncthreads_count(mine && way == 0);
    if (mine && r) atomicAdd(&sh.hist[v], r);
    __syncthreads();
    if (mine && way == 0) sk[sh.hist[v]] = x;
    __syncthreads();
    return P;
  }
  uint64_t* out2 = reinterpret_cast<uint64_t*>(sh.wd);
  constexpr int kPerT = kCap / kThreads;
  uint64_t xs[kPerT];
  uint32_t kmin = 0xFFFFFFFFu, mine = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const uint32_t i = tid + q * kThreads;
    xs[q] = (i < total) ? sk[i] : 0ull;
    if (i < total && xs[q] >= R) {
      kmin = min(kmin, (uint32_t)(xs[q] >> 32));
      ++mine;
    }
  }
  // One barrier pair gives every thread the smallest key and the count; the buckets clear before it.
  for (uint32_t b = tid; b < kBuckets; b += kThreads) sh.bcnt[b] = 0;
  kmin = wave_min_u32(kmin);
  mine = wave_sum_u32(mine);
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) {
    sh.red_u[tid / kWave] = kmin;
    sh.base[tid / kWave] = mine;
  }
  __syncthreads();
  uint32_t P = 0;
  kmin = 0xFFFFFFFFu;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    kmin = min(kmin, sh.red_u[w]);
    P += sh.base[w];
  }
  const uint32_t range = kmax - kmin;
  uint32_t shift = 0;
  while ((range >> shift) >= kBuckets) ++shift;
  uint32_t slot[kPerT];
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const uint32_t i = tid + q * kThreads;
    slot[q] = 0;
    if (i < total && xs[q] >= R) slot[q] = atomicAdd(&sh.bcnt[(kmax - (uint32_t)(xs[q] >> 32)) >> shift], 1u);
  }
  __syncthreads();
  if (tid < kWave) {
    // Bucket starts on wave 0: kB consecutive buckets per lane, then a scan over the lanes.
    constexpr uint32_t kB = kBuckets / kWave;
    uint32_t cs[kB], run = 0;
#pragma unroll
    for (uint32_t q = 0; q < kB; ++q) {
      cs[q] = sh.bcnt[tid * kB + q];
      run += cs[q];
    }
    uint32_t off = wave_scan_u32(run) - run;
#pragma unroll
    for (uint32_t q = 0; q < kB; ++q) {
      sh.bstart[tid * kB + q] = off;
      off += cs[q];
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const uint32_t i = tid + q * kThreads;
    if (i < total && xs[q] >= R) {
      const uint32_t b = (kmax - (uint32_t)(xs[q] >> 32)) >> shift;
      out2[sh.bstart[b] + slot[q]] = xs[q];
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < P; i += kThreads) {
    const uint64_t x = out2[i];
    const uint32_t b = (kmax - (uint32_t)(x >> 32)) >> shift;
    const uint32_t s0 = sh.bstart[b], nb = sh.bcnt[b];
    if (s0 >= need) continue;
    uint32_t c[4] = {0, 0, 0, 0};
    uint32_t j = 0;
    for (; j + 4 <= nb; j += 4)
#pragma unroll
      for (int u = 0; u < 4; ++u) c[u] += (out2[s0 + j + u] > x) ? 1u : 0u;
    for (; j < nb; ++j) c[0] += (out2[s0 + j] > x) ? 1u : 0u;
    sk[s0 + c[0] + c[1] + c[2] + c[3]] = x;
  }
  __syncthreads();
  return P;
}

// Inclusive prefix sums of sh.wd[0..m) (m <= kCap), eight per thread in loc[], the thread's
// offset in *off; returns the sum of all m to every thread. Parallel: each sum is within
// gamma(40) of the exact sum of its (positive) terms.
__device__ __forceinline__ double prefix_scan(Shared& sh, uint32_t m, double loc[kScanPer], double* off) {
  const uint32_t i0 = threadIdx.x * kScanPer;
  double run = 0.0;
#pragma unroll
  for (int q = 0; q < kScanPer; ++q) {
    run = __dadd_rn(run, (i0 + q < m) ? sh.wd[i0 + q] : 0.0);
    loc[q] = run;
  }
  *off = block_exclusive_scan_f64(run, sh.red_d);
#pragma unroll
  for (int q = 0; q < kScanPer; ++q)
    if (i0 + q == m - 1) sh.x = __dadd_rn(*off, loc[q]);
  __syncthreads();
  const double s = sh.x;
  __syncthreads();
  return s;
}

// The draw's decision from bounds: u (the reference's unit() * total) lies in [ulo, uhi], and the
// reference's cumulative c_j (its left fold of w_0..w_j) is within gamma(j+1) + gamma(40) of our
// scanned prefix. Returns the first j < m with c_j > u when the bounds settle it, m when u is
// certainly past every c_j of the m, kNone when they cannot decide.
__device__ __forceinline__ uint32_t decide_draw(Shared& sh, uint32_t m, const double loc[kScanPer], double off, double ulo,
                                double uhi) {
  const uint32_t i0 = threadIdx.x * kScanPer;
  const double g40 = gamma_n(40.0);
  uint32_t fp = m, fc = m;
#pragma unroll
  for (int q = 0; q < kScanPer; ++q) {
    const uint32_t i = i0 + q;
    if (i < m) {
      const double Rv = __dadd_rn(off, loc[q]);
      const double rel = gamma_ub((double)i + 1.0) + g40 + 4.0 * kU;
      if (Rv * (1.0 + rel) > ulo) fp = min(fp, i);
      if (Rv * (1.0 - rel) > uhi) fc = min(fc, i);
    }
  }
  const uint32_t jp = block_min_u32<kWaves>(fp, sh.red_u);
  const uint32_t jc = block_min_u32<kWaves>(fc, sh.red_u);
  if (jp == jc) return jc;  // jc < m, or both m: past every c_j
  return kNone;
}

// --- the fast decision for rows without a top-k ----------------------------------------------------
//
// draw_partial's cut and draw (sample.rs:208-272) from the sorted candidates with as few block-wide
// steps as possible, for a row without kept lists: one pass computes every sorted value's weights at
// T = 1 and at T, and the block sums them; wave 0 then certifies the cut from the sums and finds the
// draw among the first kWaveMax ranks from a wave prefix. Every decision is taken from bounds that
// cover the reference's own left folds, as the general path's are (the same bounds: the reference's
// cumulative at rank j within gamma(2j + 4) of its exact quotient, a parallel sum within gamma(40)
// of its terms' exact sum, a wave prefix within gamma(kWPer + 7)); when they cannot decide, or the
// draw lies past the first kWaveMax ranks, it returns false and the general path decides.
//   - Min-p's cut im is the first sorted rank below the floor (exact compares), or lies past the
//     sorted values.
//   - Top-p cannot stop before im when the reference's cumulative at rank im - 1 is certainly below
//     top_p: the sum S1 of the im values' weights at T = 1 against top_p * total1, total1's lower
//     bound from the slices' sums. Otherwise the cut may lie among the first kWaveMax ranks, where
//     the wave's prefix places it (or cannot).
//   - The draw: u = unit() * (the kept values' total at T), the kept set's total from the block sum
//     (or the wave's own total when it holds every kept value). When the kept set runs past the
//     sorted values, its weight lies between the sorted values' and that plus a bound on every value
//     below them (draw_past's: the values below the last sorted one at T, or for T <= 1 their mass
//     at T = 1 scaled by exp(d (1/T - 1)) of the last sorted one).
// On success the row's kept count (or P, a lower bound, with AS_ROW_KEPT_PARTIAL) and status are
// returned and sh.pick / sh.sum hold the rank drawn and the total.
__device__ __forceinline__ bool fast_partial(const FinishArgs& a, Shared& sh, const RowParams& p, uint32_t P,
                                             bool floor_cut, uint32_t* keep_out, uint32_t* status_out) {
  const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave, n = a.n;
  const double top = (double)key_value(sh.mk), temp = (double)p.temp, top_p = (double)p.top_p;
  const bool has_floor = p.min_p > 0.0f, topp = p.top_p < 1.0f;
  const double floor = __dadd_rn(top, p.ln_min_p);
  const uint64_t* tab = sh.tab;
  auto val = [&](uint32_t i) -> double { return (double)packed_value(sh.sk[i]); };
  uint32_t first = P;
  if (has_floor && !floor_cut)
    for (uint32_t i = tid; i < P; i += kThreads)
      if (!(val(i) >= floor)) first = min(first, i);
  const uint32_t im = block_min_u32<kWaves>(first, sh.red_u);
  // min-p's cut is known when it falls among the sorted values or right after them (floor_cut).
  const bool im_exact = (has_floor && im < P) || floor_cut;
  double X = 0.0, eps = 0.0;
  if (topp) {
    slices_total(a, sh, top, temp, false, &X, &eps);
    if (!(X - eps > 0.0 && eps == eps)) return false;
  }
  // The weights of the values before min-p's cut (all P when it lies past them): at T in sh.wd, at
  // T = 1 for the first kWaveMax past the end of sh.wd's used part.
  const uint32_t m = im;
  double* w1s = sh.wd + (kCap - kWaveMax);
  double s1 = 0.0, sT = 0.0;
  for (uint32_t i = tid; i < m; i += kThreads) {
    const double v = val(i);
    const double wt = as_exp::exp_with(tab, __ddiv_rn(__dsub_rn(v, top), temp));
    sh.wd[i] = wt;
    sT = __dadd_rn(sT, wt);
    if (topp) {
      const double w1 = as_exp::exp_with(tab, __dsub_rn(v, top));
      s1 = __dadd_rn(s1, w1);
      if (i < kWaveMax) w1s[i] = w1;
    }
  }
  s1 = wave_sum_f64(s1);
  sT = wave_sum_f64(sT);
  if (lane == 0) {
    sh.red_d[w] = s1;
    sh.red_d2[w] = sT;
  }
  __syncthreads();
  if (tid < kWave) {
    const double g40 = gamma_n(40.0);
    double S1 = sh.red_d[0], ST = sh.red_d2[0];
    for (int k = 1; k < kWaves; ++k) {
      S1 = __dadd_rn(S1, sh.red_d[k]);
      ST = __dadd_rn(ST, sh.red_d2[k]);
    }
    const uint32_t i0 = lane * kWPer;
    const double g = gamma_ub(2.0 * kWPer + 16.0);
    uint32_t kk = kNone;  // the kept count, when known
    bool past = false;    // the kept set runs past the sorted values
    if (topp) {
      const double tp_lo = top_p * (X - eps), tp_hi = top_p * (X + eps);
      if (S1 * (1.0 + 2.0 * g40 + gamma_ub(2.0 * (double)m + 2.0) + 10.0 * kU) < tp_lo) {
        if (im_exact) kk = im;
        else if (P == n) kk = n;
        else past = true;
      } else {
        const uint32_t mw = min(m, kWaveMax);
        double wv[kWPer], pre[kWPer];
#pragma unroll
        for (int q = 0; q < kWPer; ++q) wv[q] = (i0 + q < mw) ? w1s[i0 + q] : 0.0;
        wave_prefix(wv, pre);
        bool lo[kWPer], hi[kWPer];
#pragma unroll
        for (int q = 0; q < kWPer; ++q) {
          const double rel = 2.0 * g + gamma_ub(2.0 * (double)(i0 + q) + 4.0) + 10.0 * kU;
          lo[q] = pre[q] * (1.0 + rel) >= tp_lo;  // the reference's cumulative may have reached top_p
          hi[q] = pre[q] * (1.0 - rel) >= tp_hi;  // it certainly has
        }
        const uint32_t jl = wave_first(lo, mw), jh = wave_first(hi, mw);
        if (jl == jh && jh < mw) kk = jh + 1;
      }
    } else {
      if (im_exact) kk = im;
      else if (P == n) kk = n;
      else past = true;
    }
    uint32_t pick = kNone;
    double tot = 0.0, ulo = 0.0, uhi = 0.0;
    uint32_t mw = 0;
    bool past_mw = false;  // u certainly passes every cumulative of the first mw
    if (kk != kNone) {
      mw = min(kk, kWaveMax);
      // The kept total: the wave's own when it holds every kept value, else the block's sum (kk == m).
      double S = ST, dS = g40;
      if (kk <= kWaveMax) {
        double wv[kWPer], pre[kWPer];
#pragma unroll
        for (int q = 0; q < kWPer; ++q) wv[q] = (i0 + q < mw) ? sh.wd[i0 + q] : 0.0;
        S = wave_prefix(wv, pre);
        dS = g;
      }
      const double d = gamma_ub((double)kk + 1.0) + dS + 4.0 * kU;
      ulo = sh.u01 * S * (1.0 - d) * (1.0 - 3.0 * kU);
      uhi = sh.u01 * S * (1.0 + d) * (1.0 + 3.0 * kU);
      tot = S;
    } else if (past) {
      mw = min(P, kWaveMax);
      double tail = (double)(n - P) * sh.wd[P - 1] * (1.0 + 4.0 * kU);
      if (topp && p.temp <= 1.0f) {
        const double d = __dsub_rn(val(P - 1), top);
        const double rest = (X + eps) - S1 * (1.0 - 2.0 * g40);
        const double t2 = as_exp::exp_with(tab, d * (1.0 / temp - 1.0)) * (1.0 + 1e-9) * (rest > 0.0 ? rest : 0.0);
        if (t2 < tail) tail = t2;
      }
      const double gn = gamma_n((double)n);
      const double slo = ST * (1.0 - g40 - 4.0 * kU) * (1.0 - gn);
      const double shi = (ST * (1.0 + g40 + 4.0 * kU) + tail) * (1.0 + gn);
      ulo = sh.u01 * slo * (1.0 - 3.0 * kU);
      uhi = sh.u01 * shi * (1.0 + 3.0 * kU);
      tot = ST;
    }
    if (mw > 0) {
      // The first rank among the first mw whose cumulative passes u, when the bounds agree.
      double wv[kWPer], pre[kWPer];
#pragma unroll
      for (int q = 0; q < kWPer; ++q) wv[q] = (i0 + q < mw) ? sh.wd[i0 + q] : 0.0;
      wave_prefix(wv, pre);
      bool may[kWPer], sure[kWPer];
#pragma unroll
      for (int q = 0; q < kWPer; ++q) {
        const double rel = gamma_ub((double)(i0 + q) + 1.0) + g + 4.0 * kU;
        may[q] = pre[q] * (1.0 + rel) > ulo;
        sure[q] = pre[q] * (1.0 - rel) > uhi;
      }
      const uint32_t jp = wave_first(may, mw), jc = wave_first(sure, mw);
      if (jp == jc) {
        if (jc < mw) pick = jc;
        else if (kk != kNone && kk == mw) pick = kk - 1;  // past every cumulative: the last kept
        past_mw = jc == mw;
      }
    }
    if (lane == 0) {
      sh.pick = pick;
      sh.sum = tot;
      sh.keep = pick == kNone ? kNone : (kk != kNone ? kk : P);
      // u certainly past the first kWaveMax: the whole block scans the weights in place when the
      // kept set is every one of them, or runs past them (a bracket that straddles a cumulative among
      // the first kWaveMax would straddle it there too).
      const bool more = pick == kNone && past_mw && ((kk != kNone && kk == m) || past) && m > kWaveMax;
      sh.fp_m = more ? m : 0u;
      sh.fp_past = past ? 1u : 0u;
      sh.fp_lo = ulo;
      sh.fp_hi = uhi;
    }
  }
  __syncthreads();
  uint32_t keep = sh.keep;
  const uint32_t scan_m = sh.fp_m;
  if (keep == kNone && scan_m > 0) {
    double loc[kScanPer], off;
    prefix_scan(sh, scan_m, loc, &off);
    const uint32_t j = decide_draw(sh, scan_m, loc, off, sh.fp_lo, sh.fp_hi);
    // j == scan_m: u passes every cumulative, so the draw is the last kept value, unless the kept
    // set runs past the scanned values.
    if (j != kNone && (j < scan_m || !sh.fp_past) && tid == 0) {
      sh.pick = j < scan_m ? j : scan_m - 1;
      sh.keep = sh.fp_past ? P : scan_m;
    }
    __syncthreads();
    keep = sh.keep;
  }
  if (keep == kNone) return false;
  *keep_out = keep;
  *status_out = keep == P && !(im_exact || P == n) ? (uint32_t)AS_ROW_KEPT_PARTIAL : (uint32_t)AS_ROW_OK;
  return true;
}

// --- the deep path ------------------------------------------------------------------------------
//
// For a row whose cut or draw lies past the fast path's sorted candidates: one pass over the row
// histograms its values into bins (fine near the row's largest value; each bin's count and its
// weight in fixed point, added with integer LDS atomics), which fixes the lowest bin that can hold
// the cut (or the draw), with a margin; a second pass collects every value down to that bin; a
// bucket sort in HBM scratch puts them in rank order; and the same certified decisions as the fast
// path run while streaming through them. The row's exact total in index order is computed only
// when the slices' certified sums leave a decision open. When a bound still cannot decide, the
// exact-order path runs.

constexpr uint32_t kDeepBins = 4096;
constexpr uint32_t kDeepBucketMax = 4096;

// Streams the sorted values buf[c0 .. c0+m) through LDS in chunks: sh.sk gets the values, sh.wd
// their weight(value), then a block prefix scan; f(chunk_start, count, loc, base) sees the chunk,
// with the global inclusive prefix of chunk value q at base + loc[q], and returns true to stop.
// Returns the sum of every weight streamed (within gamma(80) of the exact sum).
template <class W, class F>
__device__ __forceinline__ double stream_scan(Shared& sh, const uint64_t* buf, uint32_t m, W weight, F f) {
  double carry = 0.0;
  for (uint32_t c0 = 0; c0 < m; c0 += kCap) {
    const uint32_t cn = min((uint32_t)kCap, m - c0);
    for (uint32_t i = threadIdx.x; i < cn; i += kThreads) {
      const uint64_t x = buf[c0 + i];
      sh.sk[i] = x;
      sh.wd[i] = weight((double)packed_value(x));
    }
    __syncthreads();
    double loc[kScanPer], off;
    const double tot = prefix_scan(sh, cn, loc, &off);
    const bool stop = f(c0, cn, loc, __dadd_rn(carry, off));
    carry = __dadd_rn(carry, tot);
    __syncthreads();
    if (stop) break;
  }
  return carry;
}

// First rank j with lo/hi bounds of the reference's cumulative crossing `target`: fills *jl (first
// j whose upper bound reaches it) and *jh (first j whose lower bound does), over m streamed values.
// cum_j = R_j / total with total in [x - eps, x + eps]; rel(j) bounds the rank-order fold.
template <class W>
__device__ __forceinline__ void stream_cross(Shared& sh, const uint64_t* buf, uint32_t m, W weight,
                                             double x, double eps, double target, uint32_t* jl,
                                             uint32_t* jh) {
  uint32_t fl = kNone, fh = kNone;
  stream_scan(sh, buf, m, weight, [&](uint32_t c0, uint32_t cn, const double loc[kScanPer], double base) {
    const uint32_t i0 = threadIdx.x * kScanPer;
    uint32_t a = kNone, b = kNone;
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
      const uint32_t i = i0 + q;
      if (i < cn) {
        const double Rv = __dadd_rn(base, loc[q]);
        const double rel = 2.0 * gamma_n(80.0) + gamma_n(2.0 * (double)(c0 + i) + 4.0) + 10.0 * kU;
        if (Rv * (1.0 + rel) / (x - eps) >= target) a = min(a, c0 + i);
        if (Rv * (1.0 - rel) / (x + eps) >= target) b = min(b, c0 + i);
      }
    }
    a = block_min_u32<kWaves>(a, sh.red_u);
    b = block_min_u32<kWaves>(b, sh.red_u);
    if (fl == kNone) fl = a;
    if (fh == kNone) fh = b;
    return fl != kNone && fh != kNone;
  });
  *jl = (fl == kNone) ? m : fl;
  *jh = (fh == kNone) ? m : fh;
}

// The draw over the first m streamed values with u in [ulo, uhi]: the first j with the
// reference's cumulative c_j > u when the bounds settle it, m when u is certainly past all of
// them, kNone when they cannot decide.
template <class W>
__device__ __forceinline__ uint32_t stream_draw(Shared& sh, const uint64_t* buf, uint32_t m, W weight,
                                                double ulo, double uhi) {
  uint32_t res = m;
  bool done = false;
  stream_scan(sh, buf, m, weight, [&](uint32_t c0, uint32_t cn, const double loc[kScanPer], double base) {
    const uint32_t i0 = threadIdx.x * kScanPer;
    uint32_t a = kNone, b = kNone;
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
      const uint32_t i = i0 + q;
      if (i < cn) {
        const double Rv = __dadd_rn(base, loc[q]);
        const double rel = gamma_n((double)(c0 + i) + 1.0) + gamma_n(80.0) + 4.0 * kU;
        if (Rv * (1.0 + rel) > ulo) a = min(a, c0 + i);
        if (Rv * (1.0 - rel) > uhi) b = min(b, c0 + i);
      }
    }
    a = block_min_u32<kWaves>(a, sh.red_u);
    b = block_min_u32<kWaves>(b, sh.red_u);
    if (a != kNone) {
      res = (a == b) ? a : kNone;
      done = true;
    }
    return done;
  });
  return res;
}

// The deep path's passes over a row: 16 values per thread per step, with their history counts
// (cnt, 0 when null). One workgroup streams a whole row, so its loads' latency, not HBM, bounds a
// pass. With kPipe and without counts, whole 16-byte steps go through a ring of kDepth steps' loads:
// each step's loads are issued kDepth - 1 steps before its values are used (near the end they reload
// the last step rather than branch); otherwise (counts take as many registers again, and some callers
// have none to spare) a step's loads are all issued before any value is used. Scalar loads cover an
// unaligned row and the ragged end. f(i, v, c) runs for each value.
template <bool kPipe = false, int kDepth = 2, class F>
__device__ __forceinline__ void for_each_value(const float* x, const uint32_t* cnt, uint32_t n, bool vec, F f) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr uint32_t kStep = 16 * kThreads;
  const uint32_t tid = threadIdx.x;
  auto at = [&](uint32_t s, int j) { return s * kStep + (j * kThreads + tid) * 4; };
  uint32_t b0 = 0;
  if (vec) {
    const uint32_t whole = n / kStep;
    if (kPipe && !cnt && whole > 0) {
      static_assert(kDepth >= 2, "a step in flight while another is used");
      f32x4 q[kDepth][4];
      auto load = [&](f32x4 (&r)[4], uint32_t s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = gload(reinterpret_cast<const f32x4*>(x + at(s, j)));
      };
      auto use = [&](const f32x4 (&r)[4], uint32_t s) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) f(at(s, j) + c, r[j][c], 0u);
      };
      // Slot d holds step s + d; before step s + d is used, the slot of the step used just before
      // takes step s + d + kDepth - 1.
#pragma unroll
      for (int d = 0; d < kDepth - 1; ++d) load(q[d], min((uint32_t)d, whole - 1));
      uint32_t s = 0;
      for (; s + kDepth <= whole; s += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
          load(q[(d + kDepth - 1) % kDepth], min(s + d + kDepth - 1, whole - 1));
          use(q[d], s + d);
        }
      }
#pragma unroll
      for (int d = 0; d < kDepth - 1; ++d)
        if (s + d < whole) use(q[d], s + d);
    } else {
      for (uint32_t s = 0; s < whole; ++s) {
        f32x4 q[4];
        u32x4 k[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          q[j] = gload(reinterpret_cast<const f32x4*>(x + at(s, j)));
          k[j] = cnt ? gload(reinterpret_cast<const u32x4*>(cnt + at(s, j))) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) f(at(s, j) + c, q[j][c], k[j][c]);
      }
    }
    b0 = whole * kStep;
  }
  for (; b0 < n; b0 += kStep) {
    float q[16];
    uint32_t k[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t i = b0 + j * kThreads + tid;
      q[j] = (i < n) ? gload(x + i) : 0.0f;
      k[j] = (cnt && i < n) ? gload(cnt + i) : 0u;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t i = b0 + j * kThreads + tid;
      if (i < n) f(i, q[j], k[j]);
    }
  }
}

__device__ __noinline__ float penalize_out(float x, uint32_t c, const RowParams& p) { return penalize(x, c, p); }

// --- the deep path by deciding bins ---------------------------------------------------------------
//
// A row without a top-k whose cut or draw lies past the fast path's candidates needs the rank order
// only where a decision falls: at top-p's cut (the cumulative weight at T = 1 reaching top_p of the
// total), at min-p's floor, and at the draw (the cumulative weight at T passing u times the kept
// weight). One pass over the row histograms every value by its distance below the largest into
// kDeepBins bins (the bin is monotone in the value, so bins follow the rank order) and adds each
// value's weights, each within kPassRel of the reference's term (the bounded exp of exp_poly.h, at
// (l - top) / T computed as (l - top) * (1 / T)): any sum of them differs from the reference's ordered
// folds by rounding and kPassRel of the sum. The bins' prefix sums fix, with certified bounds, the few bins that can hold each
// decision; a second pass collects only those bins' values into LDS, a sort orders them, and each
// one's rank is the count before its run of collected bins plus its place in the run. The decisions
// compare the reference's cumulatives, bounded by the prefix before the run plus the run's terms,
// with targets bounded by the exact totals. Returns false, with nothing written, when a bound cannot
// decide or the bins hold more values than LDS does; the caller then takes the full deep path.
constexpr uint32_t kBinRanges = 3;
// The histogram passes' terms against the reference's: the bounded exp's kExpPolyRel and the argument
// scaled by 1 / T instead of divided by T (two roundings, |(l - top) / T| <= 708 before the clamp:
// 1.6e-13 more), rounded up.
constexpr double kPassRel = 2.0e-12;
static_assert(kPassRel >= kExpPolyRel + 1.6e-13, "the histogram terms' bound");
// A histogram pass's weights of a value: exp(l - top) (top-p's) and exp((l - top) / T).
struct PassWeights {
  ExpPoly ep;
  double top, inv_t;
  __device__ __forceinline__ void init(double top_, double temp) {
    ep.load();
    top = top_;
    inv_t = 1.0 / temp;
  }
  __device__ __forceinline__ double d(float v) const { return __dsub_rn((double)v, top); }
  __device__ __forceinline__ double one(double dv) const { return ep.exp_neg(dv); }
  __device__ __forceinline__ double at_t(double dv) const { return ep.exp_neg(__dmul_rn(dv, inv_t)); }
};
// Element k of a run's three values, by selects (the runs' few values stay in registers).
template <class T>
__device__ __forceinline__ T sel3(uint32_t k, T v0, T v1, T v2) {
  return k == 0 ? v0 : (k == 1 ? v1 : v2);
}

// The deep passes' lower cut: min-p's floor (as an f32: v >= it exactly when v is at or above the
// reference's f64 floor) when it is the row's only cut, else -inf. Below it nothing is kept and no
// total the row's decisions use counts a value.
__device__ __forceinline__ float deep_cut(const RowParams& p, float topf) {
  const bool only_floor = p.mode == kModePartial && p.min_p > 0.0f && !(p.top_p < 1.0f);
  return only_floor ? floor_f32(__dadd_rn((double)topf, p.ln_min_p)) : -__builtin_inff();
}

// --- the deep passes shared with idle workgroups ----------------------------------------------
//
// In a small batch most of the finish kernel's workgroups have no row, or are done with theirs, while
// a deep row's two passes over its values would take one workgroup hundreds of microseconds. Those
// passes are shared: the row's workgroup publishes a pass (DeepJob) and every idle workgroup takes
// parts of kTailLen values (deep_help), as does the row's own (deep_run), which then waits only for
// parts that running workgroups took. The histogram pass adds each part's bins into the row's
// histogram with device atomics; the collecting pass lists each part's values from the chosen bins.
// Nothing waits on a workgroup that has not begun, and a helper stops once every row of the call is
// finished.

// The shared passes' data in a row's scratch, after its history counts (8-byte aligned): the
// histogram (counts, weights at 1, weights at T; kDistBins each), the list's count, a pad word, and
// the list (at most kCap packed values).
__device__ __forceinline__ uint32_t* deep_shared(const FinishArgs& a, uint32_t row) {
  return a.scratch + (uint64_t)row * a.scratch_stride + (((uint64_t)a.n + 1) & ~1ull);
}

// One part of a row's shared pass (pass 0: its histogram; pass 1: its values in the published runs
// of bins), by the whole workgroup, then the part counts itself ended. The history's positions are
// left out (the row's workgroup adds the history's values penalised). The bins are the row's
// deep_bins<true> ones: distance below the largest value, kDistBins over 32 max(T, 1). sh.wd and
// sh.sk are free: a helper's own row is done, and the row's own workgroup calls this only where
// deep_bins has nothing there.
__device__ __noinline__ void deep_part(const FinishArgs& a, uint32_t row, uint32_t q, uint32_t pass) {
  Shared& sh = shm();
  constexpr uint32_t kLen = as_launch::kTailLen, kPer = kLen / kThreads, kNB = as_launch::kDistBins;
  const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1);
  DeepJob& jb = a.deep_jobs[row];
  const uint32_t n = a.n, b0 = q * kLen, b1 = min(b0 + kLen, n), len = b1 - b0;
  const float* x = a.logits + (uint64_t)row * a.row_stride;
  const bool vec = a.vec && a.row_stride % 4 == 0 && len == kLen;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  auto at = [&](uint32_t k) { return vec ? ((k / 4) * kThreads + tid) * 4 + (k % 4) : k * kThreads + tid; };
  float v[kPer];
  if (vec) {
#pragma unroll
    for (uint32_t j = 0; j < kPer / 4; ++j) {
      const f32x4 qv = *reinterpret_cast<const f32x4*>(x + b0 + (j * kThreads + tid) * 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * j + c] = qv[c];
    }
  } else {
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) v[k] = at(k) < len ? x[b0 + at(k)] : 0.0f;
  }
  const RowParams& p = a.params[row];
  uint32_t hb;
  const uint32_t he = as_launch::history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  // The job's fields, read once by the workgroup (every workgroup reads the same words).
  if (tid == 0) {
    sh.dp_mk = ld_agent(&jb.mk);
    if (pass)
      for (uint32_t k = 0; k < kBinRanges; ++k) {
        sh.dp_r[k] = ld_agent(&jb.r0[k]);
        sh.dp_r[kBinRanges + k] = ld_agent(&jb.r1[k]);
      }
  }
  uint32_t* bm = reinterpret_cast<uint32_t*>(sh.wd);  // the part's history positions
  uint32_t* hc = bm + kLen / 32;
  double* hm = reinterpret_cast<double*>(hc + kNB);
  double* hw = hm + kNB;
  static_assert((kLen / 32 + kNB) % 2 == 0 && (kLen / 32 + kNB) * 4 + kNB * 16 <= sizeof(sh.wd), "part tables");
  if (pen)
    for (uint32_t i = tid; i < kLen / 32; i += kThreads) bm[i] = 0;
  if (pass == 0)
    for (uint32_t b = tid; b < kNB; b += kThreads) {
      hc[b] = 0;
      hm[b] = 0.0;
      hw[b] = 0.0;
    }
  if (tid == 0) sh.dp_staged = 0;
  __syncthreads();
  if (pen) {
    auto mark = [&](uint32_t id) {
      const uint32_t off = id - b0;
      if (off < len) atomicOr(&bm[off >> 5], 1u << (off & 31u));
    };
    for (uint32_t h = hb + tid; h < he; h += kThreads) mark(gload(a.hist_ids + h));
    for (uint32_t h = tid; h < extra; h += kThreads) mark(gload(a.extra_ids + h));
    __syncthreads();
  }
  const uint32_t mk = sh.dp_mk;
  uint32_t r0[kBinRanges], r1[kBinRanges];
#pragma unroll
  for (uint32_t k = 0; k < kBinRanges; ++k) {
    r0[k] = pass ? sh.dp_r[k] : kNone;
    r1[k] = pass ? sh.dp_r[kBinRanges + k] : kNone;
  }
  const float topf = key_value(mk);
  const double top = (double)topf, temp = (double)p.temp;
  const float bsc = (float)kNB / (32.0f * fmaxf(1.0f, p.temp));
  const float cut = deep_cut(p, topf);
  auto bin_of = [&](float val) -> uint32_t {
    const float t = (topf - val) * bsc;
    return t < (float)(kNB - 1) ? (uint32_t)t : kNB - 1;
  };
  auto own = [&](uint32_t k) {
    return at(k) < len && !(pen && ((bm[at(k) >> 5] >> (at(k) & 31u)) & 1u)) && v[k] >= cut;
  };
  uint32_t* sh_g = deep_shared(a, row);
  if (pass == 0) {
    const bool by_top_p = p.top_p < 1.0f;
    PassWeights pw;
    pw.init(top, temp);
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) {
      if (!own(k)) continue;
      const uint32_t b = bin_of(v[k]);
      const double d = pw.d(v[k]);
      atomicAdd(&hc[b], 1u);
      if (by_top_p) atomicAdd(&hm[b], pw.one(d));
      atomicAdd(&hw[b], pw.at_t(d));
    }
    __syncthreads();
    double* gm = reinterpret_cast<double*>(sh_g + kNB);
    double* gw = gm + kNB;
    for (uint32_t b = tid; b < kNB; b += kThreads) {
      if (hc[b] == 0u) continue;
      __hip_atomic_fetch_add(gp(sh_g + b), hc[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (by_top_p) __hip_atomic_fetch_add(gp(gm + b), hm[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(gp(gw + b), hw[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    // The part's values in the runs, staged in sh.sk with one LDS atomic per wave, then listed.
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) {
      bool in = false;
      if (own(k)) {
        const uint32_t b = bin_of(v[k]);
#pragma unroll
        for (uint32_t r = 0; r < kBinRanges; ++r) in = in || (b >= r0[r] && b <= r1[r]);  // unused: kNone
      }
      const uint64_t m = __ballot(in);
      if (m) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&sh.dp_staged, (uint32_t)__popcll(m));
        base = __builtin_amdgcn_readfirstlane(base);
        const uint32_t i = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (in) sh.sk[i] = pack(total_key(v[k]), b0 + at(k));
      }
    }
    __syncthreads();
    const uint32_t staged = sh.dp_staged;
    if (tid == 0) sh.dp_base = __hip_atomic_fetch_add(gp(sh_g + 5 * kNB), staged, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t base = sh.dp_base;
    uint64_t* list = reinterpret_cast<uint64_t*>(sh_g + 5 * kNB + 2);
    if (base + staged <= (uint32_t)kCap)
      for (uint32_t i = tid; i < staged; i += kThreads) st_agent(list + base + i, sh.sk[i]);
  }
  // Every write above has completed (in every thread) before the part counts itself ended.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) __hip_atomic_fetch_add(gp(&jb.ended[pass]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The row's own workgroup: publishes pass `pass` (the fields it needs were stored before, in every
// thread), takes its parts until none is left, then waits for the parts other workgroups took.
// False if that wait ran past its guard (it cannot when every running workgroup makes progress).
constexpr uint32_t kDeepSpin = 1u << 24;
// The shared histogram pass published: the row's histogram in its scratch cleared and the job's
// fields set (its largest key, its counters), then its stamp, once they have completed. Workgroups
// with no row left take its parts from then on.
__device__ __noinline__ void deep_publish_hist(const FinishArgs& a, uint32_t row, uint32_t mk) {
  constexpr uint32_t kNB = as_launch::kDistBins;
  const uint32_t tid = threadIdx.x;
  uint32_t* gc = deep_shared(a, row);
  double* gm = reinterpret_cast<double*>(gc + kNB);
  double* gw = gm + kNB;
  DeepJob& jb = a.deep_jobs[row];
  for (uint32_t b = tid; b < kNB; b += kThreads) {
    __hip_atomic_store(gp(gc + b), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gp(gm + b), 0.0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gp(gw + b), 0.0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) {
    __hip_atomic_store(gp(&jb.mk), mk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int k = 0; k < 2; ++k) {
      __hip_atomic_store(gp(&jb.next[k]), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gp(&jb.ended[k]), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) __hip_atomic_store(gp(&jb.stamp), 2 * a.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ bool deep_run(const FinishArgs& a, uint32_t row, uint32_t pass) {
  Shared& sh = shm();
  DeepJob& jb = a.deep_jobs[row];
  const uint32_t parts = as_launch::tail_parts(a.n);
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(gp(&jb.stamp), 2 * a.call + pass, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    if (threadIdx.x == 0)
      sh.dp_q = ld_agent(&jb.next[pass]) < parts
                    ? __hip_atomic_fetch_add(gp(&jb.next[pass]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                    : parts;
    __syncthreads();
    const uint32_t q = sh.dp_q;
    __syncthreads();
    if (q >= parts) break;
    deep_part(a, row, q, pass);
  }
  if (threadIdx.x == 0) {
    uint32_t k = 0;
    for (; ld_agent(&jb.ended[pass]) < parts && k < kDeepSpin; ++k) __builtin_amdgcn_s_sleep(2);
    sh.dp_stop = k < kDeepSpin ? 1u : 0u;
  }
  __syncthreads();
  return sh.dp_stop != 0u;
}

// A workgroup with no row left: takes parts of the rows' published passes (starting from its own
// index, so that helpers spread over the rows) until every row of the call is finished. Helpers are
// optional (each row's workgroup takes the parts nobody took), so a helper also stops after
// kHelpTicks of the device's 100 MHz clock, a guard no call reaches.
constexpr uint64_t kHelpTicks = 5000000;  // 50 ms
__device__ __attribute__((unused)) void deep_help(const FinishArgs& a, uint32_t wg) {
  Shared& sh = shm();
  const uint32_t tid = threadIdx.x, nr = a.n_rows, parts = as_launch::tail_parts(a.n);
  if (tid < 256) sh.tab[tid] = as_exp::kTable[tid];  // the parts' exps read the table in LDS
  const uint64_t s0 = 2 * a.call, t0 = wall_clock64();
  for (;;) {
    if (tid == 0) sh.dp_pick = kNone;
    __syncthreads();
    // Every row's job at once, one per thread: a published pass with parts left.
    for (uint32_t r = tid; r < nr; r += kThreads) {
      const DeepJob& jb = a.deep_jobs[r];
      const uint64_t st = ld_agent(&jb.stamp);
      const uint32_t left0 = ld_agent(&jb.next[0]), left1 = ld_agent(&jb.next[1]);
      const uint32_t pass = st == s0 ? 0u : (st == s0 + 1 ? 1u : 2u);
      if (pass < 2 && (pass ? left1 : left0) < parts) atomicMin(&sh.dp_pick, (((r + nr - wg % nr) % nr) << 1) | pass);
    }
    if (tid == 0) sh.dp_stop = (ld_agent(a.deep_done) >= a.deep_target || wall_clock64() - t0 > kHelpTicks) ? 1u : 0u;
    __syncthreads();
    const uint32_t pick = sh.dp_pick, stop = sh.dp_stop;
    if (pick != kNone) {
      const uint32_t r = ((pick >> 1) + wg % nr) % nr, pass = pick & 1u;
      if (tid == 0) sh.dp_q = __hip_atomic_fetch_add(gp(&a.deep_jobs[r].next[pass]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      const uint32_t q = sh.dp_q;
      if (q < parts) deep_part(a, r, q, pass);
      continue;
    }
    if (stop) break;
    __builtin_amdgcn_s_sleep(8);
  }
}

// The deep path's two passes over a row, each streaming through a ring of three steps' loads (two in
// flight while one is used: more would spill the caller's registers). Both leave out the history's
// positions (cnt set): their values are penalised, which the caller adds. The bins: distance below
// the largest value topf, bsc bins per unit, the last bin holding everything further down.
__device__ __forceinline__ uint32_t deep_bin(float topf, float bsc, uint32_t nb, float v) {
  const float t = (topf - v) * bsc;
  return t < (float)(nb - 1) ? (uint32_t)t : nb - 1;
}

// Pass 1: each value at or above cut, its count and weights into the LDS histogram (hc counts, hm the
// weights at T = 1 when by_top_p, hw the weights at T).
__device__ __forceinline__ void deep_hist(const float* x, const uint32_t* pcnt, uint32_t n, bool vec, uint32_t nb,
                                       float topf, float bsc, double top, double temp, bool by_top_p, float cut,
                                       uint32_t* hc, double* hm, double* hw) {
  PassWeights pw;
  pw.init(top, temp);
  for_each_value<true, 3>(x, pcnt, n, vec, [&](uint32_t, float v, uint32_t c) {
    if (__builtin_expect(c == 0, 1) && v >= cut) {
      const uint32_t b = deep_bin(topf, bsc, nb, v);
      const double d = pw.d(v);
      atomicAdd(&hc[b], 1u);
      if (by_top_p) atomicAdd(&hm[b], pw.one(d));
      atomicAdd(&hw[b], pw.at_t(d));
    }
  });
}

// Pass 2: the values of the bins in the runs [a0, e0], [a1, e1], [a2, e2] (kNone: no run) whose key is
// at least kcut into sk, packed, in any order; *pick counts them (past cap they are counted, not
// kept). kb: 6 words of LDS.
// The bin is a non-increasing function of the value, so the values whose bin lies in a run [a, e]
// are those whose key lies in an interval [lo, hi]. Lanes 0-5 find the six bounds by bisection over
// the keys at or below the largest value's (no value of the row lies above it; the keys below the
// finite values, -inf's and the NaNs', fall in the last bin as -FLT_MAX does); each value then costs
// its key and two compares per run instead of its bin and the runs' tests.
__device__ __forceinline__ void deep_collect(const float* x, const uint32_t* pcnt, uint32_t n, bool vec, uint32_t nb,
                                          float topf, float bsc, uint32_t a0, uint32_t e0, uint32_t a1, uint32_t e1,
                                          uint32_t a2, uint32_t e2, uint32_t* pick, uint64_t* sk, uint32_t cap,
                                          uint32_t* kb, uint32_t kcut) {
  static_assert(kBinRanges == 3, "three runs");
  const uint32_t tid = threadIdx.x;
  if (tid < 2 * kBinRanges) {
    const uint32_t r = tid >> 1, a = sel3(r, a0, a1, a2), e = sel3(r, e0, e1, e2), ktop = total_key(topf);
    auto bin = [&](uint32_t k) { return deep_bin(topf, bsc, nb, key_value(k)); };
    uint32_t out;
    if (a == kNone) {
      out = (tid & 1u) ? 0u : 0xFFFFFFFFu;  // an empty interval: lo above hi
    } else if ((tid & 1u) == 0) {
      // lo: the least key whose bin is at most e (the largest value's bin, 0, is).
      uint32_t lo = 0, hi = ktop;
      while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (bin(mid) <= e) hi = mid;
        else lo = mid + 1;
      }
      out = max(lo, kcut);
    } else {
      // hi: the greatest key at or below ktop whose bin is at least a (key 0's, the last bin, is).
      uint32_t lo = 0, hi = ktop;
      while (lo < hi) {
        const uint32_t mid = hi - (hi - lo) / 2;
        if (bin(mid) >= a) lo = mid;
        else hi = mid - 1;
      }
      out = lo;
    }
    kb[tid] = out;
  }
  __syncthreads();
  const uint32_t l0 = kb[0], h0 = kb[1], l1 = kb[2], h1 = kb[3], l2 = kb[4], h2 = kb[5];
  for_each_value<true, 3>(x, pcnt, n, vec, [&](uint32_t i, float v, uint32_t c) {
    const uint32_t k = total_key(v);
    const bool hit = ((k >= l0) & (k <= h0)) | ((k >= l1) & (k <= h1)) | ((k >= l2) & (k <= h2));
    if (__builtin_expect(hit && c == 0, 0)) {
      const uint32_t s = atomicAdd(pick, 1u);
      if (s < cap) sk[s] = pack(k, i);
    }
  });
}

template <bool kDist>
__device__ __noinline__ bool deep_bins(const FinishArgs& a, const RowParams& p, uint32_t row, bool pen) {
  constexpr uint32_t kNB = kDist ? as_launch::kDistBins : kDeepBins;
  Shared& sh = shm();
  const uint32_t n = a.n, tid = threadIdx.x;
  uint32_t* cnt = a.scratch + (uint64_t)row * a.scratch_stride;
  uint32_t hb;
  const uint32_t he = history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const float* x = a.logits + (uint64_t)row * a.row_stride;
  const uint32_t* pcnt = pen ? cnt : nullptr;
  const bool vec = a.vec && a.row_stride % 4 == 0;
  const uint64_t* tab = sh.tab;
  const uint32_t mk = sh.mk;
  const double top = (double)key_value(mk), temp = (double)p.temp, top_p = (double)p.top_p;
  const float topf = key_value(mk);
  const bool has_floor = p.min_p > 0.0f, by_top_p = p.top_p < 1.0f;
  // A top-k row keeps its k best ranks before top-p and min-p cut (sample.rs:157-161), and top-p's
  // total is theirs.
  const bool topk = p.mode == kModeTopK || p.mode == kModeExactTopK;
  const uint32_t kk = topk ? p.top_k : n;
  const bool unfiltered = !by_top_p && !has_floor && !topk;
  const float floorf = floor_f32(__dadd_rn(top, p.ln_min_p));
  // With min-p's floor the only cut (no top-p, no top-k), values below the floor are never kept and
  // no total counts them: both passes leave them out.
  const float cut = deep_cut(p, topf);
  // Bins of distance below the largest value, kNB over span, everything further down in the
  // last: below span a weight is under e^-32 of the largest's (span is 32 T above T = 1).
  const float span = 32.0f * fmaxf(1.0f, p.temp);
  const float bsc = (float)kNB / span;
  auto bin_of = [&](float v) -> uint32_t {
    const float t = (topf - v) * bsc;
    return t < (float)(kNB - 1) ? (uint32_t)t : kNB - 1;
  };
  // The reference's weights exp(l - top) (top-p's) and exp((l - top) / T); arguments at or below
  // -512 (terms under 1e-222) are left out, far inside the bounds below.
  auto e_core = [&](double d) -> double { return d > -512.0 ? as_exp::exp_core(tab, d) : 0.0; };
  auto w1 = [&](float v) -> double { return e_core(__dsub_rn((double)v, top)); };
  auto wt = [&](float v) -> double { return e_core(__ddiv_rn(__dsub_rn((double)v, top), temp)); };

  // Pass 1: counts (hc), weights at T = 1 (hm, top-p rows) and at T (hw). hc and hm share sh.wd,
  // hw lies in sh.sk.
  uint32_t* hc = reinterpret_cast<uint32_t*>(sh.wd);
  double* hm = sh.wd + kNB / 2;
  double* hw = reinterpret_cast<double*>(sh.sk);
  static_assert(kNB * 12 <= sizeof(sh.wd) && kNB * 8 <= sizeof(sh.sk), "histogram room");
  for (uint32_t b = tid; b < kNB; b += kThreads) {
    hc[b] = 0;
    hm[b] = 0.0;
    hw[b] = 0.0;
  }
  __syncthreads();
  PassWeights pw;
  pw.init(top, temp);
  auto count = [&](float v) {
    const uint32_t b = bin_of(v);
    const double d = pw.d(v);
    atomicAdd(&hc[b], 1u);
    if (by_top_p) atomicAdd(&hm[b], pw.one(d));
    atomicAdd(&hw[b], pw.at_t(d));
  };
  if (kDist) {
    // The histogram pass shared: the row's histogram in its scratch is cleared, the pass published,
    // and this workgroup takes parts with the others until none is left, then waits for the parts
    // the others took (the history's positions are left out of every part: they are added below).
    uint32_t* gc = deep_shared(a, row);
    double* gm = reinterpret_cast<double*>(gc + kNB);
    double* gw = gm + kNB;
    if (!sh.dp_pub) deep_publish_hist(a, row, mk);  // unless the row published it before its candidates
    if (!deep_run(a, row, 0)) return false;
    for (uint32_t b = tid; b < kNB; b += kThreads) {
      hc[b] = ld_agent(gc + b);
      hm[b] = ld_agent(gm + b);
      hw[b] = ld_agent(gw + b);
    }
    __syncthreads();  // the bins are whole before the history's values add to them
  } else {
    deep_hist(x, pcnt, n, vec, kNB, topf, bsc, top, temp, by_top_p, cut, hc, hm, hw);
  }
  if (pen) {
    // Each history id once, penalised, by the thread that sets its count's top bit first (pass 2
    // clears it again).
    auto hist_one = [&](uint32_t id) {
      if (id >= n) return;
      const uint32_t old = atomicOr(&cnt[id], 0x80000000u);
      if (!(old & 0x80000000u)) {
        const float v = penalize(x[id], old, p);
        if (v >= cut) count(v);
      }
    };
    for (uint32_t h = hb + tid; h < he; h += kThreads) hist_one(gload(a.hist_ids + h));
    for (uint32_t h = tid; h < extra; h += kThreads) hist_one(gload(a.extra_ids + h));
  }
  __syncthreads();

  // Inclusive prefixes over the bins, in place: kDPer bins per thread, then the block.
  constexpr int kDPer = kNB / kThreads;
  static_assert(kNB % kThreads == 0, "whole bins per thread");
  {
    uint32_t c4[kDPer], cs = 0;
    double m4[kDPer], w4[kDPer], ms = 0.0, ws = 0.0;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      const uint32_t b = tid * kDPer + q;
      cs += hc[b];
      ms = __dadd_rn(ms, hm[b]);
      ws = __dadd_rn(ws, hw[b]);
      c4[q] = cs;
      m4[q] = ms;
      w4[q] = ws;
    }
    uint32_t call;
    const uint32_t cb = block_exclusive_scan_u32(cs, sh.red_u, &call);
    const double mb = block_exclusive_scan_f64(ms, sh.red_d);
    const double wb = block_exclusive_scan_f64(ws, sh.red_d);
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      const uint32_t b = tid * kDPer + q;
      hc[b] = cb + c4[q];
      hm[b] = __dadd_rn(mb, m4[q]);
      hw[b] = __dadd_rn(wb, w4[q]);
    }
  }
  __syncthreads();
  // Every prefix (and the totals) is within E of the exact sum of the reference's terms: each term is
  // within kPassRel of the reference's and goes through one f64 atomic add and at most
  // kDPer + 2 log2(kThreads) + 2 more adds; the reference's own folds of its terms (total1 and the
  // unfiltered total in index order, the cumulatives in rank order, the kept weight) are within
  // gamma(n) of the same exact sums, and gj covers their ratios.
  const double M_all = hm[kNB - 1], W_all = hw[kNB - 1];
  const double g_all = gamma_ub(2.0 * (double)n + 128.0) + kPassRel * (1.0 + 1e-6);
  const double Em = g_all * M_all, Ew = g_all * W_all;
  const double gj = gamma_ub(2.0 * (double)n + 4.0) + 10.0 * kU;
  auto C = [&](uint32_t b) -> uint32_t { return b == kNone ? 0u : hc[b]; };  // through bin b; kNone: none
  auto Mc = [&](uint32_t b) -> double { return b == kNone ? 0.0 : hm[b]; };
  auto Wc = [&](uint32_t b) -> double { return b == kNone ? 0.0 : hw[b]; };
  auto before = [](uint32_t b) -> uint32_t { return b == 0 ? kNone : b - 1; };

  // top-k's count cut: rank k - 1 lies in bin bk, the first whose count reaches k.
  uint32_t bk = kNB - 1;
  if (topk) {
    uint32_t a0 = kNone;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      const uint32_t b = tid * kDPer + q;
      if (hc[b] >= kk) a0 = min(a0, b);
    }
    bk = block_min_u32<kWaves>(a0, sh.red_u);
    if (bk == kNone) return false;
  }
  // top-p's total1: the row's, or the top-k ranks' (those of the bins before bk and some of bk's:
  // bounded here, summed from bk's sorted values below; each bound three times the error of that
  // sum apart, so that the targets only narrow once it is known).
  const double Em2 = Em + 2.0 * gamma_n(64.0) * M_all;
  double M_lo = M_all - Em, M_hi = M_all + Em;
  if (topk) {
    M_lo = Mc(before(bk)) - 3.0 * Em2;
    M_hi = Mc(bk) + 3.0 * Em2;
  }
  // top-p's cut: the first rank whose reference cumulative reaches top_p, i.e. whose prefix S_j
  // reaches top_p * total1. Bins before c_lo cannot hold it (their prefixes cannot reach the least
  // target); at the end of c_hi it has surely been reached (for a top-k row, at bk's end at the
  // latest: past rank k - 1 nothing is kept).
  double tp_lo = top_p * M_lo, tp_hi = top_p * M_hi;
  uint32_t c_lo = kNone, c_hi = kNone;
  if (by_top_p) {
    uint32_t a0 = kNone, a1 = kNone;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      const uint32_t b = tid * kDPer + q;
      if ((hm[b] + Em) * (1.0 + gj) >= tp_lo) a0 = min(a0, b);
      if ((hm[b] - Em) * (1.0 - gj) >= tp_hi) a1 = min(a1, b);
    }
    c_lo = block_min_u32<kWaves>(a0, sh.red_u);
    c_hi = block_min_u32<kWaves>(a1, sh.red_u);
    if (c_hi == kNone) c_hi = kNB - 1;
    if (c_lo == kNone) c_lo = c_hi;
    c_lo = min(c_lo, bk);
    c_hi = min(c_hi, bk);
  }
  // min-p's cut, the first rank below the floor, lies in the floor value's bin f (or at its ends).
  const uint32_t f = has_floor ? bin_of(floorf) : kNone;
  const bool need_c = by_top_p && !(has_floor && f < c_lo);  // else min-p surely cuts first
  const bool need_f = has_floor && !(by_top_p && f > c_hi) && !(topk && f > bk);  // else another does
  // The count cut, unless min-p surely cuts first; bk's values are collected for it and for top-p's
  // total1.
  const bool need_k = topk && !(has_floor && f < bk);
  const bool need_bk = need_k || (topk && need_c);
  // The kept set ends in bins [k_lo, k_hi] (the last bin when nothing cuts).
  uint32_t k_lo = kNB - 1, k_hi = kNB - 1;
  if (need_c) {
    k_lo = c_lo;
    k_hi = c_hi;
  }
  if (need_f) {
    k_lo = min(k_lo, f);
    k_hi = min(k_hi, f);
  }
  if (need_k) {
    k_lo = min(k_lo, bk);
    k_hi = min(k_hi, bk);
  }
  // The draw: u = unit() * W, W the kept weight at T, in [Wc(k_lo - 1), Wc(k_hi)] (all of it when
  // nothing cuts); the bins that can hold the first cumulative above u, at most the kept set's.
  const double Wk_lo = unfiltered ? W_all : Wc(before(k_lo)), Wk_hi = unfiltered ? W_all : Wc(k_hi);
  const double u_lo = sh.u01 * (Wk_lo - Ew) * (1.0 - gj) * (1.0 - 4.0 * kU);
  const double u_hi = sh.u01 * (Wk_hi + Ew) * (1.0 + gj) * (1.0 + 4.0 * kU);
  uint32_t d_lo, d_hi;
  {
    uint32_t a0 = kNone, a1 = kNone;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      const uint32_t b = tid * kDPer + q;
      if ((hw[b] + Ew) * (1.0 + gj) > u_lo) a0 = min(a0, b);
      if ((hw[b] - Ew) * (1.0 - gj) > u_hi) a1 = min(a1, b);
    }
    d_lo = min(block_min_u32<kWaves>(a0, sh.red_u), k_hi);
    d_hi = min(block_min_u32<kWaves>(a1, sh.red_u), k_hi);  // past the kept set: its last value
  }
  // The runs of bins to collect, in bin order, merged where they touch (more than kBinRanges runs:
  // the full deep path).
  uint32_t r0[kBinRanges], r1[kBinRanges], nr = 0;
  {
    // The draw's, the cut's, the floor's and bk (kNone: not needed), sorted by start with five
    // compare-exchanges (kNone last), then merged.
    constexpr uint32_t kIn = kBinRanges + 1;
    uint32_t lo[kIn] = {d_lo, need_c ? c_lo : kNone, need_f ? f : kNone, need_bk ? bk : kNone};
    uint32_t hi[kIn] = {d_hi, need_c ? c_hi : kNone, need_f ? f : kNone, need_bk ? bk : kNone};
    auto cx = [&](int i, int j) {
      if (lo[j] < lo[i]) {
        const uint32_t t0 = lo[i], t1 = hi[i];
        lo[i] = lo[j];
        hi[i] = hi[j];
        lo[j] = t0;
        hi[j] = t1;
      }
    };
    static_assert(kIn == 4, "a sorting network of four");
    cx(0, 1);
    cx(2, 3);
    cx(0, 2);
    cx(1, 3);
    cx(1, 2);
#pragma unroll
    for (uint32_t i = 0; i < kBinRanges; ++i) {
      r0[i] = kNone;
      r1[i] = kNone;
    }
    bool over = false;
#pragma unroll
    for (uint32_t i = 0; i < kIn; ++i) {
      if (lo[i] == kNone) continue;
      if (nr > 0 && lo[i] <= sel3(nr - 1, r1[0], r1[1], r1[2]) + 1) {
        const uint32_t e = max(sel3(nr - 1, r1[0], r1[1], r1[2]), hi[i]);
#pragma unroll
        for (uint32_t k = 0; k < kBinRanges; ++k)
          if (k + 1 == nr) r1[k] = e;
      } else if (nr == kBinRanges) {
        over = true;
      } else {
#pragma unroll
        for (uint32_t k = 0; k < kBinRanges; ++k)
          if (k == nr) {
            r0[k] = lo[i];
            r1[k] = hi[i];
          }
        ++nr;
      }
    }
    if (over) return false;
  }
  // Per run: the count and weights before it, and where its values start among the collected ones.
  uint32_t cbr[kBinRanges], first[kBinRanges];
  double mbr[kBinRanges], wbr[kBinRanges];
  uint32_t collected = 0;
#pragma unroll
  for (uint32_t k = 0; k < kBinRanges; ++k) {
    cbr[k] = 0;
    mbr[k] = 0.0;
    wbr[k] = 0.0;
    first[k] = kNone;  // past every collected value: no run
    if (k < nr) {
      cbr[k] = C(before(r0[k]));
      mbr[k] = Mc(before(r0[k]));
      wbr[k] = Wc(before(r0[k]));
      first[k] = collected;
      collected += C(r1[k]) - cbr[k];
    }
  }
  const uint32_t cf_before = need_f ? C(before(f)) : 0u, cf_through = need_f ? C(f) : 0u;
  const double wf_before = need_f ? Wc(before(f)) : 0.0, wf_through = need_f ? Wc(f) : 0.0;
  const bool fits = collected <= (uint32_t)kCap;
  if (tid == 0) sh.pick = 0;
  __syncthreads();  // every thread has read the prefixes: sh.sk takes the collected values

  // Pass 2: the runs' values into sh.sk (any order); the history ids once more, which clears their
  // counts' top bits (also when the values do not fit).
  auto in_runs = [&](uint32_t b) {
    bool in = false;
#pragma unroll
    for (uint32_t k = 0; k < kBinRanges; ++k) in = in || (b >= r0[k] && b <= r1[k]);  // unused: kNone
    return in;
  };
  if (fits && kDist) {
    // The collecting pass shared: the runs published, the parts' values listed in the row's scratch,
    // then copied here (the list holds at most kCap: more and the values do not fit).
    DeepJob& jb = a.deep_jobs[row];
    uint32_t* lc = deep_shared(a, row) + 5 * kNB;
    const uint64_t* list = reinterpret_cast<const uint64_t*>(lc + 2);
    if (tid == 0) {
#pragma unroll
      for (uint32_t k = 0; k < kBinRanges; ++k) {
        __hip_atomic_store(gp(&jb.r0[k]), sel3(k, r0[0], r0[1], r0[2]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(gp(&jb.r1[k]), sel3(k, r1[0], r1[1], r1[2]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_store(gp(lc), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!deep_run(a, row, 1)) return false;
    if (tid == 0) sh.nsk = ld_agent(lc);
    __syncthreads();
    const uint32_t got = sh.nsk;
    if (got <= (uint32_t)kCap) {
      for (uint32_t i = tid; i < got; i += kThreads) sh.sk[i] = ld_agent(list + i);
      if (tid == 0) sh.pick = got;
    } else if (tid == 0) {
      sh.pick = kCap + 1;  // more than fit: not collected
    }
    __syncthreads();
  } else if (fits) {
    deep_collect(x, pcnt, n, vec, kNB, topf, bsc, r0[0], r1[0], r0[1], r1[1], r0[2], r1[2], &sh.pick, sh.sk,
                 (uint32_t)kCap, sh.base, cut > -__builtin_inff() ? total_key(cut) : 0u);
  }
  if (pen) {
    auto hist_two = [&](uint32_t id) {
      if (id >= n) return;
      const uint32_t old = atomicAnd(&cnt[id], 0x7fffffffu);
      if (!(old & 0x80000000u) || !fits) return;
      const float v = penalize(x[id], old & 0x7fffffffu, p);
      if (v >= cut && in_runs(bin_of(v))) {
        const uint32_t s = atomicAdd(&sh.pick, 1u);
        if (s < (uint32_t)kCap) sh.sk[s] = pack(total_key(v), id);
      }
    };
    for (uint32_t h = hb + tid; h < he; h += kThreads) hist_two(gload(a.hist_ids + h));
    for (uint32_t h = tid; h < extra; h += kThreads) hist_two(gload(a.extra_ids + h));
  }
  __syncthreads();
  if (!fits || sh.pick != collected || collected == 0) return false;
  // The bucket sort spreads keys below its kmax over its buckets: the collected values' own largest
  // key, since they lie in a few bins far below the row's largest (with that one most would share a
  // few buckets).
  uint32_t ck = 0;
  for (uint32_t i = tid; i < collected; i += kThreads) ck = max(ck, (uint32_t)(sh.sk[i] >> 32));
  ck = block_max_u32<kWaves>(ck, sh.red_u);
  const uint32_t P = sort_candidates(sh, collected, 0ull, ck, kNone);
  if (P != collected) return false;
  auto val = [&](uint32_t i) -> float { return packed_value(sh.sk[i]); };
  auto run_of = [&](uint32_t i) -> uint32_t { return (i >= first[2]) ? 2u : (i >= first[1] ? 1u : 0u); };
  auto rank_of = [&](uint32_t i, uint32_t k) -> uint32_t { return sel3(k, cbr[0], cbr[1], cbr[2]) + (i - sel3(k, first[0], first[1], first[2])); };
  // A scan of the collected values' weights in sh.wd: each thread's inclusive prefixes, and per run
  // the scan just before it (a run's terms through i are the difference, within 2 gamma(40) of the
  // scan's total).
  double loc[kScanPer], off;
  double* run_base = sh.red_d;  // one slot per run (kWaves >= kBinRanges)
  static_assert(kWaves >= (int)kBinRanges, "a slot per run");
  auto scan_runs = [&]() {
    prefix_scan(sh, P, loc, &off);
    if (tid < kBinRanges) run_base[tid] = 0.0;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
      const uint32_t i = tid * kScanPer + q;
#pragma unroll
      for (uint32_t k = 1; k < kBinRanges; ++k)
        if (i < P && i + 1 == first[k]) run_base[k] = __dadd_rn(off, loc[q]);
    }
    __syncthreads();
  };
  const double g40 = 2.0 * gamma_n(40.0);

  // Up to kWaveMax collected values: wave 0 takes the decisions below from registers (lane l holds
  // collected values kWPer l .. kWPer l + kWPer - 1, their prefixes come from a wave scan) with the
  // same bounds and no block-wide step, and the other waves wait at one barrier. A prefix through
  // collected value i is within gamma(kWPer + 7) of its exact sum, inside the block path's gamma(40).
  if (P <= kWaveMax) {
    if (tid < kWave) {
      const uint32_t i0 = tid * kWPer;
      float v[kWPer];
      uint32_t rn[kWPer], rk[kWPer];
#pragma unroll
      for (int q = 0; q < kWPer; ++q) {
        const uint32_t i = i0 + q;
        v[q] = i < P ? val(i) : 0.0f;
        rn[q] = run_of(i);
        rk[q] = i < P ? rank_of(i, rn[q]) : kNone;
      }
      // Where a rank's value lies among the collected ones (kNone: not collected), and the run that
      // holds it: run k holds ranks cbr[k] .. and collected values first[k] .., up to the next run's.
      auto index_of = [&](uint32_t r, uint32_t* home) -> uint32_t {
        uint32_t j = kNone;
#pragma unroll
        for (uint32_t k = 0; k < kBinRanges; ++k) {
          if (k >= nr) continue;
          const uint32_t f0 = sel3(k, first[0], first[1], first[2]);
          const uint32_t f1 = k + 1 < nr ? sel3(k + 1, first[0], first[1], first[2]) : P;
          const uint32_t c0 = sel3(k, cbr[0], cbr[1], cbr[2]);
          if (r >= c0 && r - c0 < f1 - f0) {
            j = f0 + (r - c0);
            *home = k;
          }
        }
        return j;
      };
      double w[kWPer], pre[kWPer], rb[kBinRanges];
      // The prefixes of w in pre, and per run the prefix just before it in rb.
      auto prefixes = [&]() {
        wave_prefix(w, pre);
#pragma unroll
        for (uint32_t k = 0; k < kBinRanges; ++k) {
          const uint32_t f = sel3(k, first[0], first[1], first[2]);
          double x = 0.0;
          if (k > 0 && k < nr && f > 0) {
            const uint32_t j = f - 1, qj = j % kWPer;
            double y = pre[0];
#pragma unroll
            for (int q = 1; q < kWPer; ++q)
              if ((uint32_t)q == qj) y = pre[q];
            x = wave_lane_f64(y, j / kWPer);
          }
          rb[k] = x;
        }
      };
      // The prefix through collected value j in run k, above the run's start.
      auto run_part = [&](uint32_t j, uint32_t k) -> double {
        const uint32_t qj = j % kWPer;
        double y = pre[0];
#pragma unroll
        for (int q = 1; q < kWPer; ++q)
          if ((uint32_t)q == qj) y = pre[q];
        return __dsub_rn(wave_lane_f64(y, j / kWPer), sel3(k, rb[0], rb[1], rb[2]));
      };
      bool ok = true;
      uint32_t keep_w = n, k_floor = kNone;
      double Wk = W_all, Wk_err = Ew;
      if (need_c || need_f || topk) {
        uint32_t jl = kNone, jh = kNone, jf = kNone;
        if (need_c) {
#pragma unroll
          for (int q = 0; q < kWPer; ++q) w[q] = i0 + q < P ? w1(v[q]) : 0.0;
          prefixes();
          double tlo = tp_lo, thi = tp_hi;
          if (topk) {
            uint32_t home = kNone;
            const uint32_t j = index_of(kk - 1, &home);
            if (j == kNone) {
              ok = false;
            } else {
              const double Mk = __dadd_rn(sel3(home, mbr[0], mbr[1], mbr[2]), run_part(j, home));
              tlo = top_p * (Mk - Em2);
              thi = top_p * (Mk + Em2);
            }
          }
          const double err = Em + g40 * M_all;
#pragma unroll
          for (int q = 0; q < kWPer; ++q) {
            if (i0 + q >= P || rk[q] >= kk) continue;
            const uint32_t k = rn[q];
            const double S = __dadd_rn(sel3(k, mbr[0], mbr[1], mbr[2]), __dsub_rn(pre[q], sel3(k, rb[0], rb[1], rb[2])));
            if ((S + err) * (1.0 + gj) >= tlo) jl = min(jl, rk[q]);
            if ((S - err) * (1.0 - gj) >= thi) jh = min(jh, rk[q]);
          }
        }
#pragma unroll
        for (int q = 0; q < kWPer; ++q)
          if (need_f && i0 + q < P && rk[q] < kk && !(v[q] >= floorf)) jf = min(jf, rk[q]);
        jl = wave_min_u32(jl);
        jh = wave_min_u32(jh);
        jf = wave_min_u32(jf);
        uint32_t k_topp = kNone;
        if (need_c) {
          if (topk && jl == kNone) {
            k_topp = kNone;
          } else if (jl != jh || jh == kNone) {
            ok = false;
          } else {
            k_topp = jh + 1;
          }
        }
        if (need_f) k_floor = min(jf, cf_through);
        keep_w = min(min(k_topp, k_floor), kk);
        Wk_err = Ew + 2.0 * gamma_n(64.0) * W_all;
      }
      // The weights at T and their prefixes; the kept weight, a prefix of whole bins when min-p cuts
      // at its bin's ends, else a run's prefix plus its terms through rank keep - 1.
#pragma unroll
      for (int q = 0; q < kWPer; ++q) w[q] = i0 + q < P ? wt(v[q]) : 0.0;
      prefixes();
      if (need_c || need_f || topk) {
        if (need_f && keep_w == k_floor && keep_w == cf_through) {
          Wk = wf_through;
        } else if (need_f && keep_w == k_floor && keep_w == cf_before) {
          Wk = wf_before;
        } else {
          uint32_t home = kNone;
          const uint32_t j = keep_w > 0 ? index_of(keep_w - 1, &home) : kNone;
          if (j == kNone) ok = false;
          else Wk = __dadd_rn(sel3(home, wbr[0], wbr[1], wbr[2]), run_part(j, home));
        }
      }
      // The draw, as below.
      const double ulo = sh.u01 * (Wk - Wk_err) * (1.0 - gj) * (1.0 - 4.0 * kU);
      const double uhi = sh.u01 * (Wk + Wk_err) * (1.0 + gj) * (1.0 + 4.0 * kU);
      const double err = Ew + g40 * W_all;
      uint32_t jp = kNone, jc = kNone, last = kNone;
#pragma unroll
      for (int q = 0; q < kWPer; ++q) {
        if (i0 + q >= P || rk[q] >= keep_w) continue;
        if (rk[q] + 1 == keep_w) last = i0 + q;
        const uint32_t k = rn[q];
        const double S = __dadd_rn(sel3(k, wbr[0], wbr[1], wbr[2]), __dsub_rn(pre[q], sel3(k, rb[0], rb[1], rb[2])));
        if ((S + err) * (1.0 + gj) > ulo) jp = min(jp, rk[q]);
        if ((S - err) * (1.0 - gj) > uhi) jc = min(jc, rk[q]);
      }
      jp = wave_min_u32(jp);
      jc = wave_min_u32(jc);
      last = wave_min_u32(last);
      uint32_t pick_rank = kNone;
      if (jp == kNone) {
        if (last == kNone) ok = false;
        else pick_rank = keep_w - 1;
      } else if (jp == jc) {
        pick_rank = jc;
      } else {
        ok = false;
      }
      uint32_t home = kNone;
      const uint32_t pi = ok ? index_of(pick_rank, &home) : kNone;
      if (pi == kNone) ok = false;
      if (tid == 0) {
        if (ok) {
          a.tokens[row] = packed_id(sh.sk[pi]);
          a.status[row] = AS_ROW_OK | AS_ROW_DEEP_PATH;
          if (a.kept_count) a.kept_count[row] = keep_w;
        }
        sh.pick = ok ? 1u : 0u;
      }
    }
    __syncthreads();
    return sh.pick != 0;
  }

  // The cut (sample.rs:230-252): at the first rank below the floor, or one past the first whose
  // cumulative reaches top_p, whichever comes first.
  // The run that holds rank r (kNone: not collected).
  auto home_of = [&](uint32_t r) -> uint32_t {
    uint32_t home = kNone;
    for (uint32_t i = tid; i < P; i += kThreads) {
      const uint32_t k = run_of(i);
      if (rank_of(i, k) == r) home = k;
    }
    return block_min_u32<kWaves>(home, sh.red_u);
  };
  uint32_t keep = n;
  double Wkeep = W_all, Wkeep_err = Ew;
  if (need_c || need_f || topk) {
    for (uint32_t i = tid; i < P; i += kThreads) sh.wd[i] = need_c ? w1(val(i)) : 0.0;
    __syncthreads();
    if (topk && need_c) {
      // top-p's total1 over the top-k ranks: the prefix before rank k - 1's run plus that run's
      // terms through it, within Em2 of the exact sum; the targets narrow to it.
      const uint32_t home = home_of(kk - 1);
      if (home == kNone) return false;
      double part = 0.0;
      for (uint32_t i = tid; i < P; i += kThreads)
        if (run_of(i) == home && rank_of(i, home) < kk) part += sh.wd[i];
      part = block_sum_f64<kWaves>(part, sh.red_d);
      const double Mk = __dadd_rn(sel3(home, mbr[0], mbr[1], mbr[2]), part);
      tp_lo = top_p * (Mk - Em2);
      tp_hi = top_p * (Mk + Em2);
    }
    scan_runs();
    uint32_t jl = kNone, jh = kNone, jf = kNone;
    const double err = Em + g40 * M_all;
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
      const uint32_t i = tid * kScanPer + q;
      if (i >= P) continue;
      const uint32_t k = run_of(i), r = rank_of(i, k);
      if (r >= kk) continue;  // past top-k's cut
      if (need_f && !(val(i) >= floorf)) jf = min(jf, r);
      if (need_c) {
        const double S = __dadd_rn(sel3(k, mbr[0], mbr[1], mbr[2]), __dsub_rn(__dadd_rn(off, loc[q]), run_base[k]));
        if ((S + err) * (1.0 + gj) >= tp_lo) jl = min(jl, r);
        if ((S - err) * (1.0 - gj) >= tp_hi) jh = min(jh, r);
      }
    }
    jl = block_min_u32<kWaves>(jl, sh.red_u);
    jh = block_min_u32<kWaves>(jh, sh.red_u);
    jf = block_min_u32<kWaves>(jf, sh.red_u);
    uint32_t k_topp = kNone, k_floor = kNone;
    if (need_c) {
      // A top-k row's cumulative may not reach top_p by rank k - 1 (its terms' rounding): then
      // top-p keeps all k (sample.rs:169-176).
      if (topk && jl == kNone) {
        k_topp = kNone;
      } else {
        if (jl != jh || jh == kNone) return false;
        k_topp = jh + 1;
      }
    }
    // The first value past the floor's bin is below the floor: min-p cuts there at the latest.
    if (need_f) k_floor = min(jf, cf_through);
    keep = min(min(k_topp, k_floor), kk);
    // The kept weight at T: a prefix of whole bins when min-p cuts at its bin's ends, else a run's
    // prefix plus its terms through rank keep - 1.
    __syncthreads();
    for (uint32_t i = tid; i < P; i += kThreads) sh.wd[i] = wt(val(i));
    __syncthreads();
    if (need_f && keep == k_floor && keep == cf_through) {
      Wkeep = wf_through;
    } else if (need_f && keep == k_floor && keep == cf_before) {
      Wkeep = wf_before;
    } else {
      const uint32_t home = home_of(keep - 1);
      if (home == kNone) return false;
      double part = 0.0;
      for (uint32_t i = tid; i < P; i += kThreads)
        if (run_of(i) == home && rank_of(i, home) < keep) part += sh.wd[i];
      part = block_sum_f64<kWaves>(part, sh.red_d);
      Wkeep = __dadd_rn(sel3(home, wbr[0], wbr[1], wbr[2]), part);
    }
    Wkeep_err = Ew + 2.0 * gamma_n(64.0) * W_all;
  } else {
    for (uint32_t i = tid; i < P; i += kThreads) sh.wd[i] = wt(val(i));
    __syncthreads();
  }

  // The draw (sample.rs:260-272, 274-292): u = unit() * (the kept weight), then the first kept rank
  // whose cumulative at T passes u, or the last kept one when none does.
  scan_runs();
  const double ulo = sh.u01 * (Wkeep - Wkeep_err) * (1.0 - gj) * (1.0 - 4.0 * kU);
  const double uhi = sh.u01 * (Wkeep + Wkeep_err) * (1.0 + gj) * (1.0 + 4.0 * kU);
  const double err = Ew + g40 * W_all;
  uint32_t jp = kNone, jc = kNone, last = kNone;
#pragma unroll
  for (int q = 0; q < kScanPer; ++q) {
    const uint32_t i = tid * kScanPer + q;
    if (i >= P) continue;
    const uint32_t k = run_of(i), r = rank_of(i, k);
    if (r >= keep) continue;
    if (r + 1 == keep) last = i;
    const double S = __dadd_rn(sel3(k, wbr[0], wbr[1], wbr[2]), __dsub_rn(__dadd_rn(off, loc[q]), run_base[k]));
    if ((S + err) * (1.0 + gj) > ulo) jp = min(jp, r);
    if ((S - err) * (1.0 - gj) > uhi) jc = min(jc, r);
  }
  jp = block_min_u32<kWaves>(jp, sh.red_u);
  jc = block_min_u32<kWaves>(jc, sh.red_u);
  last = block_min_u32<kWaves>(last, sh.red_u);
  // Ranks before the draw's first bin cannot pass u (their bins' prefixes cannot reach u_lo), and
  // every kept rank from there on was collected; so the first collected rank that may pass u is
  // the first of all.
  uint32_t pick_rank;
  if (jp == kNone) {
    if (last == kNone) return false;  // the last kept value was not collected
    pick_rank = keep - 1;
  } else if (jp == jc) {
    pick_rank = jc;
  } else {
    return false;
  }
  uint32_t pi = kNone;
  for (uint32_t i = tid; i < P; i += kThreads)
    if (rank_of(i, run_of(i)) == pick_rank) pi = i;
  pi = block_min_u32<kWaves>(pi, sh.red_u);
  if (pi == kNone) return false;
  if (tid == 0) {
    a.tokens[row] = packed_id(sh.sk[pi]);
    a.status[row] = AS_ROW_OK | AS_ROW_DEEP_PATH;
    if (a.kept_count) a.kept_count[row] = keep;
  }
  return true;
}


// Returns true when it settled the row.
// The row's history counts in its scratch (u32 per id), for the passes over the whole row: whether
// penalties act (false: no counts).
__device__ __noinline__ bool deep_prep(const FinishArgs& a, const RowParams& p, uint32_t row) {
  const uint32_t n = a.n, tid = threadIdx.x;
  uint32_t* cnt = a.scratch + (uint64_t)row * a.scratch_stride;
  uint32_t hb;
  const uint32_t he = history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  if (pen) {
    for (uint32_t i = tid; i < n; i += kThreads) cnt[i] = 0;
    __syncthreads();
    for (uint32_t h = hb + tid; h < he; h += kThreads) {
      const uint32_t id = gload(a.hist_ids + h);
      if (id < n) atomicAdd(&cnt[id], 1u);
    }
    for (uint32_t h = tid; h < extra; h += kThreads) {
      const uint32_t id = gload(a.extra_ids + h);
      if (id < n) atomicAdd(&cnt[id], 1u);
    }
    __syncthreads();
  }
  return pen;
}

// The full deep path, after deep_prep: returns true when it settled the row.
__device__ __noinline__ bool deep_row(const FinishArgs& a, const RowParams& p, uint32_t row, bool pen) {
  Shared& sh = shm();
  const uint32_t n = a.n, tid = threadIdx.x, lane = tid & (kWave - 1);
  uint32_t* S = a.scratch + (uint64_t)row * a.scratch_stride;
  uint32_t* cnt = S;
  uint64_t* bufA = reinterpret_cast<uint64_t*>(S + ((n + 1) & ~1u));
  uint64_t* bufB = bufA + n;
  const float* x = a.logits + (uint64_t)row * a.row_stride;

  uint32_t hb;
  const uint32_t he = history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  // The counts start 16-byte aligned (the scratch stride is a multiple of 4 words). History values
  // are few: their penalty runs out of line, so that the passes do not evaluate it for every value.
  const uint32_t* pcnt = pen ? cnt : nullptr;
  auto pvalue = [&](float v, uint32_t c) -> float { return __builtin_expect(c != 0, 0) ? penalize_out(v, c, p) : v; };
  const bool vec = a.vec && a.row_stride % 4 == 0;

  if (p.mode == kModeGreedy) {
    // greedy / greedy_penalized (sample.rs:9-17, 378-396) over the whole row.
    float gv = 0.0f;
    uint32_t gi = kNone;
    for_each_value(x, pcnt, n, vec, [&](uint32_t i, float v, uint32_t c) { greedy_merge(gv, gi, pvalue(v, c), i); });
    wave_greedy(gv, gi);
    if (lane == 0) {
      sh.wd[tid / kWave] = (double)gv;
      sh.red_u[tid / kWave] = gi;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kWaves; ++w) greedy_merge(gv, gi, (float)sh.wd[w], sh.red_u[w]);
      a.tokens[row] = gi;
      a.status[row] = AS_ROW_OK | AS_ROW_DEEP_PATH;
      if (a.kept_count) a.kept_count[row] = 1;
      if (a.kept_ids && a.kept_cap > 0) {
        a.kept_ids[(uint64_t)row * a.kept_cap] = gi;
        if (a.kept_probs) a.kept_probs[(uint64_t)row * a.kept_cap] = 1.0;
      }
    }
    return true;
  }

  // A slice whose statistics the scan could not finish (too many distinct history ids or
  // candidates) leaves the maxima and sums incomplete: the exact-order path recomputes everything.
  if (sh.stats_bad) return false;


  const uint32_t mk = sh.mk;
  const double top = (double)key_value(mk);
  const double temp = (double)p.temp, top_p = (double)p.top_p;
  const bool has_floor = p.min_p > 0.0f;
  const double floor = __dadd_rn(top, p.ln_min_p);
  const uint32_t fk = total_key(floor_f32(floor));
  const bool topk = (p.mode == kModeTopK || p.mode == kModeExactTopK);
  const uint32_t k = p.top_k;
  const bool cuts = p.top_p < 1.0f || has_floor;
  const bool unfiltered = !topk && !cuts;
  const uint64_t* tab = sh.tab;
  auto w_temp = [&](double v) { return as_exp::exp_with(tab, __ddiv_rn(__dsub_rn(v, top), temp)); };
  auto w_one = [&](double v) { return as_exp::exp_with(tab, __dsub_rn(v, top)); };

  // The row's total, when the cut or the draw needs it: first the slices' certified sums (within
  // about 1e-6 of the total); when a decision falls inside that bound (a cut this deep has
  // neighbouring cumulative weights ~1e-5 of the total apart), exact_total() sums the host-exact exp
  // of the reference's own f64 arguments, within (n + its fold's depth) * 2^-53 of the reference's
  // left fold.
  const bool need_total = !topk && (p.top_p < 1.0f || unfiltered);
  double X = 0.0, eps = 0.0;
  if (need_total) {
    slices_total(a, sh, top, temp, unfiltered, &X, &eps);
    if (!(X - eps > 0.0 && eps == eps)) return false;
  }
  bool exact = false;

  // Pass 1: a histogram of the values by distance below the largest, kDeepBins bins over dspan
  // (32, or 32 T for weights exp((l - top) / T): below it a value's weight is under e^-32 of the
  // largest), the last bin holding everything further down; with f32 weight sums. The bin is
  // monotone in the value, so every value ranking above the cut lies in a bin at or before its.
  const float topf = key_value(mk), inv_t = 1.0f / p.temp;
  const float bsc = (float)kDeepBins / (unfiltered ? 32.0f * p.temp : 32.0f);
  auto bin_of = [&](float v) -> uint32_t {
    const float t = (topf - v) * bsc;
    return t < (float)(kDeepBins - 1) ? (uint32_t)t : kDeepBins - 1;
  };
  // Counts (u32) and weights in 2^-32 units (u64: LDS integer atomics; float ones serialise).
  uint32_t* hc = reinterpret_cast<uint32_t*>(sh.wd);
  uint64_t* hm = reinterpret_cast<uint64_t*>(sh.wd) + kDeepBins / 2;
  static_assert(kDeepBins * 12 <= sizeof(sh.wd), "histogram room");
  for (uint32_t b = tid; b < kDeepBins; b += kThreads) {
    hc[b] = 0;
    hm[b] = 0ull;
  }
  __syncthreads();
  // One value into the histogram: its bin and (for the cut's bin) its weight, exp(d) <= 1 in 2^-32
  // units rounded down.
  auto count = [&](float v) {
    const uint32_t b = bin_of(v);
    atomicAdd(&hc[b], 1u);
    if (need_total) {
      const float f = unfiltered ? __expf((v - topf) * inv_t) : __expf(v - topf);
      atomicAdd(reinterpret_cast<unsigned long long*>(&hm[b]), (unsigned long long)(f * 0x1p32f));
    }
  };
  // The stream leaves history positions (count c != 0) out; each history id is then counted once,
  // penalised, by the thread that sets its count's top bit first.
  for_each_value(x, pcnt, n, vec, [&](uint32_t, float v, uint32_t c) {
    if (__builtin_expect(c == 0, 1)) count(v);
  });
  if (pen) {
    auto hist_one = [&](uint32_t id) {
      if (id >= n) return;
      const uint32_t old = atomicOr(&cnt[id], 0x80000000u);
      if (!(old & 0x80000000u)) count(penalize(x[id], old, p));
    };
    for (uint32_t h = hb + tid; h < he; h += kThreads) hist_one(gload(a.hist_ids + h));
    for (uint32_t h = tid; h < extra; h += kThreads) hist_one(gload(a.extra_ids + h));
  }
  __syncthreads();
  {
    // The cut's bin bc: the first whose running count reaches k (top-k), or whose running f32
    // weight reaches the target with 5% to spare; four bins per thread, then block scans.
    constexpr int kDPer = kDeepBins / kThreads;
    static_assert(kDeepBins % kThreads == 0, "whole bins per thread");
    uint32_t c4[kDPer], csum = 0;
    double m4[kDPer], msum = 0.0;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      c4[q] = hc[tid * kDPer + q];
      m4[q] = (double)hm[tid * kDPer + q] * 0x1p-32;
      csum += c4[q];
      msum += m4[q];
    }
    uint32_t call;
    uint32_t cb = block_exclusive_scan_u32(csum, sh.red_u, &call);
    double mb = block_exclusive_scan_f64(msum, sh.red_d);
    const double target = unfiltered ? sh.u01 * (X + eps) * 1.005 : (p.top_p < 1.0f ? top_p * (X + eps) * 1.005 : 0.0);
    uint32_t first = kDeepBins - 1;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      cb += c4[q];
      mb += m4[q];
      const bool hit = topk ? (cb >= k) : (need_total && mb >= target);
      if (hit) first = min(first, tid * kDPer + q);
    }
    uint32_t bc = block_min_u32<kWaves>(first, sh.red_u);
    if (!topk && has_floor) bc = min(bc, bin_of(key_value(fk)));
    if (tid == 0) {
      sh.keep = bc;
      sh.pick = 0;
    }
  }
  __syncthreads();
  const uint32_t bc = sh.keep;

  // Pass 2: every value in bins 0..bc, into bufA (any order): 16 values per thread per step,
  // placed by ballots with one LDS atomic per wave and step.
  {
    constexpr uint32_t kStep = 16 * kThreads;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (uint32_t b0 = 0; b0 < n; b0 += kStep) {
      float q[16];
      uint32_t idx[16], hc16[16];
      if (vec && b0 + kStep <= n) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        f32x4 t[4];
        u32x4 k[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t e = b0 + (j * kThreads + tid) * 4;
          t[j] = *reinterpret_cast<const f32x4*>(x + e);
          k[j] = pcnt ? *reinterpret_cast<const u32x4*>(pcnt + e) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            q[4 * j + c] = t[j][c];
            hc16[4 * j + c] = k[j][c];
            idx[4 * j + c] = b0 + (j * kThreads + tid) * 4 + c;
          }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          idx[j] = b0 + j * kThreads + tid;
          q[j] = (idx[j] < n) ? x[idx[j]] : 0.0f;
          hc16[j] = (pcnt && idx[j] < n) ? pcnt[idx[j]] : 0u;
        }
      }
      uint32_t keys[16];
      uint64_t m[16];
      uint32_t tot = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        keys[j] = (idx[j] < n) ? total_key(q[j]) : 0u;
        const bool take = idx[j] < n && hc16[j] == 0 && bin_of(q[j]) <= bc;
        m[j] = __ballot(take);
        tot += (uint32_t)__popcll(m[j]);
      }
      uint32_t base = 0;
      if (lane == 0 && tot) base = atomicAdd(&sh.pick, tot);
      base = __shfl(base, 0, kWave);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if ((m[j] >> lane) & 1ull) bufA[base + __popcll(m[j] & below)] = pack(keys[j], idx[j]);
        base += (uint32_t)__popcll(m[j]);
      }
    }
    if (pen) {
      // Each history id once more, penalised, by the thread that clears its count's top bit.
      auto hist_two = [&](uint32_t id) {
        if (id >= n) return;
        const uint32_t old = atomicAnd(&cnt[id], 0x7fffffffu);
        if (!(old & 0x80000000u)) return;
        const float v = penalize(x[id], old & 0x7fffffffu, p);
        if (bin_of(v) <= bc) bufA[atomicAdd(&sh.pick, 1u)] = pack(total_key(v), id);
      };
      for (uint32_t h = hb + tid; h < he; h += kThreads) hist_two(gload(a.hist_ids + h));
      for (uint32_t h = tid; h < extra; h += kThreads) hist_two(gload(a.extra_ids + h));
    }
  }
  __syncthreads();
  const uint32_t D = sh.pick;
  const bool complete = (D == n);

  // Bucket sort of bufA[0..D) into rank order (through bufB): kDeepBins value buckets over the range
  // the collected values span (monotone in the value, so bucket order is rank order).
  uint32_t kmin = 0xFFFFFFFFu;
  for (uint32_t i = tid; i < D; i += kThreads) kmin = min(kmin, (uint32_t)(bufA[i] >> 32));
  kmin = block_min_u32<kWaves>(kmin, sh.red_u);
  const float span2 = topf - key_value(kmin);
  const float bsc2 = span2 > 0.0f ? (float)(kDeepBins - 1) / span2 : 0.0f;
  auto bin_p = [&](uint64_t x) {
    const float t = (topf - packed_value(x)) * bsc2;
    return t < (float)(kDeepBins - 1) ? (uint32_t)t : kDeepBins - 1;
  };
  {
    for (uint32_t b = tid; b < kDeepBins; b += kThreads) hc[b] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < D; i += kThreads) atomicAdd(&hc[bin_p(bufA[i])], 1u);
    __syncthreads();
    // Exclusive scan of the kDeepBins counts: kDPer per thread, then the block.
    constexpr int kDPer = kDeepBins / kThreads;
    uint32_t* bs = hc + kDeepBins;  // bucket starts (over hm's space)
    uint32_t c4[kDPer], run = 0, big = 0;
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      c4[q] = hc[tid * kDPer + q];
      big = max(big, c4[q]);
      run += c4[q];
    }
    uint32_t all;
    uint32_t off = block_exclusive_scan_u32(run, sh.red_u, &all);
#pragma unroll
    for (int q = 0; q < kDPer; ++q) {
      bs[tid * kDPer + q] = off;
      off += c4[q];
    }
    big = block_max_u32<kWaves>(big, sh.red_u);
    if (big > kDeepBucketMax) return false;  // heavy ties: the exact-order path's stable sort
    // Scatter: a value's slot in its bucket from an LDS counter (reusing the counts, now zeroed
    // by subtraction as slots are taken).
    for (uint32_t i = tid; i < D; i += kThreads) {
      const uint64_t v = bufA[i];
      const uint32_t b = bin_p(v);
      const uint32_t slot = atomicSub(&hc[b], 1u) - 1u;
      bufB[bs[b] + slot] = v;
    }
    __syncthreads();
    for (uint32_t i = tid; i < D; i += kThreads) {
      const uint64_t v = bufB[i];
      const uint32_t b = bin_p(v);
      const uint32_t s0 = bs[b];
      const uint32_t e0 = (b + 1 < kDeepBins) ? bs[b + 1] : D;
      uint32_t r = 0;
      for (uint32_t j = s0; j < e0; ++j) r += (bufB[j] > v) ? 1u : 0u;
      bufA[s0 + r] = v;
    }
    __syncthreads();
  }
  auto val_at = [&](uint32_t j) -> double { return (double)packed_value(bufA[j]); };

  // The exact total: exp_core per value streamed (arguments at or below -512 give terms under
  // 1e-222 of a total of at least 1, left out, far inside eps), then the history ids penalised (each
  // claimed by setting its count's top bit, which pass 2 cleared). One loop per case, so that no
  // division is evaluated where none is needed.
  auto exact_total = [&]() {
    const uint64_t* t = shm().tab;
    double acc = 0.0;
    if (unfiltered) {
      for_each_value(x, pcnt, n, vec, [&](uint32_t, float v, uint32_t c) {
        if (__builtin_expect(c == 0, 1)) {
          const double d = __ddiv_rn(__dsub_rn((double)v, top), temp);
          acc = __dadd_rn(acc, d > -512.0 ? as_exp::exp_core(t, d) : 0.0);
        }
      });
    } else {
      for_each_value(x, pcnt, n, vec, [&](uint32_t, float v, uint32_t c) {
        if (__builtin_expect(c == 0, 1)) {
          const double d = __dsub_rn((double)v, top);
          acc = __dadd_rn(acc, d > -512.0 ? as_exp::exp_core(t, d) : 0.0);
        }
      });
    }
    if (pen) {
      auto hist_three = [&](uint32_t id) {
        if (id >= n) return;
        const uint32_t old = atomicOr(&cnt[id], 0x80000000u);
        if (old & 0x80000000u) return;
        double d = __dsub_rn((double)penalize(x[id], old, p), top);
        if (unfiltered) d = __ddiv_rn(d, temp);
        acc = __dadd_rn(acc, as_exp::exp_with(t, d));
      };
      for (uint32_t h = hb + tid; h < he; h += kThreads) hist_three(gload(a.hist_ids + h));
      for (uint32_t h = tid; h < extra; h += kThreads) hist_three(gload(a.extra_ids + h));
    }
    X = block_sum_f64<kWaves>(acc, sh.red_d);
    eps = kU * 1.02 * ((double)n + (double)(n / kThreads) + 32.0) * X;
    exact = true;
    return X - eps > 0.0 && eps == eps;
  };

  // The cut.
  uint32_t keep = kNone;
  if (topk) {
    keep = k;
    if (p.top_p < 1.0f) {
      const double Tk = stream_scan(sh, bufA, k, w_one, [](uint32_t, uint32_t, const double*, double) { return false; });
      const double ek = Tk * (gamma_n((double)k) + 2.0 * gamma_n(80.0) + 4.0 * kU);
      uint32_t jl, jh;
      stream_cross(sh, bufA, k, w_one, Tk, ek, top_p, &jl, &jh);
      if (jl == jh) keep = (jl < k) ? jl + 1 : k;
      else return false;
    }
    if (has_floor) {
      uint32_t first = keep;
      for (uint32_t j = tid; j < keep; j += kThreads)
        if (!(val_at(j) >= floor)) first = min(first, j);
      keep = block_min_u32<kWaves>(first, sh.red_u);
    }
  } else if (cuts) {
    uint32_t im = D;
    if (has_floor) {
      uint32_t first = D;
      for (uint32_t j = tid; j < D; j += kThreads)
        if (!(val_at(j) >= floor)) first = min(first, j);
      im = block_min_u32<kWaves>(first, sh.red_u);
    }
    const bool im_exact = (im < D) || complete;
    for (;;) {
      uint32_t jl = D, jh = D;
      if (p.top_p < 1.0f) stream_cross(sh, bufA, D, w_one, X, eps, top_p, &jl, &jh);
      if (im_exact && im <= jl) keep = im;
      else if (jl < D && jl == jh) keep = jh + 1;
      else if (jl == D && complete) keep = n;
      else if (!exact && p.top_p < 1.0f) {
        if (!exact_total()) return false;
        continue;
      } else return false;
      break;
    }
  }

  // The draw.
  uint32_t pick;
  double tot;
  if (unfiltered) {
    for (;;) {
      const uint32_t j = stream_draw(sh, bufA, D, w_temp, sh.u01 * (X - eps) * (1.0 - 3.0 * kU),
                                     sh.u01 * (X + eps) * (1.0 + 3.0 * kU));
      if (j != kNone && j < D) pick = j;
      else if (j == D && complete) pick = n - 1;
      else if (!exact) {
        if (!exact_total()) return false;
        continue;
      } else return false;
      break;
    }
    keep = n;
    tot = X;
  } else {
    const double Sk = stream_scan(sh, bufA, keep, w_temp, [](uint32_t, uint32_t, const double*, double) { return false; });
    const double d = gamma_n((double)keep) + 2.0 * gamma_n(80.0) + 4.0 * kU;
    const uint32_t j = stream_draw(sh, bufA, keep, w_temp, sh.u01 * Sk * (1.0 - d), sh.u01 * Sk * (1.0 + d));
    if (j == kNone) return false;
    pick = (j < keep) ? j : keep - 1;
    tot = Sk;
  }
  if (tid == 0) {
    a.tokens[row] = packed_id(bufA[pick]);
    a.status[row] = AS_ROW_OK | AS_ROW_DEEP_PATH;
    if (a.kept_count) a.kept_count[row] = keep;
  }
  if (a.kept_ids) {
    const uint32_t m = min(min(keep, a.kept_cap), D);
    for (uint32_t j = tid; j < m; j += kThreads) {
      a.kept_ids[(uint64_t)row * a.kept_cap + j] = packed_id(bufA[j]);
      if (a.kept_probs) a.kept_probs[(uint64_t)row * a.kept_cap + j] = __ddiv_rn(w_temp(val_at(j)), tot);
    }
  }
  return true;
}

// --- the draw's unsorted tail --------------------------------------------------------------------
//
// Bounds [sh.w_lo, sh.w_hi] on W, the sum of exp((l - top) / T) over S: the row's values that rank below
// R and are >= fl (min-p's floor as an f32, or -inf), and [sh.m_lo, sh.m_hi] on M, the sum of
// exp(l - top) over S. One pass over the row; the history's ids are
// marked in an LDS bitmap and counted in an LDS hash, left out of the stream and added penalised.
// Each term comes from the hardware's exp2: for |t| <= 126 its error (the instruction's, and four
// roundings of t of 2^-24 |t| each) is below 3e-5 relative, and below that terms are under 2^-126
// each; terms add in f32 in runs of at most 16 (under 1e-6 relative), then in f64. Returns false when
// the history does not fit the tables.
constexpr uint32_t kTailHash = 1024;

__device__ __noinline__ bool tail_sums(const FinishArgs& a, const RowParams& p, uint32_t row, uint64_t R,
                                       float fl, float topf) {
  Shared& sh = shm();
  const uint32_t n = a.n, tid = threadIdx.x;
  const float* x = a.logits + (uint64_t)row * a.row_stride;
  uint32_t hb;
  const uint32_t he = history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  // The bitmap over sh.wd, the hash over the sort's bucket tables (both free here).
  uint32_t* bm = reinterpret_cast<uint32_t*>(sh.wd);
  uint32_t* hid = sh.bcnt;
  uint32_t* hcnt = sh.bstart;
  static_assert(kTailHash <= sizeof(sh.bcnt) / 4 && kTailHash <= sizeof(sh.bstart) / 4, "hash room");
  if (pen) {
    const uint32_t words = (n + 31) / 32;
    if (words > sizeof(sh.wd) / 4) return false;
    for (uint32_t i = tid; i < words; i += kThreads) bm[i] = 0;
    for (uint32_t i = tid; i < kTailHash; i += kThreads) {
      hid[i] = kNone;
      hcnt[i] = 0;
    }
    if (tid == 0) sh.tail_over = 0;
    __syncthreads();
    auto mark = [&](uint32_t id) {
      if (id >= n) return;
      atomicOr(&bm[id >> 5], 1u << (id & 31u));
      uint32_t h = (id * 0x9E3779B1u) >> (32 - 10);
      static_assert(kTailHash == 1u << 10, "the hash's top bits");
      for (uint32_t probe = 0; probe < kTailHash; ++probe) {
        const uint32_t prev = atomicCAS(&hid[h], kNone, id);
        if (prev == kNone || prev == id) {
          atomicAdd(&hcnt[h], 1u);
          return;
        }
        h = (h + 1) & (kTailHash - 1);
      }
      sh.tail_over = 1;
    };
    for (uint32_t h = hb + tid; h < he; h += kThreads) mark(gload(a.hist_ids + h));
    for (uint32_t h = tid; h < extra; h += kThreads) mark(gload(a.extra_ids + h));
    __syncthreads();
    if (sh.tail_over) return false;
  }
  // In S: v >= fl, and v ranks below R: v < R's value, or (rarely) equal to it and below in the
  // packed order (which also orders -0 below +0).
  const float rv = key_value((uint32_t)(R >> 32));
  const float s1 = 1.44269502f, sw = (1.0f / p.temp) * s1;
  double w = 0.0, m = 0.0;
  // v's terms into (tw, tm) when v is in S.
  auto term = [&](float v, uint32_t id, float& tw, float& tm) {
    bool in = v >= fl && v < rv;
    if (__builtin_expect(v == rv, 0)) in = v >= fl && pack(total_key(v), id) < R;
    if (in) {
      const float d = v - topf;
      tw += __builtin_amdgcn_exp2f(d * sw);
      tm += __builtin_amdgcn_exp2f(d * s1);
    }
  };
  auto one = [&](float v, uint32_t id) {
    float tw = 0.0f, tm = 0.0f;
    term(v, id, tw, tm);
    w += (double)tw;
    m += (double)tm;
  };
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  auto masked = [&](uint32_t i) { return pen && ((bm[i >> 5] >> (i & 31u)) & 1u); };
  if (a.vec && a.row_stride % 4 == 0) {
    // 16-byte groups, kG per thread per batch, two batches in flight: batch b+1's loads are issued
    // before batch b is summed.
    constexpr uint32_t kG = 4, kS = kG * kThreads;
    const uint32_t ng = n / 4;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x);
    f32x4 qa[kG], qb[kG];
    auto load = [&](f32x4 (&q)[kG], uint32_t g0) {
#pragma unroll
      for (uint32_t k = 0; k < kG; ++k) {
        const uint32_t g = g0 + k * kThreads + tid;
        q[k] = (g < ng) ? xv[g] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    };
    auto sum = [&](const f32x4 (&q)[kG], uint32_t g0) {
      float tw = 0.0f, tm = 0.0f;
#pragma unroll
      for (uint32_t k = 0; k < kG; ++k) {
        const uint32_t g = g0 + k * kThreads + tid;
        const uint32_t mask = (g >= ng) ? 15u : pen ? (bm[g >> 3] >> ((4 * g) & 31u)) & 15u : 0u;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (!((mask >> c) & 1u)) term(q[k][c], 4 * g + c, tw, tm);
      }
      w += (double)tw;
      m += (double)tm;
    };
    load(qa, 0);
    for (uint32_t g0 = 0; g0 < ng; g0 += 2 * kS) {
      load(qb, g0 + kS);
      sum(qa, g0);
      load(qa, g0 + 2 * kS);
      sum(qb, g0 + kS);
    }
    for (uint32_t i = 4 * ng + tid; i < n; i += kThreads)
      if (!masked(i)) one(x[i], i);
  } else {
    for (uint32_t i = tid; i < n; i += kThreads)
      if (!masked(i)) one(x[i], i);
  }
  if (pen)
    for (uint32_t s = tid; s < kTailHash; s += kThreads)
      if (hid[s] != kNone) one(penalize(x[hid[s]], hcnt[s], p), hid[s]);
  w = block_sum_f64<kWaves>(w, sh.red_d);
  m = block_sum_f64<kWaves>(m, sh.red_d);
  const double flush = (double)n * 0x1p-125;
  if (tid == 0) {
    sh.w_lo = fmax(0.0, w * (1.0 - 1e-4) - flush);
    sh.w_hi = w * (1.0 + 1e-4) + flush;
    sh.m_lo = fmax(0.0, m * (1.0 - 1e-4) - flush);
    sh.m_hi = m * (1.0 + 1e-4) + flush;
  }
  __syncthreads();
  return true;
}

// The draw when neither filter stops among the P sorted values, so that the kept set runs past
// them (draw_partial, sample.rs:260-272). The draw is still settled when u falls among the sorted
// values with the unsorted tail's weight bounded. First from the sorted values alone: each unsorted
// weight is at most the last sorted one, and for T <= 1 with top-p's total known, w = e^(1/T) <=
// e * e_last^(1/T - 1) with e = exp(l - top) <= e_last, so the tail is at most e_last^(1/T - 1)
// times total1's unsorted part. When u falls within that bound of a cumulative weight, one pass
// over the row bounds S's weight W (S: the values below R, and above the floor). The kept tail is
// S's first values in rank order: its weight is at most W; all of W when only the floor cuts; and
// for T <= 1 at least K / M of W, with K the kept tail's mass at T = 1 and M S's (the ratio of the
// two weights, exp(l - top)^(1/T - 1), falls with the rank). K >= top-p's cumulative mass past the
// sorted values, or K = M when the floor cuts first. sh.x1 +- sh.eps1 is total1 and sh.r_prefix the
// sorted values' mass at T = 1 (top-p rows); with_tail: [sh.w_lo, sh.w_hi] bounds W and [sh.m_lo,
// sh.m_hi] bounds M. With bins (S's histogram, TailBins), the cut is placed
// within S by the bins' cumulative mass at T = 1: every bin whose cumulative mass stays below top-p's
// least target is kept whole, and no bin past the first whose cumulative mass reaches its largest
// target is kept at all, which bounds the kept tail's weight by sums of whole bins. Returns the rank
// drawn (P: past every sorted value; kNone: undecided); sh.sum gets the sorted weight.
__device__ __noinline__ uint32_t draw_past(const FinishArgs& a, const RowParams& p, uint32_t row, uint32_t P,
                                           bool with_tail, bool bins) {
  Shared& sh = shm();
  const double x1 = sh.x1, eps1 = sh.eps1, r_prefix = sh.r_prefix;
  const uint32_t n = a.n, tid = threadIdx.x;
  const uint64_t* tab = sh.tab;
  const double top = (double)key_value(sh.mk), temp = (double)p.temp, top_p = (double)p.top_p;
  auto val = [&](uint32_t i) -> double { return (double)packed_value(sh.sk[i]); };
  const double g40 = gamma_n(40.0), gn = gamma_n((double)n);
  // S's bins, kTailBins / kWave consecutive ones per lane of wave 0, loaded first: their latency
  // passes while the sorted values' weights are computed and scanned.
  constexpr uint32_t kBPer = as_dev::kTailBins / kWave;
  static_assert(as_dev::kTailBins % kWave == 0, "whole bins per lane");
  const bool use_bins = with_tail && bins && p.top_p < 1.0f;
  double bm[kBPer], bw[kBPer];
  if (use_bins && tid < kWave) {
    const as_dev::TailBins& tb = a.tail_bins[row];
#pragma unroll
    for (uint32_t q = 0; q < kBPer; ++q) {
      bm[q] = ld_agent(&tb.m[tid * kBPer + q]);
      bw[q] = ld_agent(&tb.w[tid * kBPer + q]);
    }
  }
  for (uint32_t i = tid; i < P; i += kThreads)
    sh.wd[i] = as_exp::exp_with(tab, __ddiv_rn(__dsub_rn(val(i), top), temp));
  __syncthreads();
  double loc[kScanPer], off;
  const double SP = prefix_scan(sh, P, loc, &off);
  double lo = 0.0, w_hi = __builtin_inf();
  if (with_tail) {
    const double w_lo = sh.w_lo, m_lo = sh.m_lo, m_hi = sh.m_hi;
    w_hi = sh.w_hi;
    // Top-p's target past the sorted values, at least kp: when S's whole mass is below it, the
    // floor cuts first (or nothing but the floor cuts) and the kept tail is all of S.
    const double kp = (p.top_p < 1.0f) ? top_p * (x1 - eps1) * (1.0 - 1e-9) - r_prefix * (1.0 + 1e-9)
                                       : __builtin_inf();
    if (m_hi < kp) {
      lo = w_lo;
    } else if (p.temp <= 1.0f) {
      const double k1 = fmin(kp, m_lo);
      if (k1 > 0.0 && m_hi > 0.0) lo = k1 / m_hi * w_lo;
    }
    if (use_bins) {
      // Top-p's target past the sorted values lies in [kp, kq]. Each bin's sums are within 1e-4
      // relative (as RowTail's) plus its flushed terms; their prefix sums add at most gamma(256).
      // On wave 0: b_min, the first bin whose cumulative mass can reach kp (the bins before it are
      // kept whole); b_max, the first whose cumulative mass surely reaches kq (no later bin is kept).
      if (tid < kWave) {
        const double kq = top_p * (x1 + eps1) * (1.0 + 1e-9) - r_prefix * (1.0 - 1e-9);
        const double fl_b = (double)n * 0x1p-125, slack = 1e-4 + gamma_n(300.0);
        double mhi[kBPer], mlo[kBPer], whi[kBPer], wlo[kBPer], rh = 0.0, rl = 0.0;
#pragma unroll
        for (uint32_t q = 0; q < kBPer; ++q) {
          mlo[q] = fmax(0.0, bm[q] * (1.0 - slack) - fl_b);
          mhi[q] = bm[q] * (1.0 + slack) + fl_b;
          wlo[q] = fmax(0.0, bw[q] * (1.0 - slack) - fl_b);
          whi[q] = bw[q] * (1.0 + slack) + fl_b;
          rh = __dadd_rn(rh, mhi[q]);
          rl = __dadd_rn(rl, mlo[q]);
          mhi[q] = rh;  // the lane's inclusive prefixes
          mlo[q] = rl;
        }
        // The lanes before this one, by an inclusive scan over the lanes.
        const double ih = wave_scan_f64(rh), il = wave_scan_f64(rl);
        const double eh = wave_prev_f64(ih), el = wave_prev_f64(il);
        uint32_t a_min = kNone, a_max = kNone;
#pragma unroll
        for (uint32_t q = 0; q < kBPer; ++q) {
          const uint32_t b = tid * kBPer + q;
          if (a_min == kNone && __dadd_rn(eh, mhi[q]) >= kp) a_min = b;
          if (a_max == kNone && __dadd_rn(el, mlo[q]) >= kq) a_max = b;
        }
        const uint32_t b_min = wave_min_u32(a_min), b_max = wave_min_u32(a_max);
        double before = 0.0, upto = 0.0;
#pragma unroll
        for (uint32_t q = 0; q < kBPer; ++q) {
          const uint32_t b = tid * kBPer + q;
          before += b < b_min ? wlo[q] : 0.0;
          upto += (b_max != kNone && b <= b_max) ? whi[q] : 0.0;
        }
        before = wave_sum_f64(before);
        upto = wave_sum_f64(upto);
        if (tid == 0) {
          sh.dp_lo = fmax(lo, before * (1.0 - gamma_n(300.0)));
          sh.dp_hi = b_max != kNone ? fmin(w_hi, upto * (1.0 + gamma_n(300.0))) : w_hi;
        }
      }
      __syncthreads();
      lo = sh.dp_lo;
      w_hi = sh.dp_hi;
    }
  }
  double tail = (double)(n - P) * sh.wd[P - 1] * (1.0 + 4.0 * kU);
  if (p.top_p < 1.0f && p.temp <= 1.0f) {
    // e_last^(1/T - 1) = exp(d (1/T - 1)), d = l_last - top (exact in f64): the product's rounding
    // and the exp's move the bound by far less than its 1e-9 margin.
    const double d = __dsub_rn(val(P - 1), top);
    const double rest = (x1 + eps1) - r_prefix * (1.0 - 2.0 * g40);
    const double t2 = as_exp::exp_with(tab, d * (1.0 / temp - 1.0)) * (1.0 + 1e-9) * (rest > 0.0 ? rest : 0.0);
    if (t2 < tail) tail = t2;
  }
  tail = fmin(tail, w_hi);
  const double slo = (SP * (1.0 - g40 - 4.0 * kU) + lo) * (1.0 - gn);
  const double shi = (SP * (1.0 + g40 + 4.0 * kU) + tail) * (1.0 + gn);
  const uint32_t j = decide_draw(sh, P, loc, off, sh.u01 * slo * (1.0 - 3.0 * kU), sh.u01 * shi * (1.0 + 3.0 * kU));
  if (tid == 0) sh.sum = SP;
  return j;
}

// --- S's sums in the finish kernel ---------------------------------------------------------------
//
// A min-p row without a top-k whose scan did not keep every value above its floor (a slice flagged
// it in the call's TailList) may need the weights of S, the values ranking below the candidates'
// bound R and at or above the floor: W = sum of exp((l - top) / T), M = sum of exp(l - top), |S|,
// S's histogram (TailBins) and, when S is small, its values (in the row's scratch). The flagged rows
// are cut into parts of kTailLen values, item i being part i mod parts of the list's row i / parts.
// The H workgroups whose row is not flagged (and those past the call's rows) are the helpers: helper
// h takes items h, h + H, ..., first of all (tail_help), once it has claimed that set by raising
// its claim word to the call's number (an atomic max: a lower number is an earlier call's; the
// claim is issued with the first item's loads and checked before anything is written). A flagged
// row's workgroup, when it needs the sums (tail_wait), claims the sets holding its row's items that
// no helper has claimed (helpers not yet running) and takes them itself, then waits only for sets
// that running workgroups hold. With no helper, each flagged row takes its own items. An item adds
// its sums with device atomics and stores its values with device-coherent stores, and counts itself
// in RowTail::ended once they are complete; the row's workgroup reads them with device-coherent
// loads, and clears them after its row (tail_end).

// An item's tables, over sh.wd (free whenever an item runs: before the row's work, or while its
// workgroup waits with the row's candidates in sh.sk).
constexpr uint32_t kPartHash = 512;   // distinct history ids in a part
constexpr uint32_t kTailStage = 2048; // values of S a part stages before they go to scratch
struct TailLds {
  double bin_m[kTailBins];
  double bin_w[kTailBins];
  float vals[as_launch::kTailLen];  // the part's raw values (the history's are read here)
  uint32_t bitmap[as_launch::kTailLen / 32];
  uint32_t hid[kPartHash];
  uint32_t hcnt[kPartHash];
  uint64_t stage[kTailStage];
  double red_w[kWaves], red_m[kWaves];
  uint32_t red_c[kWaves];
  uint32_t overflow, staged, base, skip, top, bad;
  uint64_t R;
};
static_assert(sizeof(TailLds) <= sizeof(double) * kCap, "an item's tables fit in sh.wd");
static_assert(as_launch::kTailLen % (4 * kThreads) == 0, "whole 16-byte groups per thread");
static_assert(kPartHash % kWave == 0 && kPartHash <= (uint32_t)kThreads, "whole waves take the history's slots, one each");

// One item: part `part` of flagged row `row`. With `claim`, thread 0 first claims the helper's set
// through that word; the claim is lost (returns false, nothing written) when a flagged row's
// workgroup took the set first. Loads that need only the row go out at once (the claim, the part's
// values, the row's parameters, history bounds and slice statistics), then the history's ids (whose
// raw values are read from the part's values, staged in LDS). S's count is reserved in the row's
// list while the terms are computed.
__device__ __noinline__ bool tail_item(const FinishArgs& a, uint32_t row, uint32_t part, uint64_t* claim) {
  Shared& sh = shm();
  TailLds& t = *reinterpret_cast<TailLds*>(sh.wd);
  constexpr uint32_t kLen = as_launch::kTailLen, kPer = kLen / kThreads;
  const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const uint32_t n = a.n, b0 = part * kLen, b1 = min(b0 + kLen, n), len = b1 - b0;
  const float* x = a.logits + (uint64_t)row * a.row_stride;
  const bool vec = a.vec && a.row_stride % 4 == 0 && len == kLen;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  uint64_t old = 0;
  if (claim && tid == 0)
    old = __hip_atomic_fetch_max(gp(claim), a.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Value k of this thread is at offset at(k) of the part.
  auto at = [&](uint32_t k) { return vec ? ((k / 4) * kThreads + tid) * 4 + (k % 4) : k * kThreads + tid; };
  float v[kPer];
  if (vec) {
#pragma unroll
    for (uint32_t j = 0; j < kPer / 4; ++j) {
      const f32x4 q = gload(reinterpret_cast<const f32x4*>(x + b0 + (j * kThreads + tid) * 4));
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * j + c] = q[c];
    }
  } else {
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) v[k] = at(k) < len ? gload(x + b0 + at(k)) : 0.0f;
  }
  const RowParams& p = a.params[row];
  uint32_t hb;
  const uint32_t he = as_launch::history_bounds(a, p, row, &hb);
  const uint32_t extra = a.extra_ids ? p.extra : 0;
  const bool pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  // The row's largest value and bound, and whether its statistics are whole, from its slices.
  uint32_t top = 0, bad = 0;
  uint64_t bound = 0;
  for (uint32_t s = tid; s < a.n_seg; s += kThreads) {
    const SegStats g = gload(a.stats + (uint64_t)row * a.n_seg + s);
    top = max(top, g.max_key);
    if (g.truncated & 1u) bound = max(bound, g.bound);
    if ((g.truncated & 2u) || g.nonfinite != kNone) bad = 1;
  }
#pragma unroll
  for (uint32_t k = 0; k < kPer; ++k)
    if (at(k) < kLen) t.vals[at(k)] = v[k];
  if (pen) {
    for (uint32_t i = tid; i < kLen / 32; i += kThreads) t.bitmap[i] = 0;
    for (uint32_t i = tid; i < kPartHash; i += kThreads) {
      t.hid[i] = kNone;
      t.hcnt[i] = 0;
    }
  }
  for (uint32_t b = tid; b < kTailBins; b += kThreads) {
    t.bin_m[b] = 0.0;
    t.bin_w[b] = 0.0;
  }
  if (tid == 0) {
    t.top = 0;
    t.bad = 0;
    t.R = 0;
    t.overflow = 0;
    t.staged = 0;
  }
  __syncthreads();
  if (tid < a.n_seg) {
    atomicMax(&t.top, top);
    if (bound) atomicMax(reinterpret_cast<unsigned long long*>(&t.R), (unsigned long long)bound);
    if (bad) t.bad = 1;
  }
  if (pen) {
    auto mark = [&](uint32_t id) {
      const uint32_t off = id - b0;
      if (off >= len) return;
      atomicOr(&t.bitmap[off >> 5], 1u << (off & 31u));
      uint32_t h = (id * 0x9E3779B1u) >> (32 - 9);
      static_assert(kPartHash == 1u << 9, "the hash's top bits");
      for (uint32_t probe = 0; probe < kPartHash; ++probe) {
        const uint32_t prev = atomicCAS(&t.hid[h], kNone, id);
        if (prev == kNone || prev == id) {
          atomicAdd(&t.hcnt[h], 1u);
          return;
        }
        h = (h + 1) & (kPartHash - 1);
      }
      t.overflow = 1;
    };
    for (uint32_t h = hb + tid; h < he; h += kThreads) mark(gload(a.hist_ids + h));
    for (uint32_t h = tid; h < extra; h += kThreads) mark(gload(a.extra_ids + h));
  }
  if (tid == 0) t.skip = (claim && old >= a.call) ? 1u : 0u;
  __syncthreads();
  if (t.skip) return false;
  RowTail& rt = a.tail[row];
  const float topf = key_value(t.top);
  const float fl = floor_f32(__dadd_rn((double)topf, p.ln_min_p));
  const uint64_t R = t.R;
  // S is defined for a min-p row without a top-k whose statistics are whole and whose bound lies
  // above its floor; otherwise the item only ends.
  const bool defined = p.mode == kModePartial && p.min_p > 0.0f && t.bad == 0u &&
                       ((uint64_t)total_key(fl) << 32) < R;
  if (defined && t.overflow == 0u) {
    // In S: v >= fl, and v ranks below R: v < R's value, or (rarely) equal to it and below in the
    // packed order (which also orders -0 below +0).
    const float rv = key_value((uint32_t)(R >> 32));
    auto in_s = [&](float val, uint32_t id) {
      bool in = val >= fl && val < rv;
      if (__builtin_expect(val == rv, 0)) in = val >= fl && pack(total_key(val), id) < R;
      return in;
    };
    bool in[kPer];
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) {
      const uint32_t off = at(k);
      const bool valid = off < len && !(pen && ((t.bitmap[off >> 5] >> (off & 31u)) & 1u));
      in[k] = valid && in_s(v[k], b0 + off);
      cnt += in[k] ? 1u : 0u;
    }
    // The history's ids in the part, penalised (one slot of the hash per thread).
    float hv = 0.0f;
    uint32_t hid = kNone;
    bool hin = false;
    if (pen && tid < kPartHash) {
      hid = t.hid[tid];
      if (hid != kNone) {
        hv = penalize(t.vals[hid - b0], t.hcnt[tid], p);
        hin = in_s(hv, hid);
        cnt += hin ? 1u : 0u;
      }
    }
    cnt = block_sum_u32<kWaves>(cnt, t.red_c);
    // The part's place in the row's list, reserved now and read once the terms are in.
    uint32_t base = 0;
    if (tid == 0) {
      base = __hip_atomic_fetch_add(gp(&rt.count), cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (cnt > kTailStage) __hip_atomic_fetch_or(gp(&rt.lost), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const float s1 = 1.44269502f, sw = (1.0f / p.temp) * s1;
    // The histogram's scale: (rv - v) * bscale is monotone in v, so bins follow the rank order.
    const float span = rv - fl;
    const float bscale = (span > 0.0f && span < __builtin_inff()) ? (float)kTailBins / span : 0.0f;
    float gw = 0.0f, gm = 0.0f;
    // Called by every lane of the wave at once: the values in S add their terms and bins, and are
    // staged with one LDS atomic per wave.
    auto add = [&](bool in_, float val, uint32_t id) {
      if (in_) {
        const float d = val - topf;
        const float tw = __builtin_amdgcn_exp2f(d * sw), tm = __builtin_amdgcn_exp2f(d * s1);
        gw += tw;
        gm += tm;
        const uint32_t b = (uint32_t)fminf((rv - val) * bscale, (float)(kTailBins - 1));
        atomicAdd(&t.bin_w[b], (double)tw);
        atomicAdd(&t.bin_m[b], (double)tm);
      }
      const uint64_t mk = __ballot(in_);
      if (mk) {
        uint32_t sbase = 0;
        if (lane == 0) sbase = atomicAdd(&t.staged, (uint32_t)__popcll(mk));
        sbase = __builtin_amdgcn_readfirstlane(sbase);
        const uint32_t i =
            sbase + __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
        if (in_ && i < kTailStage) t.stage[i] = pack(total_key(val), id);
      }
    };
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) add(in[k], v[k], b0 + at(k));
    double w = (double)gw, m = (double)gm;
    if (pen && tid < kPartHash) {
      gw = 0.0f;
      gm = 0.0f;
      add(hin, hv, hid);
      w += (double)gw;
      m += (double)gm;
    }
    // Both sums over the block in one round (wave sums, then the waves' in order).
    w = wave_sum_f64(w);
    m = wave_sum_f64(m);
    if (lane == 0) {
      t.red_w[wave] = w;
      t.red_m[wave] = m;
    }
    if (tid == 0) t.base = base;
    __syncthreads();  // also: the LDS bins and the staged values are whole
    if (tid == 0) {
      double sw_ = t.red_w[0], sm_ = t.red_m[0];
      for (int k = 1; k < kWaves; ++k) {
        sw_ = __dadd_rn(sw_, t.red_w[k]);
        sm_ = __dadd_rn(sm_, t.red_m[k]);
      }
      __hip_atomic_fetch_add(gp(&rt.w), sw_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(gp(&rt.m), sm_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(gp(&rt.parts), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The part's bins into the row's.
    as_dev::TailBins& tb = a.tail_bins[row];
    for (uint32_t b = tid; b < kTailBins; b += kThreads) {
      if (t.bin_w[b] != 0.0) __hip_atomic_fetch_add(gp(&tb.w[b]), t.bin_w[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t.bin_m[b] != 0.0) __hip_atomic_fetch_add(gp(&tb.m[b]), t.bin_m[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The staged values to scratch, at the part's place in the row's list, when the list can hold
    // them.
    const uint32_t at0 = t.base, staged = min(cnt, kTailStage);
    uint64_t* list = reinterpret_cast<uint64_t*>(a.scratch + (uint64_t)row * a.scratch_stride);
    if (at0 + staged <= kTailKeep)
      for (uint32_t i = tid; i < staged; i += kThreads) st_agent(list + at0 + i, t.stage[i]);
  } else if (defined && tid == 0) {
    __hip_atomic_fetch_or(gp(&rt.failed), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Every write above has completed (in every thread) before the item counts itself ended.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) __hip_atomic_fetch_add(gp(&rt.ended), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// First thing in every workgroup of the sliced finish, before its row: this call's flagged rows
// (the first kTailRows) and their ranks into LDS, with this row's rank (no barrier).
__device__ __forceinline__ void tail_list_load(const FinishArgs& a, uint32_t wg) {
  Shared& sh = shm();
  const uint32_t tid = threadIdx.x;
  if (tid < as_launch::kTailRows) {
    sh.tl_rows[tid] = a.tail_list->rows[tid];  // entries past the count are unused
    sh.tl_help[tid] = a.tail_list->help[tid];
    if (tid == 0) {
      sh.tl_me = wg < a.n_rows ? a.params[wg].help : 0u;
      // More flagged rows than the list holds, and no kept lists asked for: the rows past the list take
      // their own pass over the row (tail_sums), which sets the batch's time, so nothing is shared
      // (helping the listed rows would only delay every helper). With kept lists the rows past it
      // take the deep path, and the listed rows keep their parts.
      const uint32_t flagged = a.tail_list->count;
      sh.tl_n = (flagged <= as_launch::kTailRows || a.kept_ids) ? min(flagged, as_launch::kTailRows) : 0u;
      sh.tail_waited = 0;
    }
  }
}

// After a barrier that follows tail_list_load: this workgroup's row's place in the list
// (sh.tail_slot, read after later barriers), and, for a helper, its set of items, before its row. Helpers are
// numbered in the order their own work is expected to cost: the workgroups past the call's rows
// first, then the rows by RowParams::help (flagged rows left out), so that with fewer items than
// helpers the items go to the cheapest rows.
__device__ __attribute__((unused)) void tail_help(const FinishArgs& a, uint32_t wg, uint32_t groups) {
  Shared& sh = shm();
  const uint32_t nl = sh.tl_n;
  uint32_t slot = kNone;
  for (uint32_t k = 0; k < nl; ++k)
    if (sh.tl_rows[k] == wg) slot = k;
  __syncthreads();  // every thread has read sh.tl_* before thread 0 writes the slot
  if (threadIdx.x == 0) sh.tail_slot = slot;
  const uint32_t helpers = groups - nl;
  if (nl == 0 || slot != kNone || helpers == 0) return;
  const uint32_t extra = groups - a.n_rows, me = wg >= a.n_rows ? wg - a.n_rows : extra + sh.tl_me;
  uint32_t below = 0;  // flagged rows ranked before this workgroup
  for (uint32_t k = 0; k < nl; ++k) below += extra + sh.tl_help[k] < me ? 1u : 0u;
  const uint32_t parts = as_launch::tail_parts(a.n), items = nl * parts, h = me - below;
  for (uint32_t i = h; i < items; i += helpers)
    if (!tail_item(a, sh.tl_rows[i / parts], i % parts, i == h ? a.tail_claims + h : nullptr)) break;
  __syncthreads();
}

// The flagged row's workgroup: takes the sets holding its row's items that no helper has claimed
// (all its items when there is no helper), waits for the sets running helpers hold, and reads S's
// sums (within 1e-4 relative: each term is within 3e-5, and terms under 2^-126 may have flushed to
// 0). Once per row; sh.bcnt and sh.wd are free (the candidates' sort is done with them).
constexpr uint32_t kTailSpin = 1u << 24;  // a guard: every set claimed is being summed by a running workgroup
__device__ __noinline__ void tail_wait(const FinishArgs& a, uint32_t row) {
  Shared& sh = shm();
  const uint32_t tid = threadIdx.x, slot = sh.tail_slot, parts = as_launch::tail_parts(a.n);
  const uint32_t nl = sh.tl_n, items = nl * parts, helpers = gridDim.x - nl;
  if (helpers == 0) {
    for (uint32_t q = 0; q < parts; ++q) tail_item(a, row, q, nullptr);
  } else {
    // One claim per thread (the won sets listed in sh.bcnt; of two threads claiming the same set
    // only one wins), up to kThreads at a time.
    static_assert(sizeof(sh.bcnt) / 4 >= (uint32_t)kThreads, "a list slot per thread");
    for (uint32_t q0 = 0; q0 < parts; q0 += kThreads) {
      __syncthreads();
      if (tid == 0) sh.tail_won = 0;
      __syncthreads();
      const uint32_t q = q0 + tid, h = (slot * parts + q) % helpers;
      if (q < parts &&
          __hip_atomic_fetch_max(gp(a.tail_claims + h), a.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < a.call)
        sh.bcnt[atomicAdd(&sh.tail_won, 1u)] = h;
      __syncthreads();
      const uint32_t won = sh.tail_won;
      for (uint32_t k = 0; k < won; ++k) {
        const uint32_t hk = sh.bcnt[k];
        for (uint32_t i = hk; i < items; i += helpers) tail_item(a, sh.tl_rows[i / parts], i % parts, nullptr);
      }
    }
  }
  RowTail& rt = a.tail[row];
  if (tid == 0) {
    for (uint32_t k = 0; ld_agent(&rt.ended) < parts && k < kTailSpin; ++k) __builtin_amdgcn_s_sleep(2);
    const bool whole = ld_agent(&rt.ended) == parts;
    const double w = ld_agent(&rt.w), m = ld_agent(&rt.m);
    const uint32_t count = ld_agent(&rt.count), summed = ld_agent(&rt.parts);
    const uint32_t failed = ld_agent(&rt.failed), lost = ld_agent(&rt.lost);
    sh.have_tail = (whole && summed == parts && failed == 0u) ? 1u : 0u;
    const double flush = (double)a.n * 0x1p-125;
    sh.w_lo = fmax(0.0, w * (1.0 - 1e-4) - flush);
    sh.w_hi = w * (1.0 + 1e-4) + flush;
    sh.m_lo = fmax(0.0, m * (1.0 - 1e-4) - flush);
    sh.m_hi = m * (1.0 + 1e-4) + flush;
    sh.tail_count = count;
    sh.tail_listed = (lost == 0u && count <= kTailKeep) ? 1u : 0u;
    sh.tail_parts = summed;
    sh.tail_waited = 1;
  }
  __syncthreads();
}

// After a flagged row: its items have all ended (waiting for them if the row did not need them);
// its sums and bins go back to zero for the next call.
__device__ __noinline__ __attribute__((unused)) void tail_end(const FinishArgs& a, uint32_t row) {
  Shared& sh = shm();
  if (!sh.tail_waited) tail_wait(a, row);
  const uint32_t tid = threadIdx.x;
  if (tid < sizeof(RowTail) / 4) reinterpret_cast<uint32_t*>(a.tail + row)[tid] = 0u;
  if (tid < kTailBins) {
    a.tail_bins[row].m[tid] = 0.0;
    a.tail_bins[row].w[tid] = 0.0;
  }
}

// --- the kernel ---------------------------------------------------------------------------------

// The first loads of a row's workgroup, issued with the list of flagged rows (tail_list_load) before
// the barrier that follows it, so that they arrive in the same round trip: the slices' statistics,
// the exp table, the row's parameters and history bounds, and its RNG state when it draws from its
// own (a.rng_rows). A row that first takes parts of S (tail_help) then starts on them at once.
__device__ __forceinline__ void row_prefetch(const FinishArgs& a, uint32_t row) {
  Shared& sh = shm();
  const uint32_t tid = threadIdx.x;
  if (tid < 256) sh.tab[tid] = as_exp::kTable[tid];
  if (row >= a.n_rows) return;
  const SegStats* gst = a.stats + (uint64_t)row * a.n_seg;
  for (uint32_t s = tid; s < a.n_seg; s += kThreads) sh.seg[s] = gload(gst + s);
  static_assert(sizeof(RowParams) % 4 == 0 && sizeof(RowParams) / 4 <= (uint32_t)kThreads, "a word per thread");
  if (tid < sizeof(RowParams) / 4)
    reinterpret_cast<uint32_t*>(&sh.prm)[tid] = gload(reinterpret_cast<const uint32_t*>(a.params + row) + tid);
  if (a.rng_rows && tid >= 64 && tid < 68) sh.rng4[tid - 64] = gload(a.rng_state + 4ull * row + (tid - 64));
  if (tid == 96) {
    // history_bounds, without the row's parameters when the CSR offsets are given.
    uint32_t b = 0, e = 0;
    if (a.hist_ids) {
      if (a.hist_off) {
        b = a.hist_off[row];
        e = a.hist_off[row + 1];
      } else {
        const RowParams& pg = a.params[row];
        b = pg.hist_begin;
        e = pg.hist_begin + pg.hist_len;
      }
    }
    sh.pf_hb = b;
    sh.pf_he = e;
  }
}

__device__ __forceinline__ void finish_row(const FinishArgs& a, uint32_t row) {
  Shared& sh = shm();
  const uint32_t tid = threadIdx.x;
  // The slices' statistics, the exp table, the row's parameters, its history bounds and (drawing
  // from its own state) its RNG state are in LDS already (row_prefetch).
  const RowParams p = sh.prm;
  const uint32_t n = a.n;
  // S's sums: none until a flagged row waits for them (tail_wait).
  if (tid == 0) {
    sh.have_tail = 0;
    sh.tail_count = 0;
    sh.tail_listed = 0;
    sh.tail_parts = 0;
    sh.dp_pub = 0;
  }
  const bool draws = p.mode != kModeGreedy;
  uint64_t s4[4] = {0ull, 0ull, 0ull, 0ull};
  uint64_t* src = a.rng_state + 4ull * p.rng_index;
  uint32_t hb = 0, he = 0;
  if (tid == 0) {
    if (a.rng_rows) {
      for (int k = 0; k < 4; ++k) s4[k] = sh.rng4[k];
    } else if (draws) {
      for (int k = 0; k < 4; ++k) s4[k] = gload(src + k);
    }
    hb = sh.pf_hb;
    he = sh.pf_he;
  }
  __syncthreads();
  // The row's shared words go back to zero for the next call (this call's scan has ended, and their
  // words were read above).
  if (tid < sizeof(RowShare) / 4) reinterpret_cast<uint32_t*>(a.share + row)[tid] = 0u;
  const SegStats* st = sh.seg;

  if (tid < kWave) {
    // Wave 0 merges the slices' results, one slice per lane (a row has at most a few hundred): the
    // non-finite index and the largest key by reductions, the greedy pick by its total order (a row
    // holding a NaN or an infinity is refused before that pick matters), and each slice's first
    // candidate's place by a prefix of the counts in slice order.
    const uint32_t lane = tid;
    uint32_t bad = kNone, gi = kNone, mk = 0, trunc = 0, long_hist = 0, run = 0, vast = 0;
    float gv = 0.0f;
    uint64_t bound = 0;
    for (uint32_t b0 = 0; b0 < a.n_seg; b0 += kWave) {
      const uint32_t s = b0 + lane;
      uint32_t c = 0;
      if (s < a.n_seg) {
        const SegStats& t = st[s];
        bad = min(bad, t.nonfinite);
        greedy_merge(gv, gi, t.greedy_val, t.greedy_idx);
        mk = max(mk, t.max_key);
        c = t.n_cand;
        if (t.truncated & 1u) {
          trunc = 1;
          bound = max(bound, t.bound);
        }
        if (t.truncated & 2u) long_hist = 1;
        vast |= t.vast;
      }
      const uint32_t incl = wave_scan_u32(c);
      if (s < a.n_seg) sh.seg_off[s] = run + incl - c;
      run += wave_lane_u32(incl, kWave - 1);
    }
    bad = wave_min_u32(bad);
    mk = wave_max_u32(mk);
    trunc = wave_max_u32(trunc);
    long_hist = wave_max_u32(long_hist);
    vast = wave_max_u32(vast);
    bound = wave_max_u64(bound);
    wave_greedy(gv, gi);
    if (lane == 0) {
      sh.seg_off[a.n_seg] = run;
      sh.bad = bad;
      sh.gi = gi;
      sh.mk = mk;
      sh.total = run;
      sh.trunc = trunc;
      sh.bound_key = bound;
      sh.exact = long_hist;
      sh.vast = vast;
      sh.stats_bad = long_hist;
      sh.nsk = 0;
      sh.u01 = 0.0;
      sh.hist_over = (he - hb > a.max_history) ? he - hb : 0u;
      sh.draw_rng = (bad == kNone && draws && !sh.hist_over) ? 1u : 0u;
    }
  }
  // One unit() per sampled row (sample.rs:189, 264, 276), after the row's skipped draws: thread 0
  // advances the stream (its state loaded above) once the row's next loads are in flight, before the
  // barrier that follows them; nothing reads u01 earlier.
  auto take_u01 = [&]() {
    if (tid == 0 && sh.draw_rng) {
      for (uint32_t k = 0; k < p.rng_skip; ++k) rng_next(s4);
      sh.u01 = rng_unit(s4);
      if (p.flags & kFlagRngWrite)
        for (int k = 0; k < 4; ++k) src[k] = s4[k];
    }
  };
  __syncthreads();

  if (sh.hist_over) {
    if (tid == 0) {
      a.tokens[row] = kNone;
      a.status[row] = AS_ROW_HISTORY;
      if (a.kept_count) a.kept_count[row] = sh.hist_over;
    }
    return;
  }
  if (sh.bad != kNone) {
    if (tid == 0) {
      a.tokens[row] = kNone;
      a.status[row] = AS_ROW_NONFINITE;
      if (a.kept_count) a.kept_count[row] = sh.bad;
    }
    return;
  }
  if (p.mode == kModeGreedy && !sh.exact) {
    if (tid == 0) {
      a.tokens[row] = sh.gi;
      a.status[row] = AS_ROW_OK;
      if (a.kept_count) a.kept_count[row] = 1;
      if (a.kept_ids && a.kept_cap > 0) {
        a.kept_ids[(uint64_t)row * a.kept_cap] = sh.gi;
        if (a.kept_probs) a.kept_probs[(uint64_t)row * a.kept_cap] = 1.0;
      }
    }
    return;
  }
  // A small batch's row without a top-k (and not flagged for S's sums) may have to draw past its
  // candidates, and one whose top-k is too large for them surely does: it publishes its deep
  // histogram pass now, so that the workgroups with no row left sum it while this one sorts and
  // tries its candidates (when they settle the row, the pass goes unused).
  if (a.deep_help && !a.kept_ids && (p.mode == kModePartial || p.mode == kModeExactTopK) && !sh.stats_bad &&
      sh.tail_slot == kNone) {
    deep_publish_hist(a, row, sh.mk);
    if (tid == 0) sh.dp_pub = 1;  // read after later barriers
  }

  if ((p.mode == kModeTopK || p.mode == kModePartial) && !sh.exact) {
    const double top = (double)key_value(sh.mk);
    const double temp = (double)p.temp;
    const double top_p = (double)p.top_p;
    const bool has_floor = p.min_p > 0.0f;
    const double floor = __dadd_rn(top, p.ln_min_p);
    const uint64_t* tab = sh.tab;
    auto val = [&](uint32_t i) -> double { return (double)packed_value(sh.sk[i]); };
    auto w_temp = [&](double v) { return as_exp::exp_with(tab, __ddiv_rn(__dsub_rn(v, top), temp)); };
    auto w_one = [&](double v) { return as_exp::exp_with(tab, __dsub_rn(v, top)); };

    // The values that can matter, sorted: every value of the row ranking at or above R is a
    // candidate (R is the largest bound of a truncated segment; for a top-k row that segment also
    // holds k values >= R), and nothing below min-p's floor is ever kept.
    uint64_t R = sh.trunc ? sh.bound_key : 0ull;
    bool floor_cut = false;  // R is the floor: the value after the sorted ones is below it
    if (p.mode == kModePartial && has_floor) {
      const uint64_t F = (uint64_t)total_key(floor_f32(floor)) << 32;
      if (F >= R) {
        R = F;
        floor_cut = true;
      }
    }
    {
      // The slices' candidates ranking >= R into sh.sk, in any order: candidate g of the row is
      // slot g - seg_off[s] of slice s. Those below R (spilled before a slice's bound rose) drop.
      const uint64_t* src = a.cands + (uint64_t)row * a.n_seg * a.cand_stride;
      const uint32_t all = sh.total, lane = tid & (kWave - 1);
      constexpr int kLoad = 4;
      for (uint32_t g0 = 0; g0 < all; g0 += kLoad * kThreads) {
        uint64_t tmp[kLoad];
#pragma unroll
        for (int q = 0; q < kLoad; ++q) {
          const uint32_t g = g0 + tid + q * kThreads;
          tmp[q] = 0ull;
          if (g < all) {
            uint32_t lo = 0, hi = a.n_seg;  // seg_off[lo] <= g < seg_off[hi]
            while (hi - lo > 1) {
              const uint32_t mid = (lo + hi) / 2;
              if (sh.seg_off[mid] <= g) lo = mid;
              else hi = mid;
            }
            tmp[q] = gload(src + (uint64_t)lo * a.cand_stride + (g - sh.seg_off[lo]));
          }
        }
#pragma unroll
        for (int q = 0; q < kLoad; ++q) {
          const bool keep = tmp[q] != 0ull && tmp[q] >= R;
          const uint64_t m = __ballot(keep);
          uint32_t base = 0;
          if (lane == 0 && m) base = atomicAdd(&sh.nsk, (uint32_t)__popcll(m));
          base = __builtin_amdgcn_readfirstlane(base);
          const uint32_t pos = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
          if (keep && pos < (uint32_t)kCap) sh.sk[pos] = tmp[q];
        }
      }
      take_u01();
      __syncthreads();
    }
    const uint32_t total = min(sh.nsk, (uint32_t)kCap);
    const bool too_many = sh.nsk > (uint32_t)kCap;  // more candidates >= R than the finish holds
    // The candidates in rank order; a flagged row's parts of S are summed meanwhile, and its sums
    // are read after (tail_wait).
    uint32_t P = sort_candidates(sh, total, R, sh.mk, p.mode == kModeTopK ? p.top_k : kNone);
    if (tid == 0) sh.prefix = P;
    uint32_t keep = kNone;
    uint32_t status = AS_ROW_OK;
    bool drawn = false;
    // A row without a top-k and without kept lists first takes the fast decision, and a flagged row
    // waits for S's sums only when that does not settle it. A flagged row whose floor set is not vast
    // skips it: min-p cuts first within S, and the draw needs S's values.
    if (p.mode == kModePartial && (p.top_p < 1.0f || has_floor) && !a.kept_ids && !too_many && P > 0 &&
        P + kWaveMax <= (uint32_t)kCap && (sh.tail_slot == kNone || sh.vast))
      drawn = fast_partial(a, sh, p, P, floor_cut, &keep, &status);
    // S's listed values past the sorted candidates, not yet sorted (sorted only when the draw lands
    // past the candidates, or kept lists need them): how many, and where they start.
    uint32_t tail_unsorted = 0, sorted_p = 0;
    if (!drawn) {
      if (sh.tail_slot != kNone) tail_wait(a, row);
      // A row whose floor set S's parts listed (S: every value below R and at or above the floor),
      // and whose whole floor set's mass at T = 1 is short of top-p's target: top-p never stops inside it
      // and min-p's floor cuts first (sample.rs:237-251), so the kept set is the candidates and all of S.
      // Every value of S ranks below every candidate: S sorted on its own follows them. The
      // candidates' mass needs no order: a parallel sum of positive terms, within gamma(40) of exact,
      // and the margins below are far wider.
      bool floor_set = false;
      if (p.mode == kModePartial && has_floor && !floor_cut && !too_many && sh.have_tail && sh.tail_listed &&
          P + sh.tail_count <= (uint32_t)kCap) {
        bool cuts_first = true;
        if (p.top_p < 1.0f) {
          double X, eps;
          slices_total(a, sh, top, temp, false, &X, &eps);
          double mc = 0.0;
          for (uint32_t i = tid; i < P; i += kThreads) mc += w_one(val(i));
          mc = block_sum_f64<kWaves>(mc, sh.red_d);
          cuts_first = (X - eps > 0.0) && (eps == eps) &&
                       sh.m_hi < top_p * (X - eps) * (1.0 - 1e-9) - mc * (1.0 + 1e-9);
        }
        if (cuts_first) {
          const uint64_t* list = reinterpret_cast<const uint64_t*>(a.scratch + (uint64_t)row * a.scratch_stride);
          const uint32_t cnt = sh.tail_count;
          for (uint32_t i = tid; i < cnt; i += kThreads) sh.sk[P + i] = ld_agent(list + i);
          __syncthreads();
          if (a.kept_ids && a.kept_cap > P) {
            P += sort_candidates(sh, cnt, 0ull, (uint32_t)(R >> 32), kNone, P);
          } else {
            sorted_p = P;
            tail_unsorted = cnt;
            P += cnt;
          }
          floor_set = true;
        }
      }
      if (tid == 0) sh.prefix = P;
      const bool complete = (P == n);  // every value of the row is sorted
      // A top-k row's k best are among the sorted values only when at least k rank at or above R.
      const bool short_topk = p.mode == kModeTopK && P < p.top_k;

      double r_prefix = 0.0;  // the top-p scan's sum of exp(l - top) over the P sorted values
      double x1 = 0.0, eps1 = 0.0;  // total1 and its bound
      if (floor_set) {
        keep = P;  // every value at or above the floor
        status |= AS_ROW_TAIL_PASS;
      } else if (short_topk || too_many) {
        keep = kNone;
      } else if (p.mode == kModeTopK) {
        // draw_full_sort over the k best (sample.rs:157-197), on wave 0 from registers: top-p's cut,
        // min-p's floor (the ranks are sorted, so it keeps a prefix) and the draw, each decided by
        // bounds and by the reference's sequential folds only when the bounds cannot.
        static_assert(as_launch::kTopKMax <= kWaveMax, "one wave holds a top-k");
        static_assert(2 * kWaveMax <= (uint32_t)kCap && as_launch::kTopKMax <= (uint32_t)kThreads,
                      "the weights of a top-k, one per thread");
        const uint32_t k = p.top_k;
        topk_weights(sh.sk, k, top, temp, p.top_p < 1.0f, tab, sh.wd);
        __syncthreads();
        if (tid < kWave) {
          uint32_t kk, pick;
          double tot;
          topk_decide(sh.sk, k, top_p, p.top_p < 1.0f, has_floor, floor, sh.u01, sh.wd, &kk, &pick, &tot);
          if (tid == 0) {
            sh.keep = kk;
            sh.pick = pick;
            sh.sum = tot;
          }
        }
        __syncthreads();
        keep = sh.keep;
        drawn = true;
      } else if (p.top_p < 1.0f || has_floor) {
        // draw_partial's cut (sample.rs:230-259): the first rank below min-p's floor, or the rank at
        // which the top-p cumulative reaches top_p, whichever comes first.
        uint32_t im = P;  // first sorted rank below the floor (P: none among the sorted)
        if (has_floor && !floor_cut) {
          uint32_t first = P;
          for (uint32_t i = tid; i < P; i += kThreads)
            if (!(val(i) >= floor)) first = min(first, i);
          im = block_min_u32<kWaves>(first, sh.red_u);
        }
        // min-p's cut is known exactly when it falls among the sorted values, or right after them.
        const bool im_exact = (im < P) || floor_cut;
        uint32_t jl = P, jh = P;  // top-p: possible and certain trigger ranks among the sorted
        bool ok = true;
        if (p.top_p < 1.0f) {
          // total1 = sum of exp(l - top) over the row in index order (sample.rs:218-222): the
          // segments' sums rescaled, with |result - reference's left fold| <= eps.
          double X, eps;
          slices_total(a, sh, top, temp, false, &X, &eps);
          x1 = X;
          eps1 = eps;
          ok = (X - eps > 0.0) && (eps == eps);
          if (ok) {
            for (uint32_t i = tid; i < P; i += kThreads) sh.wd[i] = w_one(val(i));
            __syncthreads();
            double loc[kScanPer], off;
            r_prefix = prefix_scan(sh, P, loc, &off);
            const double g40 = 2.0 * gamma_n(40.0);
            const double tp_lo = top_p * (X - eps), tp_hi = top_p * (X + eps);
            uint32_t fl = P, fh = P;
            const uint32_t i0 = tid * kScanPer;
  #pragma unroll
            for (int q = 0; q < kScanPer; ++q) {
              const uint32_t i = i0 + q;
              if (i < P) {
                const double Rv = __dadd_rn(off, loc[q]);
                const double rel = g40 + gamma_ub(2.0 * (double)i + 4.0) + 10.0 * kU;
                // Rv / (X -+ eps) against top_p as Rv against top_p * (X -+ eps): the products'
                // roundings are within the 10 u of rel.
                if (Rv * (1.0 + rel) >= tp_lo) fl = min(fl, i);
                if (Rv * (1.0 - rel) >= tp_hi) fh = min(fh, i);
              }
            }
            jl = block_min_u32<kWaves>(fl, sh.red_u);
            jh = block_min_u32<kWaves>(fh, sh.red_u);
          }
        }
        if (!ok) {
          keep = kNone;
        } else if (im_exact && im <= jl) {
          keep = im;  // min-p's cut, at or before any rank top-p could stop at
        } else if (jl < P && jl == jh) {
          keep = jh + 1;  // top-p's cut, certainly, and min-p's comes later
        } else if (jl == P && complete) {
          keep = n;  // neither filter stops: every value
        } else if (jl == P && !im_exact && sh.have_tail && sh.tail_listed && P + sh.tail_count <= (uint32_t)kCap &&
                   sh.m_hi < (p.top_p < 1.0f ? top_p * (x1 - eps1) * (1.0 - 1e-9) - r_prefix * (1.0 + 1e-9)
                                             : __builtin_inf())) {
          // Neither filter stops among the sorted values, and S's whole mass is short of top-p's
          // target past them, so the floor cuts first: the kept set is the sorted values and all of
          // S, which S's parts listed. Sorted in with the candidates, they take the exact draw.
          const uint64_t* list = reinterpret_cast<const uint64_t*>(a.scratch + (uint64_t)row * a.scratch_stride);
          const uint32_t cnt = sh.tail_count;
          for (uint32_t i = tid; i < cnt; i += kThreads) sh.sk[P + i] = ld_agent(list + i);
          __syncthreads();
          // S ranks below every candidate: sorted on its own, it follows them.
          const uint32_t P2 = P + sort_candidates(sh, cnt, 0ull, (uint32_t)(R >> 32), kNone, P);
          if (tid == 0) sh.prefix = P2;
          keep = P2;
          status |= AS_ROW_TAIL_PASS;
          __syncthreads();
        } else if (jl == P && !im_exact && !a.kept_ids) {
          // Neither filter stops among the P sorted values: the kept set runs past them.
          if (tid == 0) {
            sh.x1 = x1;
            sh.eps1 = eps1;
            sh.r_prefix = r_prefix;
          }
          __syncthreads();
          // S's sums when the row was flagged; else the sorted values alone first, and one
          // pass over the row when they cannot settle the draw.
          uint32_t j;
          if (sh.have_tail) {
            status |= AS_ROW_TAIL_PASS;
            j = draw_past(a, a.params[row], row, P, true, true);
          } else {
            j = draw_past(a, a.params[row], row, P, false, false);
            // With the deep passes shared (a small batch), a row they would settle takes them at once
            // rather than one workgroup's pass over the row first.
            if (j == kNone && !a.deep_help &&
                tail_sums(a, a.params[row], row, R, has_floor ? floor_f32(floor) : -__builtin_inff(),
                          key_value(sh.mk))) {
              status |= AS_ROW_TAIL_PASS;
              j = draw_past(a, a.params[row], row, P, true, false);
            }
          }
          if (j != kNone && j < P) {
            if (tid == 0) sh.pick = j;  // sh.sum holds the sorted weight
            drawn = true;
            keep = P;  // a lower bound: the kept set's full size is not known
            status |= AS_ROW_KEPT_PARTIAL;
          } else {
            keep = kNone;
          }
          __syncthreads();
        } else {
          keep = kNone;
        }
      } else {
        // No filter (sample.rs:274-292): the total over the row in index order, from the segments'
        // sums with an error bound, then the first rank whose cumulative weight passes u.
        double X, eps;
        slices_total(a, sh, top, temp, true, &X, &eps);
        for (uint32_t i = tid; i < P; i += kThreads) sh.wd[i] = w_temp(val(i));
        __syncthreads();
        keep = kNone;
        if (X - eps > 0.0 && eps == eps) {
          double loc[kScanPer], off;
          prefix_scan(sh, P, loc, &off);
          const uint32_t j = decide_draw(sh, P, loc, off, sh.u01 * (X - eps) * (1.0 - 3.0 * kU),
                                         sh.u01 * (X + eps) * (1.0 + 3.0 * kU));
          uint32_t pick = kNone;
          if (j != kNone && j < P) pick = j;
          else if (j == P && complete) pick = n - 1;  // u past every cumulative: the last value
          if (pick != kNone) {
            if (tid == 0) {
              sh.pick = pick;
              sh.sum = X;
            }
            drawn = true;
            keep = n;
          }
          __syncthreads();
        }
      }

    }

    if (keep != kNone && !drawn) {
      // The draw over the kept prefix (sample.rs:184-197, 260-272): u = unit() * sum(w), then the
      // first rank whose cumulative weight exceeds u. Both sums are the reference's left folds in
      // rank order; past a few hundred tokens they come from a parallel scan with an error bound,
      // and the sequential folds run only when the bound cannot decide. S's listed values past the
      // sorted candidates add to the total in any order (the scan's bound holds for any order of
      // positive terms); they are sorted only when u lies past the candidates.
      if (tail_unsorted && keep <= 256) {
        sort_candidates(sh, tail_unsorted, 0ull, (uint32_t)(R >> 32), kNone, sorted_p);
        tail_unsorted = 0;
      }
      for (uint32_t i = tid; i < keep; i += kThreads) sh.wd[i] = w_temp(val(i));
      __syncthreads();
      if (keep > 256) {
        double loc[kScanPer], off;
        double S = prefix_scan(sh, keep, loc, &off);
        const double d = gamma_n((double)keep) + gamma_n(40.0) + 4.0 * kU;
        const uint32_t m = tail_unsorted ? sorted_p : keep;
        uint32_t j = decide_draw(sh, m, loc, off, sh.u01 * S * (1.0 - d), sh.u01 * S * (1.0 + d));
        if (tail_unsorted && j == m) {
          // u lies past every candidate: S in rank order (the sort works in sh.wd), then the draw
          // over all of it.
          sort_candidates(sh, tail_unsorted, 0ull, (uint32_t)(R >> 32), kNone, sorted_p);
          for (uint32_t i = tid; i < keep; i += kThreads) sh.wd[i] = w_temp(val(i));
          __syncthreads();
          S = prefix_scan(sh, keep, loc, &off);
          j = decide_draw(sh, keep, loc, off, sh.u01 * S * (1.0 - d), sh.u01 * S * (1.0 + d));
          tail_unsorted = 0;
        } else if (tail_unsorted && j == kNone) {
          // Undecided near a candidate: the sequential folds below need every weight in rank order.
          sort_candidates(sh, tail_unsorted, 0ull, (uint32_t)(R >> 32), kNone, sorted_p);
          for (uint32_t i = tid; i < keep; i += kThreads) sh.wd[i] = w_temp(val(i));
          __syncthreads();
          tail_unsorted = 0;
        }
        if (j != kNone) {
          if (tid == 0) {
            sh.pick = (j < keep) ? j : keep - 1;  // past every cumulative: the last kept
            sh.sum = S;
          }
          drawn = true;
        }
        __syncthreads();
      }
      if (!drawn) {
        if (tid < kWave) {
          // u = unit() * sum(w), then the first rank whose cumulative weight passes u
          // (sample.rs:184-197, 260-272), on wave 0: by bounds for up to kWaveMax kept values, else
          // (or when they cannot decide) by the reference's sequential folds.
          double tot = 0.0;
          uint32_t pick = kNone;
          if (keep <= kWaveMax) {
            const uint32_t i0 = tid * kWPer;
            double w[kWPer];
#pragma unroll
            for (int q = 0; q < kWPer; ++q) w[q] = (i0 + q < keep) ? sh.wd[i0 + q] : 0.0;
            pick = wave_draw(w, keep, sh.u01, &tot);
          }
          if (pick == kNone) pick = wave_seq_draw(sh.wd, keep, sh.u01, &tot);
          if (tid == 0) {
            sh.pick = pick;
            sh.sum = tot;
          }
        }
        __syncthreads();
      }
    }

    if (keep == kNone) {
      if (tid == 0) sh.exact = 1;
    } else {
      const uint32_t pick = sh.pick;
      const double tot = sh.sum;
      if (tid == 0) {
        a.tokens[row] = packed_id(sh.sk[pick]);
        a.status[row] = status;
        if (a.kept_count) a.kept_count[row] = keep;
      }
      if (a.kept_ids) {
        const uint32_t m = min(min(keep, a.kept_cap), sh.prefix);
        for (uint32_t j = tid; j < m; j += kThreads) {
          a.kept_ids[(uint64_t)row * a.kept_cap + j] = packed_id(sh.sk[j]);
          if (a.kept_probs) a.kept_probs[(uint64_t)row * a.kept_cap + j] = __ddiv_rn(sh.wd[j], tot);
        }
      }
    }
    __syncthreads();
  } else {
    take_u01();
    if (tid == 0) sh.exact = 1;
    __syncthreads();
  }

  if (sh.exact) {
    // Rows first try collecting only the bins their decisions fall in (kept lists need every kept
    // value in order: those rows take the full deep path). Each path is called at the same depth,
    // so that the kernel's stack is the largest of theirs, not their sum.
    __syncthreads();
    // A flagged row's parts write its scratch: they have all ended before the passes below use it.
    if (sh.tail_slot != kNone && !sh.tail_waited) tail_wait(a, row);
    const RowParams& pr = a.params[row];
    const bool pen = deep_prep(a, pr, row);
    bool done = false;
    if (!sh.stats_bad && !a.kept_ids) {
      done = a.deep_help ? deep_bins<true>(a, pr, row, pen) : deep_bins<false>(a, pr, row, pen);
      __syncthreads();
    }
    if (!done && !deep_row(a, pr, row, pen)) {
      __syncthreads();
      exact_row(a, pr, row);
    }
  }
}

}  // namespace AS_FIN_NS
}  // namespace

// The C ABI (include/artemis_sampler.h): context, argument checks, per-row parameter blocks and
// the launches. No host synchronisation except as_sync and the staging-buffer reuse wait.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/artemis_sampler.h"
#include "launch.h"
#include "sampler_device.h"

using as_dev::RowParams;
using as_dev::RowShare;
using as_dev::SegStats;
using as_launch::kArgsSlot;

struct as_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t max_rows = 0, max_vocab = 0, max_history = 0, max_seg = 0;
  RowParams* d_params = nullptr;           // after the FinishArgs slot of d_block
  as_launch::FinishArgs* d_args = nullptr;  // the start of d_block
  void* d_block = nullptr;
  // The parameter blocks d_params holds (as the host last uploaded them): a call uploads only the
  // range of rows whose blocks differ, from one of two pinned staging blocks.
  std::vector<RowParams> dev_rows;
  uint32_t dev_valid = 0;  // rows of dev_rows that hold an upload
  void* h_block[2] = {nullptr, nullptr};
  uint64_t* h_done = nullptr;  // pinned: the last call whose finish kernel has started (it writes it)
  uint64_t calls = 0;
  SegStats* d_stats = nullptr;
  RowShare* d_share = nullptr;
  as_dev::RowTail* d_tail = nullptr;
  as_dev::TailBins* d_tail_bins = nullptr;
  as_dev::TailList* d_tail_list = nullptr;  // two lists: call c takes list c mod 2
  uint64_t* d_tail_claims = nullptr;         // one per finish workgroup: max(max_rows, kTailGroups)
  as_dev::DeepJob* d_deep_jobs = nullptr;    // per row
  uint64_t* d_deep_done = nullptr;           // rows finished by calls that shared the deep passes
  uint64_t deep_rows_done = 0;               // the host's count of the same
  bool share_dirty = false;  // a scan ran without its finish (a failed launch): the context is unusable
  uint64_t* d_cands = nullptr;
  uint32_t* d_scratch = nullptr;
  uint64_t scratch_stride = 0;
  uint32_t* d_vstatus = nullptr;
  float* d_zero = nullptr;  // 1,024 zeros the scan's idle loads read
  as_launch::LpPart* d_lp = nullptr;  // log-probabilities: per row, its parts' sums and lists
  uint64_t* d_mv_partials = nullptr;  // head_argmax: each matvec workgroup's best key
  as_launch::RowOrder order{};  // the scan's row order for the current call
  std::vector<std::pair<double, uint32_t>> order_cost;  // its sort keys (kept: no allocation per call)
  std::vector<RowParams> rows;  // the call's parameter blocks as built on the host (max_rows, kept)
  std::string err;
  // Profiling: events before the scan, between the kernels and after the finish, per call, and
  // whether the call ran a finish kernel (a call the scan finishes has nothing between its last two
  // events but their own overhead, which counts as no finish time).
  bool profile = false;
  std::vector<hipEvent_t> ev;
  std::vector<uint8_t> ev_fin;
  size_t ev_used = 0;
};

namespace {

int fail(as_ctx* c, int code, const std::string& msg) {
  if (c) c->err = msg;
  return code;
}

int hip_fail(as_ctx* c, hipError_t e, const char* what) {
  return fail(c, AS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define AS_HIP(ctx, call)                                   \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, #call);  \
  } while (0)

bool penalties_on(const as_sampling& s) {
  return s.presence != 0.0f || s.frequency != 0.0f || s.repetition != 1.0f;
}

// The candidates each wave of a slice keeps for a row: top_k for a top-k row the fast path can take
// (a wave holding k values at or above a threshold proves that nothing below it is among the row's
// k best), kPartialRank for rows without a top-k, 0 for rows that keep none.
uint32_t wave_cand(uint32_t top_k) { return top_k; }
uint32_t wanted_cand(const as_sampling& s, uint32_t n) {
  if (s.temp <= 0.0f) return 0;
  if (s.top_k > 0 && s.top_k < n) return s.top_k <= as_launch::kTopKMax ? wave_cand(s.top_k) : 0;
  return as_launch::kPartialRank;
}

// How a call splits its rows: n_seg slices of slice_len values, and `stride` candidate slots per
// slice. Enough slices to give the GPU about kTargetGroups workgroups (a small batch's slices hold
// at least two chunks of 1,024 values: at batch 1, 2,048-value slices gave the call 1 us less than
// 4,096-value ones, and 16,384-value ones 2 us more; a call of greedy rows without history, which
// takes greedy_kernel, at least four: 12.8 against 13.2 us at batch 1, and 14.5 us at 16,384), no
// more than the finish kernel's candidate room allows for the largest per-wave count, and slices of
// at most kSliceMax.
struct Plan {
  uint32_t n_seg, slice_len, stride, limit;
};
Plan plan_slices(uint32_t n, uint32_t n_rows, uint32_t c_max, bool greedy_call = false) {
  const uint32_t s_min = (n + as_launch::kSliceMax - 1) / as_launch::kSliceMax;
  uint32_t s = (as_launch::kTargetGroups + n_rows - 1) / n_rows;
  s = std::min(s, std::max(1u, n / ((greedy_call ? 4 : 2) * as_launch::kSliceAlign)));
  if (c_max > 0) s = std::min(s, as_launch::kCandCap / (4 * c_max + as_launch::kHistReserve));
  s = std::min(s, as_launch::kMaxSlices);
  s = std::max(s, std::max(s_min, 1u));
  uint32_t len = (n + s - 1) / s;
  len = (len + as_launch::kSliceAlign - 1) / as_launch::kSliceAlign * as_launch::kSliceAlign;
  Plan p;
  p.slice_len = len;
  p.n_seg = (n + len - 1) / len;
  p.stride = as_launch::kCandCap / p.n_seg;
  p.limit = p.stride > as_launch::kHistReserve ? (p.stride - as_launch::kHistReserve) / 4 : 0;
  return p;
}

// The row's mode and parameter block (Sampler::sample's dispatch, sample.rs:129-150).
RowParams make_row(const as_sampling& s, uint32_t n, const Plan& pl) {
  RowParams r{};
  r.temp = s.temp;
  r.top_k = s.top_k;
  r.top_p = s.top_p;
  r.min_p = s.min_p;
  r.presence = s.presence;
  r.frequency = s.frequency;
  r.repetition = s.repetition;
  r.ln_min_p = s.min_p > 0.0f ? std::log((double)s.min_p) : 0.0;
  r.flags = penalties_on(s) ? as_dev::kFlagPenalties : 0u;
  r.cap = pl.stride;
  const uint32_t limit = pl.limit;
  if (s.temp <= 0.0f) {
    r.mode = as_dev::kModeGreedy;
    r.cand = 0;
  } else if (s.top_k > 0 && s.top_k < n) {
    if (s.top_k <= as_launch::kTopKMax && wave_cand(s.top_k) <= limit) {
      r.mode = as_dev::kModeTopK;
      r.cand = wave_cand(s.top_k);
    } else {
      r.mode = as_dev::kModeExactTopK;
      r.cand = 0;
    }
  } else {
    r.mode = as_dev::kModePartial;
    // A min-p row keeps every value above its floor: each wave keeps as many as its buffer and the
    // slice's candidate room allow, so that a floor set of a few thousand values stays whole.
    const uint32_t c = s.min_p > 0.0f ? as_launch::kFloorRank : as_launch::kPartialRank;
    r.cand = std::max(1u, std::min(c, limit));
    if (s.top_p < 1.0f)
      r.flags |= as_dev::kFlagSumTop;
    else if (!(s.min_p > 0.0f))
      r.flags |= as_dev::kFlagSumTemp;
  }
  return r;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The scan's expected cost of a row's slices, in rough units (a scheduling estimate only: it sets the
// order in which rows are launched, never what they compute). Greedy rows only stream; top-k rows
// append and select more as k grows; rows without a top-k keep more candidates and add sums, and
// min-p's floor set (all of it is kept) grows quickly as min_p falls.
double row_cost(const RowParams& r) {
  switch (r.mode) {
    case as_dev::kModeTopK:
      return 1.0 + r.top_k / 50.0;
    case as_dev::kModePartial: {
      double c = 2.0;
      if (r.min_p > 0.0f && r.min_p < 0.03f) c += 1.5;
      if (r.min_p > 0.0f && r.min_p < 0.005f) c += 1.0;
      return c;
    }
    default:
      return 0.0;
  }
}

// The costliest rows first (ties in row order), so that they get the older waves of their CU.
void order_rows(const RowParams* rows, uint32_t n_rows, as_launch::RowOrder* o,
                std::vector<std::pair<double, uint32_t>>& c) {
  o->on = 0;
  if (n_rows < 2 || n_rows > as_launch::kOrderMax) return;
  c.resize(n_rows);
  for (uint32_t r = 0; r < n_rows; ++r) c[r] = {-row_cost(rows[r]), r};
  std::stable_sort(c.begin(), c.end());
  for (uint32_t r = 0; r < n_rows; ++r) o->r[r] = (uint16_t)c[r].second;
  o->on = 1;
}

// Each row's place among the finish kernel's helpers of S's sums (RowParams::help), the rows whose own
// finish costs least first: greedy rows, then top-k rows, then rows without a top-k and without
// min-p's floor, then those with it (the ones S is summed for); in row order within a kind.
void help_ranks(const RowParams* rows, uint32_t n_rows, RowParams* out) {
  auto kind = [](const RowParams& r) -> uint32_t {
    if (r.mode == as_dev::kModeTopK) return 1;
    if (r.mode == as_dev::kModePartial) return r.min_p > 0.0f ? 3 : 2;
    return r.mode == as_dev::kModeGreedy ? 0 : 2;
  };
  uint32_t start[4] = {0, 0, 0, 0};
  for (uint32_t r = 0; r < n_rows; ++r)
    for (uint32_t k = kind(rows[r]) + 1; k < 4; ++k) ++start[k];
  for (uint32_t r = 0; r < n_rows; ++r) out[r].help = start[kind(rows[r])]++;
}

// The next profiling event (created on first use), or null when profiling is off.
hipEvent_t next_event(as_ctx* c) {
  if (!c->profile) return nullptr;
  if (c->ev_used == c->ev.size()) {
    if (c->ev.size() >= 3 * 4096) return nullptr;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    c->ev.push_back(e);
  }
  return c->ev[c->ev_used++];
}

// One call over n_rows rows. The rows' parameter blocks go to device memory only where they differ
// from the blocks already there (a copy from one of two pinned staging blocks, the host waiting only
// if the call that last used that block has not reached its finish kernel); the finish kernel's
// arguments travel as the scan's kernel argument. Nothing else crosses to the GPU before the scan.
int run_rows(as_ctx* c, const Plan& pl, RowParams* rows, const float* logits, uint64_t row_stride,
             uint32_t n, uint32_t n_rows, const uint32_t* hist_off, const uint32_t* hist_ids,
             const uint32_t* extra_ids, uint64_t* rng, uint32_t* tokens, uint32_t* status,
             uint32_t* kept_count, uint32_t* kept_ids, double* kept_probs, uint32_t kept_cap) {
  const uint32_t n_seg = pl.n_seg;
  const bool vec = aligned16(logits) && (row_stride % 4 == 0);
  if (c->share_dirty)
    return fail(c, AS_ERR_HIP, "an earlier call launched its scan but not its finish kernel: the context's "
                               "shared words are not clear; destroy it and create another");
  as_launch::FinishArgs a{};
  a.logits = logits;
  a.row_stride = row_stride;
  a.n = n;
  a.n_seg = n_seg;
  a.params = c->d_params;
  a.share = c->d_share;
  a.tail = c->d_tail;
  a.tail_bins = c->d_tail_bins;
  a.hist_off = hist_off;
  a.hist_ids = hist_ids;
  a.extra_ids = extra_ids;
  a.stats = c->d_stats;
  a.cands = c->d_cands;
  a.cand_stride = pl.stride;
  a.kept_cap = kept_cap;
  a.rng_state = rng;
  a.tokens = tokens;
  a.status = status;
  a.kept_count = kept_count;
  a.kept_ids = kept_ids;
  a.kept_probs = kept_probs;
  a.vec = vec ? 1u : 0u;
  a.scratch = c->d_scratch;
  a.scratch_stride = c->scratch_stride;
  a.done = c->h_done;
  const uint64_t call = c->calls + 1;  // committed once the scan is launched
  a.call = call;
  a.tail_list = c->d_tail_list + (call & 1);
  a.tail_next = c->d_tail_list + ((call + 1) & 1);
  a.tail_claims = c->d_tail_claims;
  a.deep_jobs = c->d_deep_jobs;
  a.deep_done = c->d_deep_done;
  a.n_rows = n_rows;
  a.max_history = c->max_history;
  bool own_states = true;
  for (uint32_t r = 0; r < n_rows && own_states; ++r) own_states = rows[r].rng_index == r;
  a.rng_rows = own_states ? 1u : 0u;
  // Every row greedy and no history: each row's last slice finishes it, and no finish kernel runs.
  bool all_greedy = !hist_ids && !extra_ids;
  for (uint32_t r = 0; r < n_rows && all_greedy; ++r) all_greedy = rows[r].mode == as_dev::kModeGreedy;
  a.scan_finishes = all_greedy ? 1u : 0u;
  // Small batches share the deep passes with idle workgroups: any row without a top-k, or with one
  // too large for the slices' candidates, may take them (rows with kept lists take the full deep
  // path, which is not shared).
  bool deep_rows = false;
  for (uint32_t r = 0; r < n_rows; ++r)
    deep_rows = deep_rows || rows[r].mode == as_dev::kModePartial || rows[r].mode == as_dev::kModeExactTopK;
  a.deep_help = (n_rows <= as_launch::kDeepHelpRows && !kept_ids && deep_rows) ? 1u : 0u;
  const uint64_t deep_target = c->deep_rows_done + (a.deep_help ? n_rows : 0u);
  a.deep_target = deep_target;

  // The range of rows whose blocks differ from the device's.
  help_ranks(rows, n_rows, rows);
  uint32_t lo = n_rows, hi = 0;
  for (uint32_t r = 0; r < n_rows; ++r)
    if (r >= c->dev_valid || std::memcmp(&rows[r], &c->dev_rows[r], sizeof(RowParams)) != 0) {
      lo = std::min(lo, r);
      hi = r + 1;
    }
  if (lo < hi) {
    // Staging block b was last filled by call `call - 2` or earlier, whose finish kernel writes its
    // number once that upload is over. Waits while the GPU works through the calls before it; past
    // 50 ms (a stream held up elsewhere) it waits for the stream instead.
    const int b = (int)(call & 1);
    if (call > 2 && __atomic_load_n(c->h_done, __ATOMIC_ACQUIRE) < call - 2) {
      const auto t0 = std::chrono::steady_clock::now();
      while (__atomic_load_n(c->h_done, __ATOMIC_ACQUIRE) < call - 2) {
        if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(50)) {
          AS_HIP(c, hipStreamSynchronize(c->stream));
          break;
        }
      }
    }
    RowParams* h = static_cast<RowParams*>(c->h_block[b]);
    std::memcpy(h + lo, rows + lo, sizeof(RowParams) * (hi - lo));
    AS_HIP(c, hipMemcpyAsync(c->d_params + lo, h + lo, sizeof(RowParams) * (hi - lo), hipMemcpyHostToDevice,
                             c->stream));
    std::memcpy(&c->dev_rows[lo], rows + lo, sizeof(RowParams) * (hi - lo));
    c->dev_valid = std::max(c->dev_valid, hi);
  }

  hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr;
  if (c->profile && c->ev_used + 3 <= 3 * 4096) {
    e0 = next_event(c);
    e1 = next_event(c);
    e2 = next_event(c);
  }
  if (e0) AS_HIP(c, hipEventRecord(e0, c->stream));
  order_rows(rows, n_rows, &c->order, c->order_cost);
  AS_HIP(c, as_launch::scan(c->stream, vec, logits, c->d_zero, row_stride, n, n_rows, n_seg, pl.slice_len,
                            c->d_params, a, c->d_args, c->d_share, hist_off, hist_ids, extra_ids, c->d_stats,
                            c->d_cands, pl.stride, a.tail_list, c->order));
  // The scan is queued: from here the call's numbers are the context's.
  c->calls = call;
  c->deep_rows_done = deep_target;
  if (!a.scan_finishes) c->share_dirty = true;
  if (e1) AS_HIP(c, hipEventRecord(e1, c->stream));
  if (e0) c->ev_fin[(c->ev_used - 3) / 3] = a.scan_finishes ? 0 : 1;
  if (a.scan_finishes) {
    if (e2) AS_HIP(c, hipEventRecord(e2, c->stream));
    return AS_OK;
  }
  // Only rows without a top-k that have min-p's floor can be flagged for S's sums: with any, the
  // finish kernel runs enough workgroups to take their parts at once.
  uint32_t floor_rows = 0;
  for (uint32_t r = 0; r < n_rows; ++r)
    floor_rows += (rows[r].mode == as_dev::kModePartial && rows[r].min_p > 0.0f) ? 1u : 0u;
  const uint32_t tail_items = std::min(floor_rows, as_launch::kTailRows) * as_launch::tail_parts(n);
  uint32_t groups = std::max(n_rows, std::min(tail_items, as_launch::kTailGroups));
  if (a.deep_help) groups = std::max(groups, as_launch::kTailGroups);
  AS_HIP(c, as_launch::finish(c->stream, groups, c->d_args));
  c->share_dirty = false;
  if (e2) AS_HIP(c, hipEventRecord(e2, c->stream));
  return AS_OK;
}

}  // namespace

extern "C" {

int as_check(const as_sampling* p, char* msg, size_t cap) {
  char buf[160];
  buf[0] = 0;
  if (!p) {
    std::snprintf(buf, sizeof buf, "no sampling settings");
  } else if (!(std::isfinite(p->temp) && p->temp >= 0.0f)) {
    std::snprintf(buf, sizeof buf, "--temp %g must be a finite number, 0 or more", p->temp);
  } else if (!(p->top_p > 0.0f && p->top_p <= 1.0f)) {
    std::snprintf(buf, sizeof buf, "--top-p %g must be above 0 and at most 1", p->top_p);
  } else if (!(p->min_p >= 0.0f && p->min_p <= 1.0f)) {
    std::snprintf(buf, sizeof buf, "--min-p %g must be from 0 to 1", p->min_p);
  } else if (!std::isfinite(p->presence)) {
    std::snprintf(buf, sizeof buf, "--presence-penalty %g must be a finite number", p->presence);
  } else if (!std::isfinite(p->frequency)) {
    std::snprintf(buf, sizeof buf, "--frequency-penalty %g must be a finite number", p->frequency);
  } else if (!(std::isfinite(p->repetition) && p->repetition > 0.0f)) {
    std::snprintf(buf, sizeof buf, "--repetition-penalty %g must be a finite number above 0",
                  p->repetition);
  }
  if (msg && cap) {
    std::strncpy(msg, buf, cap - 1);
    msg[cap - 1] = 0;
  }
  return buf[0] ? AS_ERR_PARAMS : AS_OK;
}

void as_rng_seed(uint64_t seed, uint64_t state[4]) {
  uint64_t x = seed;
  for (int i = 0; i < 4; ++i) {
    x += 0x9E3779B97F4A7C15ull;
    uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    state[i] = z ^ (z >> 31);
  }
}

const char* as_last_error(const as_ctx* ctx) { return ctx ? ctx->err.c_str() : "no context"; }

int as_destroy(as_ctx* c) {
  if (!c) return AS_ERR_INVALID;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  (void)hipFree(c->d_block);
  (void)hipFree(c->d_stats);
  (void)hipFree(c->d_share);
  (void)hipFree(c->d_tail);
  (void)hipFree(c->d_tail_bins);
  (void)hipFree(c->d_tail_list);
  (void)hipFree(c->d_tail_claims);
  (void)hipFree(c->d_deep_jobs);
  (void)hipFree(c->d_deep_done);
  (void)hipFree(c->d_cands);
  (void)hipFree(c->d_scratch);
  (void)hipFree(c->d_vstatus);
  (void)hipFree(c->d_zero);
  (void)hipFree(c->d_lp);
  (void)hipFree(c->d_mv_partials);
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  for (int b = 0; b < 2; ++b)
    if (c->h_block[b]) (void)hipHostFree(c->h_block[b]);
  if (c->h_done) (void)hipHostFree(c->h_done);
  delete c;
  return AS_OK;
}

int as_create(int device, void* hip_stream, uint32_t max_rows, uint32_t max_vocab,
              uint32_t max_history, as_ctx** out) {
  if (!out) return AS_ERR_INVALID;
  *out = nullptr;
  if (max_rows == 0 || max_vocab == 0) return AS_ERR_INVALID;
  const uint32_t max_seg = as_launch::kMaxSlices;
  if ((uint64_t)max_vocab > (uint64_t)as_launch::kMaxSlices * as_launch::kSliceMax) return AS_ERR_CAPACITY;
  as_ctx* c = new as_ctx();
  c->device = device;
  c->stream = (hipStream_t)hip_stream;
  c->max_rows = max_rows;
  c->max_vocab = max_vocab;
  c->max_history = max_history;
  c->max_seg = max_seg;
  c->order_cost.reserve(std::min(max_rows, as_launch::kOrderMax));
  c->rows.resize(max_rows);
  c->dev_rows.resize(max_rows);
  c->ev_fin.assign(4096, 1);
  c->scratch_stride = as_launch::scratch_words(max_vocab);
  hipError_t e = hipSetDevice(device);
  if (e == hipSuccess) e = hipMalloc(&c->d_block, kArgsSlot + sizeof(RowParams) * max_rows);
  if (e == hipSuccess) {
    c->d_args = static_cast<as_launch::FinishArgs*>(c->d_block);
    c->d_params = reinterpret_cast<RowParams*>(static_cast<char*>(c->d_block) + kArgsSlot);
  }
  if (e == hipSuccess) e = hipMalloc(&c->d_stats, sizeof(SegStats) * (uint64_t)max_rows * max_seg);
  if (e == hipSuccess) e = hipMalloc(&c->d_share, sizeof(RowShare) * max_rows);
  if (e == hipSuccess) e = hipMemset(c->d_share, 0, sizeof(RowShare) * max_rows);
  if (e == hipSuccess) e = hipMalloc(&c->d_tail, sizeof(as_dev::RowTail) * max_rows);
  if (e == hipSuccess) e = hipMemset(c->d_tail, 0, sizeof(as_dev::RowTail) * max_rows);
  if (e == hipSuccess) e = hipMalloc(&c->d_tail_bins, sizeof(as_dev::TailBins) * max_rows);
  if (e == hipSuccess) e = hipMemset(c->d_tail_bins, 0, sizeof(as_dev::TailBins) * max_rows);
  if (e == hipSuccess) e = hipMalloc(&c->d_tail_list, 2 * sizeof(as_dev::TailList));
  if (e == hipSuccess) e = hipMemset(c->d_tail_list, 0, 2 * sizeof(as_dev::TailList));
  const size_t claims = sizeof(uint64_t) * std::max(max_rows, as_launch::kTailGroups);
  if (e == hipSuccess) e = hipMalloc(&c->d_tail_claims, claims);
  if (e == hipSuccess) e = hipMemset(c->d_tail_claims, 0, claims);
  if (e == hipSuccess) e = hipMalloc(&c->d_deep_jobs, sizeof(as_dev::DeepJob) * max_rows);
  if (e == hipSuccess) e = hipMemset(c->d_deep_jobs, 0, sizeof(as_dev::DeepJob) * max_rows);
  if (e == hipSuccess) e = hipMalloc(&c->d_deep_done, sizeof(uint64_t));
  if (e == hipSuccess) e = hipMemset(c->d_deep_done, 0, sizeof(uint64_t));
  if (e == hipSuccess)
    e = hipMalloc(&c->d_cands, sizeof(uint64_t) * (uint64_t)max_rows * as_launch::kCandCap);
  if (e == hipSuccess) e = hipMalloc(&c->d_scratch, sizeof(uint32_t) * (uint64_t)max_rows * c->scratch_stride);
  if (e == hipSuccess) e = hipMalloc(&c->d_vstatus, sizeof(uint32_t) * max_rows);
  if (e == hipSuccess) e = hipMalloc(&c->d_mv_partials, sizeof(uint64_t) * as_launch::kMatvecGroups);
  if (e == hipSuccess)
    e = hipMalloc(&c->d_lp, sizeof(as_launch::LpPart) * as_launch::lp_capacity(max_rows, max_vocab));
  if (e == hipSuccess) e = hipMalloc(&c->d_zero, sizeof(float) * 1024);
  if (e == hipSuccess) e = hipMemset(c->d_zero, 0, sizeof(float) * 1024);
  for (int b = 0; b < 2 && e == hipSuccess; ++b)
    e = hipHostMalloc(&c->h_block[b], sizeof(RowParams) * max_rows, hipHostMallocDefault);
  if (e == hipSuccess) e = hipHostMalloc((void**)&c->h_done, 64, hipHostMallocCoherent);
  if (e == hipSuccess) *c->h_done = 0;
  if (e != hipSuccess) {
    std::fprintf(stderr, "as_create: %s\n", hipGetErrorString(e));
    as_destroy(c);
    return AS_ERR_HIP;
  }
  *out = c;
  return AS_OK;
}

int as_sync(as_ctx* c) {
  if (!c) return AS_ERR_INVALID;
  AS_HIP(c, hipStreamSynchronize(c->stream));
  return AS_OK;
}

int as_sample(as_ctx* c, const as_batch* b, const as_sampling* params) {
  if (!c) return AS_ERR_INVALID;
  if (!b || !params) return fail(c, AS_ERR_INVALID, "as_sample: no batch or no params");
  if (b->n_rows == 0) return AS_OK;
  if (!b->logits || !b->rng_state || !b->tokens || !b->status)
    return fail(c, AS_ERR_INVALID, "as_sample: logits, rng_state, tokens and status are required");
  if (b->n_vocab == 0 || (b->row_stride != 0 && b->row_stride < b->n_vocab))
    return fail(c, AS_ERR_INVALID, "as_sample: n_vocab must be at least 1 and at most row_stride");
  if (b->n_rows > c->max_rows || b->n_vocab > c->max_vocab)
    return fail(c, AS_ERR_CAPACITY, "as_sample: more rows or a larger vocabulary than the context holds");
  if ((b->hist_ids == nullptr) != (b->hist_offsets == nullptr))
    return fail(c, AS_ERR_INVALID, "as_sample: hist_offsets and hist_ids go together");
  if (b->kept_ids && b->kept_cap == 0)
    return fail(c, AS_ERR_INVALID, "as_sample: kept_ids needs kept_cap > 0");
  uint32_t c_max = 0;
  bool greedy_call = !b->hist_ids;  // every row greedy, no history: greedy_kernel (run_rows)
  for (uint32_t r = 0; r < b->n_rows; ++r) {
    char msg[160];
    if (as_check(&params[r], msg, sizeof msg) != AS_OK)
      return fail(c, AS_ERR_PARAMS, "row " + std::to_string(r) + ": " + msg);
    c_max = std::max(c_max, wanted_cand(params[r], b->n_vocab));
    greedy_call = greedy_call && params[r].temp <= 0.0f;
  }
  const Plan pl = plan_slices(b->n_vocab, b->n_rows, c_max, greedy_call);
  RowParams* h = c->rows.data();
  for (uint32_t r = 0; r < b->n_rows; ++r) {
    h[r] = make_row(params[r], b->n_vocab, pl);
    h[r].rng_index = r;
    h[r].rng_skip = 0;
    h[r].flags |= as_dev::kFlagRngWrite;
  }
  AS_HIP(c, hipSetDevice(c->device));
  return run_rows(c, pl, h, b->logits, b->row_stride, b->n_vocab, b->n_rows, b->hist_offsets,
                  b->hist_ids, nullptr, b->rng_state, b->tokens, b->status, b->kept_count,
                  b->kept_ids, b->kept_probs, b->kept_cap);
}

int as_verify(as_ctx* c, const float* rows, uint64_t row_stride, uint32_t n_vocab,
              const uint32_t* drafts, uint32_t k, const uint32_t* history, uint32_t hist_len,
              const uint32_t* stop_ids, uint32_t n_stop, const as_sampling* params,
              uint64_t* rng_state, uint32_t* picks, uint32_t* result) {
  if (!c) return AS_ERR_INVALID;
  if (!rows || !params || !rng_state || !picks || !result)
    return fail(c, AS_ERR_INVALID, "as_verify: rows, params, rng_state, picks and result are required");
  if ((k > 0 && !drafts) || (hist_len > 0 && !history) || (n_stop > 0 && !stop_ids))
    return fail(c, AS_ERR_INVALID, "as_verify: a list with a length has no pointer");
  if (n_vocab == 0 || row_stride < n_vocab)
    return fail(c, AS_ERR_INVALID, "as_verify: n_vocab must be at least 1 and at most row_stride");
  if ((uint64_t)k + 1 > c->max_rows || n_vocab > c->max_vocab)
    return fail(c, AS_ERR_CAPACITY, "as_verify: more rows or a larger vocabulary than the context holds");
  if ((uint64_t)hist_len + k > c->max_history)
    return fail(c, AS_ERR_CAPACITY, "as_verify: the history and the drafts hold more ids than the context's max_history");
  char msg[160];
  if (as_check(params, msg, sizeof msg) != AS_OK) return fail(c, AS_ERR_PARAMS, msg);
  const Plan pl = plan_slices(n_vocab, k + 1, wanted_cand(*params, n_vocab));
  const bool draws = params->temp > 0.0f;
  RowParams* h = c->rows.data();
  for (uint32_t i = 0; i <= k; ++i) {
    h[i] = make_row(*params, n_vocab, pl);
    h[i].rng_index = 0;
    h[i].rng_skip = draws ? i : 0;
    h[i].hist_begin = 0;
    h[i].hist_len = hist_len;
    h[i].extra = i;  // the drafts before row i were emitted when row i is sampled
  }
  AS_HIP(c, hipSetDevice(c->device));
  int rc = run_rows(c, pl, h, rows, row_stride, n_vocab, k + 1, nullptr, hist_len ? history : nullptr,
                    k ? drafts : nullptr, rng_state, picks, c->d_vstatus, nullptr, nullptr, nullptr, 0);
  if (rc != AS_OK) return rc;
  AS_HIP(c, as_launch::accept(c->stream, picks, c->d_vstatus, drafts, k, stop_ids, n_stop, rng_state,
                              draws ? 1u : 0u, result));
  return AS_OK;
}

int as_argmax_rows(as_ctx* c, const float* logits, uint64_t row_stride, uint32_t n, uint32_t n_rows,
                   uint32_t* ids, uint64_t* rows_out, uint64_t embd, uint32_t row_bytes,
                   uint32_t slot) {
  if (!c) return AS_ERR_INVALID;
  if (n_rows == 0) return AS_OK;
  if (!logits || !ids || !rows_out || row_stride < n)
    return fail(c, AS_ERR_INVALID, "as_argmax_rows: bad pointers or row_stride < n");
  AS_HIP(c, hipSetDevice(c->device));
  const bool vec = aligned16(logits) && (row_stride % 4 == 0);
  AS_HIP(c, as_launch::argmax_rows(c->stream, vec, logits, row_stride, n, n_rows, ids, rows_out,
                                   embd, row_bytes, slot));
  return AS_OK;
}

uint64_t as_row_bytes(uint32_t wtype, uint64_t n) {
  static const uint32_t per[6] = {1, 1, 32, 256, 256, 256}, bytes[6] = {4, 2, 34, 144, 176, 210};
  if (wtype > AS_WTYPE_Q6_K || n % per[wtype] != 0) return 0;
  return n / per[wtype] * bytes[wtype];
}

int as_embed_rows(as_ctx* c, const uint64_t* rows, uint32_t wtype, uint32_t n, float* y, uint32_t n_tokens) {
  if (!c) return AS_ERR_INVALID;
  if (n_tokens == 0 || n == 0) return AS_OK;
  if (!rows || !y) return fail(c, AS_ERR_INVALID, "as_embed_rows: null rows or y");
  if (as_row_bytes(wtype, n) == 0)
    return fail(c, AS_ERR_INVALID, "as_embed_rows: unknown weight type, or n is not a whole number of its blocks");
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, as_launch::embed_rows(c->stream, rows, wtype, n, y, n_tokens));
  return AS_OK;
}

// The shape and alignment checks as_matvec and as_head_argmax share.
int check_matvec(as_ctx* c, const char* who, const void* w, uint32_t wtype, uint32_t k, const float* x) {
  char msg[160];
  if (!w || !x) {
    std::snprintf(msg, sizeof msg, "%s: null weights or input", who);
    return fail(c, AS_ERR_INVALID, msg);
  }
  if (as_row_bytes(wtype, k) == 0 || k % 32 != 0 || k > as_launch::kMatvecMaxK) {
    std::snprintf(msg, sizeof msg, "%s: unknown weight type, or k is not whole 32-value units and blocks of it "
                  "(at most %u)", who, as_launch::kMatvecMaxK);
    return fail(c, AS_ERR_INVALID, msg);
  }
  const uintptr_t align = wtype <= AS_WTYPE_BF16 ? 4 : 2;
  if ((uintptr_t)w % align != 0 || (uintptr_t)x % 4 != 0) {
    std::snprintf(msg, sizeof msg, "%s: weights must be %u-byte aligned and x 4-byte aligned", who, (unsigned)align);
    return fail(c, AS_ERR_INVALID, msg);
  }
  return AS_OK;
}

int as_matvec(as_ctx* c, const void* w, uint32_t wtype, uint32_t rows, uint32_t k, const float* x, float* y) {
  if (!c) return AS_ERR_INVALID;
  if (rows == 0) return AS_OK;
  int rc = check_matvec(c, "as_matvec", w, wtype, k, x);
  if (rc != AS_OK) return rc;
  if (!y) return fail(c, AS_ERR_INVALID, "as_matvec: null y");
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, as_launch::matvec(c->stream, w, wtype, as_row_bytes(wtype, k), rows, k, x, y));
  return AS_OK;
}

int as_head_argmax(as_ctx* c, const void* w, uint32_t wtype, uint32_t rows, uint32_t k, const float* x,
                   float* logits, uint32_t* ids, uint64_t* rows_out, uint64_t embd, uint32_t embd_row_bytes,
                   uint32_t slot) {
  if (!c) return AS_ERR_INVALID;
  int rc = check_matvec(c, "as_head_argmax", w, wtype, k, x);
  if (rc != AS_OK) return rc;
  if (rows == 0 || !ids || !rows_out) return fail(c, AS_ERR_INVALID, "as_head_argmax: no rows, or null ids/rows_out");
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, as_launch::head_argmax(c->stream, w, wtype, as_row_bytes(wtype, k), rows, k, x, logits,
                                   c->d_mv_partials, ids, rows_out, embd, embd_row_bytes, slot));
  return AS_OK;
}

int as_profile(as_ctx* c, int enable) {
  if (!c) return AS_ERR_INVALID;
  c->profile = enable != 0;
  c->ev_used = 0;
  return AS_OK;
}

int as_profile_read(as_ctx* c, double* scan_ms, double* finish_ms, uint32_t* calls) {
  if (!c || !scan_ms || !finish_ms || !calls) return AS_ERR_INVALID;
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, hipStreamSynchronize(c->stream));
  double s = 0.0, f = 0.0;
  uint32_t k = 0;
  for (size_t i = 0; i + 2 < c->ev_used; i += 3) {
    float a = 0.0f, b = 0.0f;
    AS_HIP(c, hipEventElapsedTime(&a, c->ev[i], c->ev[i + 1]));
    if (c->ev_fin[i / 3]) AS_HIP(c, hipEventElapsedTime(&b, c->ev[i + 1], c->ev[i + 2]));
    s += a;
    f += b;
    ++k;
  }
  *scan_ms = s;
  *finish_ms = f;
  *calls = k;
  c->ev_used = 0;
  return AS_OK;
}

int as_debug_exp(as_ctx* c, const double* x, double* y, uint32_t n) {
  if (!c) return AS_ERR_INVALID;
  if (n == 0) return AS_OK;
  if (!x || !y) return fail(c, AS_ERR_INVALID, "as_debug_exp: no arrays");
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, as_launch::debug_exp(c->stream, x, y, n));
  return AS_OK;
}

int as_logprobs(as_ctx* c, const float* logits, uint64_t row_stride, uint32_t n_vocab, uint32_t n_rows,
                const uint32_t* tokens, uint32_t top, float* logprob, uint32_t* top_ids, float* top_logprobs,
                uint32_t* status) {
  if (!c) return AS_ERR_INVALID;
  if (!logits || !tokens || !logprob || n_vocab == 0 || n_rows == 0)
    return fail(c, AS_ERR_INVALID, "as_logprobs: null array or zero size");
  if (top > 0 && (!top_ids || !top_logprobs))
    return fail(c, AS_ERR_INVALID, "as_logprobs: top > 0 needs top_ids and top_logprobs");
  if (row_stride != 0 && row_stride < n_vocab)
    return fail(c, AS_ERR_INVALID, "as_logprobs: row_stride below n_vocab");
  if (n_rows > c->max_rows || n_vocab > c->max_vocab)
    return fail(c, AS_ERR_CAPACITY, "as_logprobs: more rows or a wider vocabulary than the context holds");
  if (as_launch::lp_parts(n_vocab) * as_launch::kLpTop > as_launch::kLpMerge)
    return fail(c, AS_ERR_CAPACITY, "as_logprobs: vocabulary wider than the merge holds");
  const bool vec = aligned16(logits) && (row_stride % 4 == 0);
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, as_launch::logprobs(c->stream, vec, logits, row_stride, n_vocab, n_rows, c->d_lp, tokens, top, logprob,
                                top_ids, top_logprobs, status));
  return AS_OK;
}

int as_debug_exp2f(as_ctx* c, const float* x, float* y, uint32_t n) {
  if (!c) return AS_ERR_INVALID;
  if (n == 0) return AS_OK;
  if (!x || !y) return fail(c, AS_ERR_INVALID, "as_debug_exp2f: no arrays");
  AS_HIP(c, hipSetDevice(c->device));
  AS_HIP(c, as_launch::debug_exp2f(c->stream, x, y, n));
  return AS_OK;
}

}  // extern "C"

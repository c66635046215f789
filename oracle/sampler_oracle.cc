// CPU oracle for the token sampler: TEST INFRASTRUCTURE ONLY (see sampler_oracle.h).
//
// Each function follows the reference's Rust line by line; the citation on each names the lines.
// Built with -O2 -ffp-contract=off so that no f64 expression is fused, as in the reference's
// release build, and with the host libm's exp/log behind f64::exp/f64::ln.
#include "sampler_oracle.h"

#include <algorithm>
#include <atomic>
#include <thread>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <ctime>
#include <map>
#include <vector>

namespace {

// ---- rng.rs ---------------------------------------------------------------------------------

inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

// rng.rs:11-23: four splitmix64 outputs fill the state.
void rng_new(uint64_t seed, uint64_t s[4]) {
  uint64_t x = seed;
  for (int i = 0; i < 4; ++i) {
    x += 0x9E3779B97F4A7C15ull;
    uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    s[i] = z ^ (z >> 31);
  }
}

// rng.rs:26-37: xoshiro256**.
uint64_t rng_next(uint64_t s[4]) {
  uint64_t out = rotl(s[1] * 5, 7) * 9;
  uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl(s[3], 45);
  return out;
}

// rng.rs:55-57: the top 53 bits scaled by 2^-53.
double rng_unit(uint64_t s[4]) { return (double)(rng_next(s) >> 11) * (1.0 / (double)(1ull << 53)); }

// rng.rs:41-52: Lemire's multiply-shift with rejection.
uint64_t rng_below(uint64_t s[4], uint64_t n) {
  unsigned __int128 m = (unsigned __int128)rng_next(s) * n;
  if ((uint64_t)m < n) {
    uint64_t floor = (0 - n) % n;
    while ((uint64_t)m < floor) m = (unsigned __int128)rng_next(s) * n;
  }
  return (uint64_t)(m >> 64);
}

// ---- ordering -------------------------------------------------------------------------------

// f32::total_cmp as an unsigned key: larger key = larger in total order (+0 above -0).
inline uint32_t total_key(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

struct Cand {
  uint32_t id;
  float v;
};

// sample.rs:106-108: logit descending by total_cmp, then id ascending. True when a comes first.
inline bool rank_before(const Cand& a, const Cand& b) {
  uint32_t ka = total_key(a.v), kb = total_key(b.v);
  if (ka != kb) return ka > kb;
  return a.id < b.id;
}

// ---- penalties ------------------------------------------------------------------------------

// The reference subtracts the presence penalty once from every id the sampler returned
// (sample.rs:315-321, 351-356, 380-386). This build generalises that to a history multiset with
// count c >= 1 for the id: t = x, or x / rep (x > 0) or x * rep (x <= 0) when rep != 1; then
// t - (float(c) * freq + pres), every step in f32. With rep = 1 and freq = 0 this is x - pres,
// bit for bit the reference's `c.1 -= pen`.
inline float oc_penalize(float x, uint32_t c, const oc_params& p) {
  float t = x;
  if (p.repetition != 1.0f) t = (x > 0.0f) ? x / p.repetition : x * p.repetition;
  float d = (float)c * p.frequency;
  d = d + p.presence;
  return t - d;
}

// The reference's `pen != 0.0` (sample.rs:130, 315, 342, 351): whether any penalty acts.
inline bool penalties_on(const oc_params& p) {
  return p.presence != 0.0f || p.frequency != 0.0f || p.repetition != 1.0f;
}

}  // namespace

struct oc_sampler {
  oc_params s;
  uint64_t rng[4];
  // sample.rs:101-102 `seen`, here with counts (ascending ids, like the BTreeSet).
  std::map<uint32_t, uint32_t> seen;
  std::vector<uint32_t> kept_ids;
  std::vector<double> kept_w;
  double kept_total = 0.0;
  int last_path = 0;
};

namespace {

// sample.rs:308-323: every (id, logit) pair, penalised ids adjusted.
std::vector<Cand> penalized_candidates(const float* l, size_t n, const oc_sampler& smp) {
  std::vector<Cand> cand(n);
  for (size_t i = 0; i < n; ++i) cand[i] = {(uint32_t)i, l[i]};
  if (penalties_on(smp.s)) {
    for (const auto& kv : smp.seen) {
      if (kv.first < n) cand[kv.first].v = oc_penalize(l[kv.first], kv.second, smp.s);
    }
  }
  return cand;
}

const size_t kTopKRun = 64;           // sample.rs:375
const size_t kTopKOnePassMax = 256;   // sample.rs:299

// sample.rs:302-304.
bool takes_one_pass(size_t k, size_t n) { return 0 < k && k <= kTopKOnePassMax && k < n; }

// sample.rs:335-372: the k best by rank in one pass, skipping 64-runs that hold no penalised id
// and whose every logit is below the k-th best.
std::vector<Cand> top_k(const float* l, size_t n, size_t k, const oc_sampler& smp) {
  const bool on = penalties_on(smp.s);
  auto seen = smp.seen.begin();
  const auto seen_end = smp.seen.end();
  std::vector<Cand> best;
  best.reserve(k + 1);
  for (size_t start = 0; start < n; start += kTopKRun) {
    size_t end = std::min(start + kTopKRun, n);
    bool penalized = on && seen != seen_end && seen->first < end;
    if (best.size() == k && !penalized) {
      float floor = best[k - 1].v;
      bool below = true;
      for (size_t i = start; i < end; ++i) below = below & (l[i] < floor);
      if (below) continue;
    }
    for (size_t i = start; i < end; ++i) {
      float v;
      if (on && seen != seen_end && seen->first == i) {
        v = oc_penalize(l[i], seen->second, smp.s);
        ++seen;
      } else {
        v = l[i];
      }
      Cand c{(uint32_t)i, v};
      if (best.size() == k) {
        const Cand& last = best[k - 1];
        if (v < last.v || rank_before(last, c)) continue;
      }
      auto at = std::partition_point(best.begin(), best.end(),
                                     [&](const Cand& b) { return rank_before(b, c); });
      best.insert(at, c);
      if (best.size() > k) best.resize(k);
    }
  }
  return best;
}

// sample.rs:9-17.
uint32_t greedy(const float* l, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (l[i] > l[best]) best = i;
  return (uint32_t)best;
}

// sample.rs:378-396.
uint32_t greedy_penalized(const float* l, size_t n, const oc_sampler& smp) {
  auto seen = smp.seen.begin();
  auto value = [&](size_t i) {
    if (seen != smp.seen.end() && seen->first == i) {
      float v = oc_penalize(l[i], seen->second, smp.s);
      ++seen;
      return v;
    }
    return l[i];
  };
  size_t best = 0;
  float best_v = value(0);
  for (size_t i = 1; i < n; ++i) {
    float v = value(i);
    if (v > best_v) {
      best = i;
      best_v = v;
    }
  }
  return (uint32_t)best;
}

void record_kept(oc_sampler& smp, const std::vector<Cand>& cand, size_t keep,
                 const std::vector<double>& w, double total) {
  smp.kept_ids.resize(keep);
  smp.kept_w.assign(w.begin(), w.begin() + keep);
  for (size_t i = 0; i < keep; ++i) smp.kept_ids[i] = cand[i].id;
  smp.kept_total = total;
}

// sample.rs:157-198.
uint32_t draw_full_sort(oc_sampler& smp, std::vector<Cand> cand) {
  size_t k = smp.s.top_k;
  if (k > 0 && k < cand.size()) {
    std::nth_element(cand.begin(), cand.begin() + (k - 1), cand.end(), rank_before);
    cand.resize(k);
  }
  std::sort(cand.begin(), cand.end(), rank_before);
  double top = (double)cand[0].v;
  if (smp.s.top_p < 1.0f) {
    std::vector<double> w(cand.size());
    for (size_t i = 0; i < cand.size(); ++i) w[i] = std::exp((double)cand[i].v - top);
    double total = 0.0;
    for (double wi : w) total += wi;
    double cum = 0.0;
    size_t keep = cand.size();
    for (size_t i = 0; i < w.size(); ++i) {
      cum += w[i] / total;
      if (cum >= (double)smp.s.top_p) {
        keep = i + 1;
        break;
      }
    }
    cand.resize(keep);
  }
  if (smp.s.min_p > 0.0f) {
    double floor = top + std::log((double)smp.s.min_p);
    cand.erase(std::remove_if(cand.begin(), cand.end(),
                              [&](const Cand& c) { return !((double)c.v >= floor); }),
               cand.end());
  }
  double temp = (double)smp.s.temp;
  std::vector<double> w(cand.size());
  for (size_t i = 0; i < cand.size(); ++i) w[i] = std::exp(((double)cand[i].v - top) / temp);
  double sum = 0.0;
  for (double wi : w) sum += wi;
  record_kept(smp, cand, cand.size(), w, sum);
  double u = rng_unit(smp.rng) * sum;
  double cum = 0.0;
  for (size_t i = 0; i < cand.size(); ++i) {
    cum += w[i];
    if (u < cum) return cand[i].id;
  }
  return cand.back().id;
}

// sample.rs:208-293.
uint32_t draw_partial(oc_sampler& smp, std::vector<Cand> cand) {
  const size_t n = cand.size();
  const double top_p = (double)smp.s.top_p, min_p = (double)smp.s.min_p, temp = (double)smp.s.temp;
  const bool cuts = smp.s.top_p < 1.0f || smp.s.min_p > 0.0f;
  uint32_t top_key = 0;
  float top_f = cand[0].v;
  for (const Cand& c : cand) {
    if (total_key(c.v) >= top_key) {
      top_key = total_key(c.v);
      top_f = c.v;
    }
  }
  const double top = (double)top_f;
  const bool has_floor = min_p > 0.0;
  const double floor = has_floor ? top + std::log(min_p) : 0.0;
  double total1 = 0.0;
  if (smp.s.top_p < 1.0f) {
    for (const Cand& c : cand) total1 += std::exp((double)c.v - top);
  }
  size_t kk = std::min<size_t>(64, n);
  auto sort_prefix = [&](size_t kk_) {
    if (kk_ < n) std::nth_element(cand.begin(), cand.begin() + (kk_ - 1), cand.end(), rank_before);
    std::sort(cand.begin(), cand.begin() + kk_, rank_before);
  };
  if (cuts) {
    size_t keep;
    for (;;) {
      sort_prefix(kk);
      double cum = 0.0;
      bool found = false;
      size_t at = 0;
      for (size_t i = 0; i < kk; ++i) {
        const Cand& c = cand[i];
        if (has_floor && (double)c.v < floor) {
          found = true;
          at = i;
          break;
        }
        if (smp.s.top_p < 1.0f) {
          cum += std::exp((double)c.v - top) / total1;
          if (cum >= top_p) {
            found = true;
            at = i + 1;
            break;
          }
        }
      }
      if (found) {
        keep = at;
        break;
      }
      if (kk == n) {
        keep = n;
        break;
      }
      kk = std::min(4 * kk, n);
    }
    cand.resize(keep);
    std::vector<double> w(cand.size());
    for (size_t i = 0; i < cand.size(); ++i) w[i] = std::exp(((double)cand[i].v - top) / temp);
    double sum = 0.0;
    for (double wi : w) sum += wi;
    record_kept(smp, cand, cand.size(), w, sum);
    double u = rng_unit(smp.rng) * sum;
    double cum = 0.0;
    for (size_t i = 0; i < cand.size(); ++i) {
      cum += w[i];
      if (u < cum) return cand[i].id;
    }
    return cand.back().id;
  }
  // No filter: the total in index order, then a walk down the growing sorted prefix.
  double total = 0.0;
  for (const Cand& c : cand) total += std::exp(((double)c.v - top) / temp);
  double u = rng_unit(smp.rng) * total;
  double cum = 0.0;
  size_t from = 0;
  smp.kept_ids.clear();
  smp.kept_w.clear();
  smp.kept_total = total;
  for (;;) {
    sort_prefix(kk);
    for (size_t i = from; i < kk; ++i) {
      double wi = std::exp(((double)cand[i].v - top) / temp);
      smp.kept_ids.push_back(cand[i].id);
      smp.kept_w.push_back(wi);
      cum += wi;
      if (u < cum) return cand[i].id;
    }
    if (kk == n) return cand[n - 1].id;
    from = kk;
    kk = std::min(4 * kk, n);
  }
}

// sample.rs:122-153.
uint32_t sample(oc_sampler& smp, const float* l, size_t n) {
  const bool on = penalties_on(smp.s);
  uint32_t t;
  smp.kept_ids.clear();
  smp.kept_w.clear();
  smp.kept_total = 0.0;
  if (smp.s.temp <= 0.0f) {
    if (on && !smp.seen.empty()) {
      t = greedy_penalized(l, n, smp);
      smp.last_path = 1;
    } else {
      t = greedy(l, n);
      smp.last_path = 0;
    }
  } else {
    size_t k = smp.s.top_k;
    if (k > 0 && k < n) {
      std::vector<Cand> cand;
      if (takes_one_pass(k, n)) {
        cand = top_k(l, n, k, smp);
        smp.last_path = 2;
      } else {
        cand = penalized_candidates(l, n, smp);
        smp.last_path = 3;
      }
      t = draw_full_sort(smp, std::move(cand));
    } else {
      t = draw_partial(smp, penalized_candidates(l, n, smp));
      smp.last_path = 4;
    }
  }
  smp.seen[t] += 1;
  return t;
}

std::vector<Cand> from_pairs(const uint32_t* ids, const float* vals, size_t n) {
  std::vector<Cand> c(n);
  for (size_t i = 0; i < n; ++i) c[i] = {ids[i], vals[i]};
  return c;
}

size_t write_cands(const std::vector<Cand>& c, uint32_t* ids, float* vals) {
  for (size_t i = 0; i < c.size(); ++i) {
    ids[i] = c[i].id;
    vals[i] = c[i].v;
  }
  return c.size();
}

}  // namespace

extern "C" {

void oc_rng_new(uint64_t seed, uint64_t state[4]) { rng_new(seed, state); }
uint64_t oc_rng_next_u64(uint64_t state[4]) { return rng_next(state); }
double oc_rng_unit(uint64_t state[4]) { return rng_unit(state); }
uint64_t oc_rng_below(uint64_t state[4], uint64_t n) { return rng_below(state, n); }

uint32_t oc_greedy(const float* logits, size_t n) { return greedy(logits, n); }

// sample.rs:22-34 (the block pass only decides whether the scan runs; the answer is the scan's).
// sample.rs:22-34: a fold over 1,024-value blocks with no early exit inside a block (it
// vectorizes), stopping at the first block that holds a non-finite value; only then the scan for it.
int64_t oc_first_non_finite(const float* logits, size_t n) {
  bool all_finite = true;
  for (size_t b = 0; b < n && all_finite; b += 1024) {
    const size_t e = std::min(n, b + 1024);
    // is_finite as an exponent test on the bits, which the compiler vectorizes.
    uint32_t ok = 1;
    for (size_t i = b; i < e; ++i) {
      uint32_t bits;
      std::memcpy(&bits, logits + i, 4);
      ok &= (uint32_t)((bits & 0x7F800000u) != 0x7F800000u);
    }
    all_finite = ok != 0;
  }
  if (all_finite) return -1;
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(logits[i])) return (int64_t)i;
  return -1;
}

// kernels/src/twin/argmax.rs:8-16.
uint32_t oc_argmax_row(const float* logits, size_t n) {
  int64_t best = -1;
  for (size_t i = 0; i < n; ++i) {
    float v = logits[i];
    if (std::isfinite(v) && (best < 0 || v > logits[best])) best = (int64_t)i;
  }
  return best < 0 ? 0xFFFFFFFFu : (uint32_t)best;
}

// sample.rs:71-94, extended with the two new penalties' ranges.
int oc_check(const oc_params* p, char* msg, size_t cap) {
  char buf[160];
  buf[0] = 0;
  if (!(std::isfinite(p->temp) && p->temp >= 0.0f))
    std::snprintf(buf, sizeof buf, "--temp %g must be a finite number, 0 or more", p->temp);
  else if (!(p->top_p > 0.0f && p->top_p <= 1.0f))
    std::snprintf(buf, sizeof buf, "--top-p %g must be above 0 and at most 1", p->top_p);
  else if (!(p->min_p >= 0.0f && p->min_p <= 1.0f))
    std::snprintf(buf, sizeof buf, "--min-p %g must be from 0 to 1", p->min_p);
  else if (!std::isfinite(p->presence))
    std::snprintf(buf, sizeof buf, "--presence-penalty %g must be a finite number", p->presence);
  else if (!std::isfinite(p->frequency))
    std::snprintf(buf, sizeof buf, "--frequency-penalty %g must be a finite number", p->frequency);
  else if (!(std::isfinite(p->repetition) && p->repetition > 0.0f))
    std::snprintf(buf, sizeof buf, "--repetition-penalty %g must be a finite number above 0",
                  p->repetition);
  if (msg && cap) {
    std::strncpy(msg, buf, cap - 1);
    msg[cap - 1] = 0;
  }
  return buf[0] ? 1 : 0;
}

oc_sampler* oc_sampler_new(const oc_params* p, uint64_t seed) {
  oc_sampler* s = new oc_sampler();
  s->s = *p;
  rng_new(seed, s->rng);
  return s;
}
void oc_sampler_free(oc_sampler* s) { delete s; }
void oc_sampler_add_history(oc_sampler* s, const uint32_t* ids, size_t n) {
  for (size_t i = 0; i < n; ++i) s->seen[ids[i]] += 1;
}
void oc_sampler_get_rng(const oc_sampler* s, uint64_t state[4]) { std::memcpy(state, s->rng, 32); }
void oc_sampler_set_rng(oc_sampler* s, const uint64_t state[4]) { std::memcpy(s->rng, state, 32); }

uint32_t oc_sampler_sample(oc_sampler* s, const float* logits, size_t n) { return sample(*s, logits, n); }

size_t oc_sampler_last_kept(const oc_sampler* s, uint32_t* ids, double* probs, size_t cap) {
  size_t n = s->kept_ids.size();
  for (size_t i = 0; i < n && i < cap; ++i) {
    ids[i] = s->kept_ids[i];
    probs[i] = s->kept_w[i] / s->kept_total;
  }
  return n;
}
int oc_sampler_last_path(const oc_sampler* s) { return s->last_path; }

uint32_t oc_sampler_draw_full_sort(oc_sampler* s, const uint32_t* ids, const float* vals, size_t n) {
  return draw_full_sort(*s, from_pairs(ids, vals, n));
}
uint32_t oc_sampler_draw_partial(oc_sampler* s, const uint32_t* ids, const float* vals, size_t n) {
  return draw_partial(*s, from_pairs(ids, vals, n));
}

size_t oc_top_k(const oc_sampler* s, const float* logits, size_t n, size_t k, uint32_t* ids,
                float* vals) {
  return write_cands(top_k(logits, n, k, *s), ids, vals);
}

size_t oc_selected(const oc_sampler* s, const float* logits, size_t n, size_t k, uint32_t* ids,
                   float* vals) {
  std::vector<Cand> c = penalized_candidates(logits, n, *s);
  std::nth_element(c.begin(), c.begin() + (k - 1), c.end(), rank_before);
  c.resize(k);
  std::sort(c.begin(), c.end(), rank_before);
  return write_cands(c, ids, vals);
}

int oc_takes_one_pass(size_t k, size_t n) { return takes_one_pass(k, n) ? 1 : 0; }

size_t oc_verify(oc_sampler* s, const float* rows, size_t n, const uint32_t* drafts, size_t k,
                 const uint32_t* stop_ids, size_t n_stop, uint32_t* picks, uint32_t* accepted,
                 uint32_t* stopped) {
  size_t read = 0;
  *stopped = 0;
  for (size_t i = 0; i <= k; ++i) {
    uint32_t y = sample(*s, rows + i * n, n);
    read = i + 1;
    picks[i] = y;
    bool stop = false;
    for (size_t j = 0; j < n_stop; ++j) stop = stop || stop_ids[j] == y;
    if (stop) {
      *stopped = 1;
      break;
    }
    if (i < k && drafts[i] != y) break;
  }
  *accepted = (uint32_t)(read - 1);
  return read;
}

// The CPU baseline's timers: the engine's per-row work, the non-finite check before the sampler
// (decode.rs:437-447, sample.rs:22-34) and Sampler::sample (sample.rs:122-153), or the verify loop
// over k+1 rows (spec/step.rs:340-385, each row checked first as verify.rs:345-348 does), timed on
// the calling thread with CLOCK_MONOTONIC. The sampler (its RNG and history set) is built by the
// caller beforehand, as the engine's Sampler already holds them. Returns nanoseconds.
static double now_ns() {
  timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec * 1e9 + (double)t.tv_nsec;
}

double oc_sampler_sample_timed(oc_sampler* s, const float* logits, size_t n, uint32_t* token) {
  const double t0 = now_ns();
  const int64_t bad = oc_first_non_finite(logits, n);
  *token = bad >= 0 ? 0xFFFFFFFFu : sample(*s, logits, n);
  return now_ns() - t0;
}

double oc_verify_timed(oc_sampler* s, const float* rows, size_t n, const uint32_t* drafts, size_t k,
                       uint32_t* picks, uint32_t* read) {
  const double t0 = now_ns();
  size_t r = 0;
  for (size_t i = 0; i <= k; ++i) {
    if (oc_first_non_finite(rows + i * n, n) >= 0) break;
    const uint32_t y = sample(*s, rows + i * n, n);
    picks[i] = y;
    r = i + 1;
    if (i < k && drafts[i] != y) break;
  }
  *read = (uint32_t)r;
  return now_ns() - t0;
}

// logprobs.rs:12-48.
float oc_logprobs(const float* logits, size_t n, uint32_t token, uint32_t top, uint32_t* ids,
                  float* lps, size_t* n_top) {
  float mf = -INFINITY;
  for (size_t i = 0; i < n; ++i) mf = std::fmax(mf, logits[i]);
  double m = (double)mf;
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) sum += std::exp((double)logits[i] - m);
  double lse = m + std::log(sum);
  size_t nt = std::min<size_t>(std::min<size_t>(top, 20), n);
  float logprob = (float)((double)logits[token] - lse);
  *n_top = nt;
  if (nt == 0) return logprob;
  std::vector<uint32_t> all(n);
  for (size_t i = 0; i < n; ++i) all[i] = (uint32_t)i;
  auto by_logit = [&](uint32_t a, uint32_t b) {
    if (logits[a] > logits[b]) return true;
    if (logits[a] < logits[b]) return false;
    return a < b;
  };
  if (nt < n) std::nth_element(all.begin(), all.begin() + (nt - 1), all.end(), by_logit);
  std::sort(all.begin(), all.begin() + nt, by_logit);
  for (size_t i = 0; i < nt; ++i) {
    ids[i] = all[i];
    lps[i] = (float)((double)logits[all[i]] - lse);
  }
  return logprob;
}

double oc_exp(double x) { return std::exp(x); }
double oc_log(double x) { return std::log(x); }
void oc_exp_array(const double* x, double* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = std::exp(x[i]);
}

void oc_sample_rows(const oc_params* params, const uint64_t* seeds, const float* logits,
                    size_t stride, size_t n, size_t rows, const uint32_t* hist_off,
                    const uint32_t* hist_ids, unsigned threads, uint32_t* tokens,
                    uint64_t* rng_out) {
  std::atomic<size_t> next{0};
  auto work = [&]() {
    for (;;) {
      const size_t r = next.fetch_add(1);
      if (r >= rows) break;
      const float* row = logits + r * stride;
      oc_sampler smp;
      smp.s = params[r];
      rng_new(seeds[r], smp.rng);
      if (hist_off)
        for (uint32_t h = hist_off[r]; h < hist_off[r + 1]; ++h) smp.seen[hist_ids[h]] += 1;
      // The engine's check before the sampler (decode.rs:437-447, sample.rs:22-34).
      tokens[r] = oc_first_non_finite(row, n) >= 0 ? 0xFFFFFFFFu : sample(smp, row, n);
      if (rng_out) std::memcpy(rng_out + 4 * r, smp.rng, 32);
    }
  };
  if (threads <= 1) {
    work();
  } else {
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t) pool.emplace_back(work);
    for (auto& t : pool) t.join();
  }
}

}  // extern "C"

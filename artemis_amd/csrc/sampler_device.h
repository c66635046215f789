// Device-side building blocks of the sampler kernels: the rank order as integer keys, the penalty,
// the seed stream, the per-row parameter block and wave64 reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exp_f64.h"
#include "exp_poly.h"

namespace as_dev {

// A load through a pointer to global memory. A pointer the compiler cannot place in an address space
// (one read from memory, as the finish kernel's arguments are) takes flat instructions, which count
// against the LDS wait counter as well: every wait for an LDS access then also waits for the loads
// in flight, and a loop that mixes the two streams its row one step at a time. Reading through a
// global-address-space view takes global instructions instead.
template <class T>
__device__ __forceinline__ T gload(const T* p) {
  if constexpr (__is_scalar(T) || __is_same(T, float __attribute__((ext_vector_type(4)))) ||
                __is_same(T, uint32_t __attribute__((ext_vector_type(4))))) {
    return *(const __attribute__((address_space(1))) T*)p;
  } else {
    // A structure, word by word (a global-address-space object has no copy constructor to bind).
    static_assert(sizeof(T) % 4 == 0, "whole words");
    struct Words {
      uint32_t w[sizeof(T) / 4];
    } r;
    const __attribute__((address_space(1))) uint32_t* q = (const __attribute__((address_space(1))) uint32_t*)p;
#pragma unroll
    for (uint32_t i = 0; i < sizeof(T) / 4; ++i) r.w[i] = q[i];
    return __builtin_bit_cast(T, r);
  }
}

constexpr int kWave = 64;
constexpr uint32_t kNone = 0xFFFFFFFFu;

// Row modes, chosen on the host from the sampling settings (sample.rs:129-150).
enum : uint32_t {
  kModeGreedy = 0,     // temp <= 0: greedy / greedy_penalized
  kModeTopK = 1,       // 0 < k < n, k small enough for the slice candidates: draw_full_sort
  kModePartial = 2,    // k == 0 or k >= n: draw_partial
  kModeExactTopK = 3,  // 0 < k < n with a k too large for the slice candidates
};

// RowParams.flags
enum : uint32_t {
  kFlagPenalties = 1u,  // some penalty acts (the reference's `pen != 0.0`)
  kFlagSumTop = 2u,     // partial with top_p < 1: slice sums of exp(l - m)
  kFlagSumTemp = 4u,    // partial with no filter: slice sums of exp((l - m) / T)
  kFlagRngWrite = 8u,   // write the advanced RNG state back (batch rows; verify defers it)
  kFlagKept = 16u,      // the caller wants kept lists
};

struct RowParams {
  float temp;
  uint32_t top_k;
  float top_p;
  float min_p;
  float presence;
  float frequency;
  float repetition;
  uint32_t mode;
  double ln_min_p;      // log((double)min_p) from the host libm, as f64::ln (sample.rs:181, 217)
  uint32_t flags;
  uint32_t cand;        // candidates each wave of a slice keeps (top-k rows: k)
  uint32_t rng_index;   // which 4-word state the row draws from
  uint32_t rng_skip;    // draws to skip first (verify row i skips i)
  uint32_t hist_begin;  // history range when no CSR offsets are given
  uint32_t hist_len;
  uint32_t extra;       // ids of the extra list appended to the history (verify drafts)
  uint32_t cap;         // candidate slots per slice (slices x cap fit the finish LDS)
  uint32_t help;        // the row's place among the finish kernel's helpers of S's sums (cheapest first)
  uint32_t pad_;        // zero: the host compares blocks byte for byte
};
static_assert(sizeof(RowParams) == 80 && sizeof(RowParams) % 16 == 0, "whole 16-byte words, no implicit padding");

// A row's words that its slices share during a scan, in device memory; zero before the scan (the
// context clears them once, and the finish kernel clears its row's after each scan; in a call the
// scan finishes, the rows' slices touch only `arrived`, which the row's last slice clears).
constexpr uint32_t kShareSlots = 16;
struct RowShare {
  uint32_t bound;  // the largest wave threshold's key any slice of the row has published
  uint32_t top;    // the largest key any slice has seen (min-p rows)
  // Top-k rows: wave i < kShareSlots of the row keeps here the key of its q-th best value so far,
  // q = ceil(k / slots); once every slot is set, their minimum has at least k values at or above it.
  uint32_t slot[kShareSlots];
  uint32_t gave_up;  // min-p rows: a slice's bound lay above its floor (not every value above it kept)
  uint32_t arrived;  // calls the scan finishes: the row's slices that have ended (the last one clears it)
};

// A min-p row whose candidates do not hold its whole floor set: the weights of S, the row's values
// that rank below the candidates' bound and lie at or above the floor, summed in parts by the finish
// kernel's workgroups (sums of f32 terms from the hardware's exp2, each within 3e-5 relative; zero
// between calls: the row's own workgroup clears it once every part has ended).
struct RowTail {
  double w;        // sum of exp((l - top) / T) over S
  double m;        // sum of exp(l - top) over S
  uint32_t count;  // values in S; when at most kTailKeep, they are in the row's scratch (packed)
  uint32_t parts;  // parts of the row summed (the sums cover S once every part has added)
  uint32_t failed; // a part could not (more distinct history ids than its table holds)
  uint32_t lost;   // a part held more of S than it could stage (the scratch list is incomplete)
  uint32_t ended;  // parts that have ended, summed or not (their writes complete before they count)
  uint32_t pad_;
};
constexpr uint32_t kTailKeep = 8192;
// The histogram of S by value: bin b holds the values v with
// floor(min(rv - v) * kTailBins / (rv - fl), kTailBins - 1) = b (rv: the value of the candidates' bound,
// fl: the floor), so that every value of bin b ranks above every value of bin b + 1; per bin the
// sums of exp(l - top) (m) and exp((l - top) / T) (w), each term as in RowTail. Zero between calls.
constexpr uint32_t kTailBins = 256;
struct TailBins {
  double m[kTailBins];
  double w[kTailBins];
};

// The rows a call's scan flagged for S's sums (RowShare::gave_up), in the order the scan flagged
// them: the first kTailListMax of them. A context holds two lists and call c takes list c mod 2; the
// finish kernel of call c clears the other list's count for the next call.
constexpr uint32_t kTailListMax = 16;
struct TailList {
  uint32_t count;  // rows flagged (may exceed kTailListMax)
  uint32_t rows[kTailListMax];
  uint32_t help[kTailListMax];  // each listed row's RowParams::help
};

// A row's deep-path passes, shared with the finish kernel's idle workgroups (small batches): the
// row's workgroup publishes each pass by stamping it (2 x the call's number for the histogram pass,
// that + 1 for the collecting pass) once the fields it needs are stored; any workgroup takes the
// pass's parts through `next`, and each part counts itself in `ended` once its writes are complete.
struct DeepJob {
  uint64_t stamp;
  uint32_t mk;            // the row's largest key
  uint32_t next[2];       // per pass: the next part to take
  uint32_t ended[2];      // per pass: parts ended
  uint32_t r0[3], r1[3];  // the collecting pass: the runs of bins to collect (kNone: none)
  uint32_t pad_;
};

// Per (row, slice) results of the scan.
struct SegStats {
  uint32_t nonfinite;   // first index holding NaN/inf in the raw logits, or kNone
  uint32_t greedy_idx;  // IEEE-greater argmax, lowest index on ties, NaN skipped; kNone if none
  float greedy_val;
  uint32_t max_key;     // largest rank key of the penalised values
  uint32_t n_cand;
  uint32_t truncated;   // bit 0: the slice held more values than it kept as candidates;
                        // bit 1: the scan could not finish the slice's statistics (more distinct
                        // history ids than its hash holds, or more candidates than its slots)
  float err_rel;        // sum's error from its own evaluation: at most err_rel * sum
  float err_abs;        //   + err_abs * sum_abs
  uint64_t bound;       // a truncated slice kept every value whose packed rank is >= bound,
                        // and at least `cand` of its values are >= bound
  double sum;           // sum of exp(d), d = l - m (or (l - m) / T), m = sum_ref
  double sum_abs;       // sum of exp(d) * |d|
  float sum_ref;        // the sums' reference m: at least every value they hold
  uint32_t vast;        // min-p rows: the slice found the floor set vast (tens of thousands of values)
};

// f32::total_cmp as an unsigned key (sample.rs:106-108): larger key = higher rank; +0 above -0.
__device__ __forceinline__ uint32_t total_key(float x) {
  uint32_t b = __float_as_uint(x);
  return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}
// Rank order as one descending u64: key, then the lower id.
__device__ __forceinline__ uint64_t pack(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint64_t)(~id);
}
__device__ __forceinline__ uint32_t packed_id(uint64_t p) { return ~(uint32_t)p; }
__device__ __forceinline__ float packed_value(uint64_t p) { return key_value((uint32_t)(p >> 32)); }

__device__ __forceinline__ bool is_finite_bits(float x) {
  return (__float_as_uint(x) & 0x7F800000u) != 0x7F800000u;
}

// The smallest f32 whose f64 value is >= f (IEEE, so a floor of 0 admits -0 as well): a value x
// passes min-p's test f64(x) >= f (sample.rs:181, 237) exactly when x >= floor_f32(f).
__device__ __forceinline__ float floor_f32(double f) {
  float x = __double2float_rn(f);
  if ((double)x < f) x = nextafterf(x, __builtin_inff());
  if (x == 0.0f) x = -0.0f;
  return x;
}

// The history penalty for an id seen c >= 1 times, in f32, each operation rounded on its own.
__device__ __forceinline__ float penalize(float x, uint32_t c, const RowParams& p) {
  float t = x;
  if (p.repetition != 1.0f) t = (x > 0.0f) ? __fdiv_rn(x, p.repetition) : __fmul_rn(x, p.repetition);
  float d = __fmul_rn((float)c, p.frequency);
  d = __fadd_rn(d, p.presence);
  return __fsub_rn(t, d);
}

// xoshiro256** (rng.rs:26-37) and unit() (rng.rs:55-57).
__device__ __forceinline__ uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
__device__ __forceinline__ uint64_t rng_next(uint64_t s[4]) {
  uint64_t out = rotl64(s[1] * 5, 7) * 9;
  uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return out;
}
__device__ __forceinline__ double rng_unit(uint64_t s[4]) {
  return (double)(rng_next(s) >> 11) * (1.0 / 9007199254740992.0);
}

// ---- wave64 / block reductions ----------------------------------------------------------------
// The device library's wavefront reductions (DPP lane moves, a fixed order).

}  // namespace as_dev
extern "C" __device__ __attribute__((const)) unsigned int __ockl_wfred_add_u32(unsigned int);
extern "C" __device__ __attribute__((const)) unsigned int __ockl_wfred_min_u32(unsigned int);
extern "C" __device__ __attribute__((const)) unsigned int __ockl_wfred_max_u32(unsigned int);
extern "C" __device__ __attribute__((const)) double __ockl_wfred_add_f64(double);
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(unsigned long long);
namespace as_dev {

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return __ockl_wfred_max_u32(v); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return __ockl_wfred_min_u32(v); }
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return __ockl_wfred_add_u32(v); }
__device__ __forceinline__ double wave_sum_f64(double v) { return __ockl_wfred_add_f64(v); }
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return __ockl_wfred_max_u64(v); }

// ---- wave64 scans by DPP lane moves -----------------------------------------------------------
// Lane i's inclusive sum of lanes 0..i by Hillis-Steele steps inside each row of 16 lanes (row_shr
// 1, 2, 4, 8), then across rows (row_bcast:15 carries a row's last lane into rows 1 and 3,
// row_bcast:31 lane 31 into rows 2 and 3): every lane's sum is a tree of depth 6 over its terms, as
// a shuffle-based Hillis-Steele scan's is, without the shuffles' trips through the LDS crossbar. A
// lane with no source lane, or outside the row mask, reads 0.
constexpr int kDppRowShr = 0x110, kDppWaveShr1 = 0x138, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kCtrl, kRowMask, 0xf, true);
}
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint64_t lo = dpp_u32<kCtrl, kRowMask>((uint32_t)b), hi = dpp_u32<kCtrl, kRowMask>((uint32_t)(b >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
  x += dpp_u32<kDppRowShr + 1>(x);
  x += dpp_u32<kDppRowShr + 2>(x);
  x += dpp_u32<kDppRowShr + 4>(x);
  x += dpp_u32<kDppRowShr + 8>(x);
  x += dpp_u32<kDppRowBcast15, 0xa>(x);
  x += dpp_u32<kDppRowBcast31, 0xc>(x);
  return x;
}
__device__ __forceinline__ double wave_scan_f64(double x) {
  x = __dadd_rn(x, dpp_f64<kDppRowShr + 1>(x));
  x = __dadd_rn(x, dpp_f64<kDppRowShr + 2>(x));
  x = __dadd_rn(x, dpp_f64<kDppRowShr + 4>(x));
  x = __dadd_rn(x, dpp_f64<kDppRowShr + 8>(x));
  x = __dadd_rn(x, dpp_f64<kDppRowBcast15, 0xa>(x));
  x = __dadd_rn(x, dpp_f64<kDppRowBcast31, 0xc>(x));
  return x;
}
// Lane i - 1's value (0 on lane 0), e.g. the exclusive sum from the inclusive one.
__device__ __forceinline__ uint32_t wave_prev_u32(uint32_t x) { return dpp_u32<kDppWaveShr1>(x); }
__device__ __forceinline__ double wave_prev_f64(double x) { return dpp_f64<kDppWaveShr1>(x); }
// Lane k's value in every lane (k the same in the whole wave).
__device__ __forceinline__ uint32_t wave_lane_u32(uint32_t x, uint32_t k) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, (int)__builtin_amdgcn_readfirstlane(k));
}
__device__ __forceinline__ double wave_lane_f64(double x, uint32_t k) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint64_t lo = wave_lane_u32((uint32_t)b, k), hi = wave_lane_u32((uint32_t)(b >> 32), k);
  return __builtin_bit_cast(double, lo | (hi << 32));
}

// Greedy's order (sample.rs:9-17): a larger value by IEEE `>`, equal values to the lower index;
// kNone loses to anything.
__device__ __forceinline__ void greedy_merge(float& v, uint32_t& i, float v2, uint32_t i2) {
  if (i2 == kNone) return;
  if (i == kNone || v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}
__device__ __forceinline__ void wave_greedy(float& v, uint32_t& i) {
  for (int o = 32; o > 0; o >>= 1) {
    float v2 = __shfl_xor(v, o, kWave);
    uint32_t i2 = (uint32_t)__shfl_xor((int)i, o, kWave);
    greedy_merge(v, i, v2, i2);
  }
}

// Block reductions through a small LDS array `red` (one slot per wave); all threads get the result.
template <int NW>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  uint32_t r = red[0];
  for (int k = 1; k < NW; ++k) r = max(r, red[k]);
  return r;
}
template <int NW>
__device__ __forceinline__ uint32_t block_min_u32(uint32_t v, uint32_t* red) {
  v = wave_min_u32(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  uint32_t r = red[0];
  for (int k = 1; k < NW; ++k) r = min(r, red[k]);
  return r;
}
template <int NW>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  v = wave_sum_u32(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  uint32_t r = 0;
  for (int k = 0; k < NW; ++k) r += red[k];
  return r;
}
template <int NW>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  double r = red[0];
  for (int k = 1; k < NW; ++k) r = __dadd_rn(r, red[k]);
  return r;
}

}  // namespace as_dev

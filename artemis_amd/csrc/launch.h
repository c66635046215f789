// Host-side launchers of the sampler kernels (each defined beside its kernel).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sampler_device.h"

namespace as_launch {

// The scan splits each row into slices, one 256-thread workgroup each, and streams a slice through
// registers. A slice holds at most kSliceMax values (its history bitmap lives in LDS) and starts at
// a multiple of kSliceAlign.
constexpr uint32_t kSliceMax = 98304;
constexpr uint32_t kSliceAlign = 1024;
constexpr uint32_t kMaxSlices = 256;
// The scan aims for about this many workgroups per call: three per CU, which its registers allow
// at once, so that a call runs in one round.
constexpr uint32_t kTargetGroups = 768;
// Candidate slots per row in HBM (the slices share them evenly), and how many of a row's candidates
// at or above its bound the finish kernel sorts in LDS.
constexpr uint32_t kCandCap = 16384;
constexpr uint32_t kFinishCap = 8192;
// Each wave of a slice keeps the values at or above its threshold in an LDS buffer of kWaveCap
// entries, and at most its best C once the buffer fills (C = top_k; kPartialRank for rows without a
// top-k; kFloorRank for those with min-p, whose buffer should hold every value above the floor); a
// slice writes at most 4 C of them plus the history values that rank at or above its bound, for
// which kHistReserve slots are kept.
constexpr uint32_t kWaveCap = 768;
constexpr uint32_t kPartialRank = 192;
constexpr uint32_t kFloorRank = 384;
constexpr uint32_t kTopKMax = 256;
constexpr uint32_t kHistReserve = 64;
// Distinct history ids a slice can count (an LDS hash; a 16,000-id history of generated text holds
// about 3,200 distinct ids, 1,100 per slice at batch 256); more send the row to the exact path.
constexpr uint32_t kHistSlots = 2048;
// The deep passes shared with idle workgroups histogram a row into kDistBins bins.
constexpr uint32_t kDistBins = 1024;
// u32 words of scratch per row for rows of n values: the history counts [n], then (8-byte aligned)
// either two u64 buffers [n] (the full deep and exact-order paths) or the shared deep passes'
// histogram (a u32 count and two f64 weights per bin) and list (a count, a pad word, kFinishCap
// packed values); a multiple of 4 words, so that every row's scratch starts 16-byte aligned.
__host__ __device__ constexpr uint64_t scratch_words(uint32_t n) {
  const uint64_t head = ((uint64_t)n + 1) & ~1ull;
  const uint64_t bufs = 4ull * n, shared = 5ull * kDistBins + 2 + 2ull * kFinishCap;
  return (head + (bufs > shared ? bufs : shared) + 3) & ~3ull;
}

// The finish kernel's arguments reach the GPU as the scan's kernel argument; the scan's first
// workgroup stores them in device memory, where every finish workgroup reads them. The rows'
// parameter blocks live in device memory across calls: the host uploads a call's blocks only when
// they differ from the ones already there (a request's settings rarely change between steps), and
// the scan reads them with scalar loads.
constexpr uint32_t kArgsSlot = 320;

struct FinishArgs {
  const float* logits;
  uint64_t row_stride;
  uint32_t n;
  uint32_t n_seg;
  const as_dev::RowParams* params;
  as_dev::RowShare* share;
  const uint32_t* hist_off;
  const uint32_t* hist_ids;
  const uint32_t* extra_ids;
  const as_dev::SegStats* stats;
  const uint64_t* cands;
  uint32_t cand_stride;
  uint32_t kept_cap;
  uint64_t* rng_state;
  uint32_t* tokens;
  uint32_t* status;
  uint32_t* kept_count;
  uint32_t* kept_ids;
  double* kept_probs;
  uint32_t vec;             // the rows are 16-byte aligned (float4 loads)
  uint32_t* scratch;        // deep and exact paths: scratch_words(n) u32 per row
  uint64_t scratch_stride;  // u32 per row
  uint64_t* done;           // pinned host word: the number of the last call whose finish kernel
  uint64_t call;            //   has started (the host reuses an upload's staging block after it)
  as_dev::RowTail* tail;    // per row: S's sums (min-p rows whose scan gave up)
  as_dev::TailBins* tail_bins;  // per row: S's histogram
  as_dev::TailList* tail_list;  // the rows this call's scan flagged for S's sums
  as_dev::TailList* tail_next;  // the next call's list (cleared by this call's finish kernel)
  uint64_t* tail_claims;    // per helper of S's sums: the number of the last call that claimed its set
  uint32_t max_history;     // a row with more history ids than this is refused (AS_ROW_HISTORY)
  uint32_t n_rows;          // rows of the call
  uint32_t deep_help;       // the deep path's passes are shared with idle workgroups (small batches)
  as_dev::DeepJob* deep_jobs;  // per row
  uint64_t* deep_done;      // rows finished, over every call of the context
  uint64_t deep_target;     // deep_done once this call's rows are finished
  uint32_t rng_rows;        // row r draws from RNG state r (as_sample): its state loads without its parameters
  uint32_t scan_finishes;   // every row greedy and no history: each row's last slice finishes it, and
                            // no finish kernel runs
  uint32_t pad2_[2];
};
static_assert(sizeof(FinishArgs) <= kArgsSlot && kArgsSlot % 16 == 0, "FinishArgs slot");

// The row's history ids are hist_ids[*hb, return value), from the CSR offsets or the row's range.
__device__ __forceinline__ uint32_t history_bounds(const FinishArgs& a, const as_dev::RowParams& p,
                                                   uint32_t row, uint32_t* hb) {
  uint32_t b = 0, e = 0;
  if (a.hist_ids) {
    if (a.hist_off) {
      b = a.hist_off[row];
      e = a.hist_off[row + 1];
    } else {
      b = p.hist_begin;
      e = p.hist_begin + p.hist_len;
    }
  }
  *hb = b;
  return e;
}

// The finish kernel covers S for each of the first kTailRows flagged rows in parts of kTailLen
// values; a call with rows that may be flagged runs at least min(kTailGroups, their parts)
// workgroups, the ones past its rows only taking parts. The parts go to the workgroups whose own
// work is expected to cost least: those past the call's rows, then the rows by RowParams::help.
constexpr uint32_t kTailLen = 8192;
constexpr uint32_t kTailRows = as_dev::kTailListMax;
constexpr uint32_t kTailGroups = 256;
__host__ __device__ constexpr uint32_t tail_parts(uint32_t n) { return (n + kTailLen - 1) / kTailLen; }

// The order in which the scan's workgroups take rows: the workgroups of launch row y (grid y) scan
// row r[y]. Workgroups launched earlier hold the older waves of their CU, which the hardware serves
// first, so a slice's time grows with its launch position (about 10% from the first 256 workgroups to
// the last); the host puts the rows it expects to cost most first. At most kOrderMax rows (a larger
// call, or on = 0, takes the rows in order). Passed by value, in the kernel's arguments.
constexpr uint32_t kOrderMax = 1024;
struct RowOrder {
  uint32_t on;
  uint16_t r[kOrderMax];
};

// n_seg slices of slice_len values per row (the last one shorter).
// zero: 1,024 readable floats (the loads of a wave with no full chunk of its slice read there).
// params: the rows' parameter blocks (device memory); args: the finish kernel's arguments, which the
// first workgroup stores at args_out.
hipError_t scan(hipStream_t stream, bool vec, const float* logits, const float* zero, uint64_t row_stride,
                uint32_t n, uint32_t n_rows, uint32_t n_seg, uint32_t slice_len, const as_dev::RowParams* params,
                const FinishArgs& args, FinishArgs* args_out, as_dev::RowShare* share, const uint32_t* hist_off,
                const uint32_t* hist_ids, const uint32_t* extra_ids, as_dev::SegStats* stats, uint64_t* cands,
                uint32_t cand_stride, as_dev::TailList* tail_list, const RowOrder& order);

// A call of at most kDeepHelpRows rows, any of which may take the deep path, runs kTailGroups
// workgroups: those past its rows, and each row's once its row is done, take parts of the rows' deep
// passes until every row is finished.
constexpr uint32_t kDeepHelpRows = 16;
// groups: the call's rows, or more (the workgroups past them only take parts of S's sums and of the
// deep passes).
hipError_t finish(hipStream_t stream, uint32_t groups, const FinishArgs* a);

// Log-probabilities (logprobs.hip): rows in parts, each part's 20 best and sums. Parts of kLpPart
// values spread a part kernel's per-wave work over the most values its registers hold; a call whose
// parts of kLpPartSmall values number under kLpOneRound (the chip's part workgroups at once: 256 CUs,
// 7 each) takes those instead, for twice the workgroups per row.
constexpr uint32_t kLpPart = 16384;
constexpr uint32_t kLpPartSmall = 8192;
constexpr uint32_t kLpOneRound = 1792;
constexpr uint32_t kLpTop = 20;     // logprobs.rs:7, MAX_TOP
constexpr uint32_t kLpMerge = 2048; // the parts' lists a row merges: parts per row * kLpTop at most
__host__ __device__ constexpr uint32_t lp_parts(uint32_t n) { return (n + kLpPart - 1) / kLpPart; }
__host__ __device__ constexpr uint32_t lp_part_len(uint32_t n, uint32_t n_rows) {
  return (uint64_t)n_rows * ((n + kLpPartSmall - 1) / kLpPartSmall) < kLpOneRound &&
                 ((n + kLpPartSmall - 1) / kLpPartSmall) * kLpTop <= kLpMerge
             ? kLpPartSmall
             : kLpPart;
}
// A call's parts per row, and the parts a context holds for any call within its sizes.
__host__ __device__ constexpr uint32_t lp_parts_of(uint32_t n, uint32_t n_rows) {
  return (n + lp_part_len(n, n_rows) - 1) / lp_part_len(n, n_rows);
}
__host__ __device__ constexpr uint64_t lp_capacity(uint32_t max_rows, uint32_t max_vocab) {
  return (uint64_t)max_rows * ((max_vocab + kLpPartSmall - 1) / kLpPartSmall);
}
struct LpPart {
  double sum;         // sum of exp(x - max) over the part
  float max;          // the part's largest value
  uint32_t n_top;     // entries in top
  uint32_t overflow;  // ties past the part's list: the row takes its best by full passes
  uint32_t pad_;
  uint64_t top[kLpTop];  // the part's best, packed (rank key of the logit with -0 as +0, ~id), in order
};
hipError_t logprobs(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride, uint32_t n,
                    uint32_t n_rows, LpPart* parts, const uint32_t* tokens, uint32_t top, float* logprob,
                    uint32_t* top_ids, float* top_lps, uint32_t* status);

hipError_t accept(hipStream_t stream, const uint32_t* picks, const uint32_t* status,
                  const uint32_t* drafts, uint32_t k, const uint32_t* stop_ids, uint32_t n_stop,
                  uint64_t* rng_state, uint32_t draws_per_row, uint32_t* result);

// matvec.hip: y = W x (the reference's matvec, bit for bit), and the same with argmax_rows fused
// (partials: kMatvecGroups u64 of scratch). k at most kMatvecMaxK (x is staged in LDS).
constexpr uint32_t kMatvecGroups = 4096;  // the most workgroups a launch uses
constexpr uint32_t kMatvecMaxK = 8192;
hipError_t matvec(hipStream_t stream, const void* w, uint32_t wtype, uint64_t row_bytes, uint32_t rows, uint32_t k,
                  const float* x, float* y);
hipError_t head_argmax(hipStream_t stream, const void* w, uint32_t wtype, uint64_t row_bytes, uint32_t rows,
                       uint32_t k, const float* x, float* y, uint64_t* partials, uint32_t* ids, uint64_t* rows_out,
                       uint64_t embd, uint32_t embd_row_bytes, uint32_t slot);

// embed.hip: y[t] = the row at rows[t] dequantized (wtype an AS_WTYPE_*, n whole blocks).
hipError_t embed_rows(hipStream_t stream, const uint64_t* rows, uint32_t wtype, uint32_t n, float* y,
                      uint32_t n_tokens);

hipError_t argmax_rows(hipStream_t stream, bool vec, const float* logits, uint64_t row_stride,
                       uint32_t n, uint32_t n_rows, uint32_t* ids, uint64_t* rows_out,
                       uint64_t embd, uint32_t row_bytes, uint32_t slot);

hipError_t debug_exp(hipStream_t stream, const double* x, double* y, uint32_t n);
hipError_t debug_exp2f(hipStream_t stream, const float* x, float* y, uint32_t n);

}  // namespace as_launch

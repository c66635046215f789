// CPU oracle for the token sampler: TEST INFRASTRUCTURE ONLY.
//
// A C++ restatement of the reference's CPU sampler (crates/engine/src/sample.rs, rng.rs,
// logprobs.rs, spec/step.rs:340-385, kernels/src/twin/argmax.rs). Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, as the checker or the
// timed CPU baseline. The product (artemis_amd) never calls it.
//
// Penalties extend the reference's presence penalty (sample.rs:308-323, 351-356, 378-396) to a
// history multiset with repetition and frequency penalties; with repetition 1 and frequency 0 they
// are bit-equal to the reference (see oc_penalize in sampler_oracle.cc).
//
// How each part is pinned (tests/test_oracle_*.py):
//   - rng: the reference's known-answer streams (rng.rs:64-87), an independent restatement, and the
//     below/unit invariants (rng.rs:90-144).
//   - greedy, first_non_finite, argmax_row, check, top_k, draw_full_sort, draw_partial, logprobs:
//     the reference's own sampler tests restated case for case (sample.rs:398-1086), including
//     draw_partial == draw_full_sort and the distribution tests.
//   - verify: the reference's accept-loop tests on integer-valued rows (spec/step.rs:972-1059).
//   - exp / log: the host libm (glibc), compared with Python's math module.
// Parity unpinned:
//   - repetition and frequency penalties: the reference has none; they are pinned only by their
//     definition here, a brute-force recomputation and the reduction to the presence penalty.
//   - absolute token ids on large seeded rows: no reference test fixes them; they rest on following
//     sample.rs line by line.
//   - the libm boundary: no reference test pins exp/ln bits.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// The reference's `Sampling` (sample.rs:38-49) plus the two new penalties.
typedef struct {
  float temp;
  uint32_t top_k;
  float top_p;
  float min_p;
  float presence;
  float frequency;
  float repetition;
  uint32_t pad;
} oc_params;

// rng.rs: xoshiro256** seeded by splitmix64.
void oc_rng_new(uint64_t seed, uint64_t state[4]);
uint64_t oc_rng_next_u64(uint64_t state[4]);
double oc_rng_unit(uint64_t state[4]);
uint64_t oc_rng_below(uint64_t state[4], uint64_t n);  // n > 0

// sample.rs:9-17, 22-34; kernels/src/twin/argmax.rs:8-16 (UINT32_MAX for none).
uint32_t oc_greedy(const float* logits, size_t n);
int64_t oc_first_non_finite(const float* logits, size_t n);  // -1 when all finite
uint32_t oc_argmax_row(const float* logits, size_t n);

// sample.rs:71-94. Returns 0 when accepted, else 1 with a one-line message naming the flag.
int oc_check(const oc_params* p, char* msg, size_t cap);

typedef struct oc_sampler oc_sampler;
oc_sampler* oc_sampler_new(const oc_params* p, uint64_t seed);
void oc_sampler_free(oc_sampler* s);
// Adds ids to the penalty history (each occurrence counts once more).
void oc_sampler_add_history(oc_sampler* s, const uint32_t* ids, size_t n);
void oc_sampler_get_rng(const oc_sampler* s, uint64_t state[4]);
void oc_sampler_set_rng(oc_sampler* s, const uint64_t state[4]);
// sample.rs:122-153. Returns the token; the token joins the history.
uint32_t oc_sampler_sample(oc_sampler* s, const float* logits, size_t n);
// The last draw's kept set in rank order with probabilities w_i / sum(w) at the temperature
// (empty after a greedy pick). Returns the kept count; writes at most `cap` entries.
size_t oc_sampler_last_kept(const oc_sampler* s, uint32_t* ids, double* probs, size_t cap);
// Which path the last sample took: 0 greedy, 1 greedy with penalties, 2 one-pass top-k + full sort,
// 3 every candidate + full sort, 4 partial.
int oc_sampler_last_path(const oc_sampler* s);

// The two draws and the top-k selections on explicit candidates, for the equivalence tests
// (sample.rs:157-198, 208-293, 308-323, 335-372). Candidates are (id, value) pairs.
uint32_t oc_sampler_draw_full_sort(oc_sampler* s, const uint32_t* ids, const float* vals, size_t n);
uint32_t oc_sampler_draw_partial(oc_sampler* s, const uint32_t* ids, const float* vals, size_t n);
// One-pass top-k over logits with the sampler's history penalties; returns the count written.
size_t oc_top_k(const oc_sampler* s, const float* logits, size_t n, size_t k, uint32_t* ids,
                float* vals);
// Selection over every penalized candidate, then sorted (the equivalence the one pass claims).
size_t oc_selected(const oc_sampler* s, const float* logits, size_t n, size_t k, uint32_t* ids,
                   float* vals);
int oc_takes_one_pass(size_t k, size_t n);

// spec/step.rs:340-385 with Picker's stop rule (turn.rs:344-352): rows 0..=k in order, each
// picked by the sampler; stop at the first pick that is a stop id or differs from the next draft.
// `rows` is [k+1][n]. Returns read (rows picked); picks[0..read) are written, *accepted = read-1
// (drafts kept), *stopped = 1 when the last pick was a stop id.
size_t oc_verify(oc_sampler* s, const float* rows, size_t n, const uint32_t* drafts, size_t k,
                 const uint32_t* stop_ids, size_t n_stop, uint32_t* picks, uint32_t* accepted,
                 uint32_t* stopped);

// logprobs.rs:12-38: returns the token's log-probability; writes min(top, 20, n) (id, logprob).
// The CPU baseline's timers (nanoseconds on the calling thread): the non-finite check and one
// sample; or the verify loop over k+1 rows ([k+1][n]), each row checked first.
double oc_sampler_sample_timed(oc_sampler* s, const float* logits, size_t n, uint32_t* token);
double oc_verify_timed(oc_sampler* s, const float* rows, size_t n, const uint32_t* drafts, size_t k,
                       uint32_t* picks, uint32_t* read);
float oc_logprobs(const float* logits, size_t n, uint32_t token, uint32_t top, uint32_t* ids,
                  float* lps, size_t* n_top);

// The exact f64 weight the sampler uses, from the host libm: exp(x).
double oc_exp(double x);
double oc_log(double x);
void oc_exp_array(const double* x, double* y, size_t n);

// A batch of independent rows, each a fresh Sampler(params[r], seeds[r]) with history
// hist_ids[hist_off[r] .. hist_off[r+1]) taking one draw from row r (logits + r * stride; stride 0
// shares one row). Rows are spread over `threads` host threads (1 = this thread). tokens[r] gets
// the draw, or UINT32_MAX for a row holding a non-finite value (the engine refuses such rows
// before sampling). rng_out, when given, gets each row's state after the draw ([rows][4]).
void oc_sample_rows(const oc_params* params, const uint64_t* seeds, const float* logits,
                    size_t stride, size_t n, size_t rows, const uint32_t* hist_off,
                    const uint32_t* hist_ids, unsigned threads, uint32_t* tokens,
                    uint64_t* rng_out);

// crates/qwen36/src/quant.rs:60-252 (quant_oracle.cc): weight types by the reference's codes
// (0 F32, 1 BF16, 2 Q8_0, 3 Q4_K, 4 Q5_K, 5 Q6_K). oc_row_bytes is 0 for an unknown type or a
// row that is not whole blocks; oc_dequant_row returns 1 for those (and writes nothing).
uint64_t oc_row_bytes(uint32_t wtype, uint64_t n);
int oc_dequant_row(uint32_t wtype, const uint8_t* row, uint64_t n, float* out);
float oc_half_to_float(uint16_t h);
// twin/matvec.rs:126-131: y = W x for `rows` rows of k values (k a multiple of 32, whole blocks),
// each output as a 32-lane row of the reference's matvec kernel sums it. 1 for a bad shape.
int oc_matvec(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t k, const float* x, float* y);

#ifdef __cplusplus
}
#endif

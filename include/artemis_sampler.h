/* MI355X (gfx950) token sampler and speculative verify: the C ABI.
 *
 * Replaces the reference's CPU sampler (crates/engine/src/sample.rs), its seed stream
 * (crates/engine/src/rng.rs), the speculative accept loop (crates/engine/src/spec/step.rs:340-385)
 * and the greedy draft kernel (crates/kernels/shaders/argmax_rows.comp) with HIP kernels that read
 * the logits where the output head wrote them, in HBM.
 *
 * Conventions: device pointers are plain `void*`-compatible addresses on the context's device;
 * host pointers are marked `host`. Every launch is ordered on the context's stream. Nothing blocks
 * the host except as_sync() and one bounded wait: as_sample and as_verify stage their rows'
 * parameters in one of two pinned host blocks, so a call made while the call two before it has not
 * started its kernels waits for it (a spin of at most 50 ms, then a wait for the stream).
 * Calls return AS_OK or an AS_ERR_* code, and never throw;
 * as_last_error() gives a one-line message. A context is thread-compatible: one per engine thread
 * (the reference samples on its single worker thread, crates/engine/src/worker.rs:1-5).
 */
#ifndef ARTEMIS_SAMPLER_H
#define ARTEMIS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AS_OK 0
#define AS_ERR_INVALID 1  /* a null pointer, a zero size, or sizes that do not fit together */
#define AS_ERR_PARAMS 2   /* a row's sampling settings fail as_check (as Sampling::check refuses) */
#define AS_ERR_CAPACITY 3 /* more rows, vocabulary or history than the context was made for */
#define AS_ERR_HIP 4      /* a HIP runtime call failed */

/* Per-row status written by as_sample / as_verify. */
#define AS_ROW_OK 0u
#define AS_ROW_NONFINITE 1u /* the row holds a NaN or an infinity: no token, the RNG is not advanced;
                               kept_count holds the first such index (Error::NonFinite,
                               crates/engine/src/decode.rs:439-444) */
/* The row's history holds more ids than the context's max_history: no token, the RNG is not
 * advanced; kept_count holds the row's history length. */
#define AS_ROW_HISTORY 2u
/* OR-ed into the status: the row was settled by the exact-order path (the reference's own
 * summation order), because a fast-path decision fell within its rounding bound or its cut lay
 * deeper than the fast path's candidates. Informational; the token is the same either way. */
#define AS_ROW_EXACT_PATH 0x100u
/* OR-ed into the status: the kept set runs deeper than the values the fast path sorted; the token
 * is exact (the unsorted tail's weight is bounded and cannot change it) and kept_count is a lower
 * bound. Only a call without kept lists (kept_ids null) takes this shortcut: with kept lists, such
 * a row is settled by the deep or exact-order path, so its kept_count, ids and probabilities are the
 * reference's. */
#define AS_ROW_KEPT_PARTIAL 0x200u
/* OR-ed into the status: the cut or the draw lay past the fast path's candidates and a second pass
 * over the row settled it (informational; the token is the reference's either way). */
#define AS_ROW_DEEP_PATH 0x400u
/* OR-ed into the status with AS_ROW_KEPT_PARTIAL: the draw needed one pass over the row to bound
 * the weight of the kept values past the sorted ones (informational). */
#define AS_ROW_TAIL_PASS 0x800u

/* The draft id argmax_rows writes for a row with no finite value
 * (crates/kernels/src/dispatch.rs:61, NO_DRAFT). */
#define AS_NO_DRAFT 0xFFFFFFFFu

/* How the sampler chooses: the reference's Sampling (sample.rs:38-49) plus two penalties it
 * accepts and ignores today (crates/server/src/params.rs:298-328).
 * temp 0 is greedy; top_k 0, top_p 1 and min_p 0 turn their filters off.
 * Penalties act on every id in the row's history with count c >= 1, in f32:
 *   t = (repetition != 1) ? (x > 0 ? x / repetition : x * repetition) : x
 *   x' = t - ((float)c * frequency + presence)
 * With repetition 1 and frequency 0 this is the reference's presence penalty, x - presence
 * (sample.rs:315-321). */
typedef struct {
  float temp;
  uint32_t top_k;
  float top_p;
  float min_p;
  float presence;
  float frequency;
  float repetition;
  uint32_t reserved; /* 0 */
} as_sampling;

typedef struct as_ctx as_ctx;

/* Context: device ordinal, the HIP stream to order work on (NULL = the null stream), and the
 * largest batch, vocabulary and per-row history it must take. The context owns all scratch.
 * max_history: the most history ids one row may carry. as_verify refuses a longer history (with its
 * drafts) with AS_ERR_CAPACITY; as_sample's offsets live on the device, so a longer row there is
 * refused on the device with status AS_ROW_HISTORY. */
int as_create(int device, void* hip_stream, uint32_t max_rows, uint32_t max_vocab,
              uint32_t max_history, as_ctx** out);
int as_destroy(as_ctx* ctx);
const char* as_last_error(const as_ctx* ctx);
/* Waits for the context's stream. */
int as_sync(as_ctx* ctx);

/* Sampling::check (sample.rs:71-94): 0 when the settings are usable, else AS_ERR_PARAMS and a
 * one-line message naming the flag in msg (host). */
int as_check(const as_sampling* s, char* msg, size_t cap);
/* Rng::new (rng.rs:11-23): the 4-word xoshiro256** state for a seed (host). */
void as_rng_seed(uint64_t seed, uint64_t state[4]);

/* One batch of independent rows: Sampler::sample (sample.rs:122-153) on each.
 * Replaces Picker::pick's self.sampler.sample(logits) (crates/engine/src/turn.rs:346) and the
 * non-finite check before it (sample.rs:22-34 via decode.rs:437-447). */
typedef struct {
  const float* logits;          /* [n_rows][row_stride] f32, n_vocab used per row */
  uint64_t row_stride;          /* in floats, >= n_vocab; 0: every row reads the same row */
  uint32_t n_vocab;
  uint32_t n_rows;
  const uint32_t* hist_offsets; /* [n_rows + 1] CSR offsets into hist_ids, or NULL: no history */
  const uint32_t* hist_ids;     /* penalty history per row: ids the sampler returned before */
  uint64_t* rng_state;          /* [n_rows][4] xoshiro256** states, advanced by one draw per
                                   row that draws (temp > 0 and finite) */
  uint32_t* tokens;             /* [n_rows] out */
  uint32_t* status;             /* [n_rows] out: AS_ROW_* */
  uint32_t* kept_count;         /* [n_rows] out or NULL: tokens the draw chose among */
  uint32_t* kept_ids;           /* [n_rows][kept_cap] out or NULL: kept ids in rank order */
  double* kept_probs;           /* [n_rows][kept_cap] out or NULL: w_i / sum(w) at temp */
  uint32_t kept_cap;
} as_batch;

/* params: host array [n_rows]. */
int as_sample(as_ctx* ctx, const as_batch* batch, const as_sampling* params);

/* Speculative verify (spec/step.rs:340-385 with Picker's stop rule, turn.rs:344-352): row i of
 * rows ([k+1][row_stride]) is sampled as the sampler would after emitting drafts[0..i), on the
 * i-th draw of the stream, so all k+1 rows run at once. read = 1 + the first i whose pick is a stop
 * id or differs from drafts[i] (k+1 when none does); accepted = read - 1; bonus = picks[read-1].
 * The stream advances by `read` draws (when temp > 0).
 * history/hist_len: the request's history (device); stop_ids/n_stop (device, may be 0).
 * out: picks [k+1]; result [4] = {read, accepted, bonus, flags} with flags bit 0 = stopped on a
 * stop id, bit 1 = a row was non-finite (read stops before it), bit 8 = the exact-order path ran. */
int as_verify(as_ctx* ctx, const float* rows, uint64_t row_stride, uint32_t n_vocab,
              const uint32_t* drafts, uint32_t k, const uint32_t* history, uint32_t hist_len,
              const uint32_t* stop_ids, uint32_t n_stop, const as_sampling* params,
              uint64_t* rng_state, uint32_t* picks, uint32_t* result);

/* argmax_rows (crates/kernels/src/dispatch.rs:121-153, shaders/argmax_rows.comp): for each of
 * n_rows rows, ids[slot + r] = the largest finite value's index (ties to the lower index) or
 * AS_NO_DRAFT, rows_out[slot + r] = embd + id * row_bytes (id 0 for AS_NO_DRAFT). */
int as_argmax_rows(as_ctx* ctx, const float* logits, uint64_t row_stride, uint32_t n,
                   uint32_t n_rows, uint32_t* ids, uint64_t* rows_out, uint64_t embd,
                   uint32_t row_bytes, uint32_t slot);

/* Weight types of embedding rows, by the reference's codes (crates/kernels/src/lib.rs:438-447,
 * shaders/quant.glsl:2-8): ggml's block layouts (crates/qwen36/src/quant.rs:60-74). */
#define AS_WTYPE_F32 0u
#define AS_WTYPE_BF16 1u
#define AS_WTYPE_Q8_0 2u
#define AS_WTYPE_Q4_K 3u
#define AS_WTYPE_Q5_K 4u
#define AS_WTYPE_Q6_K 5u

/* WType::row_bytes (crates/qwen36/src/quant.rs:66-74): bytes in a row of n values of type wtype;
 * 0 for an unknown type or an n that is not a whole number of the type's blocks (the reference
 * panics there). A host-only function. */
uint64_t as_row_bytes(uint32_t wtype, uint64_t n);

/* embed_rows (crates/kernels/src/dispatch.rs:97-120, shaders/embed_rows.comp): y[t][0..n) = the
 * embedding row at address rows[t] dequantized as dequant_row does (quant.rs:77-252), bit for
 * bit, for t < n_tokens. rows is a device array of n_tokens u64 addresses (argmax_rows writes
 * them); each must be 2-byte aligned and readable by the GPU (an HBM table, or pinned host memory)
 * and hold as_row_bytes(wtype, n) bytes. y: [n_tokens][n] f32 on the device. Stream-ordered.
 * AS_ERR_INVALID for a bad type, an n that is not whole blocks, or null pointers. */
int as_embed_rows(as_ctx* ctx, const uint64_t* rows, uint32_t wtype, uint32_t n, float* y,
                  uint32_t n_tokens);

/* matvec (crates/kernels/src/dispatch.rs Kernels::matvec, shaders/matvec.glsl): y = W x for `rows`
 * rows of k values of type wtype (row r at w + r * as_row_bytes(wtype, k)), each output bit for
 * bit as the reference's kernel and its twin (crates/kernels/src/twin/matvec.rs:86-131) give it.
 * k: a multiple of 32 and of the type's block, at most 8192. w: 4-byte aligned for F32 and BF16,
 * 2-byte aligned for the quantized types; x: [k] f32, y: [rows] f32, device memory. */
int as_matvec(as_ctx* ctx, const void* w, uint32_t wtype, uint32_t rows, uint32_t k, const float* x,
              float* y);

/* The output head with the greedy draft step fused (decode.rs:850 runs the head's matvec, then
 * mtp.rs's argmax_rows reads its logits): as_matvec of the head into `logits` (may be null: the
 * logits are then never written), and, as the outputs are produced, argmax_rows' result:
 * ids[slot] = the largest finite output's row (ties to the lower row, -0 and +0 tied) or
 * AS_NO_DRAFT, rows_out[slot] = embd + id * embd_row_bytes (id 0 for AS_NO_DRAFT), for embed_rows.
 * Stream-ordered; calls on one context must not overlap (they share its scratch). */
int as_head_argmax(as_ctx* ctx, const void* w, uint32_t wtype, uint32_t rows, uint32_t k,
                   const float* x, float* logits, uint32_t* ids, uint64_t* rows_out, uint64_t embd,
                   uint32_t embd_row_bytes, uint32_t slot);

/* Log-probabilities of the model's own distribution (crates/engine/src/logprobs.rs:12-38), which the
 * generation loop asks for per sampled token when a request wants them (turn.rs:361-364): for each of
 * n_rows rows of raw logits (before penalties, temperature and filters; the rows must be finite),
 * logprob[r] = ln softmax(row)[tokens[r]] in f32, and the `top` highest-logit ids with theirs (top
 * clamped to 20 and to n_vocab; 0: none), sorted by logit descending, -0 and +0 tied, ties to the
 * lower id (logprobs.rs:40-48). tokens: device [n_rows]; out: logprob [n_rows], top_ids and
 * top_logprobs [n_rows][top] (the first min(top, 20, n_vocab) of each row written; may be NULL when
 * top is 0), status [n_rows] or NULL: AS_LP_OK (every value the reference's bits), or AS_LP_INEXACT
 * when the bound e on the parallel sum's distance to the reference's left-to-right sum could move a
 * value's rounding to f32, or a token is out of range (its logprob is NaN). The bound is absolute:
 * |lse - lse_ref| <= e = gamma(n + 64) + 1.5e-12 + 2^-51 |ln total| + 2^-52 |lse| (gamma(m) =
 * m 2^-53 / (1 - m 2^-53); about 2.8e-11 at the model's vocabulary), so an inexact value is within
 * e + 2^-51 |lp| + one f32 ulp of the reference's (2^-51 |lp| covering the roundings of the two f64
 * differences x - lse, ours and the reference's), and its exp within about e relative. Near lp = 0
 * (a near-certain token) that can be many f32 ulps: compare log-probabilities bit for bit only on
 * rows whose status is AS_LP_OK. */
#define AS_LP_OK 0u
#define AS_LP_INEXACT 1u
int as_logprobs(as_ctx* ctx, const float* logits, uint64_t row_stride, uint32_t n_vocab, uint32_t n_rows,
                const uint32_t* tokens, uint32_t top, float* logprob, uint32_t* top_ids, float* top_logprobs,
                uint32_t* status);
/* as_logprobs with no allocation and no context. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It runs as_logprobs' kernels, with the same arguments and
 * results, on hip_stream (NULL = the null stream) on the current device. Their scratch is a static
 * device array each GPU holds for the life of the process (2,048 parts of 16,384 values, 368 KiB):
 * n_rows x ceil(n_vocab / 16384) must be at most 2,048 (128 rows at 248,320), else AS_ERR_CAPACITY.
 * Every call on one GPU shares that array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be ordered by the caller. Nothing is allocated and nothing is freed; the
 * device's first call looks the array's address up (hipGetSymbolAddress), so it must be made before
 * any graph capture on that device; later calls only launch the two kernels and may be captured and
 * replayed. err (host, may be NULL) gets a one-line message on failure. */
int as_logprobs_static(void* hip_stream, const float* logits, uint64_t row_stride, uint32_t n_vocab,
                       uint32_t n_rows, const uint32_t* tokens, uint32_t top, float* logprob,
                       uint32_t* top_ids, float* top_logprobs, uint32_t* status, char* err,
                       size_t err_cap);
/* Profiling: while enabled, each as_sample / as_verify records HIP events on the context's stream
 * around its scan and finish kernels (no counterpart in the reference, which samples on the CPU;
 * for benchmarks). as_profile_read waits for the stream and returns the summed kernel times of the
 * calls since as_profile and how many calls there were, then starts a new count; a call that runs no
 * finish kernel (greedy rows without history) adds no finish time. */
int as_profile(as_ctx* ctx, int enable);
int as_profile_read(as_ctx* ctx, double* scan_ms, double* finish_ms, uint32_t* calls);

/* Diagnostics: y[i] = exp(x[i]) on the GPU with the sampler's f64 exp (device arrays). */
int as_debug_exp(as_ctx* ctx, const double* x, double* y, uint32_t n);
/* Diagnostics: y[i] = 2^x[i] by the GPU instruction the scan's error-bounded sums use. */
int as_debug_exp2f(as_ctx* ctx, const float* x, float* y, uint32_t n);

#ifdef __cplusplus
}
#endif

#endif /* ARTEMIS_SAMPLER_H */

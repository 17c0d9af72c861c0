/*
 * rl_sampler.h — C ABI of the MI355X (gfx950) token sampler.
 *
 * This is the boundary a Rust `Sampler` (crates/rust-llm/src/sample.rs) calls
 * through `extern "C"`. The reference has no FFI on this path: its Sampler is a
 * Rust module API (re-exported at crates/rust-llm/src/lib.rs:17). Each entry
 * point below says which part of that API it replaces.
 *
 * Conventions:
 *   - Every pointer argument of rl_sampler_sample_rows, rl_argmax_rows and
 *     rl_top_probability_rows is a DEVICE pointer (HBM). Logits are read, never written: the repetition
 *     penalty is applied virtually, so repeated calls on the same buffer are
 *     idempotent.
 *   - `stream` is a hipStream_t passed as void*; NULL is the default stream.
 *     Calls are stream-ordered and return before the kernels finish.
 *   - Every entry point returns an rl_status; nothing panics or throws across
 *     the ABI. rl_sampler_last_error() gives a message for the calling thread.
 *   - A context is used by one thread and one stream at a time (the
 *     reference's Sampler is `&mut self`, sample.rs:215). A call's scratch
 *     (per-row arrival counters, chunk candidate lists, row state) lives in the
 *     context and calls return before their kernels finish, so two calls on
 *     one context that can overlap on the device (issued to different streams
 *     without an ordering between them) race and can return wrong tokens. Use
 *     one context per stream.
 *   - rl_sampler_configure uploads with a synchronous copy on the null stream,
 *     which does not wait for work on non-blocking streams: call it only once
 *     the context's earlier calls have completed (synchronize their stream
 *     first).
 *   - All device memory a call needs is allocated by rl_sampler_create;
 *     neither configure nor sampling allocates, on the device or the host
 *     (the reference's zero-allocation contract, tests/sample_allocations.rs).
 */
#ifndef RL_SAMPLER_H
#define RL_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* repr(C) mirror of `Sampling` (crates/rust-llm/src/sample.rs:50-67); the
 * reference's usize fields are uint64_t. Field meaning is unchanged:
 *   temperature   <= 0 is greedy (argmax, no draw)            sample.rs:259
 *   top_k         0 = whole vocabulary                          sample.rs:289
 *   top_p         >= 1 (or NaN) is off                          sample.rs:303,314
 *   min_p         <= 0 (or NaN) is off                          sample.rs:326
 *   repeat_penalty, repeat_last_n: active iff penalty != 1 and last_n > 0
 *                                                               sample.rs:82-84
 *   seed          consumed by the host-side Rng, not by the device.
 * Settings are not validated, exactly as the reference's Sampler does not
 * validate them (its callers do: main.rs:648-683, serve.rs:623-660). */
typedef struct rl_sampling {
    float temperature;
    float top_p;
    float min_p;
    float repeat_penalty;
    uint64_t top_k;
    uint64_t repeat_last_n;
    uint64_t seed;
} rl_sampling;

typedef enum rl_status {
    RL_OK = 0,
    RL_ERR_ARGUMENT = 1,       /* a null or out-of-range argument */
    RL_ERR_VOCAB = 2,          /* logits of another vocabulary: the reference
                                * panics here, sample.rs:222-226 */
    RL_ERR_CAPACITY = 3,       /* more rows, window or candidates than sized for */
    RL_ERR_DEVICE = 4,         /* a HIP runtime call failed */
    RL_ERR_NOT_CONFIGURED = 5, /* sample_rows before configure */
} rl_status;

typedef struct rl_sampler_ctx rl_sampler_ctx;

/* Allocates every device buffer for up to `max_rows` logit rows of `vocab`
 * entries and windows of up to `max_window` token ids. Replaces the allocation
 * half of Sampler::new (sample.rs:156-172). `device` is a HIP device index.
 *
 * Windows of any length, as the reference sizes its ring from any
 * repeat_last_n (sample.rs:166; the CLI parses it as any usize, main.rs:604,
 * :641-644). A call whose window_stride is at most 2048 keeps each row's
 * distinct window ids on chip while its logits stream past (an open-addressed
 * set of twice the stride in LDS on the stream path, eight ids a thread on the
 * full path's pass). A longer stride takes the reference's own route
 * (sample.rs:242-257): the call's rows are copied into the context, each
 * window id is penalised in the copy, and the copy is sampled with no window:
 * two more launches and three times the logits' HBM traffic. A context with
 * max_window above 2048 holds that copy, max_rows * vocab floats (rounded up
 * to a multiple of 4 per row). Windows of 65..2048 ids and of 2049 ids up to
 * longer than the vocabulary are tested against the oracle.
 *
 * One limit the reference does not have (RL_ERR_CAPACITY above it):
 *   vocab <= 2^21 (2 097 152). The reference takes any vocabulary
 *     (sample.rs:156-172). Every index and count on the device paths is 32-bit
 *     with this much room; Qwen's 248 320 is far below it.
 *
 * The stream path's window set is sized per call from window_stride, not from
 * max_window, so a context made for long windows costs nothing on calls whose
 * windows are short. */
int rl_sampler_create(int device, uint32_t max_rows, uint32_t vocab, uint32_t max_window,
                      rl_sampler_ctx **out);

/* Frees the context (Drop of Sampler). NULL is accepted. */
void rl_sampler_destroy(rl_sampler_ctx *ctx);

/* Fixes the settings of rows 0..rows-1 (host array, one rl_sampling per row),
 * as Sampler::new fixes a Sampler's settings (sample.rs:48-49). Uploads them
 * and plans which device path each row takes. Synchronous; call it when the
 * batch's settings change, not per step. */
int rl_sampler_configure(rl_sampler_ctx *ctx, const rl_sampling *settings, uint32_t rows);

/* Candidates per row the configured settings can keep: the smallest
 * cand_stride rl_sampler_sample_rows accepts with candidate output on for
 * every configured row. A call over rows 0..n-1 needs only what those rows
 * can keep (1 for greedy rows, top_k for rows with 0 < top_k < vocab, else
 * vocab). */
int rl_sampler_required_cand_stride(const rl_sampler_ctx *ctx, uint64_t *out);

/* Samples rows 0..rows-1 (rows <= configured rows). Replaces Sampler::pick
 * (sample.rs:221-359) batched over rows; the host keeps the Rng and the ring
 * (sample.rs:146-150, :205-219).
 *   logits      [rows][row_stride] f32; row r uses logits[r*row_stride ..+vocab]
 *   vocab       must equal the context's vocabulary (else RL_ERR_VOCAB)
 *   windows     [rows][window_stride] u32: row r's recent-token window, i.e.
 *               recent[..filled] of sample.rs:242, any order; may be NULL when
 *               no row penalises
 *   window_len  [rows] u32: filled for row r (<= window_stride <= max_window)
 *   uniforms    [rows] f32: the value Rng::next_f32 (sample.rs:401) would
 *               return for the row's draw, pre-drawn by the host
 *   out_token   [rows] u32: the picked token
 *   out_kept    [rows] u32: number of candidates kept (Sampler::kept)
 *   out_used_uniform [rows] u8: 1 iff the reference would have drawn from its
 *               Rng for this row (sample.rs:349): 0 for greedy rows and rows
 *               with no finite maximum
 *   out_cand_ids, out_cand_probs [rows][cand_stride]: the survivors and their
 *               normalised probabilities (Sampler::candidates,
 *               sample.rs:188-190); both NULL to skip. The order is the
 *               reference's wherever the reference fixes it: descending logit,
 *               ascending id on ties, when top-p is on (sample.rs:303-305);
 *               id order when top-p is off and top-k keeps the whole
 *               vocabulary (sample.rs:290-296, :326-340). One corner
 *               differs: with top_p >= 1 and 0 < top_k < vocab the reference
 *               leaves its candidates in the order Rust's
 *               select_nth_unstable_by produces (sample.rs:294), which this
 *               library cannot reproduce; it returns them in descending order
 *               instead. The kept set and probabilities are the same, but the
 *               draw walks another order, so the same uniform can pick a
 *               different token there. Greedy rows and rows with top-p on are
 *               unaffected.
 * Returns once the work is queued on `stream`. */
int rl_sampler_sample_rows(rl_sampler_ctx *ctx, const float *logits, uint64_t row_stride,
                           uint32_t rows, uint32_t vocab, const uint32_t *windows,
                           uint32_t window_stride, const uint32_t *window_len,
                           const float *uniforms, uint32_t *out_token, uint32_t *out_kept,
                           uint8_t *out_used_uniform, uint32_t *out_cand_ids,
                           float *out_cand_probs, uint64_t cand_stride, void *stream);

/* Per-row argmax with the reference's tie rule: IEEE '>', lowest id on a tie,
 * NaN never wins, a row with nothing above -inf gives 0. Replaces
 * `pub fn argmax` (sample.rs:118-128), batched. Device pointers; rows <=
 * max_rows of the context; independent of configure. */
int rl_argmax_rows(rl_sampler_ctx *ctx, const float *logits, uint64_t row_stride, uint32_t rows,
                   uint32_t vocab, uint32_t *out_token, void *stream);

/* No counterpart in the reference: rl_argmax_rows without a context, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Its partial results
 * live in a fixed 64 KiB device array inside the library (one copy per GPU,
 * held until the process ends) instead of a context's buffer, so the call
 * allocates nothing, on the device or the host. `device` is the HIP device
 * the logits live on. At most 8192 rows per call (RL_ERR_CAPACITY above).
 * Every call on one GPU shares that array: calls that can overlap on the
 * device (issued to different streams, or from different threads) race and
 * must be serialised by the caller. Results equal rl_argmax_rows's. */
int rl_argmax_rows_noalloc(int device, const float *logits, uint64_t row_stride, uint32_t rows,
                           uint32_t vocab, uint32_t *out_token, void *stream);

/* Per row: the argmax and its probability under a softmax over the whole row,
 * 1 / sum_i exp(l_i - l_best) as f32, with the sum in f64 in id order exactly
 * as the reference accumulates it (bit-identical). Replaces `top_probability`
 * (crates/rust-llm/src/forward.rs:1671-1680, the MTP draft confidence tested
 * against MTP_P_MIN at forward.rs:1014-1015), batched. A row holding a NaN, or
 * nothing above -inf, or +inf, gives a NaN probability, as the reference's sum
 * does. Device pointers; rows <= max_rows; independent of configure. */
int rl_top_probability_rows(rl_sampler_ctx *ctx, const float *logits, uint64_t row_stride, uint32_t rows,
                            uint32_t vocab, uint32_t *out_token, float *out_prob, void *stream);

/* Diagnostic: out[i] = the device's f32 exp of the float whose bit pattern is
 * lo_bits + i, for i < count (device pointer). This is the exp the sampler uses
 * for sample.rs:309's `.exp()`; comparing it with the host's libm expf over a
 * range proves the two agree bit for bit there. */
int rl_sampler_expf_range(uint32_t lo_bits, uint64_t count, float *out, void *stream);

/* A human-readable message for the last failing call on this thread. */
const char *rl_sampler_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* RL_SAMPLER_H */

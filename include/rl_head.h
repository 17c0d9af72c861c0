/*
 * rl_head.h — C ABI of the MI355X (gfx950) output head: device-resident logits
 * from the tied Q6_K embedding, bit-identical to rust-llm's CPU head.
 *
 * The reference's head is `Executor::matmul(Op::Head, &model.token_embd,
 * head_in, &mut bufs.logits[..rows * vocab])` (crates/rust-llm/src/forward.rs:
 * 932-937): it quantizes the normed hidden rows once
 * (crates/llm-core/src/quant.rs:337-375) and takes a Q6_K dot product per
 * (token, vocabulary row) (crates/llm-core/src/kernels/mod.rs:273-300 and its
 * AVX2/VNNI twins, which give the same bits), writing logits token-major
 * (crates/rust-llm/src/pool.rs:468-506). Here the logits land in HBM, where
 * rl_sampler_sample_rows (rl_sampler.h) reads them.
 *
 * Conventions as in rl_sampler.h: status codes, rl_sampler_last_error() for the
 * message, stream-ordered calls that return before the kernels finish, one
 * thread per handle. Every device buffer a call needs is allocated by
 * rl_head_create; rl_head_logits allocates nothing.
 */
#ifndef RL_HEAD_H
#define RL_HEAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rl_head rl_head;

/* Uploads a Q6_K weight tensor of `rows` rows of `k` values (ggml layout: each
 * row is ceil(k/256) blocks of 210 bytes, `ql[128] qh[64] scales[16] d:f16`;
 * q6k_bytes must be rows * ceil(k/256) * 210) from HOST memory, repacks it on
 * the device into the layout the head kernel streams (same byte count), and
 * sizes the activation scratch for up to `max_batch` rows per call. Replaces
 * the memory-mapped tensor view the reference's head reads (`model.token_embd`,
 * forward.rs:934; TensorView, crates/llm-core/src/gguf.rs:190-197).
 * Synchronous. */
int rl_head_create(int device, uint32_t k, uint32_t rows, uint32_t max_batch, const void *q6k,
                   uint64_t q6k_bytes, rl_head **out);

/* Frees the handle. NULL is accepted. */
void rl_head_destroy(rl_head *head);

/* logits[tt * row_stride + r] = the head's output for token tt and vocabulary
 * row r, for tt < t and r < rows, from x [t][k] f32 (device pointers). The
 * same bits as the reference's Op::Head matmul (forward.rs:932-937) for any t:
 * a batch gives each row what it gives alone (kernels/mod.rs:208-217). t <= max_batch;
 * row_stride >= rows. */
int rl_head_logits(rl_head *head, const float *x, uint32_t t, float *logits, uint64_t row_stride,
                   void *stream);

/* The embedding lookup from the same resident tensor (the tied `token_embd`):
 * out[i * row_stride + j] = row tokens[i] of the tensor expanded to f32, for
 * i < t and j < k, the same bits as the reference's Exec::embed
 * (crates/rust-llm/src/forward.rs:1127-1138), which is dequantize_row's Q6_K
 * arm (crates/llm-core/src/quant.rs:177-203). tokens [t] u32 and out are device
 * pointers, so a token the sampler drew in HBM feeds the next step without a
 * host round trip; row_stride >= k. The reference asserts a token is below
 * `rows`; a device kernel cannot stop, so such a token's row is written as NaN.
 * Columns past k in a padded row are not written. */
int rl_head_embed_rows(rl_head *head, const uint32_t *tokens, uint32_t t, float *out, uint64_t row_stride,
                       void *stream);

/* Activations::quantize_batch (quant.rs:337-375) on the device, for any k:
 * x [t][k] f32 into nb = ceil(k/256) blocks per row, written as the reference's
 * ActBlock fields (quant.rs:233-237): out_d [t][nb] f32, out_qs [t][nb*256]
 * int8 (zero past k), out_bsums [t][nb][16] int16. Device pointers; any of the
 * three outputs may be NULL. */
int rl_quantize_rows(const float *x, uint32_t t, uint32_t k, float *out_d, int8_t *out_qs,
                     int16_t *out_bsums, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RL_HEAD_H */

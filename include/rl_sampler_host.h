/*
 * rl_sampler_host.h — the reference's Sampler API (crates/rust-llm/src/sample.rs)
 * as a host-side object over the device ABI of rl_sampler.h.
 *
 * The reference's Rust `Sampler` owns its settings, the recent-token ring and
 * the Rng (sample.rs:132-151). Here the host object keeps exactly those and
 * hands the per-token work to the GPU: it pre-draws the uniform from a clone of
 * its Rng, uploads the window, runs rl_sampler_sample_rows, then commits the
 * Rng advance only if the device says the row drew (sample.rs:349), and
 * remembers the picked token (sample.rs:215-219). A Rust wrapper holds the same
 * state; these C functions are what the C++ host mirror exports so it can be
 * driven and tested without Rust.
 */
#ifndef RL_SAMPLER_HOST_H
#define RL_SAMPLER_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "rl_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Rng: xoshiro256++ seeded through splitmix64, sample.rs:368-404 ---- */
typedef struct rl_rng {
    uint64_t s[4];
} rl_rng;

void rl_rng_seeded(rl_rng *r, uint64_t seed);        /* Rng::seeded, sample.rs:373-385 */
uint64_t rl_rng_next_u64(rl_rng *r);                  /* Rng::next_u64, sample.rs:387-398 */
float rl_rng_next_f32(rl_rng *r);                     /* Rng::next_f32, sample.rs:401-403 */

/* Sampling::default() (sample.rs:88-100) and Sampling::GREEDY (:71-79). */
rl_sampling rl_sampling_default(void);
rl_sampling rl_sampling_greedy(void);

/* entropy_seed (sample.rs:107-112): a seed from the OS's entropy. */
uint64_t rl_entropy_seed(void);

/* argmax (sample.rs:118-128) over host memory, computed on the GPU. */
int rl_host_argmax(int device, const float *logits, size_t n, uint32_t *out);

/* ---- Sampler (sample.rs:132-219) ---- */
typedef struct rl_host_sampler rl_host_sampler;

/* Sampler::new(vocab, set) (sample.rs:156-172): allocates everything,
 * including device buffers for up to `max_rows` rows per call (1 for plain
 * sampling; draft+1 for verify; the batch size for rl_host_sample_batch, where
 * the first sampler's buffers serve the whole batch, so a sampler made with
 * max_rows > 1 sizes its candidate buffers for the whole vocabulary). */
int rl_host_sampler_new(int device, size_t vocab, const rl_sampling *set, uint32_t max_rows,
                        rl_host_sampler **out);
void rl_host_sampler_free(rl_host_sampler *s);
rl_sampling rl_host_sampler_settings(const rl_host_sampler *s);    /* sample.rs:180-182 */
void rl_host_sampler_reset(rl_host_sampler *s);                    /* sample.rs:194-198 */
void rl_host_sampler_remember(rl_host_sampler *s, uint32_t token); /* sample.rs:205-212 */

/* Sampler::sample (sample.rs:215-219) over host logits (copied to the GPU
 * first) or over one device row. RL_ERR_VOCAB where the reference panics. */
int rl_host_sampler_sample(rl_host_sampler *s, const float *host_logits, size_t n, uint32_t *token);
int rl_host_sampler_sample_device(rl_host_sampler *s, const float *device_row, size_t n,
                                  uint32_t *token, void *stream);

/* Sampler::candidates (sample.rs:188-190): pointers into the sampler's host
 * copy of the last call's survivors; returns how many. */
size_t rl_host_sampler_candidates(const rl_host_sampler *s, const uint32_t **ids, const float **probs);

/* The Rng state, for replay checks. */
void rl_host_sampler_rng(const rl_host_sampler *s, rl_rng *out);

/* Speculative verify (generate.rs:412-450) in one device call: rows
 * 0..n_drafts of device logits, where row i follows drafts 0..i-1. Row i is
 * sampled with the window the sampler would hold after accepting drafts
 * 0..i-1 and with the uniform it would draw next if every earlier row drew.
 * Nothing is committed: the picks land in `picks` (n_drafts+1 entries) and the
 * caller commits rows in order with rl_host_sampler_commit_verified, stopping
 * after the first row whose committed token differs from its draft, exactly
 * as the generation loop consumes them. */
int rl_host_sampler_verify(rl_host_sampler *s, const float *device_rows, uint64_t row_stride,
                           size_t n, const uint32_t *drafts, uint32_t n_drafts, uint32_t *picks,
                           void *stream);
/* Commits row `row` of the last verify (rows must be committed 0, 1, 2, ...):
 * remembers its token, advances the Rng if it drew, and makes its survivors
 * the sampler's candidates. The committed token is written to *token: it is
 * the verify pick unless an earlier committed row drew nothing (no finite
 * maximum, sample.rs:270-277), in which case the stream gives this row another
 * uniform and the row is sampled again with it. Row r > 0 was sampled with the
 * window that assumes drafts[0..r) were accepted, so it can only be committed
 * while the token committed for row r-1 equals drafts[r-1] (the generation
 * loop stops at the first mismatch, generate.rs:412-429): otherwise
 * RL_ERR_ARGUMENT and nothing changes. A sample, batch or reset call in
 * between abandons the verify. No call here allocates host or device memory
 * (everything is sized by rl_host_sampler_new). */
int rl_host_sampler_commit_verified(rl_host_sampler *s, uint32_t row, uint32_t *token);

/* ---- Batched serving: one device call over many samplers ---- */
/* Samples samplers[i] on device row i (logits + i*row_stride), as n separate
 * Sampler::sample calls would, in one launch. All samplers share the vocab;
 * the call uses samplers[0]'s device context, sized by its max_rows. */
int rl_host_sample_batch(rl_host_sampler *const *samplers, uint32_t n, const float *device_logits,
                         uint64_t row_stride, size_t vocab, uint32_t *tokens, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RL_SAMPLER_HOST_H */

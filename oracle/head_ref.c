/*
 * ORACLE — test infrastructure only.
 *
 * A CPU restatement, in plain C, of rust-llm's output head: the tied
 * `token_embd` Q6_K matrix times the normed hidden rows
 * (crates/rust-llm/src/forward.rs:932-937, `Executor::matmul(Op::Head, ..)`),
 * which quantizes the activations once (forward.rs:1165 →
 * crates/llm-core/src/quant.rs:337-375 `Activations::quantize_batch`) and then
 * takes one dot product per (token, vocabulary row) with the scalar Q6_K kernel
 * (crates/llm-core/src/kernels/mod.rs:273-300 `q6k_dot_scalar`), writing the
 * logits token-major (crates/rust-llm/src/pool.rs:468-506). Only tests/ and
 * bench.py's CPU-baseline leg load this; the head that ships is the HIP
 * library under rust-llm_amd/.
 *
 * Bits: the reference's three CPU tiers (scalar, AVX2, AVX-VNNI) give the same
 * bits (kernels/avx2.rs:480-523 states the epilogues perform the scalar line's
 * operations in its order), because every block's integer sum is exact and the
 * f32 line is fixed: `sum += (act.d * w.d) * (float)isum`, blocks in order,
 * from 0.0. Built with -ffp-contract=off so nothing is fused.
 *
 * Parity status (see tests/test_head.py):
 *   orc_quantize_rows  pinned: known answers (rows of +/-amax give +/-127;
 *                      zero rows give d = 0 and all-zero quants; NaN ignored by
 *                      the maximum and quantized to 0; halves round away from
 *                      zero), and a numpy restatement on random rows.
 *   orc_dequantize_row pinned: the reference tests' own check against a
 *                      dequantization written out again in the test, within
 *                      1e-6 relative (crates/llm-core/tests/kernels.rs:633-668);
 *                      exact known answers (d = 1 gives the integers s*(q-32),
 *                      a power-of-two d scales them exactly); elements past k
 *                      untouched.
 *   orc_q6k_matvec     pinned: the reference tests' own check, an f64 dot of
 *                      the dequantized ggml layout within 1e-5 of the absolute
 *                      terms (crates/llm-core/tests/kernels.rs:130-200); exact
 *                      known answers on the saturation fixtures
 *                      (kernels.rs:430-560); zero weights and zero activations
 *                      give 0; a tail block past k adds nothing; and a numpy
 *                      restatement of the AVX2 tier's decomposition (unsigned
 *                      6-bit quants minus 32 times the group sums), bit for bit.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK 256
#define Q6K_BYTES 210

/* IEEE binary16 → binary32, exact (every f16 is an f32); the reference reads
 * the block scale with half::f16::to_f32 (quant.rs:120-122). */
static float f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        /* subnormal: value man * 2^-24, normalised */
        int e = -1;
        do {
            man <<= 1;
            e++;
        } while ((man & 0x400) == 0);
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FF) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* One quant: (v * id).round().clamp(-127, 127) as i8 (quant.rs:368-370).
 * Rust's round is half away from zero (C roundf); clamp passes NaN through and
 * `as i8` turns NaN into 0. */
static int8_t quant_one(float v, float id)
{
    float p = v * id;
    float r = roundf(p);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    if (r != r) return 0;
    return (int8_t)r;
}

/* Activations::quantize_batch (quant.rs:337-375): t rows of k values into
 * ceil(k/256) blocks per row. d[t][nb], qs[t][nb*256] (zero past k),
 * bsums[t][nb][16]. */
void orc_quantize_rows(const float *x, size_t t, size_t k, float *d, int8_t *qs, int16_t *bsums)
{
    size_t nb = (k + QK - 1) / QK;
    for (size_t r = 0; r < t; r++) {
        const float *src = x + r * k;
        for (size_t b = 0; b < nb; b++) {
            size_t n = k - b * QK < QK ? k - b * QK : QK;
            const float *chunk = src + b * QK;
            float amax = 0.0f;
            for (size_t i = 0; i < n; i++) amax = fmaxf(amax, fabsf(chunk[i])); /* NaN ignored, as f32::max */
            float dd = amax / 127.0f;
            float id = amax > 0.0f ? 127.0f / amax : 0.0f;
            int8_t *q = qs + (r * nb + b) * QK;
            memset(q, 0, QK);
            for (size_t i = 0; i < n; i++) q[i] = quant_one(chunk[i], id);
            int16_t *bs = bsums + (r * nb + b) * 16;
            for (int i = 0; i < 16; i++) {
                int s = 0;
                for (int j = 0; j < 16; j++) s += q[i * 16 + j];
                bs[i] = (int16_t)s;
            }
            d[r * nb + b] = dd;
        }
    }
}

/* q6k_dot_scalar (kernels/mod.rs:273-300): one weight row of nb blocks against
 * one activation row. The weight quant of activation index
 * h*128 + g*32 + l is ggml's 6-bit value minus 32, with sub-block scale
 * sc[h*8 + 2g + l/16]. */
static float q6k_dot(const uint8_t *w, size_t nb, const float *ad, const int8_t *aq)
{
    float sum = 0.0f;
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *b = w + ib * Q6K_BYTES;
        const uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
        float dw = f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        const int8_t *a = aq + ib * QK;
        int32_t isum = 0;
        for (int h = 0; h < 2; h++) {
            const uint8_t *qlh = ql + h * 64, *qhh = qh + h * 32;
            for (int g = 0; g < 4; g++) {
                for (int l = 0; l < 32; l++) {
                    int low;
                    switch (g) {
                    case 0: low = qlh[l] & 0xF; break;
                    case 1: low = qlh[32 + l] & 0xF; break;
                    case 2: low = qlh[l] >> 4; break;
                    default: low = qlh[32 + l] >> 4; break;
                    }
                    int q = (low | (((qhh[l] >> (2 * g)) & 3) << 4)) - 32;
                    int s = (int8_t)sc[h * 8 + 2 * g + l / 16];
                    isum += s * q * a[h * 128 + g * 32 + l];
                }
            }
        }
        float scale = ad[ib] * dw;
        float term = scale * (float)isum;
        sum = sum + term;
    }
    return sum;
}

/* The head for rows [row_lo, row_hi) of a [rows][nb*210] Q6_K tensor: quantize
 * the t activation rows of x [t][k], then out[tt][r - row_lo] for every token
 * tt, token-major (pool.rs:491-503 writes out[(t0 + j) * rows + r]). */
int orc_q6k_matvec(const uint8_t *w, size_t k, size_t row_lo, size_t row_hi, const float *x, size_t t,
                   float *out)
{
    size_t nb = (k + QK - 1) / QK;
    float *d = malloc(sizeof(float) * t * nb);
    int8_t *qs = malloc((size_t)QK * t * nb);
    int16_t *bs = malloc(sizeof(int16_t) * 16 * t * nb);
    if (!d || !qs || !bs) {
        free(d);
        free(qs);
        free(bs);
        return -1;
    }
    orc_quantize_rows(x, t, k, d, qs, bs);
    size_t n = row_hi - row_lo;
    for (size_t r = row_lo; r < row_hi; r++) {
        const uint8_t *row = w + r * nb * Q6K_BYTES;
        for (size_t tt = 0; tt < t; tt++)
            out[tt * n + (r - row_lo)] = q6k_dot(row, nb, d + tt * nb, qs + tt * nb * QK);
    }
    free(d);
    free(qs);
    free(bs);
    return 0;
}

/* dequantize_row's Q6_K arm (crates/llm-core/src/quant.rs:177-203): the
 * embedding lookup (crates/rust-llm/src/forward.rs:1127-1138) of one row of k
 * values: out[i] = d * (float)(s * (q - 32)), the integer product exact and
 * one f32 multiply. Elements past k are not written. */
void orc_dequantize_row(const uint8_t *w, size_t k, float *out)
{
    size_t nb = (k + QK - 1) / QK;
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *b = w + ib * Q6K_BYTES;
        const uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
        float d = f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        for (int h = 0; h < 2; h++) {
            const uint8_t *qlh = ql + h * 64, *qhh = qh + h * 32;
            for (int g = 0; g < 4; g++) {
                for (int l = 0; l < 32; l++) {
                    int low;
                    switch (g) {
                    case 0: low = qlh[l] & 0xF; break;
                    case 1: low = qlh[32 + l] & 0xF; break;
                    case 2: low = qlh[l] >> 4; break;
                    default: low = qlh[32 + l] >> 4; break;
                    }
                    int q = (low | (((qhh[l] >> (2 * g)) & 3) << 4)) - 32;
                    int s = (int8_t)sc[h * 8 + 2 * g + l / 16];
                    size_t at = ib * QK + (size_t)(h * 128 + g * 32 + l);
                    if (at < k) out[at] = d * (float)(s * q);
                }
            }
        }
    }
}

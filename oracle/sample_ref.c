/*
 * ORACLE — test infrastructure only.
 *
 * A CPU restatement, in plain C, of rust-llm's token sampler
 * (crates/rust-llm/src/sample.rs) and of the naive f64 reference its tests
 * compare against (crates/rust-llm/tests/sample.rs:16-83). Only tests/, the
 * smoke check and bench.py's CPU-baseline leg load this library; the sampler
 * that ships is the HIP library under rust-llm_amd/.
 *
 * Arithmetic follows the reference exactly: f32 where Rust uses f32, f64
 * where it widens, sequential sums in candidate order, libm expf (which is
 * what Rust's f32::exp calls on x86_64 linux-gnu), IEEE division. Build with
 * -ffp-contract=off and no fast-math so no expression is fused or reordered.
 *
 * Parity status per function (how each is pinned, see tests/):
 *   orc_rng_*        pinned: published xoshiro256++ and splitmix64 vectors.
 *   orc_argmax       pinned: known answers of sample.rs:411-415,
 *                    tests/sample.rs:244-252, plus brute force.
 *   penalty/window   pinned: known answers sample.rs:442-460,
 *                    tests/sample.rs:317-329, :417-460.
 *   selection/order  pinned: brute-force full sort under the same total order
 *                    (the order is total, so the kept set and the sorted order
 *                    are unique).
 *   exp/sums/cut/draw pinned: the naive f64 reference (tests/sample.rs:16-83)
 *                    on 72 cases, edge counts tests/sample.rs:351-412, draw
 *                    frequencies tests/sample.rs:464-504.
 *   orc_top_probability  pinned: known answers with exact results (equal
 *                    logits: 1/n; one finite logit among -inf: 1), its NaN
 *                    and infinity cases, and a step-by-step recomputation
 *                    (Python float additions of this library's expf).
 *   One corner is parity unpinned: with top_p >= 1 and 0 < top_k < vocab the
 *   reference walks the candidates in the order Rust's select_nth_unstable_by
 *   leaves them (sample.rs:294, :349-356). That order is an implementation
 *   detail of Rust's core library; this restatement walks them in the
 *   descending total order instead.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Same layout as rl_sampling in include/rl_sampler.h; mirrors Sampling
 * (sample.rs:50-67) with usize as uint64_t. */
typedef struct orc_sampling {
    float temperature;
    float top_p;
    float min_p;
    float repeat_penalty;
    uint64_t top_k;
    uint64_t repeat_last_n;
    uint64_t seed;
} orc_sampling;

/* ---------------------------------------------------------------- Rng ---- */
/* sample.rs:368-404: xoshiro256++ seeded through splitmix64. */
typedef struct orc_rng {
    uint64_t s[4];
} orc_rng;

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t orc_splitmix64_next(uint64_t *z) {
    *z += 0x9E3779B97F4A7C15ull;
    uint64_t v = *z;
    v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
    v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
    return v ^ (v >> 31);
}

void orc_rng_seeded(orc_rng *r, uint64_t seed) { /* sample.rs:373-385 */
    uint64_t z = seed;
    for (int i = 0; i < 4; i++) r->s[i] = orc_splitmix64_next(&z);
}

void orc_rng_from_state(orc_rng *r, const uint64_t s[4]) {
    for (int i = 0; i < 4; i++) r->s[i] = s[i];
}

uint64_t orc_rng_next_u64(orc_rng *r) { /* sample.rs:387-398 */
    uint64_t *s = r->s;
    uint64_t out = rotl64(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return out;
}

float orc_rng_next_f32(orc_rng *r) { /* sample.rs:401-403 */
    return (float)(orc_rng_next_u64(r) >> 40) / (float)(1u << 24);
}

/* ------------------------------------------------------------- argmax ---- */
/* sample.rs:118-128: IEEE '>', lowest id on a tie, NaN never wins. */
uint32_t orc_argmax(const float *l, size_t n) {
    size_t best = 0;
    float best_v = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (l[i] > best_v) {
            best_v = l[i];
            best = i;
        }
    }
    return (uint32_t)best;
}

/* ------------------------------------------------------ total order ---- */
/* f32::total_cmp as an unsigned key: larger key = later in total order. */
static inline uint32_t total_key(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

/* Descending logit, then ascending id (sample.rs:282-286), as one u64 that
 * sorts descending: the key above, then the complemented id. */
static inline uint64_t composite(const float *l, uint32_t id) {
    return ((uint64_t)total_key(l[id]) << 32) | (uint32_t)~id;
}

static void swap64(uint64_t *a, uint64_t *b) {
    uint64_t t = *a;
    *a = *b;
    *b = t;
}

/* Puts the kth largest (0-based) at a[kth], larger ones before it. Keys are
 * unique, so the set a[0..=kth] is unique too. */
static void select_desc(uint64_t *a, size_t n, size_t kth) {
    size_t lo = 0, hi = n - 1;
    while (hi > lo) {
        if (hi - lo < 16) { /* insertion sort the small remainder */
            for (size_t i = lo + 1; i <= hi; i++) {
                uint64_t v = a[i];
                size_t j = i;
                while (j > lo && a[j - 1] < v) {
                    a[j] = a[j - 1];
                    j--;
                }
                a[j] = v;
            }
            return;
        }
        size_t mid = lo + (hi - lo) / 2;
        /* median of three, descending */
        if (a[mid] > a[lo]) swap64(&a[mid], &a[lo]);
        if (a[hi] > a[lo]) swap64(&a[hi], &a[lo]);
        if (a[hi] > a[mid]) swap64(&a[hi], &a[mid]);
        uint64_t pivot = a[mid];
        size_t i = lo, j = hi;
        while (i <= j) {
            while (a[i] > pivot) i++;
            while (a[j] < pivot) j--;
            if (i <= j) {
                swap64(&a[i], &a[j]);
                i++;
                if (j == 0) break;
                j--;
            }
        }
        if (kth <= j)
            hi = j;
        else if (kth >= i)
            lo = i;
        else
            return;
    }
}

static int cmp_desc(const void *pa, const void *pb) {
    uint64_t a = *(const uint64_t *)pa, b = *(const uint64_t *)pb;
    return (a < b) - (a > b);
}

static void sort_desc(uint64_t *a, size_t n) {
    if (n < 32) {
        for (size_t i = 1; i < n; i++) {
            uint64_t v = a[i];
            size_t j = i;
            while (j > 0 && a[j - 1] < v) {
                a[j] = a[j - 1];
                j--;
            }
            a[j] = v;
        }
        return;
    }
    qsort(a, n, sizeof(uint64_t), cmp_desc);
}

/* -------------------------------------------------- the pipeline ---- */
/* Scratch a pick needs, sized from the vocabulary once (the reference sizes
 * every buffer in Sampler::new, sample.rs:156-172). */
typedef struct orc_scratch {
    size_t vocab;
    float *penalized; /* sample.rs:139 */
    uint64_t *keys;   /* the index vector of sample.rs:142, as composite keys */
    uint32_t *idx;
    float *probs;     /* sample.rs:144 */
} orc_scratch;

orc_scratch *orc_scratch_new(size_t vocab) {
    orc_scratch *s = calloc(1, sizeof *s);
    if (!s) return NULL;
    s->vocab = vocab;
    s->penalized = malloc(vocab * sizeof(float) + 4);
    s->keys = malloc(vocab * sizeof(uint64_t) + 8);
    s->idx = malloc(vocab * sizeof(uint32_t) + 4);
    s->probs = malloc(vocab * sizeof(float) + 4);
    if (!s->penalized || !s->keys || !s->idx || !s->probs) {
        free(s->penalized);
        free(s->keys);
        free(s->idx);
        free(s->probs);
        free(s);
        return NULL;
    }
    return s;
}

void orc_scratch_free(orc_scratch *s) {
    if (!s) return;
    free(s->penalized);
    free(s->keys);
    free(s->idx);
    free(s->probs);
    free(s);
}

static int penalises(const orc_sampling *set) { /* sample.rs:82-84 */
    return set->repeat_penalty != 1.0f && set->repeat_last_n > 0;
}

/*
 * One pick over one row: sample.rs:221-359 with the recent-token window given
 * as recent[..filled] (any order: the penalty is per distinct id) and the
 * uniform given instead of drawn. *used_uniform says whether the reference
 * would have consumed it (sample.rs:349). Candidates land in s->idx/s->probs.
 * Returns the token, or UINT32_MAX on a vocabulary mismatch (the reference
 * panics there, sample.rs:222-226).
 */
uint32_t orc_pick(orc_scratch *s, const float *raw, size_t n, const orc_sampling *set,
                  const uint32_t *recent, size_t filled, float u, size_t *kept,
                  int *used_uniform) {
    if (n != s->vocab) return UINT32_MAX;
    *used_uniform = 0;
    uint32_t *idx = s->idx;
    float *probs = s->probs;

    /* Repetition penalty, once per distinct id, f32 (sample.rs:239-257). */
    int penalty = penalises(set) && filled > 0;
    const float *logits = raw;
    if (penalty) {
        memcpy(s->penalized, raw, n * sizeof(float));
        for (size_t i = 0; i < filled; i++) {
            uint32_t t = recent[i];
            int seen = 0;
            for (size_t j = 0; j < i; j++)
                if (recent[j] == t) {
                    seen = 1;
                    break;
                }
            if (seen) continue;
            if ((size_t)t < n) {
                float v = s->penalized[t];
                s->penalized[t] = v > 0.0f ? v / set->repeat_penalty : v * set->repeat_penalty;
            }
        }
        logits = s->penalized;
    }

    /* Greedy (sample.rs:259-265). */
    if (set->temperature <= 0.0f) {
        uint32_t token = orc_argmax(logits, n);
        idx[0] = token;
        probs[0] = 1.0f;
        *kept = 1;
        return token;
    }

    /* f32::max fold, NaN ignored; no finite maximum gives argmax
     * (sample.rs:267-277). */
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, logits[i]);
    if (!isfinite(max)) {
        uint32_t token = orc_argmax(logits, n);
        idx[0] = token;
        probs[0] = 1.0f;
        *kept = 1;
        return token;
    }

    /* top-k under the total order (sample.rs:279-305). */
    size_t k = set->top_k == 0 ? n : (set->top_k < n ? (size_t)set->top_k : n);
    if (k == n && !(set->top_p < 1.0f)) {
        /* No truncation and no order needed: the identity order of
         * sample.rs:290-292 is what the draw walks. */
        for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
    } else {
        uint64_t *keys = s->keys;
        for (size_t i = 0; i < n; i++) keys[i] = composite(logits, (uint32_t)i);
        if (k < n) select_desc(keys, n, k - 1);
        /* The reference sorts only when top_p < 1; with top_p >= 1 and k < n it
         * walks select_nth's order, which this restatement replaces with the
         * descending order (the unpinned corner named in the header). */
        sort_desc(keys, k);
        for (size_t i = 0; i < k; i++) idx[i] = ~(uint32_t)keys[i];
    }

    /* exp and the f64 mass, sequential in candidate order (sample.rs:307-311). */
    double sum = 0.0;
    for (size_t j = 0; j < k; j++) {
        float d = logits[idx[j]] - max;
        float q = d / set->temperature;
        float p = expf(q);
        probs[j] = p;
        sum += (double)p;
    }

    /* top-p (sample.rs:313-324). */
    size_t m = k;
    if (set->top_p < 1.0f) {
        double target = (double)set->top_p * sum;
        double cum = 0.0;
        for (size_t j = 0; j < k; j++) {
            cum += (double)probs[j];
            if (cum >= target) {
                m = j + 1;
                break;
            }
        }
    }

    /* min-p (sample.rs:326-340). */
    if (set->min_p > 0.0f) {
        size_t w = 0;
        for (size_t j = 0; j < m; j++) {
            if (probs[j] >= set->min_p) {
                idx[w] = idx[j];
                probs[w] = probs[j];
                w++;
            }
        }
        m = w > 1 ? w : 1;
    }

    /* Normalise (sample.rs:342-347). */
    double total = 0.0;
    for (size_t j = 0; j < m; j++) total += (double)probs[j];
    float inv = (float)(1.0 / total);
    for (size_t j = 0; j < m; j++) probs[j] *= inv;
    *kept = m;

    /* The draw (sample.rs:349-358). */
    *used_uniform = 1;
    float cum = 0.0f;
    for (size_t j = 0; j < m; j++) {
        cum += probs[j];
        if (cum > u) return idx[j];
    }
    return idx[m - 1];
}

const uint32_t *orc_scratch_ids(const orc_scratch *s) { return s->idx; }
const float *orc_scratch_probs(const orc_scratch *s) { return s->probs; }

/* Rows in a batch: row r reads logits + r*stride, its window
 * windows + r*wstride (wlen[r] entries) and uniforms[r]. Candidates are copied
 * out up to cand_cap per row. Returns 0, or -1 on allocation failure or a
 * vocabulary mismatch. */
int orc_pick_rows(const float *logits, uint64_t stride, size_t rows, size_t n,
                  const orc_sampling *settings, int per_row_settings, const uint32_t *windows,
                  size_t wstride, const uint32_t *wlen, const float *uniforms,
                  uint32_t *out_token, uint32_t *out_kept, uint8_t *out_used,
                  uint32_t *out_ids, float *out_probs, size_t cand_cap) {
    orc_scratch *s = orc_scratch_new(n);
    if (!s) return -1;
    for (size_t r = 0; r < rows; r++) {
        const orc_sampling *set = per_row_settings ? &settings[r] : settings;
        size_t kept = 0;
        int used = 0;
        uint32_t tok = orc_pick(s, logits + r * stride, n, set,
                                windows ? windows + r * wstride : NULL, wlen ? wlen[r] : 0,
                                uniforms ? uniforms[r] : 0.0f, &kept, &used);
        if (tok == UINT32_MAX) {
            orc_scratch_free(s);
            return -1;
        }
        out_token[r] = tok;
        out_kept[r] = (uint32_t)kept;
        out_used[r] = (uint8_t)used;
        if (out_ids) {
            size_t c = kept < cand_cap ? kept : cand_cap;
            memcpy(out_ids + r * cand_cap, s->idx, c * sizeof(uint32_t));
            memcpy(out_probs + r * cand_cap, s->probs, c * sizeof(float));
        }
    }
    orc_scratch_free(s);
    return 0;
}

/* ------------------------------------------------------- the Sampler ---- */
/* The stateful object of sample.rs:132-219: settings, ring window, Rng. */
typedef struct orc_sampler {
    orc_sampling set;
    size_t vocab;
    orc_scratch *scratch;
    uint32_t *recent;
    size_t recent_len, at, filled, kept;
    orc_rng rng;
} orc_sampler;

orc_sampler *orc_sampler_new(size_t vocab, const orc_sampling *set) {
    orc_sampler *s = calloc(1, sizeof *s);
    if (!s) return NULL;
    s->set = *set;
    s->vocab = vocab;
    s->scratch = orc_scratch_new(vocab);
    s->recent_len = (size_t)set->repeat_last_n;
    s->recent = calloc(s->recent_len + 1, sizeof(uint32_t));
    if (!s->scratch || !s->recent) {
        orc_scratch_free(s->scratch);
        free(s->recent);
        free(s);
        return NULL;
    }
    orc_rng_seeded(&s->rng, set->seed);
    return s;
}

void orc_sampler_free(orc_sampler *s) {
    if (!s) return;
    orc_scratch_free(s->scratch);
    free(s->recent);
    free(s);
}

void orc_sampler_reset(orc_sampler *s) { /* sample.rs:194-198 */
    s->at = 0;
    s->filled = 0;
    s->kept = 0;
}

void orc_sampler_remember(orc_sampler *s, uint32_t token) { /* sample.rs:205-212 */
    if (s->recent_len == 0) return;
    s->recent[s->at] = token;
    s->at = (s->at + 1) % s->recent_len;
    s->filled = s->filled + 1 < s->recent_len ? s->filled + 1 : s->recent_len;
}

/* sample.rs:215-219: pick, drawing the uniform from the sampler's own stream
 * only when the pipeline reaches the draw, then remember. */
uint32_t orc_sampler_sample(orc_sampler *s, const float *logits, size_t n) {
    orc_rng probe = s->rng;
    float u = orc_rng_next_f32(&probe);
    size_t kept = 0;
    int used = 0;
    uint32_t tok = orc_pick(s->scratch, logits, n, &s->set, s->recent, s->filled, u, &kept, &used);
    if (tok == UINT32_MAX) return tok;
    if (used) s->rng = probe;
    s->kept = kept;
    orc_sampler_remember(s, tok);
    return tok;
}

size_t orc_sampler_candidates(const orc_sampler *s, const uint32_t **ids, const float **probs) {
    *ids = s->scratch->idx;
    *probs = s->scratch->probs;
    return s->kept;
}

size_t orc_sampler_filled(const orc_sampler *s) { return s->filled; }
const uint32_t *orc_sampler_recent(const orc_sampler *s) { return s->recent; }
void orc_sampler_rng_state(const orc_sampler *s, uint64_t out[4]) {
    for (int i = 0; i < 4; i++) out[i] = s->rng.s[i];
}

/* ------------------------------------------- the naive f64 reference ---- */
/* tests/sample.rs:16-83: full sort of the whole vector, f64 softmax.
 * `recent` is chronological; the window is its last repeat_last_n entries.
 * Writes survivors in descending order into out_ids/out_probs (capacity n) and
 * returns how many. */
size_t orc_naive(const float *logits, size_t n, const orc_sampling *set, const uint32_t *recent,
                 size_t recent_len, uint32_t *out_ids, double *out_probs) {
    float *l = malloc(n * sizeof(float));
    uint64_t *keys = malloc(n * sizeof(uint64_t));
    double *p = malloc(n * sizeof(double));
    memcpy(l, logits, n * sizeof(float));
    if (set->repeat_penalty != 1.0f && set->repeat_last_n > 0) {
        size_t start = recent_len > set->repeat_last_n ? recent_len - (size_t)set->repeat_last_n : 0;
        for (size_t i = start; i < recent_len; i++) {
            uint32_t t = recent[i];
            int seen = 0;
            for (size_t j = start; j < i; j++)
                if (recent[j] == t) seen = 1;
            if (seen) continue;
            float v = l[t];
            l[t] = v > 0.0f ? v / set->repeat_penalty : v * set->repeat_penalty;
        }
    }
    size_t out = 0;
    if (set->temperature <= 0.0f) {
        out_ids[0] = orc_argmax(l, n);
        out_probs[0] = 1.0;
        out = 1;
        goto done;
    }
    for (size_t i = 0; i < n; i++) keys[i] = composite(l, (uint32_t)i);
    sort_desc(keys, n);
    size_t k = set->top_k == 0 ? n : (set->top_k < n ? (size_t)set->top_k : n);
    double max = (double)l[~(uint32_t)keys[0]];
    for (size_t j = 0; j < k; j++)
        p[j] = exp(((double)l[~(uint32_t)keys[j]] - max) / (double)set->temperature);
    size_t keep = k;
    if (set->top_p < 1.0f) {
        double total = 0.0, cum = 0.0;
        for (size_t j = 0; j < k; j++) total += p[j];
        for (size_t j = 0; j < k; j++) {
            cum += p[j];
            if (cum >= (double)set->top_p * total) {
                keep = j + 1;
                break;
            }
        }
    }
    size_t w = 0;
    if (set->min_p > 0.0f) {
        double pmax = 0.0;
        for (size_t j = 0; j < keep; j++) pmax = fmax(pmax, p[j]);
        for (size_t j = 0; j < keep; j++) {
            if (p[j] >= (double)set->min_p * pmax) {
                keys[w] = keys[j];
                p[w] = p[j];
                w++;
            }
        }
        keep = w;
    }
    double total = 0.0;
    for (size_t j = 0; j < keep; j++) total += p[j];
    for (size_t j = 0; j < keep; j++) {
        out_ids[j] = ~(uint32_t)keys[j];
        out_probs[j] = p[j] / total;
    }
    out = keep;
done:
    free(l);
    free(keys);
    free(p);
    return out;
}

/* ---------------------------------------- the reference tests' logits ---- */
/* tests/sample.rs:87-98: xorshift64, uniform in [-spread, spread). */
void orc_test_logits(float *out, size_t n, uint64_t seed, float spread) {
    uint64_t s = seed | 1;
    for (size_t i = 0; i < n; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = ((float)(s >> 11) / (float)(1ull << 53) * 2.0f - 1.0f) * spread;
    }
}

/* tests/sample_allocations.rs:63-73: the same generator, fixed to [-6, 6). */
void orc_alloc_test_logits(float *out, size_t n, uint64_t seed) {
    uint64_t s = seed | 1;
    for (size_t i = 0; i < n; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = (float)(s >> 11) / (float)(1ull << 53) * 12.0f - 6.0f;
    }
}

/* ---------------------------------------------------- top probability ---- */
/* forward.rs:1671-1680 `top_probability`: the argmax (IEEE '>', lowest id on a
 * tie, starting from -inf and id 0) and (1 / sum) as f32, where sum is the f64
 * sum, in id order, of exp(v - best) (f32 subtraction, libm expf). Rust's
 * f64 Sum folds from -0.0, which gives the same bits as 0.0 for these terms
 * (all >= +0 or NaN) and n >= 1. */
uint32_t orc_top_probability(const float *l, size_t n, float *prob) {
    size_t best = 0;
    float best_v = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (l[i] > best_v) {
            best_v = l[i];
            best = i;
        }
    }
    double sum = -0.0;
    for (size_t i = 0; i < n; i++) sum += (double)expf(l[i] - best_v);
    *prob = (float)(1.0 / sum);
    return (uint32_t)best;
}

void orc_top_probability_rows(const float *logits, uint64_t stride, size_t rows, size_t n, uint32_t *tok,
                              float *prob) {
    for (size_t r = 0; r < rows; r++) tok[r] = orc_top_probability(logits + r * stride, n, prob + r);
}

/* libm expf, the function Rust's f32::exp lowers to; exposed so the GPU's
 * expf can be compared against this host's. */
float orc_libm_expf(float x) { return expf(x); }

/* Counts inputs in [lo_bits, hi_bits] (as u32 bit patterns, walked upward)
 * where got[] differs bitwise from libm expf; NaN equals NaN. got[i] is the
 * result for bit pattern lo_bits + i. Writes up to max_report mismatching
 * inputs into report. */
uint64_t orc_expf_compare(const float *got, uint32_t lo_bits, uint64_t count, uint32_t *report,
                          uint64_t max_report) {
    uint64_t bad = 0;
    for (uint64_t i = 0; i < count; i++) {
        uint32_t b = lo_bits + (uint32_t)i;
        float x;
        memcpy(&x, &b, 4);
        float want = expf(x);
        uint32_t wb, gb;
        memcpy(&wb, &want, 4);
        memcpy(&gb, &got[i], 4);
        if (wb != gb && !(isnan(want) && isnan(got[i]))) {
            if (bad < max_report) report[bad] = b;
            bad++;
        }
    }
    return bad;
}

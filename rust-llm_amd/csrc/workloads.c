/*
 * Synthetic logit workloads for the sampler's five benchmark shapes. Host-only,
 * deterministic, and per-row: row r of a workload depends only on the
 * workload's seed and r, so any slice of rows can be regenerated on its own.
 *
 * Randomness: splitmix64 (Steele, Lea, Flood 2014) streams, one per row;
 * uniform doubles take the top 53 bits; normals are Box-Muller pairs in double
 * (libm log, sqrt, cos, sin), rounded to f32 once at the end.
 *
 * Workloads (V1 = 151936, V2 = 248320, window = 64 ids):
 *   WL_SINGLE  1 x V1: N(0, 2.5^2); 8 distinct row-chosen ids set to +12.0.
 *   WL_ZIPF    64 x V1: N(0, 3^2) - 1.1 * ln(rank), where rank 1..V is a
 *              seed-permuted vocabulary order shared by all rows; windows of 64
 *              ids uniform in [0, V).
 *   WL_SPIKES  1024 x V2: N(0, 2^2); 16 distinct ids per row set to values
 *              uniform in [8, 14); windows of 64 ids uniform in [0, V).
 *   WL_VERIFY  9 x V1: rows as WL_SINGLE; row i's window is the last 64 of
 *              (64 seeded history ids, then drafts 0..i-1), drafts seeded.
 *   WL_TIES    256 x V1 on the bf16 grid: 40% of each row (row-chosen ids) hold
 *              the shared value -0.0234375 (= -3/128, exact in bf16); the rest
 *              are N(0, 0.01^2) rounded to bf16 (nearest-even). The shared
 *              value sits about 2.3 sigma below the mean, so the top-p 0.99
 *              boundary falls inside the tie block.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { WL_SINGLE = 1, WL_ZIPF = 2, WL_SPIKES = 3, WL_VERIFY = 4, WL_TIES = 5 };

#define WL_WINDOW 64u

typedef struct {
    uint64_t z;
} sm64;

static uint64_t sm_next(sm64 *s) {
    s->z += 0x9E3779B97F4A7C15ull;
    uint64_t v = s->z;
    v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
    v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
    return v ^ (v >> 31);
}

static double sm_unit(sm64 *s) { /* [0, 1) */
    return (double)(sm_next(s) >> 11) * 0x1.0p-53;
}

static uint32_t sm_below(sm64 *s, uint32_t n) { /* uniform in [0, n), n <= 2^32 */
    return (uint32_t)(((sm_next(s) >> 32) * (uint64_t)n) >> 32);
}

static sm64 row_stream(uint64_t seed, uint64_t row, uint64_t salt) {
    sm64 s;
    s.z = seed ^ (row * 0xD1B54A32D192ED03ull) ^ (salt * 0xA0761D6478BD642Full);
    sm_next(&s);
    return s;
}

/* n normals N(0, sigma^2) as doubles. */
static void normals(sm64 *s, double *out, size_t n, double sigma) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = sm_unit(s);
        const double u2 = sm_unit(s);
        if (u1 < 0x1.0p-60) u1 = 0x1.0p-60;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = sigma * r * cos(two_pi * u2);
        if (i + 1 < n) out[i + 1] = sigma * r * sin(two_pi * u2);
    }
}

static float to_bf16_grid(float x) { /* round to nearest-even bf16, keep as f32 */
    uint32_t b;
    memcpy(&b, &x, 4);
    if ((b & 0x7f800000u) == 0x7f800000u) return x;
    const uint32_t lsb = (b >> 16) & 1u;
    b += 0x7fffu + lsb;
    b &= 0xffff0000u;
    float y;
    memcpy(&y, &b, 4);
    return y;
}

/* k distinct ids in [0, n) by rejection. */
static void distinct_ids(sm64 *s, uint32_t *ids, uint32_t k, uint32_t n) {
    for (uint32_t i = 0; i < k; i++) {
        for (;;) {
            const uint32_t c = sm_below(s, n);
            uint32_t dup = 0;
            for (uint32_t j = 0; j < i; j++) dup |= ids[j] == c;
            if (!dup) {
                ids[i] = c;
                break;
            }
        }
    }
}

typedef struct {
    int kind;
    uint64_t seed;
    uint32_t vocab, row0, rows;
    float *logits;      /* rows x vocab */
    uint32_t *windows;  /* rows x WL_WINDOW, may be NULL */
    uint32_t *wlen;     /* rows, may be NULL */
    const float *zipf;  /* vocab boosts, WL_ZIPF only */
    double *tmp;        /* per-thread vocab doubles */
} job;

static void gen_row(const job *j, uint32_t local, double *tmp) {
    const uint32_t row = j->row0 + local;
    const uint32_t V = j->vocab;
    float *out = j->logits + (size_t)local * V;
    sm64 s = row_stream(j->seed, row, 1);
    switch (j->kind) {
    case WL_SINGLE:
    case WL_VERIFY: {
        normals(&s, tmp, V, 2.5);
        for (uint32_t i = 0; i < V; i++) out[i] = (float)tmp[i];
        uint32_t spikes[8];
        distinct_ids(&s, spikes, 8, V);
        for (int i = 0; i < 8; i++) out[spikes[i]] = 12.0f;
        break;
    }
    case WL_ZIPF:
        normals(&s, tmp, V, 3.0);
        for (uint32_t i = 0; i < V; i++) out[i] = (float)(tmp[i] + (double)j->zipf[i]);
        break;
    case WL_SPIKES: {
        normals(&s, tmp, V, 2.0);
        for (uint32_t i = 0; i < V; i++) out[i] = (float)tmp[i];
        uint32_t spikes[16];
        distinct_ids(&s, spikes, 16, V);
        for (int i = 0; i < 16; i++) out[spikes[i]] = (float)(8.0 + 6.0 * sm_unit(&s));
        break;
    }
    case WL_TIES: {
        normals(&s, tmp, V, 0.01);
        for (uint32_t i = 0; i < V; i++) out[i] = to_bf16_grid((float)tmp[i]);
        /* 40% of ids take the shared value: a partial Fisher-Yates over an id
         * permutation held in tmp's memory as u32. */
        uint32_t *perm = (uint32_t *)tmp;
        for (uint32_t i = 0; i < V; i++) perm[i] = i;
        const uint32_t tie = (uint32_t)((uint64_t)V * 2 / 5);
        for (uint32_t i = 0; i < tie; i++) {
            const uint32_t r = i + sm_below(&s, V - i);
            const uint32_t t = perm[i];
            perm[i] = perm[r];
            perm[r] = t;
            out[perm[i]] = -0.0234375f;
        }
        break;
    }
    default:
        break;
    }
    if (j->windows) {
        uint32_t *w = j->windows + (size_t)local * WL_WINDOW;
        if (j->kind == WL_VERIFY) {
            /* history then drafts; row i keeps the last 64 of history + drafts[..i] */
            sm64 h = row_stream(j->seed, 0, 2);
            uint32_t hist[WL_WINDOW + 16];
            for (uint32_t i = 0; i < WL_WINDOW + 16; i++) hist[i] = sm_below(&h, V);
            for (uint32_t i = 0; i < WL_WINDOW; i++) w[i] = hist[row + i];
        } else {
            sm64 ws = row_stream(j->seed, row, 3);
            for (uint32_t i = 0; i < WL_WINDOW; i++) w[i] = sm_below(&ws, V);
        }
        if (j->wlen) j->wlen[local] = WL_WINDOW;
    }
}

typedef struct {
    const job *j;
    uint32_t first, step;
} worker_arg;

static void *worker(void *p) {
    const worker_arg *a = p;
    double *tmp = malloc(sizeof(double) * (a->j->vocab + 2));
    if (!tmp) return (void *)1;
    for (uint32_t r = a->first; r < a->j->rows; r += a->step) gen_row(a->j, r, tmp);
    free(tmp);
    return NULL;
}

/* The Zipf boost -1.1 * ln(rank) over a seed-permuted vocabulary order. */
static float *zipf_boost(uint64_t seed, uint32_t V) {
    float *b = malloc(sizeof(float) * V);
    uint32_t *perm = malloc(sizeof(uint32_t) * V);
    if (!b || !perm) {
        free(b);
        free(perm);
        return NULL;
    }
    sm64 s = row_stream(seed, 0, 4);
    for (uint32_t i = 0; i < V; i++) perm[i] = i;
    for (uint32_t i = V - 1; i > 0; i--) {
        const uint32_t r = sm_below(&s, i + 1);
        const uint32_t t = perm[i];
        perm[i] = perm[r];
        perm[r] = t;
    }
    for (uint32_t rank = 0; rank < V; rank++) b[perm[rank]] = (float)(-1.1 * log((double)(rank + 1)));
    free(perm);
    return b;
}

/*
 * Fills rows row0..row0+rows-1 of workload `kind` with vocabulary `vocab`:
 * logits [rows][vocab], and, when non-NULL, windows [rows][64] and wlen
 * [rows]. `threads` >= 1 host threads. Returns 0, or -1 on failure.
 */
int wl_generate(int kind, uint64_t seed, uint32_t vocab, uint32_t row0, uint32_t rows, float *logits,
                uint32_t *windows, uint32_t *wlen, int threads) {
    if (!logits || vocab < 64 || kind < WL_SINGLE || kind > WL_TIES) return -1;
    job j = {kind, seed, vocab, row0, rows, logits, windows, wlen, NULL, NULL};
    float *zb = NULL;
    if (kind == WL_ZIPF) {
        zb = zipf_boost(seed, vocab);
        if (!zb) return -1;
        j.zipf = zb;
    }
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > rows) threads = (int)rows;
    pthread_t th[64];
    worker_arg args[64];
    if (threads > 64) threads = 64;
    int rc = 0;
    for (int t = 0; t < threads; t++) {
        args[t].j = &j;
        args[t].first = (uint32_t)t;
        args[t].step = (uint32_t)threads;
        if (pthread_create(&th[t], NULL, worker, &args[t]) != 0) {
            threads = t;
            rc = -1;
            break;
        }
    }
    for (int t = 0; t < threads; t++) {
        void *ret = NULL;
        pthread_join(th[t], &ret);
        if (ret) rc = -1;
    }
    free(zb);
    return rc;
}

/* Draft ids of WL_VERIFY: row i's window ends with drafts 0..i-1, which are
 * the history stream's entries 64.. (so drafts[i] = that stream's 64+i). */
int wl_verify_drafts(uint64_t seed, uint32_t vocab, uint32_t *drafts, uint32_t n) {
    if (n > 16) return -1;
    sm64 h = row_stream(seed, 0, 2);
    uint32_t hist[WL_WINDOW + 16];
    for (uint32_t i = 0; i < WL_WINDOW + 16; i++) hist[i] = sm_below(&h, vocab);
    for (uint32_t i = 0; i < n; i++) drafts[i] = hist[WL_WINDOW + i];
    return 0;
}

/* The 64 history ids of WL_VERIFY, oldest first. */
int wl_verify_history(uint64_t seed, uint32_t vocab, uint32_t *hist64) {
    sm64 h = row_stream(seed, 0, 2);
    for (uint32_t i = 0; i < WL_WINDOW; i++) hist64[i] = sm_below(&h, vocab);
    return 0;
}

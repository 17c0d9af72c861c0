// Host side of the drop-in: the reference's Sampler API over the device ABI.
//
// crates/rust-llm/src/sample.rs keeps, per Sampler, the settings, a ring of
// recent tokens and an Rng (:132-151), and runs the whole pick on the CPU. Here
// the same state stays on the host and the pick runs on the GPU: the window is
// uploaded as recent[..filled], the uniform is pre-drawn from a clone of the
// Rng, and the clone is committed only when the device reports that the row
// drew (sample.rs:349), so the stream advances exactly as the reference's does.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <new>
#include <random>
#include <string>
#include <vector>

#include "rl_error.h"
#include "rl_pack.h"
#include "rl_sampler.h"
#include "rl_sampler_host.h"

namespace {

int herr(int code, const std::string &m) {
    rl::set_last_error(m);
    return code;
}

uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

bool penalises(const rl_sampling &s) { return s.repeat_penalty != 1.0f && s.repeat_last_n > 0; }

bool same(const rl_sampling &a, const rl_sampling &b) { return std::memcmp(&a, &b, sizeof a) == 0; }

// A row's kept count while its results are pending (a real count is at most
// the vocabulary, below 2^21).
constexpr uint32_t KEPT_PENDING = 0xFFFFFFFFu;
// How long a call polls its results before it waits on the stream instead.
constexpr double POLL_US = 2000.0;

}  // namespace

extern "C" {

void rl_rng_seeded(rl_rng *r, uint64_t seed) {
    uint64_t z = seed;
    for (int i = 0; i < 4; ++i) {  // splitmix64, sample.rs:375-381
        z += 0x9E3779B97F4A7C15ull;
        uint64_t v = z;
        v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
        v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
        r->s[i] = v ^ (v >> 31);
    }
}

uint64_t rl_rng_next_u64(rl_rng *r) {  // xoshiro256++, sample.rs:387-398
    uint64_t *s = r->s;
    const uint64_t out = rotl(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return out;
}

float rl_rng_next_f32(rl_rng *r) {  // sample.rs:401-403
    return (float)(rl_rng_next_u64(r) >> 40) / (float)(1u << 24);
}

rl_sampling rl_sampling_default(void) {  // sample.rs:88-100
    rl_sampling s{};
    s.temperature = 0.6f;
    s.top_k = 20;
    s.top_p = 0.95f;
    s.min_p = 0.0f;
    s.repeat_penalty = 1.0f;
    s.repeat_last_n = 64;
    s.seed = 0;
    return s;
}

rl_sampling rl_sampling_greedy(void) {  // sample.rs:71-79
    rl_sampling s{};
    s.temperature = 0.0f;
    s.top_k = 0;
    s.top_p = 1.0f;
    s.min_p = 0.0f;
    s.repeat_penalty = 1.0f;
    s.repeat_last_n = 0;
    s.seed = 0;
    return s;
}

uint64_t rl_entropy_seed(void) {
    std::random_device rd;
    return ((uint64_t)rd() << 32) ^ rd();
}

}  // extern "C"

// Every buffer a call touches is sized in rl_host_sampler_new, as the
// reference's Sampler sizes its own in Sampler::new (sample.rs:156-172): no
// per-call path below allocates host memory (tests/sample_allocations.rs).
struct rl_host_sampler {
    int device = 0;
    size_t vocab = 0;
    rl_sampling set{};
    uint32_t max_rows = 1;
    uint32_t wcap = 0;  // window capacity per row on the device
    std::vector<uint32_t> recent;
    size_t at = 0, filled = 0;
    rl_rng rng{};
    rl_sampler_ctx *ctx = nullptr;
    // What ctx was last configured with (capacity max_rows), `same_set` holds
    // max_rows copies of `set`, `batch_set` the settings of a batch call.
    std::vector<rl_sampling> configured, same_set, batch_set;
    std::vector<rl_rng> batch_probe;
    uint64_t cand_cap = 1;
    // Device buffers (d_in: a call's inputs when they are uploaded).
    float *d_row = nullptr;
    uint32_t *d_in = nullptr, *d_token = nullptr, *d_kept = nullptr;
    uint8_t *d_used = nullptr;
    uint32_t *d_ids = nullptr;
    float *d_probs = nullptr;
    // Coherent pinned host memory, with the device's address of each block
    // (hd_*). h_in holds a call's inputs: uniforms[max_rows] (f32), window
    // lengths[max_rows], then the windows at the call's stride (its longest
    // window). h_res receives a call's results (rl_pack.h): token, kept and
    // used[max_rows], then the first candidates of every row. A call whose
    // rows all take the stream path reads h_in and writes h_res from its
    // kernel; any other call uploads h_in to d_in (the full path re-reads a
    // row's window in every pass) and packs its results into h_res.
    uint32_t *h_in = nullptr, *hd_in = nullptr;
    uint8_t *h_res = nullptr, *hd_res = nullptr;
    size_t res_cands_at = 0;  // byte offset of the candidates in h_res
    // the last call's survivors (Sampler::candidates), capacity cand_cap
    std::vector<uint32_t> cand_ids;
    std::vector<float> cand_probs;
    size_t kept = 0;
    // The last verify, uncommitted: per row the pick, its kept count, whether
    // it drew and the uniform it was given (capacity max_rows each). Row i's
    // candidates stay in device row i until it is committed.
    uint32_t v_rows_n = 0, next_commit = 0;
    std::vector<uint32_t> v_token, v_kept, v_drafts;
    std::vector<uint8_t> v_used;
    std::vector<float> v_uniform;
    uint32_t last_committed = 0;
    const float *v_rows = nullptr;
    uint64_t v_stride = 0;
    void *v_stream = nullptr;

    ~rl_host_sampler() {
        for (void *p : {(void *)d_row, (void *)d_in, (void *)d_token, (void *)d_kept, (void *)d_used, (void *)d_ids,
                        (void *)d_probs})
            if (p) (void)hipFree(p);
        for (void *p : {(void *)h_in, (void *)h_res})
            if (p) (void)hipHostFree(p);
        rl_sampler_destroy(ctx);
    }

    float *h_uniforms() { return reinterpret_cast<float *>(h_in); }
    uint32_t *h_wlen() { return h_in + max_rows; }
    uint32_t *h_windows() { return h_in + 2 * (size_t)max_rows; }
    // The result block's arrays, in host (dev = false) or device addresses.
    uint32_t *res_token(bool dev = false) { return reinterpret_cast<uint32_t *>(dev ? hd_res : h_res); }
    uint32_t *res_kept(bool dev = false) { return res_token(dev) + max_rows; }
    uint8_t *res_used(bool dev = false) { return reinterpret_cast<uint8_t *>(res_token(dev) + 2 * (size_t)max_rows); }
    rl::PackedCands *res_cands(bool dev = false) {
        return reinterpret_cast<rl::PackedCands *>((dev ? hd_res : h_res) + res_cands_at);
    }
    static size_t res_layout(uint32_t rows, size_t *cands_at) {
        *cands_at = ((size_t)rows * 9 + 15) / 16 * 16;  // token, kept, used; candidates 16-byte aligned
        return *cands_at + (size_t)rows * sizeof(rl::PackedCands);
    }

    void remember(uint32_t t) {  // sample.rs:205-212
        if (recent.empty()) return;
        recent[at] = t;
        at = (at + 1) % recent.size();
        filled = std::min(filled + 1, recent.size());
    }

    // Configures the device context for rows 0..n-1 of `want`, unless the
    // rows it is configured for already begin with exactly these settings
    // (sample_rows takes any prefix of the configured rows).
    int ensure_configured(const rl_sampling *want, uint32_t n) {
        if (n <= configured.size() && std::equal(want, want + n, configured.begin(), same)) return RL_OK;
        const int rc = rl_sampler_configure(ctx, want, n);
        if (rc != RL_OK) {
            configured.clear();
            return rc;
        }
        configured.assign(want, want + n);  // n <= max_rows = capacity
        return RL_OK;
    }

    // The window row `i` of a verify sees, recent[..filled] of the ring after
    // remembering drafts[0..i) (sample.rs:205-212), written to `out`. Draft m
    // lands in slot (at + m) % len; a later draft overwrites an earlier one.
    size_t window_after(const uint32_t *drafts, uint32_t i, uint32_t *out) const {
        const size_t len = recent.size();
        if (len == 0) return 0;
        const size_t f = std::min(filled + (size_t)i, len);
        std::copy(recent.begin(), recent.begin() + f, out);
        for (uint32_t m = i > len ? (uint32_t)(i - len) : 0u; m < i; ++m) {
            const size_t slot = (at + m) % len;
            if (slot < f) out[slot] = drafts[m];
        }
        return f;
    }

    // Runs rows 0..rows-1 (windows in h_in at stride ws) and leaves every
    // row's results in h_res. A call whose rows all take the stream path is
    // one launch that reads h_in and writes h_res; any other call uploads
    // h_in (one copy), launches, and packs the results (one more launch).
    // Either way the host then polls the results (wait_results).
    int run(const float *d_logits, uint64_t stride, uint32_t rows, uint32_t ws, void *stream) {
        hipStream_t st = static_cast<hipStream_t>(stream);
        const bool direct = rl::rows_all_stream(ctx, rows);
        std::fill(res_kept(), res_kept() + rows, KEPT_PENDING);
        const uint32_t *in = hd_in;
        hipError_t e = hipSuccess;
        if (!direct) {
            const size_t words = 2 * (size_t)max_rows + (size_t)rows * ws;
            e = hipMemcpyAsync(d_in, h_in, words * 4, hipMemcpyHostToDevice, st);
            if (e != hipSuccess) return herr(RL_ERR_DEVICE, hipGetErrorString(e));
            in = d_in;
        }
        // No window arrays when no row has a window: the kernels then read none.
        bool any_win = false;
        for (uint32_t r = 0; r < rows; ++r) any_win = any_win || h_wlen()[r] > 0;
        const uint32_t *win = any_win ? in + 2 * (size_t)max_rows : nullptr;
        const uint32_t *wlen = any_win ? in + max_rows : nullptr;
        const float *uni = reinterpret_cast<const float *>(in);
        int rc;
        if (direct) {
            rl::PackedCands *c = res_cands(true);
            rc = rl_sampler_sample_rows(ctx, d_logits, stride, rows, (uint32_t)vocab, win, ws, wlen, uni,
                                        res_token(true), res_kept(true), res_used(true), c->ids, c->probs,
                                        rl::PACK_STRIDE, stream);
        } else {
            rc = rl_sampler_sample_rows(ctx, d_logits, stride, rows, (uint32_t)vocab, win, ws, wlen, uni, d_token,
                                        d_kept, d_used, d_ids, d_probs, cand_cap, stream);
            if (rc == RL_OK)
                rc = rl::launch_pack_rows(d_token, d_kept, d_used, d_ids, d_probs, cand_cap, rows, res_token(true),
                                          res_kept(true), res_used(true), res_cands(true), stream);
        }
        if (rc != RL_OK) return rc;
        return wait_results(rows, stream);
    }

    // Every row's kept count is the last word of its results the device
    // writes (it was set to KEPT_PENDING before the launch), so the call is
    // complete once every row's has changed: the host polls them, which
    // returns several microseconds sooner than a stream synchronisation.
    // After POLL_US it waits on the stream instead, which also reports a
    // device error; a row still pending after that is a device error too.
    int wait_results(uint32_t rows, void *stream) {
        using clk = std::chrono::steady_clock;
        const clk::time_point t0 = clk::now();
        uint32_t r = 0;
        for (;;) {
            while (r < rows && __atomic_load_n(res_kept() + r, __ATOMIC_ACQUIRE) != KEPT_PENDING) ++r;
            if (r == rows) return RL_OK;
            if (std::chrono::duration<double, std::micro>(clk::now() - t0).count() > POLL_US) break;
        }
        const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return herr(RL_ERR_DEVICE, hipGetErrorString(e));
        for (; r < rows; ++r)
            if (__atomic_load_n(res_kept() + r, __ATOMIC_ACQUIRE) == KEPT_PENDING)
                return herr(RL_ERR_DEVICE, "a row's results never arrived");
        return RL_OK;
    }

    // Packed row `slot`'s survivors into ids/probs (capacity reserved at
    // creation for any kept count the settings allow): the first PACK_CANDS
    // from the packed results; the rest of a row that keeps more is copied
    // from device row `slot` on `stream`, and *queued is set (the caller
    // synchronises once for all its rows).
    int take_candidates(uint32_t slot, std::vector<uint32_t> &ids, std::vector<float> &probs, void *stream,
                        bool *queued) {
        const rl::PackedCands &pc = res_cands()[slot];
        const uint32_t n = res_kept()[slot];
        if (n > ids.capacity() || n > probs.capacity())
            return herr(RL_ERR_CAPACITY, "more candidates than the sampler was sized for");
        ids.resize(n);
        probs.resize(n);
        const uint32_t head = std::min(n, rl::PACK_CANDS);
        std::copy(pc.ids, pc.ids + head, ids.begin());
        std::copy(pc.probs, pc.probs + head, probs.begin());
        if (n > head) {  // only a call with full-path rows keeps more: its candidates are in d_ids/d_probs
            hipStream_t st = static_cast<hipStream_t>(stream);
            const uint64_t at = (uint64_t)slot * cand_cap + head;
            hipError_t e = hipMemcpyAsync(ids.data() + head, d_ids + at, (n - head) * 4, hipMemcpyDeviceToHost, st);
            if (e == hipSuccess)
                e = hipMemcpyAsync(probs.data() + head, d_probs + at, (n - head) * 4, hipMemcpyDeviceToHost, st);
            if (e != hipSuccess) return herr(RL_ERR_DEVICE, hipGetErrorString(e));
            *queued = true;
        }
        return RL_OK;
    }

    static int finish_copies(bool queued, void *stream) {
        if (!queued) return RL_OK;
        const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return herr(RL_ERR_DEVICE, hipGetErrorString(e));
        return RL_OK;
    }

    void forget_verify() {
        v_rows_n = 0;
        next_commit = 0;
    }

    int sample_device(const float *d_logits, size_t n, uint32_t *token, void *stream) {
        if (n != vocab) return herr(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
        int rc = ensure_configured(&set, 1);
        if (rc != RL_OK) return rc;
        const bool pen = penalises(set) && filled > 0;
        h_wlen()[0] = pen ? (uint32_t)filled : 0u;
        if (pen) std::copy(recent.begin(), recent.begin() + filled, h_windows());
        rl_rng probe = rng;
        h_uniforms()[0] = rl_rng_next_f32(&probe);
        forget_verify();  // the device rows a verify left are overwritten
        rc = run(d_logits, vocab, 1, std::max<uint32_t>(1u, h_wlen()[0]), stream);
        if (rc != RL_OK) return rc;
        bool queued = false;
        rc = take_candidates(0, cand_ids, cand_probs, stream, &queued);
        if (rc == RL_OK) rc = finish_copies(queued, stream);
        if (rc != RL_OK) return rc;
        kept = res_kept()[0];
        if (res_used()[0]) rng = probe;
        *token = res_token()[0];
        remember(*token);  // sample.rs:217
        return RL_OK;
    }
};

extern "C" {

int rl_host_sampler_new(int device, size_t vocab, const rl_sampling *set, uint32_t max_rows,
                        rl_host_sampler **out) {
    if (!out || !set || vocab == 0 || vocab > 0xFFFFFFF0u || max_rows == 0)
        return herr(RL_ERR_ARGUMENT, "bad argument");
    *out = nullptr;
    if (set->repeat_last_n > 0xFFFFFFFFull) return herr(RL_ERR_CAPACITY, "repeat_last_n above 2^32 - 1");
    auto *s = new (std::nothrow) rl_host_sampler();
    if (!s) return herr(RL_ERR_CAPACITY, "out of host memory");
    s->device = device;
    s->vocab = vocab;
    s->set = *set;
    s->max_rows = max_rows;
    try {
        s->recent.assign((size_t)set->repeat_last_n, 0u);
    } catch (const std::bad_alloc &) {
        delete s;
        return herr(RL_ERR_CAPACITY, "out of host memory");
    }
    s->wcap = std::max<uint32_t>(1u, (uint32_t)set->repeat_last_n);
    rl_rng_seeded(&s->rng, set->seed);
    // Candidate slots the settings can keep (sample.rs:159: the whole
    // vocabulary unless greedy).
    s->cand_cap = max_rows > 1 ? vocab
                  : !(set->temperature <= 0.0f) ? ((set->top_k == 0 || set->top_k >= vocab) ? vocab : set->top_k)
                                                : 1;
    int rc = rl_sampler_create(device, max_rows, (uint32_t)vocab, s->wcap, &s->ctx);
    if (rc != RL_OK) {
        delete s;
        return rc;
    }
    rl::set_results_polled(s->ctx, true);  // wait_results polls the kept counts
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    const size_t in_words = 2 * (size_t)max_rows + (size_t)max_rows * s->wcap;
    const size_t res_bytes = rl_host_sampler::res_layout(max_rows, &s->res_cands_at);
    constexpr unsigned pinned = hipHostMallocMapped | hipHostMallocCoherent;
    hipError_t e = hipMalloc(&s->d_row, vocab * 4);
    if (e == hipSuccess) e = hipMalloc(&s->d_in, in_words * 4);
    if (e == hipSuccess) e = hipMalloc(&s->d_token, max_rows * 4);
    if (e == hipSuccess) e = hipMalloc(&s->d_kept, max_rows * 4);
    if (e == hipSuccess) e = hipMalloc(&s->d_used, max_rows);
    if (e == hipSuccess) e = hipMalloc(&s->d_ids, (size_t)max_rows * s->cand_cap * 4);
    if (e == hipSuccess) e = hipMalloc(&s->d_probs, (size_t)max_rows * s->cand_cap * 4);
    if (e == hipSuccess) e = hipHostMalloc(&s->h_in, in_words * 4, pinned);
    if (e == hipSuccess) e = hipHostMalloc(&s->h_res, res_bytes, pinned);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void **>(&s->hd_in), s->h_in, 0);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void **>(&s->hd_res), s->h_res, 0);
    if (e == hipSuccess) {
        std::fill(s->h_in, s->h_in + in_words, 0u);
        std::fill(s->h_res, s->h_res + res_bytes, (uint8_t)0);
    }
    (void)hipSetDevice(prev);
    if (e != hipSuccess) {
        delete s;
        return herr(RL_ERR_DEVICE, hipGetErrorString(e));
    }
    try {
        s->cand_ids.reserve(s->cand_cap);
        s->cand_probs.reserve(s->cand_cap);
        s->configured.reserve(max_rows);
        s->same_set.assign(max_rows, *set);
        s->batch_set.reserve(max_rows);
        s->batch_probe.reserve(max_rows);
        s->v_token.assign(max_rows, 0u);
        s->v_kept.assign(max_rows, 0u);
        s->v_drafts.assign(max_rows, 0u);
        s->v_used.assign(max_rows, 0);
        s->v_uniform.assign(max_rows, 0.0f);
    } catch (const std::bad_alloc &) {
        delete s;
        return herr(RL_ERR_CAPACITY, "out of host memory");
    }
    // Every row of this sampler has its settings: configured once, here, for
    // all max_rows rows, so a call over any number of them reconfigures nothing.
    rc = s->ensure_configured(s->same_set.data(), max_rows);
    if (rc != RL_OK) {
        delete s;
        return rc;
    }
    *out = s;
    return RL_OK;
}

void rl_host_sampler_free(rl_host_sampler *s) { delete s; }

rl_sampling rl_host_sampler_settings(const rl_host_sampler *s) { return s->set; }

void rl_host_sampler_reset(rl_host_sampler *s) {  // sample.rs:194-198
    s->at = 0;
    s->filled = 0;
    s->kept = 0;
    s->forget_verify();
}

void rl_host_sampler_remember(rl_host_sampler *s, uint32_t token) { s->remember(token); }

int rl_host_sampler_sample_device(rl_host_sampler *s, const float *device_row, size_t n, uint32_t *token,
                                  void *stream) {
    if (!s || !device_row || !token) return herr(RL_ERR_ARGUMENT, "null argument");
    return s->sample_device(device_row, n, token, stream);
}

int rl_host_sampler_sample(rl_host_sampler *s, const float *host_logits, size_t n, uint32_t *token) {
    if (!s || !host_logits || !token) return herr(RL_ERR_ARGUMENT, "null argument");
    if (n != s->vocab) return herr(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
    const hipError_t e = hipMemcpy(s->d_row, host_logits, n * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return herr(RL_ERR_DEVICE, hipGetErrorString(e));
    return s->sample_device(s->d_row, n, token, nullptr);
}

size_t rl_host_sampler_candidates(const rl_host_sampler *s, const uint32_t **ids, const float **probs) {
    *ids = s->cand_ids.data();
    *probs = s->cand_probs.data();
    return s->kept;
}

void rl_host_sampler_rng(const rl_host_sampler *s, rl_rng *out) { *out = s->rng; }

int rl_host_sampler_verify(rl_host_sampler *s, const float *device_rows, uint64_t row_stride, size_t n,
                           const uint32_t *drafts, uint32_t n_drafts, uint32_t *picks, void *stream) {
    if (!s || !device_rows || !picks || (n_drafts && !drafts)) return herr(RL_ERR_ARGUMENT, "null argument");
    if (n != s->vocab) return herr(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
    if (n_drafts >= s->max_rows) return herr(RL_ERR_CAPACITY, "more verify rows than max_rows");
    const uint32_t rows = n_drafts + 1;
    int rc = s->ensure_configured(s->same_set.data(), rows);
    if (rc != RL_OK) return rc;
    const bool pen = penalises(s->set);
    rl_rng probe = s->rng;
    const bool greedy = s->set.temperature <= 0.0f;
    // Row i's window holds min(filled + i, len) ids: the last row's is the
    // longest, and the call's stride.
    const uint32_t ws = std::max<uint32_t>(
        1u, pen && !s->recent.empty() ? (uint32_t)std::min(s->filled + n_drafts, s->recent.size()) : 0u);
    for (uint32_t i = 0; i < rows; ++i) {
        const size_t f = pen ? s->window_after(drafts, i, s->h_windows() + (size_t)i * ws) : 0;
        s->h_wlen()[i] = (uint32_t)f;
        s->h_uniforms()[i] = greedy ? 0.0f : rl_rng_next_f32(&probe);  // one draw per drawing row
    }
    s->forget_verify();
    rc = s->run(device_rows, row_stride, rows, ws, stream);
    if (rc != RL_OK) return rc;
    for (uint32_t i = 0; i < rows; ++i) {
        s->v_token[i] = s->res_token()[i];
        s->v_kept[i] = s->res_kept()[i];
        s->v_used[i] = s->res_used()[i];
        s->v_uniform[i] = s->h_uniforms()[i];
        picks[i] = s->v_token[i];
    }
    std::copy(drafts, drafts + n_drafts, s->v_drafts.begin());
    s->v_rows_n = rows;
    s->next_commit = 0;
    s->v_rows = device_rows;
    s->v_stride = row_stride;
    s->v_stream = stream;
    return RL_OK;
}

int rl_host_sampler_commit_verified(rl_host_sampler *s, uint32_t row, uint32_t *token) {
    if (!s || !token) return herr(RL_ERR_ARGUMENT, "null argument");
    if (row != s->next_commit || row >= s->v_rows_n)
        return herr(RL_ERR_ARGUMENT, "verify rows are committed in order, once");
    // Row `row` was sampled with the window after drafts[0..row): committing
    // it is only meaningful while every earlier committed token was its draft
    // (generate.rs:412-429 stops at the first mismatch).
    if (row > 0 && s->last_committed != s->v_drafts[row - 1])
        return herr(RL_ERR_ARGUMENT, "the previous committed token differs from its draft: the generation loop "
                                     "stops there, and this row's window assumed the draft");
    // The row was sampled with the uniform the stream would give if every
    // earlier row drew; an earlier row with no finite maximum drew nothing, so
    // recompute this one with the uniform the stream really gives now.
    rl_rng probe = s->rng;
    const float u = rl_rng_next_f32(&probe);
    uint32_t slot = row;
    if (!(s->set.temperature <= 0.0f) && u != s->v_uniform[row]) {
        const bool pen = penalises(s->set) && s->filled > 0;
        s->h_wlen()[0] = pen ? (uint32_t)s->filled : 0u;
        if (pen) std::copy(s->recent.begin(), s->recent.begin() + s->filled, s->h_windows());
        s->h_uniforms()[0] = u;
        // Result row 0 belongs to a row already committed; later rows keep theirs.
        const int rc = s->run(s->v_rows + (uint64_t)row * s->v_stride, s->vocab, 1,
                              std::max<uint32_t>(1u, s->h_wlen()[0]), s->v_stream);
        if (rc != RL_OK) return rc;
        s->v_token[row] = s->res_token()[0];
        s->v_kept[row] = s->res_kept()[0];
        s->v_used[row] = s->res_used()[0];
        slot = 0;
    }
    bool queued = false;
    int rc = s->take_candidates(slot, s->cand_ids, s->cand_probs, s->v_stream, &queued);
    if (rc == RL_OK) rc = s->finish_copies(queued, s->v_stream);
    if (rc != RL_OK) return rc;
    if (s->v_used[row]) s->rng = probe;
    s->kept = s->v_kept[row];
    s->remember(s->v_token[row]);
    s->last_committed = s->v_token[row];
    s->next_commit = row + 1;
    *token = s->v_token[row];
    return RL_OK;
}

int rl_host_sample_batch(rl_host_sampler *const *samplers, uint32_t n, const float *device_logits,
                         uint64_t row_stride, size_t vocab, uint32_t *tokens, void *stream) {
    if (!samplers || n == 0 || !device_logits || !tokens) return herr(RL_ERR_ARGUMENT, "bad argument");
    rl_host_sampler *h = samplers[0];
    if (n > h->max_rows) return herr(RL_ERR_CAPACITY, "more samplers than the first one's max_rows");
    h->batch_set.clear();
    h->batch_probe.clear();
    uint32_t ws = 1;  // the call's window stride: its longest window
    for (uint32_t i = 0; i < n; ++i) {
        rl_host_sampler *s = samplers[i];
        if (s->vocab != vocab || vocab != h->vocab)
            return herr(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
        if (s->filled > h->wcap) return herr(RL_ERR_CAPACITY, "a window longer than the first sampler's");
        if (s->cand_cap > h->cand_cap) return herr(RL_ERR_CAPACITY, "a sampler keeps more candidates than the first");
        if (penalises(s->set)) ws = std::max(ws, (uint32_t)s->filled);
    }
    for (uint32_t i = 0; i < n; ++i) {
        rl_host_sampler *s = samplers[i];
        h->batch_set.push_back(s->set);  // within the capacity reserved at creation
        const bool pen = penalises(s->set) && s->filled > 0;
        h->h_wlen()[i] = pen ? (uint32_t)s->filled : 0u;
        if (pen) std::copy(s->recent.begin(), s->recent.begin() + s->filled, h->h_windows() + (size_t)i * ws);
        h->batch_probe.push_back(s->rng);
        h->h_uniforms()[i] = rl_rng_next_f32(&h->batch_probe[i]);
    }
    int rc = h->ensure_configured(h->batch_set.data(), n);
    if (rc != RL_OK) return rc;
    for (uint32_t i = 0; i < n; ++i) samplers[i]->forget_verify();  // h's device rows are overwritten
    rc = h->run(device_logits, row_stride, n, ws, stream);
    if (rc != RL_OK) return rc;
    // Every row's candidates: from the packed results, plus one copy for each
    // row that keeps more, all waited for by one synchronisation.
    bool queued = false;
    for (uint32_t i = 0; i < n && rc == RL_OK; ++i) rc = h->take_candidates(i, samplers[i]->cand_ids,
                                                                          samplers[i]->cand_probs, stream, &queued);
    const int rc2 = h->finish_copies(queued, stream);
    if (rc != RL_OK) return rc;
    if (rc2 != RL_OK) return rc2;
    for (uint32_t i = 0; i < n; ++i) {
        rl_host_sampler *s = samplers[i];
        s->kept = h->res_kept()[i];
        if (h->res_used()[i]) s->rng = h->batch_probe[i];
        tokens[i] = h->res_token()[i];
        s->remember(tokens[i]);
    }
    return RL_OK;
}

int rl_host_argmax(int device, const float *logits, size_t n, uint32_t *out) {
    if (!logits || !out || n == 0 || n > 0xFFFFFFF0u) return herr(RL_ERR_ARGUMENT, "bad argument");
    struct Cache {
        rl_sampler_ctx *ctx = nullptr;
        float *d = nullptr;
        uint32_t *tok = nullptr;
        size_t cap = 0;
        int device = -1;
        ~Cache() {
            if (d) (void)hipFree(d);
            if (tok) (void)hipFree(tok);
            rl_sampler_destroy(ctx);
        }
    };
    thread_local Cache c;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    if (c.cap != n || c.device != device) {
        if (c.d) (void)hipFree(c.d);
        if (c.tok) (void)hipFree(c.tok);
        rl_sampler_destroy(c.ctx);
        c = Cache();
        int rc = rl_sampler_create(device, 1, (uint32_t)n, 0, &c.ctx);
        if (rc != RL_OK) {
            (void)hipSetDevice(prev);
            return rc;
        }
        if (hipMalloc(&c.d, n * 4) != hipSuccess || hipMalloc(&c.tok, 4) != hipSuccess) {
            (void)hipSetDevice(prev);
            return herr(RL_ERR_DEVICE, "hipMalloc");
        }
        c.cap = n;
        c.device = device;
    }
    hipError_t e = hipMemcpy(c.d, logits, n * 4, hipMemcpyHostToDevice);
    int rc = RL_OK;
    if (e == hipSuccess) rc = rl_argmax_rows(c.ctx, c.d, n, 1, (uint32_t)n, c.tok, nullptr);
    if (e == hipSuccess && rc == RL_OK) e = hipMemcpy(out, c.tok, 4, hipMemcpyDeviceToHost);
    (void)hipSetDevice(prev);
    if (e != hipSuccess) return herr(RL_ERR_DEVICE, hipGetErrorString(e));
    return rc;
}

}  // extern "C"

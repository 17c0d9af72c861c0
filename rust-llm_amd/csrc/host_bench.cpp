// Host-wall timing of the host Sampler's calls, for bench.py's --op
// host_verify / host_batch / host_sample: the calls run from C++ exactly as a
// native caller (the Rust wrapper) makes them, each timed with steady_clock,
// so the figures carry no interpreter overhead. Not part of the sampler's ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <vector>

#include "rl_sampler.h"
#include "rl_sampler_host.h"

namespace {

using clk = std::chrono::steady_clock;

double us_since(clk::time_point t0) { return std::chrono::duration<double, std::micro>(clk::now() - t0).count(); }

}  // namespace

extern "C" {

// `walks` speculative-verify walks over `rows` device rows (generate.rs:412-450):
// a sampler made with `set` remembers `history`; before each walk the drafts
// that every row accepts from the sampler's current state are found with
// uncommitted verify calls (untimed; row i's pick depends on drafts 0..i-1 and
// its uniform only); the timed walk is one rl_host_sampler_verify and one
// rl_host_sampler_commit_verified per row until a pick differs from its
// draft. out_us[w] is walk w's host wall time, out_committed[w] its rows.
int rlb_verify_walks(int device, const float *d_rows, uint64_t stride, size_t vocab, const rl_sampling *set,
                     const uint32_t *history, size_t hist_len, uint32_t rows, uint32_t walks, double *out_us,
                     uint32_t *out_committed) {
    if (rows < 1) return RL_ERR_ARGUMENT;
    rl_host_sampler *s = nullptr;
    int rc = rl_host_sampler_new(device, vocab, set, rows, &s);
    if (rc != RL_OK) return rc;
    for (size_t i = 0; i < hist_len; ++i) rl_host_sampler_remember(s, history[i]);
    std::vector<uint32_t> drafts(rows > 1 ? rows - 1 : 1, 0u), picks(rows, 0u);
    const uint32_t nd = rows - 1;
    for (uint32_t w = 0; w < walks && rc == RL_OK; ++w) {
        std::fill(drafts.begin(), drafts.end(), 0u);
        for (uint32_t it = 0; it < rows && rc == RL_OK; ++it) {
            rc = rl_host_sampler_verify(s, d_rows, stride, vocab, drafts.data(), nd, picks.data(), nullptr);
            if (std::equal(picks.begin(), picks.begin() + nd, drafts.begin())) break;
            std::copy(picks.begin(), picks.begin() + nd, drafts.begin());
        }
        if (rc != RL_OK) break;
        const clk::time_point t0 = clk::now();
        rc = rl_host_sampler_verify(s, d_rows, stride, vocab, drafts.data(), nd, picks.data(), nullptr);
        uint32_t committed = 0;
        for (uint32_t r = 0; r < rows && rc == RL_OK; ++r) {
            uint32_t t = 0;
            rc = rl_host_sampler_commit_verified(s, r, &t);
            ++committed;
            if (r < nd && t != drafts[r]) break;
        }
        out_us[w] = us_since(t0);
        out_committed[w] = committed;
    }
    rl_host_sampler_free(s);
    return rc;
}

// `calls` rl_host_sample_batch calls over n samplers (sampler i made with
// sets[i] and remembering windows[i][0..wlen[i])), device row i for sampler i.
int rlb_batch_calls(int device, const float *d_rows, uint64_t stride, size_t vocab, const rl_sampling *sets,
                    uint32_t n, const uint32_t *windows, uint32_t wstride, const uint32_t *wlen, uint32_t calls,
                    double *out_us) {
    std::vector<rl_host_sampler *> ss(n, nullptr);
    int rc = RL_OK;
    for (uint32_t i = 0; i < n && rc == RL_OK; ++i) {
        rc = rl_host_sampler_new(device, vocab, &sets[i], i == 0 ? n : 1, &ss[i]);
        for (uint32_t j = 0; rc == RL_OK && j < wlen[i]; ++j)
            rl_host_sampler_remember(ss[i], windows[(size_t)i * wstride + j]);
    }
    std::vector<uint32_t> tokens(n, 0u);
    for (uint32_t c = 0; c < calls && rc == RL_OK; ++c) {
        const clk::time_point t0 = clk::now();
        rc = rl_host_sample_batch(ss.data(), n, d_rows, stride, vocab, tokens.data(), nullptr);
        out_us[c] = us_since(t0);
    }
    for (rl_host_sampler *s : ss) rl_host_sampler_free(s);
    return rc;
}

// `calls` rl_host_sampler_sample_device calls on one device row, a sampler
// made with `set` remembering `history` (Sampler::sample, sample.rs:215-219).
int rlb_sample_calls(int device, const float *d_row, size_t vocab, const rl_sampling *set, const uint32_t *history,
                     size_t hist_len, uint32_t calls, double *out_us) {
    rl_host_sampler *s = nullptr;
    int rc = rl_host_sampler_new(device, vocab, set, 1, &s);
    if (rc != RL_OK) return rc;
    for (size_t i = 0; i < hist_len; ++i) rl_host_sampler_remember(s, history[i]);
    for (uint32_t c = 0; c < calls && rc == RL_OK; ++c) {
        uint32_t t = 0;
        const clk::time_point t0 = clk::now();
        rc = rl_host_sampler_sample_device(s, d_row, vocab, &t, nullptr);
        out_us[c] = us_since(t0);
    }
    rl_host_sampler_free(s);
    return rc;
}

}  // extern "C"

// Counts the heap allocations the host Sampler makes per call (test
// infrastructure; needs a GPU).
//
// The reference proves that `Sampler::sample` allocates nothing by swapping in
// a counting global allocator (crates/rust-llm/tests/sample_allocations.rs:
// 17-136): four settings that reach different stages, a full penalty window,
// two warm-up calls, then 8 counted calls over 248 320 logits. This program
// does the same to librl_sampler.so's host Sampler. It defines malloc and its
// relatives itself, so every allocation in the process, from any thread and
// library, passes through them, and attributes each one to the code that
// asked for it: the innermost stack frame outside the C and C++ runtime
// libraries. A frame in librl_sampler.so is the library's own allocation (the
// contract: there must be none); a frame in the HIP runtime is the runtime's
// bookkeeping for the copies and launches a call issues (reported, not part of
// the library's contract); anything else is reported as other.
//
// Prints one JSON object: per case, the counts over the counted calls.
#include <dlfcn.h>
#include <execinfo.h>
#include <hip/hip_runtime_api.h>
#include <malloc.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "rl_sampler.h"
#include "rl_sampler_host.h"

extern "C" {
void *__libc_malloc(size_t);
void *__libc_calloc(size_t, size_t);
void *__libc_realloc(void *, size_t);
void *__libc_memalign(size_t, size_t);
}

namespace {

std::atomic<bool> g_counting{false};
std::atomic<long> g_ours{0}, g_runtime{0}, g_other{0};
thread_local int t_inside = 0;

bool ends_with(const char *s, const char *suffix) {
    const size_t a = strlen(s), b = strlen(suffix);
    return a >= b && strcmp(s + a - b, suffix) == 0;
}

// Libraries an allocation passes through on its way from the caller.
bool is_runtime_plumbing(const char *path) {
    const char *base = strrchr(path, '/');
    base = base ? base + 1 : path;
    return strncmp(base, "libc.so", 7) == 0 || strncmp(base, "libstdc++.so", 12) == 0 ||
           strncmp(base, "libgcc_s.so", 11) == 0 || strncmp(base, "ld-linux", 8) == 0 ||
           strncmp(base, "libm.so", 7) == 0;
}

// Frame 0 is this function, frame 1 the allocation function that called it;
// the search starts at the allocation's caller.
__attribute__((noinline)) void classify() {
    if (!g_counting.load(std::memory_order_relaxed) || t_inside) return;
    ++t_inside;
    void *frames[96];
    const int n = backtrace(frames, 96);
    int verdict = 2;  // other
    for (int i = 2; i < n; ++i) {
        Dl_info info{};
        if (!dladdr(frames[i], &info) || !info.dli_fname) continue;
        if (is_runtime_plumbing(info.dli_fname)) continue;
        if (ends_with(info.dli_fname, "librl_sampler.so")) verdict = 0;
        else if (strstr(info.dli_fname, "libamdhip64") || strstr(info.dli_fname, "libhsa-runtime") ||
                 strstr(info.dli_fname, "librocprof") || strstr(info.dli_fname, "libamd_comgr"))
            verdict = 1;
        else verdict = 2;
        break;
    }
    (verdict == 0 ? g_ours : verdict == 1 ? g_runtime : g_other).fetch_add(1, std::memory_order_relaxed);
    --t_inside;
}

}  // namespace

extern "C" {
void *malloc(size_t n) {
    classify();
    return __libc_malloc(n);
}
void *calloc(size_t a, size_t b) {
    classify();
    return __libc_calloc(a, b);
}
void *realloc(void *p, size_t n) {
    classify();
    return __libc_realloc(p, n);
}
void *memalign(size_t al, size_t n) {
    classify();
    return __libc_memalign(al, n);
}
void *aligned_alloc(size_t al, size_t n) {
    classify();
    return __libc_memalign(al, n);
}
int posix_memalign(void **out, size_t al, size_t n) {
    classify();
    void *p = __libc_memalign(al, n);
    if (!p) return 12;  // ENOMEM
    *out = p;
    return 0;
}
}

namespace {

constexpr size_t VOCAB = 248320;

// The logit generator of tests/sample_allocations.rs:63-73 (xorshift64, the
// top 53 bits scaled to [-6, 6)).
std::vector<float> logits(uint64_t seed) {
    std::vector<float> v(VOCAB);
    uint64_t s = seed | 1;
    for (auto &x : v) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        x = (float)(s >> 11) / (float)(1ull << 53) * 12.0f - 6.0f;
    }
    return v;
}

struct Counts {
    long ours, runtime, other;
};

Counts window_begin() {
    g_ours = 0;
    g_runtime = 0;
    g_other = 0;
    g_counting = true;
    return {0, 0, 0};
}

Counts window_end() {
    g_counting = false;
    return {g_ours.load(), g_runtime.load(), g_other.load()};
}

bool ok(int rc, const char *what) {
    if (rc != RL_OK) {
        fprintf(stderr, "%s failed: %d %s\n", what, rc, rl_sampler_last_error());
        return false;
    }
    return true;
}

void print_case(bool &first, const char *name, int calls, Counts c) {
    printf("%s\n  \"%s\": {\"calls\": %d, \"library\": %ld, \"hip_runtime\": %ld, \"other\": %ld}", first ? "" : ",",
           name, calls, c.ours, c.runtime, c.other);
    first = false;
    fflush(stdout);
}

}  // namespace

int main() {
    void *warm[4];
    backtrace(warm, 4);  // loads the unwinder before anything is counted
    const std::vector<float> host = logits(3);
    float *d_logits = nullptr;
    const size_t rows_for_batch = 4, verify_rows = 9;
    if (hipMalloc(&d_logits, VOCAB * 4 * verify_rows) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        return 1;
    }
    for (size_t r = 0; r < verify_rows; ++r)
        if (hipMemcpy(d_logits + r * VOCAB, host.data(), VOCAB * 4, hipMemcpyHostToDevice) != hipSuccess) return 1;

    struct Case {
        const char *name;
        rl_sampling set;
    };
    rl_sampling topk_off{1.0f, 0.9f, 0.05f, 1.2f, 0, 64, 1};
    rl_sampling every{0.8f, 0.9f, 0.05f, 1.1f, 40, 64, 2};
    const Case cases[] = {{"greedy", rl_sampling_greedy()},
                          {"the defaults", rl_sampling_default()},
                          {"top-k off, so the candidate set is the whole vocabulary", topk_off},
                          {"every stage on", every}};
    const int calls = 8;
    bool first = true;
    printf("{");
    for (const Case &c : cases) {
        rl_host_sampler *s = nullptr;
        if (!ok(rl_host_sampler_new(0, VOCAB, &c.set, 1, &s), "new")) return 1;
        for (uint32_t t = 0; t < (uint32_t)c.set.repeat_last_n; ++t) rl_host_sampler_remember(s, t / 2);
        uint32_t tok = 0;
        for (int i = 0; i < 2; ++i)
            if (!ok(rl_host_sampler_sample_device(s, d_logits, VOCAB, &tok, nullptr), "sample")) return 1;
        window_begin();
        bool good = true;
        for (int i = 0; i < calls; ++i) good = good && rl_host_sampler_sample_device(s, d_logits, VOCAB, &tok, nullptr) == RL_OK;
        const Counts dev = window_end();
        if (!good) return ok(1, "sample (device logits)"), 1;
        print_case(first, (std::string("device logits: ") + c.name).c_str(), calls, dev);
        for (int i = 0; i < 2; ++i)
            if (!ok(rl_host_sampler_sample(s, host.data(), VOCAB, &tok), "sample (host)")) return 1;
        window_begin();
        for (int i = 0; i < calls; ++i) good = good && rl_host_sampler_sample(s, host.data(), VOCAB, &tok) == RL_OK;
        const Counts hst = window_end();
        if (!good) return ok(1, "sample (host logits)"), 1;
        print_case(first, (std::string("host logits: ") + c.name).c_str(), calls, hst);
        rl_host_sampler_free(s);
    }

    // Speculative verify: 8 drafts, then commits in order until a mismatch.
    {
        rl_sampling set{0.6f, 0.95f, 0.0f, 1.3f, 20, 64, 4};
        rl_host_sampler *s = nullptr;
        if (!ok(rl_host_sampler_new(0, VOCAB, &set, (uint32_t)verify_rows, &s), "new (verify)")) return 1;
        for (uint32_t t = 0; t < 64; ++t) rl_host_sampler_remember(s, t * 7);
        uint32_t drafts[8], picks[9], tok = 0;
        auto round = [&](bool &good) {
            // Drafts equal to the picks of a first verify are accepted in
            // full, so every row is committed on the second.
            good = good && rl_host_sampler_verify(s, d_logits, VOCAB, VOCAB, drafts, 8, picks, nullptr) == RL_OK;
            for (uint32_t r = 0; good && r < 9; ++r) {
                good = rl_host_sampler_commit_verified(s, r, &tok) == RL_OK;
                if (r < 8 && tok != drafts[r]) break;
            }
        };
        for (int i = 0; i < 8; ++i) drafts[i] = 0;
        bool good = true;
        for (int w = 0; w < 2; ++w) {
            if (!ok(rl_host_sampler_verify(s, d_logits, VOCAB, VOCAB, drafts, 8, picks, nullptr), "verify")) return 1;
            for (int i = 0; i < 8; ++i) drafts[i] = picks[i];
            round(good);
        }
        window_begin();
        for (int i = 0; i < calls; ++i) round(good);
        const Counts v = window_end();
        if (!good) return ok(1, "verify/commit"), 1;
        print_case(first, "verify 8 drafts and commit", calls, v);
        rl_host_sampler_free(s);
    }

    // Batched serving: four samplers with different settings, one call.
    {
        rl_host_sampler *ss[rows_for_batch] = {};
        const rl_sampling sets[rows_for_batch] = {rl_sampling_default(), rl_sampling_greedy(), topk_off, every};
        for (size_t i = 0; i < rows_for_batch; ++i) {
            if (!ok(rl_host_sampler_new(0, VOCAB, &sets[i], (uint32_t)rows_for_batch, &ss[i]), "new (batch)")) return 1;
            for (uint32_t t = 0; t < 64; ++t) rl_host_sampler_remember(ss[i], t / 2 + (uint32_t)i);
        }
        uint32_t toks[rows_for_batch];
        for (int i = 0; i < 2; ++i)
            if (!ok(rl_host_sample_batch(ss, rows_for_batch, d_logits, VOCAB, VOCAB, toks, nullptr), "batch")) return 1;
        bool good = true;
        window_begin();
        for (int i = 0; i < calls; ++i)
            good = good && rl_host_sample_batch(ss, rows_for_batch, d_logits, VOCAB, VOCAB, toks, nullptr) == RL_OK;
        const Counts b = window_end();
        if (!good) return ok(1, "batch"), 1;
        print_case(first, "batch of 4 samplers", calls, b);
        for (auto *s : ss) rl_host_sampler_free(s);
    }
    printf("\n}\n");
    (void)hipFree(d_logits);
    return 0;
}

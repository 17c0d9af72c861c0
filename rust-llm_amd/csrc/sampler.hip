// C ABI of the gfx950 token sampler (include/rl_sampler.h): context lifetime,
// per-row path planning, and the launches. Kernels are in sampler_kernels.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "rl_error.h"
#include "rl_pack.h"
#include "rl_runtime.h"
#include "rl_sampler.h"
#include "full_rest.h"
#include "greedy.h"
#include "top_probability.h"

using namespace rl;

namespace {

thread_local std::string g_last_error;

// The longest window the kernels hold on chip (the stream path's LDS set, the
// full path's ids per thread). A call with a longer window stride runs on a
// penalised copy of its rows (k_pen_copy, k_pen_window) with no window.
constexpr uint32_t SET_WINDOW_MAX = 2048;
static_assert(SET_WINDOW_MAX <= ONE_TILE_WIN_MAX, "the one-tile kernel marks every window the stream path takes");
static_assert(ONE_TILE_U * ONE_TILE_THREADS == UNROLL * FAST_THREADS, "both stream instantiations have one tile size");
// Vocabularies up to 2^21 ids (every index and count on the device paths
// fits 32 bits with room to spare).
constexpr uint32_t MAX_VOCAB = 1u << 21;
constexpr uint32_t TARGET_WGS = 1024;  // enough workgroups to cover 256 CUs four deep
constexpr uint32_t FULL_GROUP_MAX = 256;
constexpr uint32_t CHUNK_SLOTS = 2 * TARGET_WGS;

enum class Path : uint8_t { Greedy, Stream, Full };

// log2 of the stream kernel's window-set slots for windows of up to n ids: at
// least twice n (a half-full open-addressed set), at least 64. The set is
// sized per call from the call's window stride, which bounds every row's
// window, so a context made for long windows costs the kernel no LDS on calls
// with short ones.
uint32_t window_hash_bits(uint32_t n) {
    uint32_t bits = 6;
    while ((1u << bits) < 2 * n) ++bits;
    return bits;
}

// Which device path a row's settings take (see sampler_kernels.h).
Path plan_row(const rl_sampling &s, uint32_t vocab) {
    if (s.temperature <= 0.0f) return Path::Greedy;
    if (s.top_k >= 1 && s.top_k <= KMAX && s.top_k < vocab) return Path::Stream;
    return Path::Full;
}

uint64_t row_cand_need(const rl_sampling &s, uint32_t vocab) {
    if (s.temperature <= 0.0f) return 1;
    if (s.top_k == 0 || s.top_k >= vocab) return vocab;
    return s.top_k;
}

// rl_argmax_rows's grid: (chunks, rows); one 64-bit partial result per
// (row, chunk) in `part`, merged per row by k_argmax_final.
uint32_t argmax_chunks(uint32_t rows, uint32_t vocab) {
    const uint32_t chunks = std::min(MAX_CHUNKS, (TARGET_WGS + rows - 1) / rows);
    return std::max(1u, std::min(chunks, vocab / 4096));
}

int launch_argmax(const float *logits, uint64_t row_stride, uint32_t rows, uint32_t vocab, uint32_t *out_token,
                  uint64_t *part, void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint64_t stride = rows > 1 ? row_stride : vocab;
    const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) && (stride % 4 == 0);
    const uint32_t chunks = argmax_chunks(rows, vocab);
    dim3 grid(chunks, rows);
    if (vec)
        hipLaunchKernelGGL(k_argmax_part<true>, grid, dim3(FAST_THREADS), 0, st, logits, stride, vocab, chunks, part);
    else
        hipLaunchKernelGGL(k_argmax_part<false>, grid, dim3(FAST_THREADS), 0, st, logits, stride, vocab, chunks, part);
    hipLaunchKernelGGL(k_argmax_final, dim3((rows + 255) / 256), dim3(256), 0, st, part, rows, chunks, out_token);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "argmax kernels");
    return RL_OK;
}

// The allocation-free argmax (rl_argmax_rows_noalloc) keeps its partial
// results in this fixed device array instead of a context's buffer: one per
// (row, chunk). With rows <= NOALLOC_MAX_ROWS a call needs at most
// max(rows, 2 * TARGET_WGS) entries (rows >= TARGET_WGS take one chunk each,
// fewer rows take at most ceil(TARGET_WGS / rows) chunks). Every entry a call
// reads is written by the same call first, so nothing needs clearing. Each
// GPU holds its own copy from the library's load until the process ends
// (64 KiB). Calls that overlap on one GPU share it and race.
constexpr uint32_t NOALLOC_MAX_ROWS = 8192;
constexpr size_t NOALLOC_SCRATCH = NOALLOC_MAX_ROWS;
static_assert(NOALLOC_SCRATCH >= 2 * TARGET_WGS, "scratch below the split rows' partials");
static __device__ __align__(256) uint64_t scratch[NOALLOC_SCRATCH];

// The array's device address on each GPU, looked up once per device (with
// that device current). The array's name in host code is not a device
// address: only these pointers go to kernels.
constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<uint64_t *> g_scratch[NOALLOC_MAX_DEVICES];

int noalloc_scratch(int device, uint64_t **out) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return fail(RL_ERR_ARGUMENT, "device index out of range");
    uint64_t *p = g_scratch[device].load(std::memory_order_acquire);
    if (!p) {
        void *addr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress (argmax scratch)");
        p = static_cast<uint64_t *>(addr);
        g_scratch[device].store(p, std::memory_order_release);
    }
    *out = p;
    return RL_OK;
}

// One wave per row: the row's token, kept count and used flag, and its first
// PACK_CANDS candidates, into the host's result block (the kept count last).
__global__ __launch_bounds__(WAVE) void k_pack_rows(const uint32_t *token, const uint32_t *kept, const uint8_t *used,
                                                    const uint32_t *ids, const float *probs, uint64_t cand_stride,
                                                    uint32_t *out_token, uint32_t *out_kept, uint8_t *out_used,
                                                    PackedCands *out_cands) {
    const uint32_t row = blockIdx.x, lane = threadIdx.x;
    const uint32_t k = kept[row];
    const uint32_t n = k < PACK_CANDS ? k : PACK_CANDS;
    // System-scope stores into host memory, the kept count last once the
    // row's other stores have completed: the host polls it (store_sys).
    if (lane < n) {
        store_sys(out_cands[row].ids + lane, ids[(uint64_t)row * cand_stride + lane]);
        store_sys(out_cands[row].probs + lane, probs[(uint64_t)row * cand_stride + lane]);
    }
    if (lane == 0) {
        store_sys(out_token + row, token[row]);
        store_sys(out_used + row, used[row]);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) store_sys(out_kept + row, k);
}

// Windows longer than SET_WINDOW_MAX ids take the reference's own route
// (sample.rs:239-257): the row is copied (:242), then each window id below the
// vocabulary is penalised in the copy (:248-255), and the call samples the copy
// with no window. Every occurrence of an id writes the same value,
// penalize(raw[t]), so writing it once per occurrence leaves what the
// reference's once-per-distinct-id loop leaves, and repeats need no
// deduplication. The copy's rows are `pen_stride` floats (a multiple of 4), 16-byte
// aligned.
constexpr uint32_t PEN_THREADS = 256;
constexpr uint32_t PEN_TARGET_WGS = 2048;

// grid (x, min(rows, 65535)), PEN_THREADS: rows 0..rows-1 of src into dst.
template <bool VEC>
__global__ __launch_bounds__(PEN_THREADS) void k_pen_copy(const float *src, uint64_t stride, uint32_t vocab,
                                                          uint32_t rows, float *dst, uint64_t dstride) {
    const uint32_t t0 = blockIdx.x * PEN_THREADS + threadIdx.x, step = gridDim.x * PEN_THREADS;
    for (uint32_t row = blockIdx.y; row < rows; row += gridDim.y) {
        const float *s = src + (uint64_t)row * stride;
        float *d = dst + (uint64_t)row * dstride;
        uint32_t from = 0;
        if constexpr (VEC) {
            const uint32_t n4 = vocab / 4;
            for (uint32_t q = t0; q < n4; q += step)
                __builtin_nontemporal_store(__builtin_nontemporal_load((const f32x4 *)s + q), (f32x4 *)d + q);
            from = 4 * n4;
        }
        for (uint32_t i = from + t0; i < vocab; i += step) d[i] = s[i];
    }
}

// grid (x, min(rows, 65535)), PEN_THREADS: for each penalising row, every id t
// < vocab of recent[..filled] gets penalize(src[t]) in dst (after k_pen_copy).
__global__ __launch_bounds__(PEN_THREADS) void k_pen_window(const float *src, uint64_t stride, uint32_t vocab,
                                                            uint32_t rows, const rl_sampling *settings,
                                                            const uint32_t *windows, uint32_t wstride,
                                                            const uint32_t *wlen, float *dst, uint64_t dstride) {
    const uint32_t t0 = blockIdx.x * PEN_THREADS + threadIdx.x, step = gridDim.x * PEN_THREADS;
    for (uint32_t row = blockIdx.y; row < rows; row += gridDim.y) {
        const rl_sampling s = settings[row];
        if (!penalises(s)) continue;
        const uint32_t l = wlen[row];
        const uint32_t wl = l < wstride ? l : wstride;
        const uint32_t *w = windows + (uint64_t)row * wstride;
        for (uint32_t i = t0; i < wl; i += step) {
            const uint32_t t = w[i];
            if (t < vocab) dst[(uint64_t)row * dstride + t] = penalize(src[(uint64_t)row * stride + t], s.repeat_penalty);
        }
    }
}

}  // namespace

void rl::set_last_error(const std::string &msg) { g_last_error = msg; }

int rl::launch_pack_rows(const uint32_t *token, const uint32_t *kept, const uint8_t *used, const uint32_t *ids,
                         const float *probs, uint64_t cand_stride, uint32_t rows, uint32_t *out_token,
                         uint32_t *out_kept, uint8_t *out_used, PackedCands *out_cands, void *stream) {
    if (rows == 0) return RL_OK;
    static_assert(PACK_CANDS <= WAVE, "one lane per packed candidate");
    hipLaunchKernelGGL(k_pack_rows, dim3(rows), dim3(WAVE), 0, static_cast<hipStream_t>(stream), token, kept, used,
                       ids, probs, cand_stride, out_token, out_kept, out_used, out_cands);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "pack kernel");
    return RL_OK;
}

struct rl_sampler_ctx {
    int device = 0;
    uint32_t max_rows = 0, vocab = 0, max_window = 0, full_group = 0;
    rl_sampling *d_settings = nullptr;
    uint32_t *d_stream_rows = nullptr, *d_full_rows = nullptr, *d_greedy_rows = nullptr;
    uint64_t *d_greedy_best = nullptr;   // the greedy path's row slots, zero between calls
    uint32_t *d_greedy_arrive = nullptr; // and arrival counters
    uint64_t *d_chunk_cands = nullptr;
    uint32_t *d_chunk_counts = nullptr;
    uint32_t *d_arrive = nullptr;
    uint32_t *d_keyA = nullptr, *d_idA = nullptr, *d_keyB = nullptr, *d_idB = nullptr;
    float *d_probs = nullptr;
    float *d_part_max = nullptr;
    uint64_t *d_part_am = nullptr;
    double *d_psum = nullptr;
    uint64_t *d_surv = nullptr;
    FullRow *d_full_row = nullptr;
    uint32_t *d_full_arrive = nullptr;
    uint64_t *d_argmax_part = nullptr;
    uint32_t *d_tp_nan = nullptr;
    double *d_tp_sum = nullptr;
    uint32_t *d_tp_small = nullptr;  // per chunk: nonzero terms below 2^-26
    float *d_pen = nullptr;          // max_window > SET_WINDOW_MAX: the penalised rows
    uint64_t pen_stride = 0;         // floats per row of d_pen
    std::vector<void *> owned;
    // Host copy of the plan made by configure.
    uint32_t configured = 0;
    std::vector<uint32_t> stream_rows, full_rows, greedy_rows;  // ascending; capacity max_rows
    std::vector<uint64_t> need_upto;               // [r]: candidates rows 0..r can keep; capacity max_rows
    uint64_t cand_need = 0;
    bool any_drawing = false;
    bool polled = false;  // set_results_polled

    template <class T>
    hipError_t alloc(T **p, size_t count) {
        void *v = nullptr;
        const hipError_t e = hipMalloc(&v, std::max<size_t>(count, 1) * sizeof(T));
        if (e == hipSuccess) {
            owned.push_back(v);
            *p = static_cast<T *>(v);
        }
        return e;
    }
    ~rl_sampler_ctx() {
        for (void *p : owned) (void)hipFree(p);
    }
};

void rl::set_results_polled(rl_sampler_ctx *ctx, bool polled) { ctx->polled = polled; }

bool rl::rows_all_stream(const rl_sampler_ctx *ctx, uint32_t rows) {
    return ctx->full_rows.empty() || ctx->full_rows.front() >= rows;  // ascending
}

extern "C" {

const char *rl_sampler_last_error(void) { return g_last_error.c_str(); }

int rl_sampler_create(int device, uint32_t max_rows, uint32_t vocab, uint32_t max_window,
                      rl_sampler_ctx **out) {
    if (!out) return fail(RL_ERR_ARGUMENT, "out is null");
    *out = nullptr;
    if (max_rows == 0 || vocab == 0) return fail(RL_ERR_ARGUMENT, "max_rows and vocab must be positive");
    if (vocab > MAX_VOCAB) return fail(RL_ERR_CAPACITY, "vocab above " + std::to_string(MAX_VOCAB));
    DeviceGuard g(device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device " + std::to_string(device));
    auto *c = new (std::nothrow) rl_sampler_ctx();
    if (!c) return fail(RL_ERR_CAPACITY, "out of host memory");
    c->device = device;
    c->max_rows = max_rows;
    c->vocab = vocab;
    c->max_window = max_window;
    c->full_group = std::min(max_rows, FULL_GROUP_MAX);
    try {  // configure fills these in place
        c->stream_rows.reserve(max_rows);
        c->full_rows.reserve(max_rows);
        c->greedy_rows.reserve(max_rows);
        c->need_upto.reserve(max_rows);
    } catch (const std::bad_alloc &) {
        delete c;
        return fail(RL_ERR_CAPACITY, "out of host memory");
    }
    const size_t fg = c->full_group, V = vocab;
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = c->alloc(&c->d_settings, max_rows);
    if (e == hipSuccess) e = c->alloc(&c->d_stream_rows, max_rows);
    if (e == hipSuccess) e = c->alloc(&c->d_full_rows, max_rows);
    if (e == hipSuccess) e = c->alloc(&c->d_greedy_rows, max_rows);
    if (e == hipSuccess) e = c->alloc(&c->d_greedy_best, max_rows);
    if (e == hipSuccess) e = c->alloc(&c->d_greedy_arrive, max_rows);
    if (e == hipSuccess) e = hipMemset(c->d_greedy_best, 0, (size_t)max_rows * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(c->d_greedy_arrive, 0, (size_t)max_rows * sizeof(uint32_t));
    // Rows are split into chunks only while rows < TARGET_WGS, with
    // chunks <= ceil(TARGET_WGS / rows), so rows * chunks < 2 * TARGET_WGS.
    if (e == hipSuccess) e = c->alloc(&c->d_chunk_cands, (size_t)CHUNK_SLOTS * KMAX);
    if (e == hipSuccess) e = c->alloc(&c->d_chunk_counts, (size_t)CHUNK_SLOTS);
    if (e == hipSuccess) e = c->alloc(&c->d_arrive, (size_t)max_rows);
    // Arrival counters return to zero at the end of every call.
    if (e == hipSuccess) e = hipMemset(c->d_arrive, 0, (size_t)max_rows * sizeof(uint32_t));
    if (e == hipSuccess) e = c->alloc(&c->d_keyA, fg * V);
    if (e == hipSuccess) e = c->alloc(&c->d_idA, fg * V);
    if (e == hipSuccess) e = c->alloc(&c->d_keyB, fg * V);
    if (e == hipSuccess) e = c->alloc(&c->d_idB, fg * V);
    if (e == hipSuccess) e = c->alloc(&c->d_probs, fg * V);
    if (e == hipSuccess) e = c->alloc(&c->d_part_max, fg * MAX_CHUNKS);
    if (e == hipSuccess) e = c->alloc(&c->d_part_am, fg * MAX_CHUNKS);
    if (e == hipSuccess) e = c->alloc(&c->d_psum, fg * MAX_CHUNKS);
    if (e == hipSuccess) e = c->alloc(&c->d_surv, fg * SURV_CAP);
    if (e == hipSuccess) e = c->alloc(&c->d_full_row, fg);
    if (e == hipSuccess) e = c->alloc(&c->d_full_arrive, fg);
    if (e == hipSuccess) e = hipMemset(c->d_full_arrive, 0, fg * sizeof(uint32_t));
    if (e == hipSuccess) e = c->alloc(&c->d_argmax_part, std::max<size_t>(CHUNK_SLOTS, max_rows));
    if (e == hipSuccess) e = c->alloc(&c->d_tp_nan, std::max<size_t>(CHUNK_SLOTS, max_rows));
    if (e == hipSuccess) e = c->alloc(&c->d_tp_sum, std::max<size_t>(CHUNK_SLOTS, max_rows));
    if (e == hipSuccess) e = c->alloc(&c->d_tp_small, std::max<size_t>(CHUNK_SLOTS, max_rows));
    if (max_window > SET_WINDOW_MAX) {
        c->pen_stride = (V + 3) & ~(size_t)3;
        if (e == hipSuccess) e = c->alloc(&c->d_pen, (size_t)max_rows * c->pen_stride);
    }
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "hipMalloc");
    }
    *out = c;
    return RL_OK;
}

void rl_sampler_destroy(rl_sampler_ctx *ctx) {
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    (void)hipDeviceSynchronize();
    delete ctx;
}

int rl_sampler_configure(rl_sampler_ctx *ctx, const rl_sampling *settings, uint32_t rows) {
    if (!ctx || !settings) return fail(RL_ERR_ARGUMENT, "null argument");
    if (rows == 0 || rows > ctx->max_rows)
        return fail(RL_ERR_CAPACITY, "rows must be in 1..max_rows");
    DeviceGuard g(ctx->device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device");
    // The plan is rebuilt in place (the lists' capacity is max_rows, so this
    // allocates nothing); until the upload succeeds the context is unconfigured.
    ctx->configured = 0;
    ctx->stream_rows.clear();
    ctx->full_rows.clear();
    ctx->greedy_rows.clear();
    ctx->need_upto.clear();
    uint64_t need = 0;
    bool drawing = false;
    for (uint32_t r = 0; r < rows; ++r) {
        const Path p = plan_row(settings[r], ctx->vocab);
        (p == Path::Greedy ? ctx->greedy_rows : p == Path::Stream ? ctx->stream_rows : ctx->full_rows).push_back(r);
        need = std::max(need, row_cand_need(settings[r], ctx->vocab));
        ctx->need_upto.push_back(need);
        drawing = drawing || !(settings[r].temperature <= 0.0f);
    }
    const auto &sr = ctx->stream_rows;
    const auto &fr = ctx->full_rows;
    const auto &gr = ctx->greedy_rows;
    hipError_t e = hipMemcpy(ctx->d_settings, settings, rows * sizeof(rl_sampling), hipMemcpyHostToDevice);
    if (e == hipSuccess && !sr.empty())
        e = hipMemcpy(ctx->d_stream_rows, sr.data(), sr.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess && !fr.empty())
        e = hipMemcpy(ctx->d_full_rows, fr.data(), fr.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess && !gr.empty())
        e = hipMemcpy(ctx->d_greedy_rows, gr.data(), gr.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy (configure)");
    ctx->configured = rows;
    ctx->cand_need = need;
    ctx->any_drawing = drawing;
    return RL_OK;
}

int rl_sampler_required_cand_stride(const rl_sampler_ctx *ctx, uint64_t *out) {
    if (!ctx || !out) return fail(RL_ERR_ARGUMENT, "null argument");
    if (!ctx->configured) return fail(RL_ERR_NOT_CONFIGURED, "configure first");
    *out = ctx->cand_need;
    return RL_OK;
}

int rl_sampler_sample_rows(rl_sampler_ctx *ctx, const float *logits, uint64_t row_stride,
                           uint32_t rows, uint32_t vocab, const uint32_t *windows,
                           uint32_t window_stride, const uint32_t *window_len,
                           const float *uniforms, uint32_t *out_token, uint32_t *out_kept,
                           uint8_t *out_used_uniform, uint32_t *out_cand_ids,
                           float *out_cand_probs, uint64_t cand_stride, void *stream) {
    if (!ctx) return fail(RL_ERR_ARGUMENT, "ctx is null");
    if (!ctx->configured) return fail(RL_ERR_NOT_CONFIGURED, "configure first");
    if (vocab != ctx->vocab)
        return fail(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
    if (rows == 0) return RL_OK;
    if (rows > ctx->configured) return fail(RL_ERR_CAPACITY, "more rows than configured");
    if (!logits || !out_token || !out_kept || !out_used_uniform)
        return fail(RL_ERR_ARGUMENT, "null logits or outputs");
    if (rows > 1 && row_stride < vocab) return fail(RL_ERR_ARGUMENT, "row_stride below vocab");
    if ((out_cand_ids == nullptr) != (out_cand_probs == nullptr))
        return fail(RL_ERR_ARGUMENT, "candidate ids and probs must both be given or both be null");
    // The call's own rows decide the stride it needs (a prefix of the
    // configured rows may keep fewer candidates than all of them).
    if (out_cand_ids && cand_stride < ctx->need_upto[rows - 1])
        return fail(RL_ERR_CAPACITY, "cand_stride below what the call's rows can keep "
                                     "(rl_sampler_required_cand_stride for all configured rows)");
    if (window_len && windows && window_stride > ctx->max_window)
        return fail(RL_ERR_CAPACITY, "window_stride above max_window");
    if (ctx->any_drawing && !uniforms) return fail(RL_ERR_ARGUMENT, "uniforms are null");
    DeviceGuard g(ctx->device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device");
    hipStream_t st = static_cast<hipStream_t>(stream);

    RowIO io{};
    io.logits = logits;
    io.stride = rows > 1 ? row_stride : vocab;
    io.vocab = vocab;
    io.settings = ctx->d_settings;
    io.windows = (windows && window_len) ? windows : nullptr;
    io.wstride = (windows && window_len) ? window_stride : 0;
    io.wlen = (windows && window_len) ? window_len : nullptr;
    io.uniforms = uniforms;
    io.out_token = out_token;
    io.out_kept = out_kept;
    io.out_used = out_used_uniform;
    io.out_ids = out_cand_ids;
    io.out_probs = out_cand_probs;
    io.cand_stride = cand_stride;
    io.polled = ctx->polled ? 1u : 0u;
    if (io.windows && io.wstride > SET_WINDOW_MAX) {
        // A window longer than the kernels hold on chip: sample a penalised
        // copy of the rows, with no window (k_pen_copy).
        const bool svec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) && (io.stride % 4 == 0);
        const uint32_t gy = std::min(rows, 65535u);
        const uint32_t per_row = std::max(1u, (PEN_TARGET_WGS + rows - 1) / rows);
        const uint32_t cx = std::max(1u, std::min(per_row, (vocab / 4 + PEN_THREADS - 1) / PEN_THREADS));
        const uint32_t wx = std::max(1u, std::min(per_row, (io.wstride + PEN_THREADS - 1) / PEN_THREADS));
        if (svec)
            hipLaunchKernelGGL(k_pen_copy<true>, dim3(cx, gy), dim3(PEN_THREADS), 0, st, logits, io.stride, vocab, rows,
                               ctx->d_pen, ctx->pen_stride);
        else
            hipLaunchKernelGGL(k_pen_copy<false>, dim3(cx, gy), dim3(PEN_THREADS), 0, st, logits, io.stride, vocab,
                               rows, ctx->d_pen, ctx->pen_stride);
        hipLaunchKernelGGL(k_pen_window, dim3(wx, gy), dim3(PEN_THREADS), 0, st, logits, io.stride, vocab, rows,
                           ctx->d_settings, io.windows, io.wstride, io.wlen, ctx->d_pen, ctx->pen_stride);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "penalty copy kernels");
        io.logits = ctx->d_pen;
        io.stride = ctx->pen_stride;
        io.windows = nullptr;
        io.wstride = 0;
        io.wlen = nullptr;
    }
    io.hash_bits = window_hash_bits(io.wstride);
    const bool vec = (reinterpret_cast<uintptr_t>(io.logits) % 16 == 0) && (io.stride % 4 == 0);

    // Rows below `rows` on each path (the lists are ascending).
    const uint32_t ns = (uint32_t)(std::lower_bound(ctx->stream_rows.begin(), ctx->stream_rows.end(), rows) -
                                   ctx->stream_rows.begin());
    const uint32_t nf = (uint32_t)(std::lower_bound(ctx->full_rows.begin(), ctx->full_rows.end(), rows) -
                                   ctx->full_rows.begin());
    const uint32_t ngr = (uint32_t)(std::lower_bound(ctx->greedy_rows.begin(), ctx->greedy_rows.end(), rows) -
                                   ctx->greedy_rows.begin());
    if (ngr > 0) {
        RowIO gio = io;
        gio.rows = ctx->greedy_rows[ngr - 1] == ngr - 1 ? nullptr : ctx->d_greedy_rows;
        gio.row0 = 0;
        // Chunks as the stream path's: while rows are few, at most one tile a chunk.
        const uint32_t n4 = vocab / 4;
        constexpr uint32_t STEP4 = FAST_THREADS * UNROLL;
        uint32_t chunks = (TARGET_WGS + ngr - 1) / ngr;
        chunks = std::min(chunks, MAX_CHUNKS);
        chunks = std::min(chunks, std::max(1u, (n4 + STEP4 - 1) / STEP4));
        gio.chunks = std::max(chunks, 1u);
        // The window bitmap: the largest chunk's elements (the last one also
        // takes the row's vocab % 4).
        const size_t glds = gio.windows ? chunk_bitmap_words(4 * ((n4 + gio.chunks - 1) / gio.chunks) + 3) * 4 : 0;
        GreedyScratch gs{ctx->d_greedy_best, ctx->d_greedy_arrive};
        const dim3 grid(gio.chunks, ngr);
        if (vec)
            hipLaunchKernelGGL(k_greedy<true>, grid, dim3(FAST_THREADS), glds, st, gio, gs);
        else
            hipLaunchKernelGGL(k_greedy<false>, grid, dim3(FAST_THREADS), glds, st, gio, gs);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "greedy kernel");
    }
    if (ns > 0) {
        RowIO s = io;
        // The stream rows are ascending and distinct: they are 0 .. ns-1
        // exactly when the last is ns - 1, and the kernel then needs no list.
        s.rows = ctx->stream_rows[ns - 1] == ns - 1 ? nullptr : ctx->d_stream_rows;
        s.row0 = 0;
        const uint32_t n4 = vocab / 4;
        // Rows are split into chunks while there are fewer workgroups than
        // fill the GPU, but no further than one tile a chunk (a chunk a little
        // over one tile pays a second round trip to memory for its rest).
        constexpr uint32_t STEP4 = FAST_THREADS * UNROLL;
        uint32_t chunks = (TARGET_WGS + ns - 1) / ns;
        chunks = std::min(chunks, MAX_CHUNKS);
        chunks = std::min(chunks, std::max(1u, (n4 + STEP4 - 1) / STEP4));
        s.chunks = std::max(chunks, 1u);
        FastScratch sc{ctx->d_chunk_cands, ctx->d_chunk_counts, ctx->d_arrive};
        dim3 grid(s.chunks, ns);
        // Chunks of at most one tile each take the one-tile kernel, whose
        // window is a bitmap over the chunk's elements (the last chunk's
        // take the row's vocab % 4 more).
        const uint32_t per = (n4 + s.chunks - 1) / s.chunks;
        size_t wlds = window_lds_bytes(io.hash_bits);
        if (per <= STEP4) {
            wlds = std::max(wlds, (size_t)chunk_bitmap_words(4 * per + 3) * sizeof(uint32_t));
            if (vec)
                hipLaunchKernelGGL((k_stream<true, ONE_TILE_U, ONE_TILE_THREADS, true>), grid, dim3(ONE_TILE_THREADS),
                                   wlds, st, s, sc);
            else
                hipLaunchKernelGGL((k_stream<false, ONE_TILE_U, ONE_TILE_THREADS, true>), grid, dim3(ONE_TILE_THREADS),
                                   wlds, st, s, sc);
        } else if (vec) {
            hipLaunchKernelGGL((k_stream<true, UNROLL, FAST_THREADS>), grid, dim3(FAST_THREADS), wlds, st, s, sc);
        } else {
            hipLaunchKernelGGL((k_stream<false, UNROLL, FAST_THREADS>), grid, dim3(FAST_THREADS), wlds, st, s, sc);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "stream kernels");
    }
    for (uint32_t g0 = 0; g0 < nf; g0 += ctx->full_group) {
        const uint32_t ng = std::min(ctx->full_group, nf - g0);
        RowIO f = io;
        // A group whose rows are consecutive needs no list: the kernels index
        // row0 + slot directly (no dependent load before the row's address).
        const bool consecutive = ctx->full_rows[g0 + ng - 1] - ctx->full_rows[g0] == ng - 1;
        f.rows = consecutive ? nullptr : ctx->d_full_rows + g0;
        f.row0 = ctx->full_rows[g0];
        f.chunks = std::max(1u, std::min(MAX_CHUNKS, (TARGET_WGS + ng - 1) / ng));
        f.chunks = std::min(f.chunks, std::max(1u, vocab / 4096));
        FullScratch fs{ctx->d_keyA,    ctx->d_idA,     ctx->d_keyB, ctx->d_idB,     ctx->d_probs, ctx->d_part_max,
                       ctx->d_part_am, ctx->d_psum,    ctx->d_surv, ctx->d_full_row, ctx->d_full_arrive};
        const dim3 cgrid(f.chunks, ng);
        const size_t pass_lds = k_full_pass_lds_bytes(vocab, f.chunks);
        if (vec)
            hipLaunchKernelGGL(k_full_pass<true>, cgrid, dim3(FULL_THREADS), pass_lds, st, f, fs);
        else
            hipLaunchKernelGGL(k_full_pass<false>, cgrid, dim3(FULL_THREADS), pass_lds, st, f, fs);
        hipLaunchKernelGGL(k_full_rest, dim3(ng), dim3(REST_THREADS), 0, st, f, fs);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "full-path kernels");
    }
    return RL_OK;
}

int rl_argmax_rows(rl_sampler_ctx *ctx, const float *logits, uint64_t row_stride, uint32_t rows,
                   uint32_t vocab, uint32_t *out_token, void *stream) {
    if (!ctx) return fail(RL_ERR_ARGUMENT, "ctx is null");
    if (vocab != ctx->vocab)
        return fail(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
    if (rows == 0) return RL_OK;
    if (rows > ctx->max_rows) return fail(RL_ERR_CAPACITY, "more rows than max_rows");
    if (!logits || !out_token) return fail(RL_ERR_ARGUMENT, "null logits or output");
    if (rows > 1 && row_stride < vocab) return fail(RL_ERR_ARGUMENT, "row_stride below vocab");
    DeviceGuard g(ctx->device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device");
    return launch_argmax(logits, row_stride, rows, vocab, out_token, ctx->d_argmax_part, stream);
}

int rl_argmax_rows_noalloc(int device, const float *logits, uint64_t row_stride, uint32_t rows, uint32_t vocab,
                           uint32_t *out_token, void *stream) {
    if (rows == 0) return RL_OK;
    if (vocab == 0) return fail(RL_ERR_ARGUMENT, "vocab must be positive");
    if (rows > NOALLOC_MAX_ROWS)
        return fail(RL_ERR_CAPACITY, "rl_argmax_rows_noalloc takes at most " + std::to_string(NOALLOC_MAX_ROWS) +
                                         " rows (its scratch is a fixed device array); use rl_argmax_rows");
    if (!logits || !out_token) return fail(RL_ERR_ARGUMENT, "null logits or output");
    if (rows > 1 && row_stride < vocab) return fail(RL_ERR_ARGUMENT, "row_stride below vocab");
    DeviceGuard g(device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device " + std::to_string(device));
    uint64_t *part = nullptr;
    const int rc = noalloc_scratch(device, &part);
    if (rc != RL_OK) return rc;
    return launch_argmax(logits, row_stride, rows, vocab, out_token, part, stream);
}

int rl_top_probability_rows(rl_sampler_ctx *ctx, const float *logits, uint64_t row_stride, uint32_t rows,
                            uint32_t vocab, uint32_t *out_token, float *out_prob, void *stream) {
    if (!ctx) return fail(RL_ERR_ARGUMENT, "ctx is null");
    if (vocab != ctx->vocab)
        return fail(RL_ERR_VOCAB, "this sampler was built for a different vocabulary");
    if (rows == 0) return RL_OK;
    if (rows > ctx->max_rows) return fail(RL_ERR_CAPACITY, "more rows than max_rows");
    if (!logits || !out_token || !out_prob) return fail(RL_ERR_ARGUMENT, "null logits or outputs");
    if (rows > 1 && row_stride < vocab) return fail(RL_ERR_ARGUMENT, "row_stride below vocab");
    DeviceGuard g(ctx->device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint64_t stride = rows > 1 ? row_stride : vocab;
    const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) && (stride % 4 == 0);
    // Two workgroups a CU slot (the sum pass is bound by its arithmetic, and
    // more, shorter workgroups even out the CUs), within the chunk arrays'
    // max(CHUNK_SLOTS, max_rows) entries.
    const uint32_t slots = std::max(CHUNK_SLOTS, ctx->max_rows);
    uint32_t chunks = std::min(MAX_CHUNKS, (2 * TARGET_WGS + rows - 1) / rows);
    chunks = std::max(1u, std::min({chunks, vocab / 4096, slots / rows}));
    dim3 grid(chunks, rows);
    if (vec) {
        hipLaunchKernelGGL(k_tp_max<true>, grid, dim3(FAST_THREADS), 0, st, logits, stride, vocab, chunks,
                           ctx->d_argmax_part, ctx->d_tp_nan);
        hipLaunchKernelGGL(k_tp_sum<true>, grid, dim3(FAST_THREADS), 0, st, logits, stride, vocab, chunks,
                           ctx->d_argmax_part, ctx->d_tp_nan, ctx->d_tp_sum, ctx->d_tp_small, ctx->d_arrive,
                           out_token, out_prob);
    } else {
        hipLaunchKernelGGL(k_tp_max<false>, grid, dim3(FAST_THREADS), 0, st, logits, stride, vocab, chunks,
                           ctx->d_argmax_part, ctx->d_tp_nan);
        hipLaunchKernelGGL(k_tp_sum<false>, grid, dim3(FAST_THREADS), 0, st, logits, stride, vocab, chunks,
                           ctx->d_argmax_part, ctx->d_tp_nan, ctx->d_tp_sum, ctx->d_tp_small, ctx->d_arrive,
                           out_token, out_prob);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "top_probability kernels");
    return RL_OK;
}

int rl_sampler_expf_range(uint32_t lo_bits, uint64_t count, float *out, void *stream) {
    if (!out) return fail(RL_ERR_ARGUMENT, "out is null");
    if (count == 0) return RL_OK;
    if (count > (1ull << 32) - lo_bits) return fail(RL_ERR_ARGUMENT, "range past 0xFFFFFFFF");
    const uint64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(k_expf_range, dim3((uint32_t)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), lo_bits,
                       count, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "expf kernel");
    return RL_OK;
}

}  // extern "C"

// C ABI of the gfx950 output head (include/rl_head.h): weight upload and
// repack, activation quantization, and the head launches. Kernels are in
// head_kernels.h.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <new>
#include <string>

#include "head_kernels.h"
#include "rl_head.h"
#include "rl_runtime.h"

using namespace rl;

struct rl_head {
    int device = 0;
    uint32_t k = 0, rows = 0, nb = 0, groups = 0, max_batch = 0, tcap = 0;
    uint4 *wq = nullptr;
    uint32_t *ws = nullptr;
    uint16_t *wd = nullptr;
    float *ad = nullptr;    // activation scales [tcap][nb]
    uint4 *af = nullptr;    // activation fragments [tcap / 16][nb][HEAD_FRAG_UINT4]
    ~rl_head() {
        (void)hipFree(wq);
        (void)hipFree(ws);
        (void)hipFree(wd);
        (void)hipFree(ad);
        (void)hipFree(af);
    }
};

namespace {

// LDS the dot path's own quantization takes for `t` rows of `nb` blocks.
size_t dot_lds_bytes(uint32_t t, uint32_t nb) { return (size_t)t * nb * DOT_ACT_WORDS * 4; }
constexpr size_t DOT_LDS_MAX = 48 * 1024;

// Whether rows t0 .. t0 + n take the dot path (which quantizes them itself).
bool dot_path(const rl_head *h, uint32_t n) { return n <= 2 && dot_lds_bytes(n, h->nb) <= DOT_LDS_MAX; }

// Rows t0 .. t0 + n of the batch, n <= 32: the dot path for one or two rows
// (memory-bound, least arithmetic per weight), the matrix cores for more.
void launch_head(const rl_head *h, const float *x, uint32_t t0, uint32_t n, float *out, uint64_t stride,
                 hipStream_t s) {
    const uint32_t blocks = (h->groups + HEAD_WAVES - 1) / HEAD_WAVES;
    const uint64_t ao = (uint64_t)t0 * h->nb;
    const uint64_t fo = (uint64_t)(t0 / HEAD_NTILE) * h->nb * HEAD_FRAG_UINT4;  // t0 is a multiple of 32
    if (dot_path(h, n)) {
        auto kern = n == 1 ? k_head_dot<1> : k_head_dot<2>;
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(HEAD_THREADS), dot_lds_bytes(n, h->nb), s, h->wq, h->ws,
                           h->wd, x + (uint64_t)t0 * h->k, h->k, h->nb, h->rows, h->groups, out, stride);
    } else if (n <= HEAD_NTILE) {
        hipLaunchKernelGGL(k_head_mfma_regs<1>, dim3(blocks), dim3(HEAD_THREADS), 0, s, h->wq, h->ws, h->wd,
                           h->af + fo, h->ad + ao, n, h->nb, h->rows, h->groups, out, stride);
    } else {
        hipLaunchKernelGGL(k_head_mfma_lds<2>, dim3(blocks), dim3(HEAD_THREADS), 0, s, h->wq, h->ws, h->wd,
                           h->af + fo, h->ad + ao, n, h->nb, h->rows, h->groups, out, stride);
    }
}

void launch_quantize(const float *x, uint32_t t, uint32_t k, uint32_t nb, float *d, int8_t *qs, int16_t *bs,
                     uint4 *frag, hipStream_t s) {
    const uint64_t waves = (uint64_t)t * nb;
    const uint32_t blocks = (uint32_t)((waves + 3) / 4);
    hipLaunchKernelGGL(k_quantize_rows, dim3(blocks), dim3(256), 0, s, x, t, k, nb, d, qs, bs, frag);
}

}  // namespace

extern "C" {

int rl_head_create(int device, uint32_t k, uint32_t rows, uint32_t max_batch, const void *q6k, uint64_t q6k_bytes,
                   rl_head **out) {
    if (!out) return fail(RL_ERR_ARGUMENT, "out is null");
    *out = nullptr;
    if (!q6k) return fail(RL_ERR_ARGUMENT, "q6k is null");
    if (k == 0 || rows == 0 || max_batch == 0) return fail(RL_ERR_ARGUMENT, "k, rows and max_batch must be positive");
    const uint32_t nb = (k + QK - 1) / QK;
    if (q6k_bytes != (uint64_t)rows * nb * Q6K_BLOCK_BYTES)
        return fail(RL_ERR_ARGUMENT, "q6k_bytes is not rows * ceil(k/256) * 210");
    DeviceGuard g(device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select device " + std::to_string(device));
    auto *h = new (std::nothrow) rl_head();
    if (!h) return fail(RL_ERR_CAPACITY, "out of host memory");
    h->device = device;
    h->k = k;
    h->rows = rows;
    h->nb = nb;
    h->groups = (rows + HEAD_GROUP - 1) / HEAD_GROUP;
    h->max_batch = max_batch;
    h->tcap = (max_batch + HEAD_NTILE - 1) / HEAD_NTILE * HEAD_NTILE;
    const uint64_t bgt = (uint64_t)nb * h->groups * HEAD_TILES;
    hipError_t e = hipMalloc(&h->wq, bgt * HEAD_QCH * 64 * sizeof(uint4));
    if (e == hipSuccess) e = hipMalloc(&h->ws, bgt * 64 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&h->wd, bgt * HEAD_TILE * sizeof(uint16_t));
    if (e == hipSuccess) e = hipMalloc(&h->ad, (uint64_t)h->tcap * nb * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&h->af, (uint64_t)(h->tcap / HEAD_NTILE) * nb * HEAD_FRAG_UINT4 * sizeof(uint4));
    // Rows of a column tile past a call's t are read and their products
    // discarded; start them at zero.
    if (e == hipSuccess) e = hipMemset(h->ad, 0, (uint64_t)h->tcap * nb * sizeof(float));
    if (e == hipSuccess) e = hipMemset(h->af, 0, (uint64_t)(h->tcap / HEAD_NTILE) * nb * HEAD_FRAG_UINT4 * sizeof(uint4));
    uint8_t *staging = nullptr;
    if (e == hipSuccess) e = hipMalloc(&staging, q6k_bytes);
    if (e == hipSuccess) e = hipMemcpy(staging, q6k, q6k_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        const uint64_t threads = bgt * 64;
        hipLaunchKernelGGL(k_q6k_repack, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, 0, staging, rows,
                           nb, h->groups, h->wq, h->ws, h->wd);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        delete h;
        return hip_fail(e, "rl_head_create");
    }
    *out = h;
    return RL_OK;
}

void rl_head_destroy(rl_head *head) {
    if (!head) return;
    DeviceGuard g(head->device);
    delete head;
}

int rl_head_logits(rl_head *h, const float *x, uint32_t t, float *logits, uint64_t row_stride, void *stream) {
    if (!h) return fail(RL_ERR_ARGUMENT, "head is null");
    if (t == 0) return RL_OK;
    if (!x || !logits) return fail(RL_ERR_ARGUMENT, "x and logits must be device pointers");
    if (t > h->max_batch) return fail(RL_ERR_CAPACITY, "t above the head's max_batch");
    if (row_stride < h->rows) return fail(RL_ERR_ARGUMENT, "row_stride below the vocabulary");
    DeviceGuard g(h->device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select the head's device");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t per_pass = HEAD_MAX_NT * HEAD_NTILE;
    // The matrix-core passes read the quantized rows; the dot path quantizes its own.
    if (!dot_path(h, t)) launch_quantize(x, t, h->k, h->nb, h->ad, nullptr, nullptr, h->af, s);
    for (uint32_t t0 = 0; t0 < t; t0 += per_pass)
        launch_head(h, x, t0, std::min(per_pass, t - t0), logits + (uint64_t)t0 * row_stride, row_stride, s);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? RL_OK : hip_fail(e, "rl_head_logits launch");
}

int rl_head_embed_rows(rl_head *h, const uint32_t *tokens, uint32_t t, float *out, uint64_t row_stride,
                       void *stream) {
    if (!h) return fail(RL_ERR_ARGUMENT, "head is null");
    if (t == 0) return RL_OK;
    if (!tokens || !out) return fail(RL_ERR_ARGUMENT, "tokens and out must be device pointers");
    if (row_stride < h->k) return fail(RL_ERR_ARGUMENT, "row_stride below k");
    const uint64_t threads = (uint64_t)t * h->nb * 16;
    const uint64_t blocks = (threads + EMBED_THREADS - 1) / EMBED_THREADS;
    if (blocks > 0xFFFFFFFFull) return fail(RL_ERR_CAPACITY, "too many tokens for one launch");
    DeviceGuard g(h->device);
    if (!g.ok) return fail(RL_ERR_DEVICE, "cannot select the head's device");
    hipLaunchKernelGGL(k_embed_rows, dim3((uint32_t)blocks), dim3(EMBED_THREADS), 0, static_cast<hipStream_t>(stream),
                       h->wq, h->ws, h->wd, tokens, t, h->k, h->nb, h->rows, h->groups, out, row_stride);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? RL_OK : hip_fail(e, "rl_head_embed_rows launch");
}

int rl_quantize_rows(const float *x, uint32_t t, uint32_t k, float *out_d, int8_t *out_qs, int16_t *out_bsums,
                     void *stream) {
    if (t == 0) return RL_OK;
    if (!x || k == 0) return fail(RL_ERR_ARGUMENT, "x must be a device pointer and k positive");
    const uint32_t nb = (k + QK - 1) / QK;
    launch_quantize(x, t, k, nb, out_d, out_qs, out_bsums, nullptr, static_cast<hipStream_t>(stream));
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? RL_OK : hip_fail(e, "rl_quantize_rows launch");
}

}  // extern "C"

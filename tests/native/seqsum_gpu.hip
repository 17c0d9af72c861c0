// Test harness (not part of the library): runs the device replay of
// sequential sums (rust-llm_amd/csrc/rl_seqsum.h) on arbitrary term arrays,
// one workgroup per case, with the library's own workgroup shape and with a
// second one, so that tests/test_gpu_seqsum.py can compare every result with
// plain sequential loops on the host.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "full_rest.h"
#include "top_probability.h"

namespace {

// mode 0: never stops; 1: stops at the first partial sum >= thr; 2: > thr.
struct CasePred {
    double thr;
    uint32_t mode;
    __device__ bool operator()(double v) const { return mode == 1 ? v >= thr : (mode == 2 ? v > thr : false); }
};

template <int P, uint32_t NT, uint32_t ITEMS>
__global__ __launch_bounds__(NT) void k_seqsum_cases(const float *terms, const uint64_t *off, const uint32_t *n,
                                                     const double *thr, const uint32_t *mode, uint32_t *out_idx,
                                                     double *out_sum) {
    __shared__ rl::SeqLds<NT> seq;
    const uint32_t c = blockIdx.x;
    const float *x = terms + off[c];
    const CasePred pred{thr[c], mode[c]};
    double sum = -1.0;
    const uint32_t idx = rl::seq_replay<P, NT, ITEMS>(
        [x](uint32_t j) { return ((const RL_GLB float *)x)[j]; }, n[c], pred, &seq, &sum);
    if (threadIdx.x == 0) {
        out_idx[c] = idx;
        out_sum[c] = sum;
    }
}

// The chunked replay (rl::chunk_replay), one workgroup of REST_THREADS per case.
template <int P>
__global__ __launch_bounds__(rl::REST_THREADS) void k_chunk_cases(const float *terms, const uint64_t *off,
                                                                  const uint32_t *n, const double *thr,
                                                                  const uint32_t *mode, uint32_t *out_idx,
                                                                  double *out_sum) {
    __shared__ rl::ChunkLds cr_;
    RL_LDS rl::ChunkLds *cr = (RL_LDS rl::ChunkLds *)&cr_;
    const uint32_t c = blockIdx.x;
    const uint32_t *x = (const uint32_t *)(terms + off[c]);
    const CasePred pred{thr[c], mode[c]};
    double sum = -1.0;
    const uint32_t idx = rl::chunk_replay<P, rl::REST_THREADS>(
        x, [](uint32_t b) { return __uint_as_float(b); }, n[c], pred, cr, &sum);
    if (threadIdx.x == 0) {
        out_idx[c] = idx;
        out_sum[c] = sum;
    }
}

// The chunked replay as the sampler's draw runs it: in place (each staged
// round's terms are stored over its words; the term here doubles the word,
// exactly), with a range of words [hot_lo, hot_hi) that reads as hot_word
// whatever memory holds there. out_staged gets the written prefix.
template <int P>
__global__ __launch_bounds__(rl::REST_THREADS) void k_chunk_cases_wb(uint32_t *words, const uint64_t *off,
                                                                     const uint32_t *n, const double *thr,
                                                                     const uint32_t *mode, const uint32_t *hot_lo,
                                                                     const uint32_t *hot_hi, const uint32_t *hot_word,
                                                                     uint32_t *out_idx, double *out_sum,
                                                                     uint32_t *out_staged) {
    __shared__ rl::ChunkLds cr_;
    RL_LDS rl::ChunkLds *cr = (RL_LDS rl::ChunkLds *)&cr_;
    const uint32_t c = blockIdx.x;
    uint32_t *x = words + off[c];
    const CasePred pred{thr[c], mode[c]};
    rl::HotRange hr;
    hr.lo = hot_lo[c];
    hr.hi = hot_hi[c];
    hr.word = hot_word[c];
    double sum = -1.0;
    uint32_t staged = 0xFFFFFFFFu;
    const uint32_t idx = rl::chunk_replay<P, rl::REST_THREADS>(
        x, [](uint32_t b) { return 2.0f * __uint_as_float(b); }, n[c], pred, cr, &sum, x, &staged, hr);
    if (threadIdx.x == 0) {
        out_idx[c] = idx;
        out_sum[c] = sum;
        out_staged[c] = staged;
    }
}

template <int P, uint32_t NT, uint32_t ITEMS>
int launch(const float *terms, const uint64_t *off, const uint32_t *n, const double *thr, const uint32_t *mode,
           uint32_t cases, uint32_t *out_idx, double *out_sum, hipStream_t st) {
    hipLaunchKernelGGL((k_seqsum_cases<P, NT, ITEMS>), dim3(cases), dim3(NT), 0, st, terms, off, n, thr, mode, out_idx,
                       out_sum);
    return (int)hipGetLastError();
}

}  // namespace

// shape 0: REST_THREADS threads, SEQ_ITEMS terms each; shape 1: 128
// threads, 3 terms each; shape 2: top_probability's (FAST_THREADS
// threads, SEQ_ITEMS terms each); shape 3: the chunked replay the sampler
// uses (REST_THREADS threads). Every pointer is device memory; a
// case's terms are terms[off[c] .. off[c] + n[c]).
extern "C" int seqsum_gpu_run(int precision, int shape, const float *terms, const uint64_t *off, const uint32_t *n,
                              const double *thr, const uint32_t *mode, uint32_t cases, uint32_t *out_idx,
                              double *out_sum, void *stream) {
    if (cases == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    if (shape == 0) {
        if (precision == 24)
            return launch<24, rl::REST_THREADS, rl::SEQ_ITEMS>(terms, off, n, thr, mode, cases, out_idx, out_sum, st);
        if (precision == 53)
            return launch<53, rl::REST_THREADS, rl::SEQ_ITEMS>(terms, off, n, thr, mode, cases, out_idx, out_sum, st);
    } else if (shape == 1) {
        if (precision == 24) return launch<24, 128, 3>(terms, off, n, thr, mode, cases, out_idx, out_sum, st);
        if (precision == 53) return launch<53, 128, 3>(terms, off, n, thr, mode, cases, out_idx, out_sum, st);
    } else if (shape == 3) {
        if (precision == 24) {
            hipLaunchKernelGGL(k_chunk_cases<24>, dim3(cases), dim3(rl::REST_THREADS), 0, st, terms, off, n, thr, mode,
                               out_idx, out_sum);
            return (int)hipGetLastError();
        }
        if (precision == 53) {
            hipLaunchKernelGGL(k_chunk_cases<53>, dim3(cases), dim3(rl::REST_THREADS), 0, st, terms, off, n, thr, mode,
                               out_idx, out_sum);
            return (int)hipGetLastError();
        }
    } else if (shape == 2) {
        if (precision == 24)
            return launch<24, rl::FAST_THREADS, rl::SEQ_ITEMS>(terms, off, n, thr, mode, cases, out_idx, out_sum, st);
        if (precision == 53)
            return launch<53, rl::FAST_THREADS, rl::SEQ_ITEMS>(terms, off, n, thr, mode, cases, out_idx, out_sum, st);
    }
    return -1;
}

// The in-place chunked replay with a hot range (k_chunk_cases_wb); words is
// device memory that the call overwrites.
extern "C" int seqsum_gpu_run_wb(int precision, uint32_t *words, const uint64_t *off, const uint32_t *n,
                                 const double *thr, const uint32_t *mode, const uint32_t *hot_lo,
                                 const uint32_t *hot_hi, const uint32_t *hot_word, uint32_t cases, uint32_t *out_idx,
                                 double *out_sum, uint32_t *out_staged, void *stream) {
    if (cases == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    if (precision == 24)
        hipLaunchKernelGGL(k_chunk_cases_wb<24>, dim3(cases), dim3(rl::REST_THREADS), 0, st, words, off, n, thr, mode,
                           hot_lo, hot_hi, hot_word, out_idx, out_sum, out_staged);
    else if (precision == 53)
        hipLaunchKernelGGL(k_chunk_cases_wb<53>, dim3(cases), dim3(rl::REST_THREADS), 0, st, words, off, n, thr, mode,
                           hot_lo, hot_hi, hot_word, out_idx, out_sum, out_staged);
    else
        return -1;
    return (int)hipGetLastError();
}

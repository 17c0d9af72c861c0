// Test harness (gfx950; test infrastructure): the hardware base-2
// exponential, v_exp_f32, evaluated at every f32 whose bit pattern lies in
// [lo, lo + n), so a test can compare it with exp2 in f64 and check the error
// bound the min-p path's mass interval assumes for it; and the branch-free
// expf for non-positive arguments compared with the general device expf.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_expf.h"

__global__ void k_exp2_hw(uint32_t lo, uint64_t n, float *out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __builtin_amdgcn_exp2f(__uint_as_float(lo + (uint32_t)i));
}

// out: device, n floats; n <= 2^31 and lo + n <= 2^32.
extern "C" int exp2_hw_range(uint32_t lo, uint64_t n, float *out, void *stream) {
    if (!out || n == 0 || n > (1ull << 31) || (uint64_t)lo + n > (1ull << 32)) return 1;
    const uint32_t blocks = (uint32_t)((n + 255) / 256);
    hipLaunchKernelGGL(k_exp2_hw, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), lo, n, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Counts, into *count, the bit patterns in [lo, lo + n) at which
// expf_libm_nonpos_t and expf_libm_t return different bits.
__global__ void k_expf_nonpos_diff(uint32_t lo, uint64_t n, uint32_t *count) {
    __shared__ uint64_t tab[32];
    rl::copy_exp_table((__attribute__((address_space(3))) uint64_t *)tab);
    const rl::LdsExpTable etab{(__attribute__((address_space(3))) uint64_t *)tab};
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool differ = false;
    if (i < n) {
        const float x = __uint_as_float(lo + (uint32_t)i);
        differ = __float_as_uint(rl::expf_libm_nonpos_t(x, etab)) != __float_as_uint(rl::expf_libm_t(x, etab));
    }
    const uint64_t m = __ballot(differ);
    if ((threadIdx.x & 63u) == 0 && m != 0) atomicAdd(count, (uint32_t)__popcll(m));
}

// count: device, one u32 the caller has zeroed; n <= 2^31 and lo + n <= 2^32.
extern "C" int expf_nonpos_diff(uint32_t lo, uint64_t n, uint32_t *count, void *stream) {
    if (!count || n == 0 || n > (1ull << 31) || (uint64_t)lo + n > (1ull << 32)) return 1;
    const uint32_t blocks = (uint32_t)((n + 255) / 256);
    hipLaunchKernelGGL(k_expf_nonpos_diff, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), lo, n,
                       count);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

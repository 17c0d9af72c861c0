// Test harness (gfx950; test infrastructure): the hardware base-2
// exponential, v_exp_f32, evaluated at every f32 whose bit pattern lies in
// [lo, lo + n), so a test can compare it with exp2 in f64 and check the error
// bound the min-p path's mass interval assumes for it.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

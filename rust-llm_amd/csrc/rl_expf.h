// Single-precision exp on gfx950, bit-identical to the host's libm expf.
//
// The reference computes p = ((l - max) / t).exp() in f32 (sample.rs:309);
// Rust's f32::exp calls libm expf on x86_64-unknown-linux-gnu. To reproduce its
// bits this evaluates the published table-driven method that libm implements
// (ARM Optimized Routines expf, Szabolcs Nagy, 2017; shipped as glibc's expf
// since 2.27):
//   x * 32/ln2 = k + r, |r| <= 1/2, k integer (round-to-nearest by the
//   1.5*2^52 shift trick);
//   2^(k/32) = 2^(k>>5) * 2^((k&31)/32), the second factor from a 32-entry
//   table whose entry i holds the bits of RN(2^(i/32)) minus i<<47, so adding
//   k<<47 also applies the 2^(k>>5) exponent;
//   2^(r/32) ~ 1 + C2 r + C1 r^2 + C0 r^3 (minimax, evaluated as
//   (C0 r + C1) r^2 + (C2 r + 1));
//   one rounding from double to float at the end.
// Every multiply-add is a fused multiply-add, which is the evaluation an
// FMA-capable x86-64 host's libm performs; with that choice the result equals
// libm expf on all 2^32 inputs (checked exhaustively on the host against the
// C restatement, and on the GPU against the host's libm by the GPU tests).
// The table entries are RN(2^(i/32)) recomputed from exact decimal
// arithmetic. Compile with -ffp-contract=off so nothing else is fused.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rl {

__device__ __constant__ uint64_t EXP2_32_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// tab(i) returns EXP2_32_TAB[i]; kernels that evaluate many exps pass a copy
// of the table in LDS (copy_exp_table), since a per-lane index into constant
// memory is a dependent global load on every call.
// The main path: x * 32/ln2 split into k + r, the table and the polynomial.
// Equals libm expf wherever its special cases do not apply (|x| < 88, and the
// finite x up to the overflow and down to the underflow bounds).
template <class Tab>
__device__ __forceinline__ float expf_libm_core(float x, Tab tab) {
    // Polynomial for 2^(r/32), coefficients pre-divided by 32^3, 32^2, 32.
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double INV_LN2_32 = 0x1.71547652b82fep+0 * 32.0;
    const double SHIFT = 0x1.8p+52;

    const double xd = (double)x;
    double kd = __builtin_fma(INV_LN2_32, xd, SHIFT);
    // k in the low word of kd's bits; s = the bits of tab(k & 31) + (k << 47),
    // which leaves the low word alone and adds k << 15 to the high word
    // (mod 2^32, as the 64-bit sum does).
    const uint32_t ki = (uint32_t)__double_as_longlong(kd);
    kd -= SHIFT;
    const double r = __builtin_fma(INV_LN2_32, xd, -kd);
    const uint64_t tb = tab(ki & 31u);
    const double s = __hiloint2double((int)((uint32_t)(tb >> 32) + (ki << 15)), (int)(uint32_t)tb);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// Underflow bound: libm expf returns +0 below it.
constexpr float EXPF_UNDERFLOW = -0x1.9fe368p6f;

template <class Tab>
__device__ __forceinline__ float expf_libm_t(float x, Tab tab) {
    const uint32_t bits = __float_as_uint(x);
    const uint32_t abstop = (bits >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                            // |x| >= 88 or NaN
        if (bits == 0xff800000u) return 0.0f;          // exp(-inf)
        if (abstop >= 0x7f8u) return x + x;            // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff(); // overflows
        if (x < EXPF_UNDERFLOW) return 0.0f;           // underflows to +0
    }
    return expf_libm_core(x, tab);
}

// The float just below EXPF_UNDERFLOW: the main path there gives a double
// under 2^-150, which rounds to +0 in f32.
constexpr float EXPF_BELOW_UNDERFLOW = -0x1.9fe36ap6f;

// expf_libm_t for x <= 0 (either zero, -inf included), not NaN: of its
// special cases only the underflow to +0 (which covers -inf) can apply, and
// raising x to EXPF_BELOW_UNDERFLOW gives that +0 from the main path itself,
// with no branch.
template <class Tab>
__device__ __forceinline__ float expf_libm_nonpos_t(float x, Tab tab) {
    return expf_libm_core(__builtin_fmaxf(x, EXPF_BELOW_UNDERFLOW), tab);
}

__device__ __forceinline__ float expf_libm(float x) {
    return expf_libm_t(x, [](uint32_t i) { return EXP2_32_TAB[i]; });
}

// Whole-workgroup: copies the table into `lds` (32 entries). Ends with a
// barrier.
__device__ __forceinline__ void copy_exp_table(__attribute__((address_space(3))) uint64_t *lds) {
    if (threadIdx.x < 32) lds[threadIdx.x] = EXP2_32_TAB[threadIdx.x];
    __syncthreads();
}

struct LdsExpTable {
    const __attribute__((address_space(3))) uint64_t *t;
    __device__ uint64_t operator()(uint32_t i) const { return t[i]; }
};

// This lane's entry of the table spread over a wave: entry i sits in lanes i
// and 32 + i.
__device__ __forceinline__ uint64_t lane_exp_entry() { return EXP2_32_TAB[__lane_id() & 31u]; }

// The table spread over a wave (v = lane_exp_entry(), loaded ahead of need),
// read by index through the wave's lane permute: a tail evaluating a few exps
// waits for no memory round trip. Every lane of the wave must be active
// where it is called (a permute reads nothing from an inactive lane), so use
// it only with the branch-free expf_libm_nonpos_t, outside any divergent
// branch.
struct LaneExpTable {
    uint64_t v;
    __device__ uint64_t operator()(uint32_t i) const {
        const int at = (int)(i << 2);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(at, (int)(uint32_t)v);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(at, (int)(uint32_t)(v >> 32));
        return ((uint64_t)hi << 32) | lo;
    }
};

}  // namespace rl

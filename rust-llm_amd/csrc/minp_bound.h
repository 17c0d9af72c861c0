// The min-p path's mass certificate: the interval k_full_pass (full_kernels.h)
// proves to hold the reference's top-p target, top_p * S_ref
// (sample.rs:307-324), from the mass it sums in its one read of the row.
// Plain C++ with no device dependency, so that a host-built test can evaluate
// the same constants and the same interval the kernel uses.
//
// The reference's mass is S_ref = sum of p_j in sorted order (f64,
// sequential), p_j = expf(fl(fl(l_j - M) / T)). With y_j = (l_j - M) / T
// exactly, the two roundings of the argument put it within 2^-23 |y_j| of y_j,
// and libm expf is within 0.502 ulp, so p_j = e^(y_j) (1 + e_j) with
// |e_j| <= 2^-23 |y_j| + 1.004 2^-24 to first order (plus 2^-149 absolute in
// the subnormal range).
//
// The pass computes, relative to a running maximum m <= M that its wave has
// already seen, q_j = exp2_hw(fl(fl(l_j - m) * c2)) with c2 = fl(log2(e) / T)
// rounded once from the f64 quotient: the exponent carries at most three
// roundings of 2^-24 relative, and |l_j - m| <= |l_j - M|, so
// q_j e^((m - M) / T) = e^(y_j) (1 + g_j) with |g_j| <= 3 2^-24 |y_j| + H
// (H = HW_EXP2_REL bounds the hardware exp2's own error). Splitting at
// |y| = K: a term with |y_j| <= K has p_j / (its pass term) within
// 1 +- EPS_NEAR / (1 - EPS_NEAR); a term beyond differs by at most
// 2.01 e^(-K) + 2^-124 absolute (both are below e^(-K) (1 + tiny), or flushed
// subnormals).
//
// The pass's own sum: each lane adds the PASS_TERMS = 4 PASS_U terms of one
// step in f32 from zero (PASS_TERMS - 1 roundings: gamma_(PASS_TERMS - 1) <=
// PASS_TERMS 2^-24 relative, all terms being positive), then everything else
// in f64 (the steps, the wave, the chunks, the finisher: below 2^-40 relative
// together); each time the wave's maximum rises, the lane's partial sum is
// rescaled by 2^floor(z) exp2_hw(frac z) with the fraction rounded to f32
// (RESCALE_REL per rescaling, at most one per step); the other rescalings are
// f64 exp. The reference's sequential sum of V terms adds gamma_(V - 1)
// relative, and its target top_p * S_ref one f64 rounding.
//
// So with sigma = F32_STEP_REL + 2^-40 + steps RESCALE_REL (the pass's sum)
// and eps = EPS_NEAR / (1 - EPS_NEAR) (the terms), the exact sum of the
// reference's p lies in Smid (1 -+ (eps + sigma)) -+ V ABS (first order; the
// (1 + 2^-7) factor on EPS_NEAR covers the products of the small terms), and
// the interval below widens that by gamma_(V + 64) and the roundings of the
// target.
#pragma once
#include <stdint.h>

#ifndef RL_HD
#ifdef __HIPCC__
#define RL_HD __host__ __device__
#else
#define RL_HD
#endif
#endif

namespace rl {
namespace minp {

constexpr uint32_t PASS_THREADS = 256;                  // k_full_pass's workgroup
constexpr uint32_t PASS_U = 10;                         // float4 per thread per step
constexpr uint32_t PASS_STEP = PASS_THREADS * PASS_U;   // float4 per step
constexpr uint32_t PASS_TERMS = 4 * PASS_U;             // f32 terms one lane adds per step
constexpr double HW_EXP2_REL = 0x1p-21;                 // v_exp_f32 bound assumed (4 ulp; tested <= 1.42 2^-24)
constexpr double MASS_K = 32.0;
constexpr double EPS_NEAR =
    ((0x1p-23 + 3.0 * 0x1p-24) * MASS_K + 1.004 * 0x1p-24 + HW_EXP2_REL) * (1.0 + 0x1p-7);
// gamma_(PASS_TERMS - 1) = (n - 1) u / (1 - (n - 1) u) <= n u for u = 2^-24
// and n <= 2^20.
constexpr double F32_STEP_REL = (double)PASS_TERMS * 0x1p-24;
static_assert(PASS_TERMS >= 2 && PASS_TERMS <= (1u << 20), "the f32 step sum's bound assumes n u << 1");
constexpr double MASS_REL = EPS_NEAR / (1.0 - EPS_NEAR) + F32_STEP_REL + 0x1p-40;
constexpr double RESCALE_REL = (0x1p-24 + HW_EXP2_REL) * 1.001;  // one in-loop rescaling factor
// 2.01 e^(-K) + 2^-124 per term (e^-32 = 1.2664165549e-14).
constexpr double MASS_ABS_PER_TERM = 2.01 * 1.2664165549094176e-14 + 0x1p-124;

// [t_lo, t_hi] holds the reference's target top_p * S_ref, given the pass's
// mass Smid (relative to the row's maximum) of a row of V logits read in
// `chunks` chunks. A lane's partial sum is rescaled at most once per step of
// its chunk; the largest chunk has at most (V / 4) / chunks + 1 float4 (plus
// the last chunk's vocab % 4 elements, rescaled in f64), so the step count
// below bounds every chunk's.
RL_HD inline void target_interval(double Smid, uint32_t V, uint32_t chunks, float top_p, double *t_lo,
                                  double *t_hi) {
    const uint32_t steps = (uint32_t)(((uint64_t)(V / 4) / chunks + PASS_STEP) / PASS_STEP);
    const double rel = MASS_REL + (double)steps * RESCALE_REL;
    const double abs_err = MASS_ABS_PER_TERM * (double)V + (double)V * 0x1p-1000;
    const double gam = ((double)V + 64.0) * 0x1p-53;
    const double S_lo = (Smid * (1.0 - rel) - abs_err) * (1.0 - gam);
    const double S_hi = (Smid * (1.0 + rel) + abs_err) * (1.0 + gam);
    const double tp = (double)top_p;
    *t_lo = tp * S_lo * (1.0 - 0x1p-48);
    *t_hi = tp * S_hi * (1.0 + 0x1p-48);
}

}  // namespace minp
}  // namespace rl

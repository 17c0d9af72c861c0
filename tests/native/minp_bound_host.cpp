// Test harness (host only; test infrastructure): the min-p path's mass
// certificate exactly as k_full_pass evaluates it (rust-llm_amd/csrc/
// minp_bound.h, compiled here by the host compiler), so a CPU test can check
// the interval against the reference's sequential mass on rows whose pass
// arithmetic it emulates.
#include <stdint.h>

#include "minp_bound.h"

extern "C" {

void minp_target_interval(double smid, uint32_t vocab, uint32_t chunks, float top_p, double *t_lo, double *t_hi) {
    rl::minp::target_interval(smid, vocab, chunks, top_p, t_lo, t_hi);
}

// The constants the interval rests on, in this order.
void minp_constants(double *out) {
    using namespace rl::minp;
    out[0] = PASS_THREADS;
    out[1] = PASS_U;
    out[2] = PASS_TERMS;
    out[3] = HW_EXP2_REL;
    out[4] = MASS_K;
    out[5] = EPS_NEAR;
    out[6] = F32_STEP_REL;
    out[7] = MASS_REL;
    out[8] = RESCALE_REL;
    out[9] = MASS_ABS_PER_TERM;
}

}  // extern "C"

// C entry points over the reference sampler (src/gsv_sampler.{h,cpp}), compiled from the
// reference sources where they lie into oracle/_ref/ by oracle/Makefile. Test infrastructure:
// used only to pin the oracle's sampler and to write the golden vectors under tests/golden/.
#include <cstdint>

#include "gsv_sampler.h"

extern "C" {

void ref_logits_to_probs(int top_k, float top_p, float temperature, float rep, float * logits,
                         int V, const int32_t * prev, int n_prev, float * probs) {
    gsv_sampler_cfg cfg;
    cfg.top_k = top_k;
    cfg.top_p = top_p;
    cfg.temperature = temperature;
    cfg.repetition_penalty = rep;
    gsv_logits_to_probs(cfg, logits, V, prev, n_prev, probs);
}

// n draws of gsv_rng::next() from seed; returns the final state
uint64_t ref_rng_stream(uint64_t seed, int n, uint64_t * out) {
    gsv_rng r(seed);
    for (int i = 0; i < n; i++) out[i] = r.next();
    return r.s;
}

uint64_t ref_rng_exponential(uint64_t seed, int n, float * out) {
    gsv_rng r(seed);
    for (int i = 0; i < n; i++) out[i] = r.exponential();
    return r.s;
}

int ref_sample(const float * probs, int V, uint64_t seed, uint64_t * state_out) {
    gsv_rng r(seed);
    const int t = gsv_sample(probs, V, r, nullptr);
    if (state_out) *state_out = r.s;
    return t;
}

int ref_argmax_probs_over_q(const float * probs, const float * q, int V) {
    return gsv_argmax_probs_over_q(probs, q, V);
}

}  // extern "C"

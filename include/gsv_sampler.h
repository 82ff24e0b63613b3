// gsv_sampler.h — sampler settings and RNG of the AR decoder.
//
// Interface of src/gsv_sampler.h (reference) kept identical, because gsv_ar::generate takes a
// gsv_sampler_cfg and other modules of the engine construct gsv_rng (src/gsv_dit.cpp:1430,
// src/gsv_engine.cpp:601): field names, defaults, the xorshift64* update and the uniform /
// exponential draws must match for the engine to compile and behave unchanged. The sampling
// functions declared at the end are implemented by the reference's src/gsv_sampler.cpp, which
// stays in the engine build (it has no ggml dependency); the HIP build samples on the device.
#pragma once

#include <cmath>
#include <cstdint>
#include <vector>

struct gsv_sampler_cfg {
    int   top_k = 15;                 // <= 0 disables top-k
    float top_p = 1.0f;               // >= 1 disables top-p
    float temperature = 1.0f;
    float repetition_penalty = 1.35f;
};

void gsv_logits_to_probs(const gsv_sampler_cfg & cfg,
                         float * logits, int V,
                         const int32_t * prev, int n_prev,
                         float * probs);

// xorshift64* (state 0 is replaced by 1)
struct gsv_rng {
    uint64_t s;
    explicit gsv_rng(uint64_t seed = 0x9E3779B97F4A7C15ull) : s(seed ? seed : 1) {}
    uint64_t next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 0x2545F4914F6CDD1Dull;
    }
    float uniform01() { return (float) ((next() >> 40) * (1.0 / 16777216.0)); }   // [0, 1)
    float exponential() { return -logf(1.0f - uniform01()); }
};

int gsv_argmax_probs_over_q(const float * probs, const float * q, int V);
int gsv_sample(const float * probs, int V, gsv_rng & rng, float * q_scratch);

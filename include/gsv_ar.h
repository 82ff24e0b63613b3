// gsv_ar.h — the AR (text-to-semantic) decoder, MI355X / HIP build.
//
// Drop-in for src/gsv_ar.h (reference): the same types, members and signatures, so that
// gsv_engine (src/gsv_engine.cpp:215-219, 407, 467, 479), the batched-AR scheduler
// (tools/svc_core.h) and tests/bench_ar_width.cpp compile and run against it unchanged. The
// implementation (gsv.cpp_amd/csrc/gsv_ar.cpp) drives the C ABI of include/gsvk.h.
//
// Semantics kept from the reference: batch sequences are left-padded and decoded in lockstep;
// the EOS token is masked while fewer than 11 steps ran; early_stop_num stops every sequence once
// sequence 0 has generated more than early_stop_num tokens; oracle_tokens replaces the sampled
// token of every sequence at step i by (*oracle_tokens)[i]; seeds[b] (or seed_base +
// 0x9E3779B9*b) seeds sequence b's xorshift64* stream.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "gsv_sampler.h"

struct gsv_ar_request {
    std::vector<int32_t> phones;   // phoneme ids (any length; left-padded inside)
    std::vector<float>   bert;     // [bert_dim][phones.size()] row-major: bert[k*T + t]
    std::vector<int32_t> prompt;   // reference semantic tokens (same length for the whole batch)
};

struct gsv_ar_cfg {
    int  n_threads  = 0;      // unused by the HIP build
    int  max_batch  = 8;      // reserved (the KV cache is sized by the actual batch)
    bool verbose    = false;
    std::string device;       // "" / "gpu" / "hip" / "vulkan" = HIP device 0; "gpu:N" or "N" = device N
    bool disable_coopmat2 = true;  // Vulkan-only switch of the reference; ignored
};

struct gsv_ar_result {
    std::vector<std::vector<int32_t>> tokens;   // per sequence: prompt + generated, minus the stopping token
    std::vector<int> lens;                      // generated-token counts, in finish order
};

class gsv_ar {
public:
    static gsv_ar * load(const std::string & gguf_path, const gsv_ar_cfg & cfg);
    ~gsv_ar();

    int hidden_dim()          const;
    int vocab_size()          const;
    int eos()                 const;
    int bert_dim()            const;
    int prompt_len_expected() const;   // 0 = none yet

    gsv_ar_result generate(const std::vector<gsv_ar_request> & reqs,
                           const gsv_sampler_cfg & sampler,
                           uint64_t seed_base,
                           int early_stop_num = -1,
                           int max_steps = 1500,
                           const std::vector<int32_t> * oracle_tokens = nullptr,
                           const std::vector<uint64_t> * seeds = nullptr);

    // test / diagnostics: last-position logits of the prefill (B rows x vocab)
    void first_logits(const std::vector<gsv_ar_request> & reqs, std::vector<float> & logits_out);

    // free the KV cache (large after batched decoding)
    void release_cache();

private:
    gsv_ar();
    struct impl;
    impl * p;
};

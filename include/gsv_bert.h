// gsv_bert.h — the BERT text encoder (chinese-roberta-wwm-ext-large), MI355X / HIP build.
//
// Drop-in for src/gsv_bert.h (reference): the same config type, members and signatures, so that
// the engine and tools that encode text with gsv_bert compile and run against it unchanged. The
// implementation (gsv.cpp_amd/csrc/gsv_bert.cpp) drives the C ABI of include/gsvk.h
// (gsvk_bert_*).
//
// Semantics kept from the reference: layers 0 .. layers_used-1 (hidden_states[-3] of the
// 24-layer model), post-LN, gelu(erf); encode returns [hidden][T] row-major including
// [CLS]/[SEP]; encode_feat drops them ([hidden][T-2]); encode_feat_cached keeps an LRU of
// feat_cache entries keyed by the full id sequence; encode_feat_batch encodes B sequences at
// once, each attending only to its own tokens; encode_layers returns every layer's output.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

struct gsv_bert_cfg {
    int  n_threads = 0;       // unused by the HIP build
    bool verbose   = false;
    std::string device;       // "" / "gpu" / "hip" / "vulkan" = HIP device 0; "gpu:N" or "N" = device N
    int  feat_cache = 0;      // LRU entries of encode_feat_cached (0 = off)
};

class gsv_bert {
public:
    static gsv_bert * load(const std::string & gguf_path, const gsv_bert_cfg & cfg);
    ~gsv_bert();

    int hidden()      const;
    int layers_used() const;
    int max_pos()     const;

    void encode(const int32_t * ids, int T, std::vector<float> & features);
    void encode_feat(const int32_t * ids, int T, std::vector<float> & feat);
    void encode_feat_cached(const int32_t * ids, int T, std::vector<float> & feat);
    void feat_cache_stats(int & hits, int & misses) const;
    bool encode_feat_batch(int B, const int32_t * ids_flat, const int * lens, int Tmax,
                           std::vector<std::vector<float>> & feats);
    void encode_layers(const int32_t * ids, int T, std::vector<float> & features,
                       std::vector<std::vector<float>> & per_layer);

private:
    gsv_bert();
    struct impl;
    impl * p;
};

// Drives the gsv_bert drop-in class (include/gsv_bert.h, linked from libgsvk.so) through every
// member on a BERT GGUF and prints what tests/test_gpu_bert.py checks: the getters, encode's
// output and its checksum, encode_feat against encode without [CLS]/[SEP], the LRU of
// encode_feat_cached, encode_feat_batch against one-by-one calls, encode_layers' depths and the
// error behaviour of load and encode.
#include <cmath>
#include <cstdio>
#include <vector>

#include "gsv_bert.h"

static double checksum(const std::vector<float> & v) {
    double s = 0.0;
    for (size_t i = 0; i < v.size(); i++) s += (double) v[i] * (double) ((i % 7) + 1);
    return s;
}

int main(int argc, char ** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s bert.gguf\n", argv[0]);
        return 2;
    }
    gsv_bert_cfg bad;
    bad.device = "cpu";   // no CPU path in this build: load fails with nullptr
    printf("load_cpu_null %d\n", gsv_bert::load(argv[1], bad) == nullptr ? 1 : 0);
    printf("load_missing_null %d\n", gsv_bert::load("/nonexistent.gguf", gsv_bert_cfg()) == nullptr ? 1 : 0);

    gsv_bert_cfg cfg;
    cfg.device = "vulkan";   // the reference's GPU string: HIP device 0 here
    cfg.feat_cache = 2;
    gsv_bert * b = gsv_bert::load(argv[1], cfg);
    if (!b) return 3;
    const int D = b->hidden();
    printf("info %d %d %d\n", D, b->layers_used(), b->max_pos());

    const std::vector<int32_t> s1 = {1, 17, 29, 4, 811, 2}, s2 = {1, 5, 6, 7, 8, 9, 10, 11, 2},
                               s3 = {1, 300, 2};
    std::vector<float> full, feat;
    b->encode(s1.data(), (int) s1.size(), full);
    b->encode_feat(s1.data(), (int) s1.size(), feat);
    const int T = (int) s1.size();
    bool feat_ok = full.size() == (size_t) D * T && feat.size() == (size_t) D * (T - 2);
    for (int d = 0; feat_ok && d < D; d++)
        for (int t = 0; t < T - 2; t++)
            if (feat[(size_t) d * (T - 2) + t] != full[(size_t) d * T + t + 1]) feat_ok = false;
    printf("encode_checksum %.9e\n", checksum(full));
    printf("feat_ok %d\n", feat_ok ? 1 : 0);

    // LRU of 2: s1 miss, s1 hit, s2 miss, s3 miss (evicts s1), s1 miss
    std::vector<float> c;
    bool cache_same = true;
    for (const std::vector<int32_t> * s : {&s1, &s1, &s2, &s3, &s1}) {
        b->encode_feat_cached(s->data(), (int) s->size(), c);
        if (s == &s1 && c != feat) cache_same = false;
    }
    int hits = -1, misses = -1;
    b->feat_cache_stats(hits, misses);
    printf("cache %d %d %d\n", hits, misses, cache_same ? 1 : 0);
    // the cache now holds s3 (older) and s1. s3 hits and becomes the newest, s2 misses and must
    // evict s1 (least recently used; first-in-first-out would evict s3), so s3 hits again
    for (const std::vector<int32_t> * s : {&s3, &s2, &s3}) b->encode_feat_cached(s->data(), (int) s->size(), c);
    int hits2 = -1, misses2 = -1;
    b->feat_cache_stats(hits2, misses2);
    printf("lru %d %d\n", hits2 - hits, misses2 - misses);

    // batch of s1, s2 (Tmax 9) against one-by-one
    std::vector<int32_t> flat(2 * 9, 0);
    for (size_t i = 0; i < s1.size(); i++) flat[i] = s1[i];
    for (size_t i = 0; i < s2.size(); i++) flat[9 + i] = s2[i];
    const int lens[2] = {(int) s1.size(), (int) s2.size()};
    std::vector<std::vector<float>> feats;
    const bool ok = b->encode_feat_batch(2, flat.data(), lens, 9, feats);
    std::vector<float> f2;
    b->encode_feat(s2.data(), (int) s2.size(), f2);
    double md = 0.0, mx = 0.0;
    for (int k = 0; k < 2 && ok; k++) {
        const std::vector<float> & ref = k == 0 ? feat : f2;
        for (size_t i = 0; i < ref.size() && i < feats[k].size(); i++) {
            md = std::fmax(md, std::fabs((double) feats[k][i] - ref[i]));
            mx = std::fmax(mx, std::fabs((double) ref[i]));
        }
    }
    printf("batch %d %zu %zu %.3e\n", ok ? 1 : 0, ok ? feats[0].size() : 0, ok ? feats[1].size() : 0,
           mx > 0 ? md / mx : 1.0);
    printf("batch_bad_args %d\n", b->encode_feat_batch(2, flat.data(), lens, 2, feats) ? 0 : 1);

    std::vector<float> last;
    std::vector<std::vector<float>> per;
    b->encode_layers(s3.data(), (int) s3.size(), last, per);
    std::vector<float> e3;
    b->encode(s3.data(), (int) s3.size(), e3);
    printf("layers %zu %d\n", per.size(), last == e3 && per.back() == e3 ? 1 : 0);

    std::vector<int32_t> too_long((size_t) b->max_pos() + 1, 1);
    std::vector<float> none = {1.0f};
    b->encode(too_long.data(), (int) too_long.size(), none);
    printf("too_long_empty %d\n", none.empty() ? 1 : 0);
    delete b;
    printf("done\n");
    return 0;
}

// gsv_bert (include/gsv_bert.h) on the HIP C ABI (include/gsvk.h): the drop-in replacement of
// the reference's src/gsv_bert.cpp. The encoder runs in gsvk_bert_encode; this file keeps the
// reference's post-processing (dropping [CLS]/[SEP]), its feature LRU and its error behaviour
// (load -> nullptr with a message on stderr; a failed encode leaves the output empty).
#include "gsv_bert.h"

#include <cstdio>
#include <cstring>
#include <vector>

#include "gsvk.h"

struct gsv_bert::impl {
    gsvk_bert * m = nullptr;
    gsvk_bert_info info{};
    // encode_feat_cached's LRU, keyed by the full id sequence (src/gsv_bert.cpp:246-283)
    int feat_cache_n = 0;
    uint64_t feat_use = 0;
    int hits = 0, misses = 0;
    struct entry {
        uint64_t h, use;
        std::vector<int32_t> ids;
        std::vector<float> feat;
    };
    std::vector<entry> cache;

    // [hidden][T] of one sequence after n_layers layers; false (and out empty) on error
    bool run(const int32_t * ids, int T, int n_layers, std::vector<float> & out) {
        out.clear();
        if (!m || !ids || T < 1) return false;
        std::vector<float> y((size_t) info.hidden * T);
        const int32_t len = T;
        if (gsvk_bert_encode(m, 1, ids, &len, T, n_layers, y.data()) != GSVK_OK) {
            fprintf(stderr, "[gsv_bert] encode failed: %s\n", gsvk_last_error());
            return false;
        }
        out.swap(y);
        return true;
    }
};

namespace {

uint64_t hash_ids(const int32_t * ids, int T) {   // FNV-1a over the ids, then T
    uint64_t h = 1469598103934665603ull;
    for (int i = 0; i < T; i++) {
        h ^= (uint32_t) ids[i];
        h *= 1099511628211ull;
    }
    h ^= (uint64_t) (uint32_t) T;
    h *= 1099511628211ull;
    return h;
}

// [hidden][T] -> [hidden][T-2] without [CLS] and [SEP]
void drop_cls_sep(const std::vector<float> & full, int D, int T, std::vector<float> & feat) {
    const int T2 = T - 2;
    feat.clear();
    if (T2 <= 0 || full.size() < (size_t) D * T) return;
    feat.resize((size_t) D * T2);
    for (int d = 0; d < D; d++)
        memcpy(&feat[(size_t) d * T2], &full[(size_t) d * T + 1], (size_t) T2 * sizeof(float));
}

}  // namespace

gsv_bert::gsv_bert() : p(new impl()) {}

gsv_bert::~gsv_bert() {
    if (p) {
        gsvk_bert_free(p->m);
        delete p;
    }
}

gsv_bert * gsv_bert::load(const std::string & gguf_path, const gsv_bert_cfg & cfg) {
    int device = 0;
    if (gsvk_parse_device(cfg.device.c_str(), &device) != GSVK_OK) {
        fprintf(stderr, "[gsv_bert] %s\n", gsvk_last_error());
        return nullptr;
    }
    gsvk_bert * m = nullptr;
    if (gsvk_bert_load(gguf_path.c_str(), device, cfg.verbose ? 1 : 0, &m) != GSVK_OK) {
        fprintf(stderr, "[gsv_bert] failed to load %s: %s\n", gguf_path.c_str(), gsvk_last_error());
        return nullptr;
    }
    gsv_bert * b = new gsv_bert();
    b->p->m = m;
    gsvk_bert_get_info(m, &b->p->info);
    b->p->feat_cache_n = cfg.feat_cache > 0 ? cfg.feat_cache : 0;
    return b;
}

int gsv_bert::hidden() const { return p->info.hidden; }
int gsv_bert::layers_used() const { return p->info.layers_used; }
int gsv_bert::max_pos() const { return p->info.max_pos; }

void gsv_bert::encode(const int32_t * ids, int T, std::vector<float> & features) {
    p->run(ids, T, -1, features);
}

void gsv_bert::encode_feat(const int32_t * ids, int T, std::vector<float> & feat) {
    std::vector<float> full;
    feat.clear();
    if (!p->run(ids, T, -1, full)) return;
    drop_cls_sep(full, p->info.hidden, T, feat);
}

void gsv_bert::encode_feat_cached(const int32_t * ids, int T, std::vector<float> & feat) {
    impl & s = *p;
    if (s.feat_cache_n <= 0) {
        encode_feat(ids, T, feat);
        return;
    }
    const uint64_t h = hash_ids(ids, T);
    for (impl::entry & e : s.cache) {
        if (e.h == h && (int) e.ids.size() == T && memcmp(e.ids.data(), ids, (size_t) T * 4) == 0) {
            feat = e.feat;
            e.use = ++s.feat_use;
            s.hits++;
            return;
        }
    }
    s.misses++;
    encode_feat(ids, T, feat);
    if ((int) s.cache.size() >= s.feat_cache_n) {   // evict the least recently used
        size_t victim = 0;
        for (size_t i = 1; i < s.cache.size(); i++)
            if (s.cache[i].use < s.cache[victim].use) victim = i;
        s.cache.erase(s.cache.begin() + (long) victim);
    }
    s.cache.push_back(impl::entry{h, ++s.feat_use, std::vector<int32_t>(ids, ids + T), feat});
}

void gsv_bert::feat_cache_stats(int & hits, int & misses) const {
    hits = p->hits;
    misses = p->misses;
}

bool gsv_bert::encode_feat_batch(int B, const int32_t * ids_flat, const int * lens, int Tmax,
                                 std::vector<std::vector<float>> & feats) {
    feats.assign((size_t) (B > 0 ? B : 0), {});
    if (B <= 0 || !ids_flat || !lens || Tmax < 3 || Tmax > p->info.max_pos) {
        fprintf(stderr, "[gsv_bert] encode_feat_batch: bad args (B=%d Tmax=%d max_pos=%d)\n", B, Tmax,
                p->info.max_pos);
        return false;
    }
    const int D = p->info.hidden;
    std::vector<int32_t> len(B);
    size_t total = 0;
    for (int b = 0; b < B; b++) {
        len[b] = lens[b];
        total += (size_t) (lens[b] > 0 ? lens[b] : 0);
    }
    std::vector<float> out(total * D);
    if (gsvk_bert_encode(p->m, B, ids_flat, len.data(), Tmax, -1, out.data()) != GSVK_OK) {
        fprintf(stderr, "[gsv_bert] encode_feat_batch: %s\n", gsvk_last_error());
        return false;
    }
    size_t off = 0;
    for (int b = 0; b < B; b++) {
        std::vector<float> full(out.begin() + (long) (off * D), out.begin() + (long) ((off + len[b]) * D));
        drop_cls_sep(full, D, len[b], feats[b]);
        off += len[b];
    }
    return true;
}

void gsv_bert::encode_layers(const int32_t * ids, int T, std::vector<float> & features,
                             std::vector<std::vector<float>> & per_layer) {
    features.clear();
    per_layer.assign((size_t) p->info.layers_used + 1, {});
    for (int k = 0; k <= p->info.layers_used; k++) {
        std::vector<float> out;
        p->run(ids, T, k, out);
        if (k == p->info.layers_used) features = out;
        per_layer[k] = std::move(out);
    }
}

// gsv_bert (include/gsv_bert.h) on the HIP C ABI (include/gsvk.h): the drop-in replacement of
// the reference's src/gsv_bert.cpp. The encoder runs in gsvk_bert_encode; this file keeps the
// reference's post-processing (dropping [CLS]/[SEP]), its feature LRU and its error behaviour
// (load -> nullptr with a message on stderr; a failed encode leaves the output empty).
#include "gsv_bert.h"

#include <cstdio>
#include <cstring>
#include <list>
#include <string>
#include <unordered_map>
#include <vector>

#include "gsvk.h"

struct gsv_bert::impl {
    gsvk_bert * m = nullptr;
    gsvk_bert_info info{};
    // encode_feat_cached's cache of at most `capacity` id sequences (the reference's observable
    // behaviour, src/gsv_bert.cpp:242-264: a hit refreshes the entry, a miss inserts it and, when
    // full, first drops the entry unused for longest). A recency list, most recent first, and an
    // index from the sequence's bytes to its list node.
    int capacity = 0;
    int hits = 0, misses = 0;
    struct Cached {
        std::string key;   // the ids as raw bytes
        std::vector<float> feat;
    };
    std::list<Cached> recency;
    std::unordered_map<std::string, std::list<Cached>::iterator> index;

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
    b->p->capacity = cfg.feat_cache > 0 ? cfg.feat_cache : 0;
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
    impl & c = *p;
    if (c.capacity <= 0) {
        encode_feat(ids, T, feat);
        return;
    }
    std::string key(reinterpret_cast<const char *>(ids), (ids && T > 0) ? (size_t) T * sizeof(int32_t) : 0);
    const auto found = c.index.find(key);
    if (found != c.index.end()) {
        c.recency.splice(c.recency.begin(), c.recency, found->second);   // now the most recent
        feat = found->second->feat;
        c.hits++;
        return;
    }
    c.misses++;
    encode_feat(ids, T, feat);   // a failed encode is remembered too (empty), as the reference does
    if ((int) c.recency.size() >= c.capacity) {
        c.index.erase(c.recency.back().key);
        c.recency.pop_back();
    }
    c.recency.push_front(impl::Cached{std::move(key), feat});
    c.index.emplace(c.recency.front().key, c.recency.begin());
}

void gsv_bert::feat_cache_stats(int & hits, int & misses) const {
    hits = p->hits;
    misses = p->misses;
}

bool gsv_bert::encode_feat_batch(int B, const int32_t * ids_flat, const int * lens, int Tmax,
                                 std::vector<std::vector<float>> & feats) {
    feats.assign((size_t) (B > 0 ? B : 0), {});
    const bool ok = B > 0 && ids_flat && lens && Tmax >= 3 && Tmax <= p->info.max_pos;
    if (!ok) {
        fprintf(stderr, "[gsv_bert] encode_feat_batch refused: %d sequences of up to %d tokens (positions: %d)\n",
                B, Tmax, p->info.max_pos);
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
    // hidden state k (the embedding for k = 0) is the encoder stopped after k layers
    const int depth = p->info.layers_used;
    per_layer.resize((size_t) depth + 1);
    int k = 0;
    for (std::vector<float> & h : per_layer) p->run(ids, T, k++, h);
    features = per_layer[(size_t) depth];
}

// gsv_ar (include/gsv_ar.h) on the HIP C ABI (include/gsvk.h): the drop-in replacement of the
// reference's src/gsv_ar.cpp. All arithmetic runs in the gfx950 kernels; this file converts the
// C++ request/result types, keeps the reference's diagnostics switches and reports errors the
// way the reference's callers expect (load -> nullptr, generate -> empty result).
#include "gsv_ar.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "gsv_progress.h"   // the engine's /progress counters (src/gsv_progress.h)
#include "gsvk.h"

struct gsv_ar::impl {
    gsvk_model * m = nullptr;
    gsvk_model_info info{};
    bool verbose = false;
    bool profile = false;
    int prompt_len = 0;
};

namespace {

double now_ms() {
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch()).count();
}

std::vector<gsvk_request> to_c(const std::vector<gsv_ar_request> & reqs) {
    std::vector<gsvk_request> out(reqs.size());
    for (size_t i = 0; i < reqs.size(); i++) {
        const gsv_ar_request & r = reqs[i];
        out[i].phones = r.phones.data();
        out[i].n_phones = (int32_t) r.phones.size();
        // the reference reads bert[k*T + t] unconditionally; an empty vector means zeros here
        out[i].bert = r.bert.size() >= (size_t) 1024 * r.phones.size() && !r.bert.empty() ? r.bert.data() : nullptr;
        out[i].prompt = r.prompt.data();
        out[i].n_prompt = (int32_t) r.prompt.size();
    }
    return out;
}

void progress_tick(void *, int) { gsvprog::tick(); }

}  // namespace

gsv_ar::gsv_ar() : p(new impl()) {}

gsv_ar::~gsv_ar() {
    if (p) {
        gsvk_model_free(p->m);
        delete p;
    }
}

int gsv_ar::hidden_dim() const { return p->info.d_model; }
int gsv_ar::vocab_size() const { return p->info.vocab; }
int gsv_ar::eos() const { return p->info.eos; }
int gsv_ar::bert_dim() const { return p->info.bert_dim; }
int gsv_ar::prompt_len_expected() const { return p->prompt_len; }

gsv_ar * gsv_ar::load(const std::string & gguf_path, const gsv_ar_cfg & cfg) {
    int device = 0;
    if (gsvk_parse_device(cfg.device.c_str(), &device) != GSVK_OK) {
        fprintf(stderr, "[gsv_ar] %s\n", gsvk_last_error());
        return nullptr;
    }
    gsv_ar * a = new gsv_ar();
    a->p->verbose = cfg.verbose;
    a->p->profile = getenv("GSV_AR_PROFILE") != nullptr;
    if (gsvk_model_load(gguf_path.c_str(), device, cfg.verbose ? 1 : 0, &a->p->m) != GSVK_OK) {
        fprintf(stderr, "[gsv_ar] load failed: %s\n", gsvk_last_error());
        delete a;
        return nullptr;
    }
    gsvk_model_get_info(a->p->m, &a->p->info);
    if (cfg.verbose)
        printf("[gsv_ar] loaded %s: D=%d head=%d layers=%d vocab=%d EOS=%d bert=%d alpha=(%.4f, %.4f) "
               "| HIP device %d\n", gguf_path.c_str(), a->p->info.d_model, a->p->info.n_head,
               a->p->info.n_layer, a->p->info.vocab, a->p->info.eos, a->p->info.bert_dim,
               a->p->info.text_alpha, a->p->info.audio_alpha, device);
    return a;
}

void gsv_ar::first_logits(const std::vector<gsv_ar_request> & reqs, std::vector<float> & logits_out) {
    if (reqs.empty()) return;
    if (p->prompt_len == 0) p->prompt_len = (int) reqs[0].prompt.size();
    std::vector<gsvk_request> c = to_c(reqs);
    logits_out.assign((size_t) p->info.vocab * reqs.size(), 0.0f);
    if (gsvk_first_logits(p->m, c.data(), (int) c.size(), logits_out.data()) != GSVK_OK)
        fprintf(stderr, "[gsv_ar] first_logits failed: %s\n", gsvk_last_error());
}

gsv_ar_result gsv_ar::generate(const std::vector<gsv_ar_request> & reqs,
                               const gsv_sampler_cfg & sampler, uint64_t seed_base,
                               int early_stop_num, int max_steps,
                               const std::vector<int32_t> * oracle_tokens,
                               const std::vector<uint64_t> * seeds) {
    gsv_ar_result res;
    const int B = (int) reqs.size();
    if (B == 0) return res;
    for (const auto & r : reqs)
        if (r.prompt.size() != reqs[0].prompt.size())
            fprintf(stderr, "[gsv_ar] warning: prompt lengths differ within the batch\n");
    p->prompt_len = (int) reqs[0].prompt.size();
    const int P = p->prompt_len;
    if (max_steps < 0) max_steps = 0;
    std::vector<gsvk_request> c = to_c(reqs);
    gsvk_sampler_cfg sc{sampler.top_k, sampler.top_p, sampler.temperature, sampler.repetition_penalty};
    std::vector<uint64_t> sd;
    if (seeds) {   // explicit seeds for the first seeds->size() sequences, defaults after
        sd.resize(B);
        for (int b = 0; b < B; b++)
            sd[b] = (size_t) b < seeds->size() ? (*seeds)[b] : seed_base + 0x9E3779B9ull * (uint64_t) b;
    }
    const int stride = P + max_steps;
    std::vector<int32_t> tokens((size_t) B * stride), tok_len(B), lens(B);
    const char * dump_path = getenv("GSV_AR_PROB_DUMP");
    std::vector<float> probs;
    if (dump_path) probs.resize((size_t) max_steps * p->info.vocab);
    gsvk_gen_out out{};
    out.tokens = tokens.data();
    out.tok_stride = stride;
    out.tok_len = tok_len.data();
    out.lens = lens.data();
    out.probs0 = dump_path ? probs.data() : nullptr;
    out.progress = progress_tick;
    gsvprog::begin(2, max_steps);
    const double t0 = now_ms();
    const int rc = gsvk_generate(p->m, c.data(), B, &sc, seed_base, early_stop_num, max_steps,
                                 oracle_tokens ? oracle_tokens->data() : nullptr,
                                 oracle_tokens ? (int) oracle_tokens->size() : 0,
                                 seeds ? sd.data() : nullptr, dump_path ? GSVK_GEN_PROB_DUMP : 0u, &out);
    if (rc != GSVK_OK) {
        fprintf(stderr, "[gsv_ar] generate failed: %s\n", gsvk_last_error());
        return res;   // empty: callers check tokens.size() == reqs.size()
    }
    if (p->profile) {
        // the reference's three report lines (src/gsv_ar.cpp:33-42); the embedding, masks and
        // sampling run on the device inside `compute`, so the host buckets are zero
        gsvk_profile pr{};
        gsvk_model_get_profile(p->m, &pr);
        const int n = std::max(1, pr.steps);
        printf("[prof:decode] prefill(build/copy/compute/io) = %.1f/%.1f/%.1f/%.1f ms\n", pr.pf_build_ms,
               pr.pf_copy_ms, pr.pf_compute_ms, pr.pf_io_ms);
        printf("[prof:decode] steps=%d build=%.1fms copy=%.1fms compute=%.1fms other=%.1fms (per-step: %.2f/%.2f/%.2f)\n",
               pr.steps, pr.dec_build_ms, pr.dec_copy_ms, pr.dec_compute_ms, pr.dec_other_ms, pr.dec_build_ms / n,
               pr.dec_copy_ms / n, pr.dec_compute_ms / n);
        printf("[prof:decode] host per-step: mask=%.3fms sampling=%.3fms emb+pe=%.3fms\n", 0.0, 0.0, 0.0);
        printf("[prof:decode] B=%d total=%.1f ms\n", B, now_ms() - t0);
    }
    res.tokens.resize(B);
    for (int b = 0; b < B; b++)
        res.tokens[b].assign(tokens.begin() + (size_t) b * stride, tokens.begin() + (size_t) b * stride + tok_len[b]);
    res.lens.assign(lens.begin(), lens.end());
    if (dump_path && out.n_steps > 0) {
        FILE * f = fopen(dump_path, "wb");
        if (f) {
            fwrite(probs.data(), 4, (size_t) out.n_steps * p->info.vocab, f);
            fclose(f);
            fprintf(stderr, "[gsv_ar] prob dump: %d steps -> %s\n", out.n_steps, dump_path);
        }
    }
    return res;
}

void gsv_ar::release_cache() {
    if (p && p->m) gsvk_release_cache(p->m);
}

// Host replay of the GEMV-chain decode step (the launches of runtime.hip's enqueue_decode_rows and
// decode_head, then the sampler of the next step) with the library's kernels compiled for the CPU
// (hip/hip_runtime.h, emu.h) under AddressSanitizer. Every buffer has the exact size the runtime
// allocates for that shape (ensure_state, alloc_kv, do_prefill's lmax = S + max_steps + 8), so an
// access outside one of them is reported with its kernel and line. Test infrastructure only.
//
//   decode_replay B S steps idx layers...   e.g.  decode_replay 32 400 500 7 0 1 23
//
// B sequences with valid lengths spread over [S/4, S] (left padding), a cache for `steps` decode
// steps, the step at loop index idx (the new key at column S + idx), the listed layers.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "common.h"
#include "layer.h"
#include "qkv_attn.h"
#include "sampler.h"

namespace gsvk {
static std::string g_err;
void set_error(const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}
const char * get_error() { return g_err.c_str(); }
int launch_head_ln(const void * W, int wtype, int64_t n, const float * res, const float * r, const float * bias,
                   const float * wb, int64_t m, float * Y, int64_t ys, hipStream_t stream);
// the prefill's many-row projection on the matrix cores (fdot_mfma.hip) is not part of the decode
// step: linked here, never run
int launch_fdot_mfma(const float *, int64_t, int64_t, const float *, int64_t, int64_t, float *, int64_t,
                     hipStream_t) {
    std::fprintf(stderr, "hostemu: matrix-core kernel not emulated\n");
    std::abort();
}
}  // namespace gsvk

using namespace gsvk;

static std::mt19937_64 g_rng(0x6A5E0002);

// exact-size heap buffers (AddressSanitizer bounds each allocation)
template <typename T>
static T * buf(size_t n, const char * what) {
    T * p = (T *) std::malloc(std::max<size_t>(n, 1) * sizeof(T));
    if (!p) {
        std::fprintf(stderr, "allocation of %s (%zu elements) failed\n", what, n);
        std::exit(2);
    }
    std::memset(p, 0, std::max<size_t>(n, 1) * sizeof(T));
    return p;
}
static void fill_q(int8_t * q, size_t n) {
    for (size_t i = 0; i < n; i++) q[i] = (int8_t) ((int) (g_rng() % 255) - 127);
}
static void fill_d(uint16_t * d, size_t n) {
    for (size_t i = 0; i < n; i++) d[i] = (uint16_t) (0x1800 + g_rng() % 0x400);   // fp16 ~ 2^-9
}
static void fill_f(float * f, size_t n, float s) {
    std::normal_distribution<float> nd(0.0f, s);
    for (size_t i = 0; i < n; i++) f[i] = nd(g_rng);
}

struct Lin {
    int8_t * qs;
    uint16_t * d;
    float * b;
};
static Lin make_lin(int n, int k) {
    Lin l{buf<int8_t>((size_t) n * k, "quants"), buf<uint16_t>((size_t) n * k / 32, "scales"), buf<float>(n, "bias")};
    fill_q(l.qs, (size_t) n * k);
    fill_d(l.d, (size_t) n * k / 32);
    fill_f(l.b, n, 0.02f);
    return l;
}

#define CHECK(call)                                                                        \
    do {                                                                                   \
        int s_ = (call);                                                                   \
        if (s_ != GSVK_OK) {                                                               \
            std::fprintf(stderr, "%s failed: %s\n", #call, get_error());                    \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

int main(int argc, char ** argv) {
    if (argc < 6) {
        std::fprintf(stderr, "usage: %s B S steps idx layer...\n", argv[0]);
        return 2;
    }
    const int B = std::atoi(argv[1]), S = std::atoi(argv[2]), steps = std::atoi(argv[3]), idx = std::atoi(argv[4]);
    std::vector<int> layers;
    for (int i = 5; i < argc; i++) layers.push_back(std::atoi(argv[i]));
    const int D = 512, NH = 16, HD = 32, F = 2048, V = 1025, NL = 24, P = 64, PE_MAX = 4096, EOS = 1024;
    const int lmax = S + steps + 8, lstride = lmax + 1;
    const int hist_len = P + steps;
    const size_t Bp = ((size_t) B + 31) / 32 * 32;
    std::printf("replay: B=%d S=%d lstride=%d idx=%d (new key at column %d)\n", B, S, lstride, idx, S + idx);

    // weights (the layers replayed; each keeps its own buffers)
    std::vector<Lin> qkv(NL), out(NL), f1(NL), f2(NL);
    std::vector<float *> ln1(NL), ln2(NL);
    for (int li : layers) {
        qkv[li] = make_lin(3 * D, D);
        out[li] = make_lin(D, D);
        f1[li] = make_lin(F, D);
        f2[li] = make_lin(D, F);
        ln1[li] = buf<float>(2 * D, "ln1");
        ln2[li] = buf<float>(2 * D, "ln2");
        for (int i = 0; i < D; i++) ln1[li][i] = ln2[li][i] = 1.0f;
    }
    // the previous layer of a replayed layer > 0 supplies b_2 and LN2 (its FFN2 bias)
    for (int li : layers)
        if (li > 0 && !f2[li - 1].b) {
            f2[li - 1].b = buf<float>(D, "prev f2 bias");
            ln2[li - 1] = buf<float>(2 * D, "prev ln2");
            for (int i = 0; i < D; i++) ln2[li - 1][i] = 1.0f;
        }
    float * audio_emb = buf<float>((size_t) V * D, "audio_emb");
    fill_f(audio_emb, (size_t) V * D, 0.02f);
    float * pe = buf<float>((size_t) PE_MAX * D, "pe");
    fill_f(pe, (size_t) PE_MAX * D, 0.5f);
    uint16_t * head = buf<uint16_t>((size_t) V * D, "head");
    fill_d(head, (size_t) V * D);

    // ensure_state
    float * xx = buf<float>((size_t) B * D, "x.x");
    int8_t * xq = buf<int8_t>(Bp * D, "x.q");
    float * xd = buf<float>(Bp * D / 32, "x.d");
    float * ax = buf<float>((size_t) B * D, "attn.x");
    int8_t * aq = buf<int8_t>(Bp * D, "attn.q");
    float * ad = buf<float>(Bp * D / 32, "attn.d");
    float * n1x = buf<float>((size_t) B * D, "n1.x");
    fill_f(n1x, (size_t) B * D, 1.0f);
    int8_t * hq = buf<int8_t>(Bp * F, "hq.q");
    float * hd = buf<float>(Bp * F / 32, "hq.d");
    float * qkvb = buf<float>((size_t) B * 3 * D, "qkv");
    float * o = buf<float>((size_t) B * D, "o");
    float * h2 = buf<float>((size_t) B * D, "h2");
    fill_f(h2, (size_t) B * D, 0.1f);
    float * logits = buf<float>((size_t) B * V, "logits");
    fill_f(logits, (size_t) B * V, 1.0f);
    int32_t * kv_begin = buf<int32_t>(B, "kv_begin");
    int32_t * kv_end = buf<int32_t>(B, "kv_end");
    int32_t * d_step = buf<int32_t>(1, "d_step");
    int32_t * hist = buf<int32_t>((size_t) B * hist_len, "hist");
    int32_t * ny = buf<int32_t>(B, "ny");
    int32_t * fin_step = buf<int32_t>(B, "fin_step");
    int32_t * fin_kind = buf<int32_t>(B, "fin_kind");
    int32_t * last_tok = buf<int32_t>(B, "last_tok");
    int32_t * done_counter = buf<int32_t>(1, "done_counter");
    int32_t * n_unfinished = buf<int32_t>(1, "n_unfinished");
    int32_t * sampled = buf<int32_t>((size_t) steps * B, "sampled");
    uint64_t * rng = buf<uint64_t>(B, "rng");
    // alloc_kv (EMU_PLANT=1: the K cache short by the rows from this step's column on, for the
    // last (sequence, head) pair of the last layer, a planted mistake that the check must report)
    const size_t per = (size_t) NL * B * NH * (size_t) lstride * HD;
    const bool plant = std::getenv("EMU_PLANT") && std::atoi(std::getenv("EMU_PLANT")) == 1;
    uint16_t * kc = buf<uint16_t>(plant ? per - (size_t) (lstride - (S + idx)) * HD : per, "kc");
    uint16_t * vc = buf<uint16_t>(per, "vc");
    // valid lengths over [S/4, S], left padding
    for (int b = 0; b < B; b++) {
        const int len = S / 4 + (int) ((int64_t) (S - S / 4) * b / std::max(B - 1, 1));
        kv_begin[b] = S - len;
        ny[b] = P + idx;
        fin_step[b] = -1;
        fin_kind[b] = -1;
        last_tok[b] = (int) (g_rng() % 1024);
        rng[b] = 1 + b;
        for (int i = 0; i < P + idx; i++) hist[(size_t) b * hist_len + i] = (int) (g_rng() % 1024);
    }
    *d_step = idx + 1;   // the decode of loop index idx runs with the counter already advanced
    const int chunk = (V + 63) / 64;
    uint64_t * jump = buf<uint64_t>(RNG_JUMP_WORDS, "rng jump");
    uint64_t * adv = buf<uint64_t>(RNG_ADV_WORDS, "rng adv");
    rng_tables(V, chunk, jump, adv);

    const float scale = 1.0f / std::sqrt((float) HD);
    const size_t row_kv = (size_t) NH * lstride * HD;
    for (int li : layers) {
        std::printf("layer %d\n", li);
        std::fflush(stdout);
        const size_t loff = (size_t) li * B * row_kv;
        LayerIn in{};
        if (li == 0) {
            in.mode = IN_EMB;
            in.emb = audio_emb;
            in.pe = pe;
            in.tok = last_tok;
            in.pos_ptr = d_step;
            in.pos_add = P - 1;
            in.alpha = 1.0f;
            in.vocab = V;
            in.kv_end = kv_end;
            in.kv_end_add = S;
            in.pos_sub = nullptr;
            in.pe_rows = PE_MAX;
        } else {
            in.mode = IN_LN;
            in.res = n1x;
            in.r = h2;
            in.bias = f2[li - 1].b;
            in.wb = ln2[li - 1];
        }
        in.out_x = xx;
        // QKV + attention in one launch (the GEMV chain's choice for every batch it ran at)
        QkvAttnArgs qa{};
        qa.ws = qkv[li].qs;
        qa.wd = qkv[li].d;
        qa.bias = qkv[li].b;
        qa.in = in;
        qa.kc = kc + loff;
        qa.vc = vc + loff;
        qa.lstride = lstride;
        qa.kv_begin = kv_begin;
        qa.col_ptr = d_step;
        qa.col_add = S - 1;
        qa.n_head = NH;
        qa.scale_log2 = scale * 1.4426950408889634f;
        qa.out = ax;
        qa.oq = aq;
        qa.od = ad;
        CHECK(launch_qkv_attn(qa, B, lstride, nullptr));
        // layer_tail, GEMV form
        LayerIn qin{};
        qin.mode = IN_Q8;
        qin.xs = aq;
        qin.xd = ad;
        LayerOut oo{};
        oo.y = o;
        oo.y_stride = D;
        oo.n_store = D;
        CHECK(launch_layer_gemv(out[li].qs, out[li].d, D, D, B, qin, oo, nullptr));
        LayerIn lin{};
        lin.mode = IN_LN;
        lin.res = xx;
        lin.r = o;
        lin.bias = out[li].b;
        lin.wb = ln1[li];
        lin.out_x = n1x;
        LayerOut ho{};
        ho.bias = f1[li].b;
        ho.act = 1;
        ho.yq = hq;
        ho.yd = hd;
        CHECK(launch_layer_gemv(f1[li].qs, f1[li].d, F, D, B, lin, ho, nullptr));
        LayerIn hin{};
        hin.mode = IN_Q8;
        hin.xs = hq;
        hin.xd = hd;
        LayerOut h2o{};
        h2o.y = h2;
        h2o.y_stride = D;
        h2o.n_store = D;
        CHECK(launch_layer_gemv(f2[li].qs, f2[li].d, D, F, B, hin, h2o, nullptr));
    }
    // decode_head: LN2 of the last replayed layer in the F16 head's input stage
    const int last = layers.back();
    std::printf("head\n");
    std::fflush(stdout);
    CHECK(launch_head_ln(head, 1, V, n1x, h2, f2[last].b, ln2[last], B, logits, V, nullptr));
    // the next step's sampler (top-k 15, repetition 1.35, EOS masked)
    std::printf("sampler\n");
    std::fflush(stdout);
    SampleArgs sa{};
    sa.logits = logits;
    sa.V = V;
    sa.eos = EOS;
    sa.B = B;
    sa.P = P;
    sa.hist = hist;
    sa.hist_stride = hist_len;
    sa.ny = ny;
    sa.fin_step = fin_step;
    sa.fin_kind = fin_kind;
    sa.rng = rng;
    sa.jump = jump;
    sa.adv = adv;
    sa.chunk = chunk;
    sa.top_k = 15;
    sa.top_p = 1.0f;
    sa.temperature = 1.0f;
    sa.rep = 1.35f;
    sa.step = d_step;
    sa.flags = 1u;
    sa.last_tok = last_tok;
    sa.sampled_dump = sampled;
    sa.max_steps = steps;
    sa.done_counter = done_counter;
    sa.n_unfinished = n_unfinished;
    sa.early_stop = -1;
    CHECK(launch_sample(sa, nullptr));
    std::printf("replay done: no access outside the buffers\n");
    return 0;
}

// Host runtime of the gfx950 AR decoder: GGUF load and device upload (src/gsv_ar.cpp:490-705),
// resident fp16 KV cache (:94-147), device-side prefill (:186-293), the decode step (:380-467)
// captured as one HIP graph together with the device sampler, and the generate loop (:719-824).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "decode_layer.h"
#include "gguf.h"
#include "layer.h"
#include "qkv_attn.h"
#include "sampler.h"

namespace gsvk {

// kernels defined in the other translation units
int launch_head_ln(const void * W, int wtype, int64_t n, const float * res, const float * r, const float * bias,
                   const float * wb, int64_t m, float * Y, int64_t ys, hipStream_t stream);
int launch_head_ln_parts(const void * W, int wtype, int64_t n, const float * res, const float * parts,
                         int nparts, int64_t pstride, const float * bias, const float * wb, int64_t m,
                         float * Y, int64_t ys, hipStream_t stream);
int launch_fdot(const void * W, int wtype, int64_t n, int64_t k, const float * X, int64_t xs,
                int64_t m, float * Y, int64_t ys, int mode, hipStream_t stream);
int launch_build_xy(const float * text_emb, const float * audio_emb, const float * pe,
                    const int32_t * phones, const int32_t * pad, const int32_t * prompt, int B,
                    int S, int max_len, int d, float ta, float aa, float * xy, hipStream_t stream);
int launch_bert_feat(const float * bert, const int64_t * boff, const int32_t * row_b,
                     const int32_t * row_t, const int32_t * tlen, int bert_dim, int R, float * feat,
                     hipStream_t stream);
int launch_add_proj(float * xy, const float * proj, const float * bias, const int32_t * row_b,
                    const int32_t * row_t, const int32_t * pad, int S, int d, int R, int R1,
                    hipStream_t stream);
int launch_gather_last(const float * in, int B, int S, int d, float * out, hipStream_t stream);
int launch_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                        int d_model, float scale, float * out, int8_t * oq, float * od,
                        hipStream_t stream);
int launch_attn_exact_decode(const float * q, int64_t q_stride, const uint16_t * k, const uint16_t * v, int B,
                             int nh, int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end,
                             float scale, float * out, int8_t * oq, float * od, hipStream_t stream,
                             int oq_layout);
int launch_attn_exact_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                              int d_model, float scale, float * out, int8_t * oq, float * od, hipStream_t stream);

constexpr int PE_MAX = 4096;   // Y_PE_MAX, src/gsv_ar.cpp:44
// decode steps per graph launch of generate on the persistent decode (no launch passes max_steps)
constexpr int GEN_STEPS_PER_LAUNCH = 4;
// K/V rows per step from which the persistent decode streams the cache (the MALL holds 256 MB)
constexpr int64_t PERSIST_NT_BYTES = (int64_t) 256 << 20;

// ---- device allocation helpers ------------------------------------------------------------

struct DevArena {
    std::vector<void *> ptrs;
    ~DevArena() { release(); }
    void release() {
        for (void * p : ptrs) (void) hipFree(p);
        ptrs.clear();
    }
    template <typename T>
    int alloc(T *& out, size_t count) {
        out = nullptr;
        if (count == 0) count = 1;
        void * p = nullptr;
        const hipError_t e = hipMalloc(&p, count * sizeof(T));
        if (e != hipSuccess) {
            (void) hipGetLastError();
            set_error("hipMalloc of %zu bytes failed: %s", count * sizeof(T), hipGetErrorString(e));
            return GSVK_ERR_NOMEM;
        }
        ptrs.push_back(p);
        out = (T *) p;
        return GSVK_OK;
    }
};

// Bump allocation from a model-owned pool that is kept between calls; what does not fit is
// allocated apart (and freed with the arena), and `need` records the size the pool should have so
// that the next call of the same shape allocates nothing.
struct PoolArena {
    char * base = nullptr;
    size_t cap = 0, off = 0, need = 0;
    DevArena extra;
    template <typename T>
    int alloc(T *& out, size_t count) {
        const size_t bytes = ((std::max<size_t>(count, 1) * sizeof(T)) + 255) & ~(size_t) 255;
        need += bytes;
        if (off + bytes <= cap) {
            out = (T *) (base + off);
            off += bytes;
            return GSVK_OK;
        }
        return extra.alloc(out, count);
    }
};

struct Lin {
    int8_t * qs = nullptr;    // sliced quants (GEMV)
    int8_t * qn = nullptr;    // the same quants in natural order (GEMM, large batch)
    uint16_t * d = nullptr;
    int8_t * qt = nullptr;    // quants and scales in the matrix-core operand order (GEMM, small
    uint16_t * dt = nullptr;  // batch); rows % 32 == 0 only
    uint16_t * w16 = nullptr; // fp16(d * q) [n][k]: the prefill's fp16 mode (made at its first use)
    float * b = nullptr;
    int n = 0, k = 0;
    int type = GGML_Q8_0;     // GGML_Q8_0, or GGML_F16 / GGML_F32 with the rows [n][k] in wf
    void * wf = nullptr;
};

struct LayerW {
    Lin qkv, out, f1, f2;
    float * ln1 = nullptr;   // [w; b]
    float * ln2 = nullptr;
};

// Activation buffer: fp32 rows plus their Q8_0 copy (sliced quants + fp32 scales).
struct Act {
    float * x = nullptr;
    int8_t * q = nullptr;
    float * d = nullptr;
};

}  // namespace gsvk

using namespace gsvk;

struct gsvk_model {
    int device = 0;
    hipStream_t stream = nullptr;
    int verbose = 0;
    // hparams
    int D = 512, NH = 16, HD = 32, NL = 24, V = 1025, EOS = 1024, PH = 732, BERT = 1024, FFN = 2048;
    int head_type = 1;
    float text_alpha = 1.0f, audio_alpha = 1.0f;
    // weights
    DevArena wmem;
    std::vector<LayerW> L;
    void * head = nullptr;        // F16/F32 [V][D]
    Lin head_q8;                  // Q8_0 head
    float * text_emb = nullptr, * audio_emb = nullptr, * bert_aug = nullptr, * pe = nullptr;
    float * bert_b = nullptr;     // bias column of bert_aug, contiguous [D]
    uint64_t * rng_jump = nullptr, * rng_adv = nullptr;
    int rng_chunk = 17;
    // KV cache
    DevArena kvmem;
    uint16_t * kc = nullptr, * vc = nullptr;   // [NL][B][NH][lstride][HD]
    int kv_B = 0, kv_lmax = 0;
    int64_t lstride = 0;
    // decode / state buffers (sized for kv_B)
    DevArena smem;
    // prefill workspace (activations of all B*S rows), grown to the largest prefill seen
    void * pf_pool = nullptr;
    size_t pf_cap = 0;
    int s_B = 0, s_hist = 0, s_steps = 0;
    int64_t s_lstride = 0;
    Act x, attn, n1, hq;
    float * qkv = nullptr, * o = nullptr, * h2 = nullptr, * logits = nullptr;
    float * p1 = nullptr, * p2 = nullptr;   // partial rows of the two-launch decode layer
    float * hx = nullptr;                   // FFN1 output rows (F16 / F32 projections)
    // the persistent decode (decode_layer.h k_dec_persist): per-layer launch arguments in device
    // memory, its barrier words + error word; usable on this device; failed once (then not used)
    DecAttnArgs * d_pattn = nullptr;
    DecFfnArgs * d_pffn = nullptr;
    int * d_pflags = nullptr;           // [8 * 32] flags, then the error word
    bool persist_dev_ok = false, persist_failed = false, persist_now = false;
    bool generic = false;   // some projection is F16 / F32: the per-op path (enqueue_decode_generic)
    int decode_path = GSVK_DECODE_AUTO;
    bool exact = false;   // gsvk_model_set_exact: ggml-cpu's arithmetic order throughout
    bool prefill_f16 = false;   // gsvk_model_set_prefill_f16: prefill projections on fp16 matrix cores
    DevArena w16mem;            // the fp16 weight copies of that mode
    void * attn_ws = nullptr;
    int32_t * kv_begin = nullptr, * kv_end = nullptr;
    int32_t * d_step = nullptr, * hist = nullptr, * ny = nullptr, * fin_step = nullptr,
            * fin_kind = nullptr, * last_tok = nullptr, * done_counter = nullptr,
            * n_unfinished = nullptr, * oracle = nullptr, * sampled = nullptr;
    uint64_t * rng = nullptr;
    float * probs_dump = nullptr;
    int32_t * h_pinned = nullptr;   // pinned host word for the unfinished count
    // generate's completion check: the sampler also stores the unfinished count into this
    // mapped pinned word (d_unfinished_host: its device address); one event per step in flight
    int32_t * h_unfinished = nullptr, * d_unfinished_host = nullptr;
    hipEvent_t step_ev[2] = {nullptr, nullptr};
    // GSV_AR_PROFILE buckets of the last prefill / generate (gsvk_model_get_profile); the prefill's
    // device phases are timed with these events (uploads, kernels, logits read-back)
    hipEvent_t pf_ev[4] = {nullptr, nullptr, nullptr, nullptr};
    gsvk_profile prof{};
    // sequence state
    int prompt_len = 0, S = 0, max_len = 0, B = 0, host_step = 0;
    bool prefilled = false;
    // graph of one decode step; generate on the persistent decode also captures GEN_STEPS_PER_LAUNCH
    // steps in one graph (gexec_k), and its steps' sampler records whether any row took part, which
    // the persistent kernel checks (persist_gate) so that the steps run after the last row finished
    // return at once
    hipGraphExec_t gexec = nullptr, gexec_k = nullptr;
    hipGraph_t graph = nullptr, graph_k = nullptr;
    bool use_graph = true;
    bool persist_gate = false;
    // a batch that sequences join and leave while it decodes (gsvk_cb_*): per-row loop index at
    // which the row joined and its step limit (both non-null only while a session is open), the
    // session's shape and its host-side slot table
    DevArena cbmem;
    int32_t * row_start = nullptr, * row_max = nullptr;
    bool cb_open = false;
    int cb_smax = 0, cb_steps = 0, cb_step = 0;
    std::vector<int> cb_used, cb_start, cb_max;
    SampleArgs cb_sa{};

    ~gsvk_model() {
        if (pf_pool) (void) hipFree(pf_pool);
        if (gexec) (void) hipGraphExecDestroy(gexec);
        if (graph) (void) hipGraphDestroy(graph);
        if (gexec_k) (void) hipGraphExecDestroy(gexec_k);
        if (graph_k) (void) hipGraphDestroy(graph_k);
        if (h_pinned) (void) hipHostFree(h_pinned);
        if (h_unfinished) (void) hipHostFree(h_unfinished);
        for (hipEvent_t & e : step_ev)
            if (e) (void) hipEventDestroy(e);
        for (hipEvent_t & e : pf_ev)
            if (e) (void) hipEventDestroy(e);
        if (stream) (void) hipStreamDestroy(stream);
    }
};

namespace {

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        (void) hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void) hipSetDevice(prev);
    }
};

void drop_graph(gsvk_model * m) {
    if (m->gexec) (void) hipGraphExecDestroy(m->gexec);
    if (m->graph) (void) hipGraphDestroy(m->graph);
    if (m->gexec_k) (void) hipGraphExecDestroy(m->gexec_k);
    if (m->graph_k) (void) hipGraphDestroy(m->graph_k);
    m->gexec = m->gexec_k = nullptr;
    m->graph = m->graph_k = nullptr;
}

// Close an open batch session (its graph and per-row arrays); the cache and state stay allocated.
void cb_drop(gsvk_model * m) {
    if (!m->cb_open) return;
    (void) hipStreamSynchronize(m->stream);
    drop_graph(m);
    m->cbmem.release();
    m->row_start = m->row_max = nullptr;
    m->cb_open = false;
    m->cb_used.clear();
    m->cb_start.clear();
    m->cb_max.clear();
    m->prefilled = false;
}

int upload(void * dst, const void * src, size_t bytes, hipStream_t st) {
    GSVK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st));
    return GSVK_OK;
}

// Read a Q8_0 [rows][k] tensor and repack it to the device layout.
int load_q8(gsvk_model * m, const GgufFile & g, const GgufTensor * t, Lin & lin, void * staging,
            size_t staging_bytes, std::vector<uint8_t> & host) {
    if (t->type != GGML_Q8_0 || t->ne.size() != 2) {
        set_error("%s: expected a 2-D Q8_0 tensor (type %u)", t->name.c_str(), t->type);
        return GSVK_ERR_FORMAT;
    }
    lin.k = (int) t->ne[0];
    lin.n = (int) t->ne[1];
    if (lin.k % 128 != 0) {
        set_error("%s: row length %d must be a multiple of 128", t->name.c_str(), lin.k);
        return GSVK_ERR_FORMAT;
    }
    if (t->nbytes > staging_bytes) {
        set_error("%s: staging buffer too small", t->name.c_str());
        return GSVK_ERR_FORMAT;
    }
    host.resize(t->nbytes);
    if (!g.read(*t, host.data())) {
        set_error("read of %s failed", t->name.c_str());
        return GSVK_ERR_IO;
    }
    GSVK_TRY(m->wmem.alloc(lin.qs, (size_t) lin.n * lin.k));
    GSVK_TRY(m->wmem.alloc(lin.qn, (size_t) lin.n * lin.k));
    GSVK_TRY(m->wmem.alloc(lin.d, (size_t) lin.n * (lin.k / 32)));
    if (lin.n % 32 == 0) {
        GSVK_TRY(m->wmem.alloc(lin.qt, (size_t) lin.n * lin.k));
        GSVK_TRY(m->wmem.alloc(lin.dt, (size_t) lin.n * (lin.k / 32)));
    }
    GSVK_HIP(hipMemcpyAsync(staging, host.data(), t->nbytes, hipMemcpyHostToDevice, m->stream));
    GSVK_TRY(launch_q8_repack(staging, lin.n, lin.k, lin.qs, lin.d, m->stream, lin.qn, lin.qt, lin.dt));
    GSVK_HIP(hipStreamSynchronize(m->stream));   // host buffer is reused
    return GSVK_OK;
}

// Read a projection of a pre-swizzled file: quants (I8) and scales (F16) already in the Q8_TILED
// order go to the device as they are; the sliced and natural copies are derived there.
int load_q8_tiled(gsvk_model * m, const GgufFile & g, const GgufTensor * tq, const GgufTensor * td, Lin & lin,
                  std::vector<uint8_t> & host) {
    if (tq->type != GGML_I8 || tq->ne.size() != 2 || td->type != GGML_F16 || td->ne.size() != 2 ||
        td->ne[0] * 32 != tq->ne[0] || td->ne[1] != tq->ne[1]) {
        set_error("%s / %s: expected I8 [k, n] quants and F16 [k/32, n] scales", tq->name.c_str(), td->name.c_str());
        return GSVK_ERR_FORMAT;
    }
    lin.k = (int) tq->ne[0];
    lin.n = (int) tq->ne[1];
    if (lin.k % 128 != 0 || lin.n % 32 != 0) {
        set_error("%s: row length %d must be a multiple of 128 and rows %d of 32", tq->name.c_str(), lin.k, lin.n);
        return GSVK_ERR_FORMAT;
    }
    const size_t nq = (size_t) lin.n * lin.k, nd = (size_t) lin.n * (lin.k / 32);
    GSVK_TRY(m->wmem.alloc(lin.qs, nq));
    GSVK_TRY(m->wmem.alloc(lin.qn, nq));
    GSVK_TRY(m->wmem.alloc(lin.d, nd));
    GSVK_TRY(m->wmem.alloc(lin.qt, nq));
    GSVK_TRY(m->wmem.alloc(lin.dt, nd));
    host.resize(tq->nbytes);
    if (!g.read(*tq, host.data())) { set_error("read of %s failed", tq->name.c_str()); return GSVK_ERR_IO; }
    GSVK_HIP(hipMemcpy(lin.qt, host.data(), nq, hipMemcpyHostToDevice));
    host.resize(td->nbytes);
    if (!g.read(*td, host.data())) { set_error("read of %s failed", td->name.c_str()); return GSVK_ERR_IO; }
    GSVK_HIP(hipMemcpy(lin.dt, host.data(), nd * 2, hipMemcpyHostToDevice));
    GSVK_TRY(launch_q8_untile(lin.qt, lin.dt, lin.n, lin.k, lin.qs, lin.d, lin.qn, m->stream));
    return GSVK_OK;
}

int load_f32(gsvk_model * m, const GgufFile & g, const char * name, int64_t expect, float *& dst,
             std::vector<float> * keep = nullptr) {
    const GgufTensor * t = g.tensor(name);
    if (!t) { set_error("missing tensor %s", name); return GSVK_ERR_FORMAT; }
    if (t->type != GGML_F32) { set_error("%s must be F32 (type %u)", name, t->type); return GSVK_ERR_FORMAT; }
    int64_t nel = 1;
    for (int64_t v : t->ne) nel *= v;
    if (expect >= 0 && nel != expect) {
        set_error("%s: %lld elements, expected %lld", name, (long long) nel, (long long) expect);
        return GSVK_ERR_FORMAT;
    }
    std::vector<float> host((size_t) nel);
    if (!g.read(*t, host.data())) { set_error("read of %s failed", name); return GSVK_ERR_IO; }
    GSVK_TRY(m->wmem.alloc(dst, (size_t) nel));
    GSVK_HIP(hipMemcpy(dst, host.data(), (size_t) nel * 4, hipMemcpyHostToDevice));
    if (keep) *keep = std::move(host);
    return GSVK_OK;
}

// Resident buffers of the decode step, prefill excluded (sized by B and the KV capacity).
int ensure_state(gsvk_model * m, int B, int hist_len, int max_steps) {
    if (m->s_B == B && m->s_hist >= hist_len && m->s_steps >= max_steps && m->s_lstride == m->lstride &&
        m->x.x)
        return GSVK_OK;
    drop_graph(m);
    m->smem.release();
    const int D = m->D;
    auto & a = m->smem;
    // Q8_0 activations hold whole 32-row tiles (the matrix-core operand order of the large-batch
    // path); the padding rows are zero and stay so
    const size_t Bp = ((size_t) B + 31) / 32 * 32;
    GSVK_TRY(a.alloc(m->x.x, (size_t) B * D));
    GSVK_TRY(a.alloc(m->x.q, Bp * D));
    GSVK_TRY(a.alloc(m->x.d, Bp * D / 32));
    GSVK_TRY(a.alloc(m->attn.x, (size_t) B * D));
    GSVK_TRY(a.alloc(m->attn.q, Bp * D));
    GSVK_TRY(a.alloc(m->attn.d, Bp * D / 32));
    GSVK_TRY(a.alloc(m->n1.x, (size_t) B * D));
    GSVK_TRY(a.alloc(m->n1.q, Bp * D));
    GSVK_TRY(a.alloc(m->n1.d, Bp * D / 32));
    GSVK_TRY(a.alloc(m->hq.q, Bp * m->FFN));
    GSVK_TRY(a.alloc(m->hq.d, Bp * m->FFN / 32));
    for (Act * act : {&m->x, &m->attn, &m->n1}) {
        GSVK_HIP(hipMemset(act->q, 0, Bp * D));
        GSVK_HIP(hipMemset(act->d, 0, Bp * D / 32 * sizeof(float)));
    }
    GSVK_HIP(hipMemset(m->hq.q, 0, Bp * m->FFN));
    GSVK_HIP(hipMemset(m->hq.d, 0, Bp * m->FFN / 32 * sizeof(float)));
    GSVK_TRY(a.alloc(m->qkv, (size_t) B * 3 * D));
    GSVK_TRY(a.alloc(m->o, (size_t) B * D));
    GSVK_TRY(a.alloc(m->h2, (size_t) B * D));
    GSVK_TRY(a.alloc(m->logits, (size_t) B * m->V));
    GSVK_TRY(a.alloc(m->p1, (size_t) m->NH * B * D));
    GSVK_TRY(a.alloc(m->p2, (size_t) DEC_FFN_GROUPS_MAX * B * D));
    GSVK_TRY(a.alloc(m->hx, (size_t) B * m->FFN));
    char * ws = nullptr;
    GSVK_TRY(a.alloc(ws, attn_workspace_bytes(B, m->NH, m->lstride)));
    GSVK_HIP(hipMemset(ws, 0, attn_workspace_bytes(B, m->NH, m->lstride)));
    m->attn_ws = ws;
    GSVK_TRY(a.alloc(m->kv_begin, B));
    GSVK_TRY(a.alloc(m->kv_end, B));
    GSVK_TRY(a.alloc(m->d_step, 1));
    GSVK_TRY(a.alloc(m->hist, (size_t) B * hist_len));
    GSVK_TRY(a.alloc(m->ny, B));
    GSVK_TRY(a.alloc(m->fin_step, B));
    GSVK_TRY(a.alloc(m->fin_kind, B));
    GSVK_TRY(a.alloc(m->last_tok, B));
    GSVK_TRY(a.alloc(m->done_counter, 1));
    GSVK_HIP(hipMemset(m->done_counter, 0, sizeof(int32_t)));
    GSVK_TRY(a.alloc(m->n_unfinished, 1));
    GSVK_TRY(a.alloc(m->oracle, max_steps));
    GSVK_TRY(a.alloc(m->sampled, (size_t) max_steps * B));
    GSVK_TRY(a.alloc(m->rng, B));
    GSVK_TRY(a.alloc(m->probs_dump, (size_t) max_steps * m->V));
    m->s_B = B;
    m->s_hist = hist_len;
    m->s_steps = max_steps;
    m->s_lstride = m->lstride;
    return GSVK_OK;
}

int alloc_kv(gsvk_model * m, int B, int lmax) {
    if (m->kc && m->kv_lmax >= lmax && m->kv_B == B) return GSVK_OK;
    drop_graph(m);
    m->kvmem.release();
    m->smem.release();
    m->s_B = 0;
    m->kc = m->vc = nullptr;
    m->kv_B = m->kv_lmax = 0;
    const size_t per = (size_t) m->NL * B * m->NH * (size_t) (lmax + 1) * m->HD;
    GSVK_TRY(m->kvmem.alloc(m->kc, per));
    GSVK_TRY(m->kvmem.alloc(m->vc, per));
    GSVK_HIP(hipMemsetAsync(m->kc, 0, per * 2, m->stream));
    GSVK_HIP(hipMemsetAsync(m->vc, 0, per * 2, m->stream));
    m->kv_B = B;
    m->kv_lmax = lmax;
    m->lstride = lmax + 1;
    return GSVK_OK;
}

int head_logits(gsvk_model * m, const Act & x, int B, int mode, float * out, hipStream_t st) {
    if (m->head_type == GGML_Q8_0) {
        GemvEpilogue epi{};
        return launch_q8_gemv(m->head_q8.qs, m->head_q8.d, m->V, m->D, x.q, x.d, B, epi, out,
                              st);
    }
    return launch_fdot(m->head, m->head_type == GGML_F16 ? 1 : 0, m->V, m->D, x.x, m->D, B, out,
                       m->V, mode, st);
}

// The projections of one layer after attention (shared by prefill and decode), with the
// LayerNorms folded into the input stage of the consuming GEMV:
//   o  = Wo . attn
//   n1 = LN1(cur + o + bo)                       (FFN1 input stage; stored to n1x)
//   hq = Q8_0(relu(W1 . n1 + b1))                (quantised in FFN1's output stage)
//   h2 = W2 . hq
// LN2 (cur' = LN2(n1 + h2 + b2)) is the input stage of the next layer's QKV or of final_ln().
Q8Weights q8w(const Lin & l) { return Q8Weights{l.qn, l.d, l.qt, l.dt}; }

// The fp16 copies of the four projections of every layer (gsvk_model_set_prefill_f16), made once.
int ensure_w16(gsvk_model * m) {
    for (LayerW & w : m->L)
        for (Lin * l : {&w.qkv, &w.out, &w.f1, &w.f2})
            if (!l->w16) {
                GSVK_TRY(m->w16mem.alloc(l->w16, (size_t) l->n * l->k));
                GSVK_TRY(launch_q8_dequant_f16(l->qn, l->d, l->n, l->k, l->w16, m->stream));
            }
    return GSVK_OK;
}

// A projection of the prefill's rows on the matrix cores: the int8 GEMM, or in the fp16 mode the
// fp16 GEMM on the dequantised weights (the shapes it takes: above 256 rows, n % 128 == 0, k 512
// or 2048).
int prefill_gemm(const gsvk_model * m, const Lin & l, int64_t rows, const int8_t * xs, const float * xd,
                 const LayerOut & out, hipStream_t st) {
    if (m->prefill_f16 && l.w16 && rows > 256 && l.n % 128 == 0 && (l.k == 512 || l.k == 2048))
        return launch_q8h_gemm(l.w16, l.n, l.k, rows, xs, xd, out, st);
    return launch_q8_gemm(q8w(l), l.n, l.k, rows, xs, xd, Q8_NATURAL, out, st);
}

int layer_tail(gsvk_model * m, hipStream_t st, const LayerW & w, int64_t R, const float * cur_x, const Act & attn,
               float * o, float * n1x, Act & hq, float * h2, Act * n1 = nullptr,
               int layout = Q8_NATURAL, const int32_t * row_pad = nullptr, int rows_per_seq = 0,
               bool prefill = false) {
    const int D = m->D, F = m->FFN;
    if (n1) {
        // many rows (the caller's choice): the projections on the matrix cores, LN1 as its own
        // launch (with the Q8_0 copy the FFN1 GEMM reads); the Q8_0 activations (attention output,
        // LN1, FFN1 output) in the given layout
        LayerOut oo{};
        oo.y = o;
        oo.y_stride = D;
        oo.n_store = D;
        oo.row_pad = row_pad;           // (prefill: tiles of left-padding rows are skipped)
        oo.rows_per_seq = rows_per_seq;
        // (prefill: natural order; prefill_gemm picks the int8 or the fp16 GEMM)
        auto gemm = [&](const Lin & l, int64_t n, int64_t k, const int8_t * xs, const float * xd,
                        const LayerOut & out) {
            return prefill ? prefill_gemm(m, l, R, xs, xd, out, st)
                           : launch_q8_gemm(q8w(l), n, k, R, xs, xd, layout, out, st);
        };
        GSVK_TRY(gemm(w.out, D, D, attn.q, attn.d, oo));
        // (prefill: the left-padding rows are normalised from zeros, without reading their
        // rows: no valid row reads them, and the FFN GEMM tiles that mix them with valid rows get
        // finite values)
        GSVK_TRY(launch_layernorm(cur_x, o, w.out.b, w.ln1, R, D, 1e-5f, n1x, n1->q, n1->d, st, layout, nullptr,
                                  row_pad, rows_per_seq));
        LayerOut ho{};
        ho.bias = w.f1.b;
        ho.act = 1;
        ho.yq = hq.q;
        ho.yd = hq.d;
        ho.yq_layout = layout;
        ho.row_pad = row_pad;
        ho.rows_per_seq = rows_per_seq;
        GSVK_TRY(gemm(w.f1, F, D, n1->q, n1->d, ho));
        LayerOut h2o{};
        h2o.y = h2;
        h2o.y_stride = D;
        h2o.n_store = D;
        h2o.row_pad = row_pad;
        h2o.rows_per_seq = rows_per_seq;
        return gemm(w.f2, D, F, hq.q, hq.d, h2o);
    }
    LayerIn qin{};
    qin.mode = IN_Q8;
    qin.xs = attn.q;
    qin.xd = attn.d;
    LayerOut oo{};
    oo.y = o;
    oo.y_stride = D;
    oo.n_store = D;
    GSVK_TRY(launch_layer_gemv(w.out.qs, w.out.d, D, D, R, qin, oo, st));
    LayerIn lin{};
    lin.mode = IN_LN;
    lin.res = cur_x;
    lin.r = o;
    lin.bias = w.out.b;
    lin.wb = w.ln1;
    lin.out_x = n1x;
    LayerOut ho{};
    ho.bias = w.f1.b;
    ho.act = 1;
    ho.yq = hq.q;
    ho.yd = hq.d;
    GSVK_TRY(launch_layer_gemv(w.f1.qs, w.f1.d, F, D, R, lin, ho, st));
    LayerIn hin{};
    hin.mode = IN_Q8;
    hin.xs = hq.q;
    hin.xd = hq.d;
    LayerOut h2o{};
    h2o.y = h2;
    h2o.y_stride = D;
    h2o.n_store = D;
    GSVK_TRY(launch_layer_gemv(w.f2.qs, w.f2.d, D, F, R, hin, h2o, st));
    return GSVK_OK;
}

// QKV projection output stage: q (and k, v when n_store = 3D) as fp32, plus the K/V append.
LayerOut qkv_out(gsvk_model * m, const LayerW & w, size_t loff, float * y, int n_store,
                 int rows_per_seq, const int32_t * col_ptr, int col_add) {
    LayerOut qo{};
    qo.y = y;
    qo.y_stride = n_store;
    qo.n_store = n_store;
    qo.bias = w.qkv.b;
    qo.kc = m->kc + loff;
    qo.vc = m->vc + loff;
    qo.kv_row0 = m->D;
    qo.d_model = m->D;
    qo.n_head = m->NH;
    qo.lstride = m->lstride;
    qo.rows_per_seq = rows_per_seq;
    qo.col_ptr = col_ptr;
    qo.col_add = col_add;
    return qo;
}

// LN2 of the last layer: x = LN2(n1 + h2 + b2), quantised too when the head is Q8_0.
int final_ln(gsvk_model * m, hipStream_t st, int64_t R, const float * n1x, const float * h2, Act & x) {
    const LayerW & w = m->L[m->NL - 1];
    const bool q = m->head_type == GGML_Q8_0;
    return launch_layernorm(n1x, h2, w.f2.b, w.ln2, R, m->D, 1e-5f, x.x, q ? x.q : nullptr,
                            q ? x.d : nullptr, st);
}

// Logits of a decode step: the last layer's LN2 then the head. An F16 / F32 head takes the
// LayerNorm as its input stage (the same arithmetic as the LayerNorm launch, one launch fewer).
int decode_head(gsvk_model * m, int n, const float * n1x, const float * h2, Act & x, float * logits,
                hipStream_t st) {
    if (m->head_type != GGML_Q8_0 && m->D == 512) {
        const LayerW & w = m->L[m->NL - 1];
        return launch_head_ln(m->head, m->head_type == GGML_F16 ? 1 : 0, m->V, n1x, h2, w.f2.b, w.ln2, n,
                              logits, m->V, st);
    }
    GSVK_TRY(final_ln(m, st, n, n1x, h2, x));
    return head_logits(m, x, n, 0, logits, st);
}

// Kernels of one decode step at loop index idx = *d_step - 1: the layer-0 QKV embeds last_tok at
// PE position prompt_len + idx (and sets kv_end = S + idx + 1); every QKV appends K/V at column
// S + idx; logits of the head.
//
// Matrix-core path (batch >= DECODE_GEMM_MIN_BATCH): the whole batch on the model's stream.
int enqueue_decode_mfma(gsvk_model * m) {
    const int B = m->B, D = m->D;
    const float scale = 1.0f / std::sqrt((float) m->HD);
    for (int li = 0; li < m->NL; li++) {
        const LayerW & w = m->L[li];
        const size_t loff = (size_t) li * B * m->NH * m->lstride * m->HD;
        // large batch: embedding / LN2 of the previous layer as their own launches, the QKV
        // GEMM with the K/V append, attention, then the GEMM tail; every Q8_0 activation in
        // the matrix-core operand order (rows padded to 32)
        if (li == 0) {
            GSVK_TRY(launch_embed_pe(m->audio_emb, m->pe, m->last_tok, m->V, m->d_step,
                                     m->prompt_len - 1, m->audio_alpha, D, B, m->x.x, m->x.q,
                                     m->x.d, m->kv_end, m->S, m->row_start, PE_MAX, m->stream, Q8_TILED));
        } else {
            const LayerW & p = m->L[li - 1];
            GSVK_TRY(launch_layernorm(m->n1.x, m->h2, p.f2.b, p.ln2, B, D, 1e-5f, m->x.x, m->x.q,
                                      m->x.d, m->stream, Q8_TILED));
        }
        GSVK_TRY(launch_q8_gemm(q8w(w.qkv), 3 * D, D, B, m->x.q, m->x.d, Q8_TILED,
                                qkv_out(m, w, loff, m->qkv, D, 1, m->d_step, m->S - 1), m->stream));
        GSVK_TRY(launch_attn_decode(m->qkv, D, m->kc + loff, m->vc + loff, B, m->NH, m->HD,
                                    m->lstride, m->kv_begin, m->kv_end, m->lstride, scale,
                                    m->attn.x, nullptr, m->attn.q, m->attn.d, m->attn_ws, m->stream,
                                    Q8_TILED));
        GSVK_TRY(layer_tail(m, m->stream, w, B, m->x.x, m->attn, m->o, m->n1.x, m->hq, m->h2, &m->n1, Q8_TILED));
    }
    return decode_head(m, B, m->n1.x, m->h2, m->x, m->logits, m->stream);
}

// GEMV path, batch rows [r0, r0 + n) on stream st. Every kernel of it computes each row on its
// own: the per-row arithmetic does not depend on which or how many rows a launch holds. (Cutting
// a batch-16 step in row groups on 2 or 4 streams, forked and joined inside the captured graph,
// was measured slower, 0.57 -> 0.78 / 1.41 ms per step: the graph ran every branch on one
// hardware queue, one after the other.)
int enqueue_decode_rows(gsvk_model * m, int r0, int n, hipStream_t st) {
    // the GEMV chain decodes (and is tested at) up to GEMV_DECODE_MAX_BATCH rows only
    GSVK_REQUIRE(n >= 1 && n <= GEMV_DECODE_MAX_BATCH, "decode: %d rows on the GEMV path (at most %d)", n,
                 GEMV_DECODE_MAX_BATCH);
    const int B = m->B, D = m->D, F = m->FFN;
    const float scale = 1.0f / std::sqrt((float) m->HD);
    const size_t row_kv = (size_t) m->NH * m->lstride * m->HD;
    auto rows_of = [r0](const Act & a, int k) {
        return Act{a.x ? a.x + (size_t) r0 * k : nullptr, a.q ? a.q + (size_t) r0 * k : nullptr,
                   a.d ? a.d + (size_t) r0 * (k / 32) : nullptr};
    };
    Act x = rows_of(m->x, D), attn = rows_of(m->attn, D), n1 = rows_of(m->n1, D), hq = rows_of(m->hq, F);
    float * o = m->o + (size_t) r0 * D, * h2 = m->h2 + (size_t) r0 * D, * qkv = m->qkv + (size_t) r0 * D;
    for (int li = 0; li < m->NL; li++) {
        const LayerW & w = m->L[li];
        const size_t loff = (size_t) li * B * row_kv + (size_t) r0 * row_kv;
        LayerIn in{};
        if (li == 0) {
            in.mode = IN_EMB;
            in.emb = m->audio_emb;
            in.pe = m->pe;
            in.tok = m->last_tok + r0;
            in.pos_ptr = m->d_step;
            in.pos_add = m->prompt_len - 1;
            in.alpha = m->audio_alpha;
            in.vocab = m->V;
            in.kv_end = m->kv_end + r0;
            in.kv_end_add = m->S;
            in.pos_sub = m->row_start ? m->row_start + r0 : nullptr;
            in.pe_rows = PE_MAX;
        } else {
            const LayerW & p = m->L[li - 1];
            in.mode = IN_LN;
            in.res = n1.x;
            in.r = h2;
            in.bias = p.f2.b;
            in.wb = p.ln2;
        }
        in.out_x = x.x;
        const bool exact_fused = m->exact && m->NH * m->HD == 512 && m->HD == 32;
        if (m->exact && !exact_fused) {
            // the GEMV QKV, then attention in ggml-cpu's sequential order with glibc's expf
            GSVK_TRY(launch_layer_gemv(w.qkv.qs, w.qkv.d, 3 * D, D, n, in,
                                       qkv_out(m, w, loff, qkv, D, 1, m->d_step, m->S - 1), st));
            GSVK_TRY(launch_attn_exact_decode(qkv, D, m->kc + loff, m->vc + loff, n, m->NH, m->lstride,
                                              m->kv_begin + r0, m->kv_end + r0, scale, attn.x, attn.q, attn.d, st,
                                              Q8_SLICED));
        } else if (exact_fused || qkv_attn_preferred(n, m->NH, m->lstride)) {
            // QKV + attention in one launch per layer (exact mode: the attention in ggml-cpu's
            // sequential order with glibc's expf)
            QkvAttnArgs qa{};
            qa.ws = w.qkv.qs;
            qa.wd = w.qkv.d;
            qa.bias = w.qkv.b;
            qa.in = in;
            qa.kc = m->kc + loff;
            qa.vc = m->vc + loff;
            qa.lstride = m->lstride;
            qa.kv_begin = m->kv_begin + r0;
            qa.col_ptr = m->d_step;
            qa.col_add = m->S - 1;
            qa.n_head = m->NH;
            qa.scale_log2 = scale * 1.4426950408889634f;
            qa.scale = scale;
            qa.out = attn.x;
            qa.oq = attn.q;
            qa.od = attn.d;
            GSVK_TRY(launch_qkv_attn(qa, n, m->lstride, st, exact_fused));
        } else {
            GSVK_TRY(launch_layer_gemv(w.qkv.qs, w.qkv.d, 3 * D, D, n, in,
                                       qkv_out(m, w, loff, qkv, D, 1, m->d_step, m->S - 1), st));
            GSVK_TRY(launch_attn_decode(qkv, D, m->kc + loff, m->vc + loff, n, m->NH, m->HD,
                                        m->lstride, m->kv_begin + r0, m->kv_end + r0, m->lstride, scale,
                                        attn.x, nullptr, attn.q, attn.d, m->attn_ws, st));
        }
        GSVK_TRY(layer_tail(m, st, w, n, x.x, attn, o, n1.x, hq, h2));
    }
    return decode_head(m, n, n1.x, h2, x, m->logits + (size_t) r0 * m->V, st);
}

// Two launches per layer (decode_layer.hip) for the whole batch on the model's stream: the
// attention launch (input LayerNorm over the previous layer's partial rows, QKV, K/V append,
// attention, out-projection partial rows per head) and the FFN launch (LN1 over those partials,
// FFN1 + ReLU of a group of hidden units, FFN2 partial rows per group); the head sums the last
// layer's partials in its LayerNorm input stage.
void dec_layer_args(const gsvk_model * m, int li, DecAttnArgs & aa, DecFfnArgs & fa) {
    const int B = m->B;
    const int G = dec_ffn_groups(B);   // hidden groups of the FFN launch = partial rows of the next LN
    const float scale = 1.0f / std::sqrt((float) m->HD);
    const LayerW & w = m->L[li];
    const size_t loff = (size_t) li * B * m->NH * m->lstride * m->HD;
    aa = DecAttnArgs{};
    if (li == 0) {
        aa.mode = IN_EMB;
        aa.emb = m->audio_emb;
        aa.pe = m->pe;
        aa.tok = m->last_tok;
        aa.pos_ptr = m->d_step;
        aa.pos_add = m->prompt_len - 1;
        aa.pos_sub = m->row_start;
        aa.pe_rows = PE_MAX;
        aa.alpha = m->audio_alpha;
        aa.vocab = m->V;
        aa.kv_end = m->kv_end;
        aa.kv_end_add = m->S;
    } else {
        const LayerW & p = m->L[li - 1];
        aa.mode = IN_LN;
        aa.res = m->n1.x;
        aa.parts = m->p2;
        aa.nparts = G;
        aa.bias = p.f2.b;
        aa.wb = p.ln2;
    }
    aa.x_out = m->x.x;
    aa.wq = w.qkv.qs;
    aa.wd = w.qkv.d;
    aa.bqkv = w.qkv.b;
    aa.kc = m->kc + loff;
    aa.vc = m->vc + loff;
    aa.lstride = m->lstride;
    aa.kv_begin = m->kv_begin;
    aa.col_ptr = m->d_step;
    aa.col_add = m->S - 1;
    aa.scale_log2 = scale * 1.4426950408889634f;
    aa.woq = w.out.qt;
    aa.wod = w.out.dt;
    aa.p1 = m->p1;
    aa.B = B;
    fa = DecFfnArgs{};
    fa.res = m->x.x;
    fa.p1 = m->p1;
    fa.bo = w.out.b;
    fa.wb1 = w.ln1;
    fa.n1_out = m->n1.x;
    fa.w1q = w.f1.qs;
    fa.w1d = w.f1.d;
    fa.b1 = w.f1.b;
    fa.w2q = w.f2.qt;
    fa.w2d = w.f2.dt;
    fa.p2 = m->p2;
    fa.groups = G;
    fa.B = B;
}

int decode_head_parts(gsvk_model * m) {
    const LayerW & last = m->L[m->NL - 1];
    return launch_head_ln_parts(m->head, m->head_type == GGML_F16 ? 1 : 0, m->V, m->n1.x, m->p2,
                                dec_ffn_groups(m->B), (int64_t) m->B * m->D, last.f2.b, last.ln2, m->B, m->logits,
                                m->V, m->stream);
}

int enqueue_decode_fused(gsvk_model * m) {
    for (int li = 0; li < m->NL; li++) {
        DecAttnArgs aa;
        DecFfnArgs fa;
        dec_layer_args(m, li, aa, fa);
        GSVK_TRY(launch_dec_attn(aa, m->stream));
        GSVK_TRY(launch_dec_ffn(fa, m->stream));
    }
    return decode_head_parts(m);
}

// The persistent decode: one launch for the 24 layers (the arguments prepare_persist uploaded),
// then the head.
DecPersistArgs persist_args(const gsvk_model * m) {
    DecPersistArgs pa{};
    pa.attn = m->d_pattn;
    pa.ffn = m->d_pffn;
    pa.n_layer = m->NL;
    pa.B = m->B;
    pa.groups = dec_ffn_groups(m->B);
    pa.step = m->d_step;
    pa.flags = m->d_pflags;
    pa.err = m->d_pflags + 8 * 32;
    pa.active = m->persist_gate ? m->d_pflags + 8 * 32 + 1 : nullptr;
    // the cache rows one step reads (keys from S to lstride, about half way on average): beyond the
    // MALL, stream them (batch 16, 500 steps, ~400 MB per step: 0.351 -> 0.340 ms per step; batch
    // 1, 17 MB, stays cached: streaming it cost 0.293 -> 0.305)
    const int64_t step_kv = (int64_t) m->B * ((m->S + m->lstride) / 2) * m->NL * m->NH * m->HD * 2 * 2;
    pa.nt = step_kv > PERSIST_NT_BYTES ? 1 : 0;
    return pa;
}

int enqueue_decode_persist(gsvk_model * m) {
    GSVK_TRY(launch_dec_persist(persist_args(m), m->stream));
    return decode_head_parts(m);
}

// y[R][n] = W[n][k] . x[R][k] of one projection in ggml-cpu's order: a Q8_0 weight through the GEMV
// on the sliced Q8_0 copy of x (xq, xd); an F16 / F32 weight through ggml_vec_dot (mode 0) or
// tinyBLAS (mode 1) on the fp32 rows x, F16 with the activations rounded to fp16.
int proj_rows(const Lin & l, const float * x, const int8_t * xq, const float * xd, int64_t R, float * y, int mode,
              hipStream_t st) {
    if (l.type == GGML_Q8_0) {
        LayerIn qin{};
        qin.mode = IN_Q8;
        qin.xs = xq;
        qin.xd = xd;
        LayerOut o{};
        o.y = y;
        o.y_stride = l.n;
        o.n_store = l.n;
        return launch_layer_gemv(l.qs, l.d, l.n, l.k, R, qin, o, st);
    }
    return launch_fdot(l.wf, l.type == GGML_F16 ? 1 : 0, l.n, l.k, x, l.k, R, y, l.n, mode, st);
}

// Decode step of a model with F16 / F32 projections (the reference exporter's attn= / ffn=
// options; the engine's fallback model): one launch per op of src/gsv_ar.cpp:380-467, each in
// ggml-cpu's order (the projections as proj_rows, the LayerNorms as the Q8_0 path's), the attention
// the default decode kernel or, in exact mode, ggml's sequential one.
int enqueue_decode_generic(gsvk_model * m) {
    const int B = m->B, D = m->D, F = m->FFN;
    const float scale = 1.0f / std::sqrt((float) m->HD);
    hipStream_t st = m->stream;
    const size_t row_kv = (size_t) m->NH * m->lstride * m->HD;
    for (int li = 0; li < m->NL; li++) {
        const LayerW & w = m->L[li];
        const size_t loff = (size_t) li * B * row_kv;
        if (li == 0) {
            GSVK_TRY(launch_embed_pe(m->audio_emb, m->pe, m->last_tok, m->V, m->d_step, m->prompt_len - 1,
                                     m->audio_alpha, D, B, m->x.x, m->x.q, m->x.d, m->kv_end, m->S, m->row_start,
                                     PE_MAX, st));
        } else {
            const LayerW & p = m->L[li - 1];
            GSVK_TRY(launch_layernorm(m->n1.x, m->h2, p.f2.b, p.ln2, B, D, 1e-5f, m->x.x, m->x.q, m->x.d, st));
        }
        GSVK_TRY(proj_rows(w.qkv, m->x.x, m->x.q, m->x.d, B, m->qkv, 0, st));
        GSVK_TRY(launch_bias_kv(m->qkv, w.qkv.b, B, D, m->kc + loff, m->vc + loff, m->NH, m->lstride, 1, m->d_step,
                                m->S - 1, st));
        if (m->exact)
            GSVK_TRY(launch_attn_exact_decode(m->qkv, 3 * D, m->kc + loff, m->vc + loff, B, m->NH, m->lstride,
                                              m->kv_begin, m->kv_end, scale, m->attn.x, m->attn.q, m->attn.d, st,
                                              Q8_SLICED));
        else
            GSVK_TRY(launch_attn_decode(m->qkv, 3 * D, m->kc + loff, m->vc + loff, B, m->NH, m->HD, m->lstride,
                                        m->kv_begin, m->kv_end, m->lstride, scale, m->attn.x, nullptr, m->attn.q,
                                        m->attn.d, m->attn_ws, st));
        GSVK_TRY(proj_rows(w.out, m->attn.x, m->attn.q, m->attn.d, B, m->o, 0, st));
        GSVK_TRY(launch_layernorm(m->x.x, m->o, w.out.b, w.ln1, B, D, 1e-5f, m->n1.x, m->n1.q, m->n1.d, st));
        GSVK_TRY(proj_rows(w.f1, m->n1.x, m->n1.q, m->n1.d, B, m->hx, 0, st));
        GSVK_TRY(launch_add_act(m->hx, w.f1.b, (int64_t) B * F, F, 1, m->hx, st));
        if (w.f2.type == GGML_Q8_0) GSVK_TRY(launch_q8_quantize(m->hx, B, F, m->hq.q, m->hq.d, st));
        GSVK_TRY(proj_rows(w.f2, m->hx, m->hq.q, m->hq.d, B, m->h2, 0, st));
    }
    return decode_head(m, B, m->n1.x, m->h2, m->x, m->logits, st);
}

// The two-launch layer covers the shape and the weights it reads (tiled out / FFN2 copies, an
// F16 / F32 head).
bool fused_decode_ok(const gsvk_model * m) {
    if (m->generic || m->head_type == GGML_Q8_0 || !dec_layer_supported(m->B, m->NH, m->D, m->FFN, m->lstride))
        return false;
    for (const LayerW & w : m->L)
        if (!w.out.qt || !w.f2.qt) return false;
    return true;
}

// The persistent decode covers the shape: the two-launch layer's range up to 32 sequences, the device
// it assumes, no earlier failure, not in exact mode or a continuous-batching session.
bool persist_decode_ok(const gsvk_model * m) {
    return m->persist_dev_ok && !m->persist_failed && !m->exact && !m->cb_open && m->B <= DEC_PERSIST_MAX_BATCH &&
           m->NL <= 64 && fused_decode_ok(m);
}

// Before the decode steps of a run (outside any graph capture): the persistent decode's per-layer
// arguments for the current state uploaded and its barrier words cleared, when it will run.
int prepare_persist(gsvk_model * m) {
    m->persist_now = false;
    const bool want = m->decode_path == GSVK_DECODE_PERSIST ||
                      (m->decode_path == GSVK_DECODE_AUTO && m->B <= DEC_PERSIST_AUTO_MAX_BATCH);
    if (!want || !persist_decode_ok(m)) return GSVK_OK;
    if (!m->d_pattn) {
        GSVK_TRY(m->wmem.alloc(m->d_pattn, (size_t) m->NL));
        GSVK_TRY(m->wmem.alloc(m->d_pffn, (size_t) m->NL));
        GSVK_TRY(m->wmem.alloc(m->d_pflags, 8 * 32 + 2));   // flags, error word, step-active word
    }
    std::vector<DecAttnArgs> aa((size_t) m->NL);
    std::vector<DecFfnArgs> fa((size_t) m->NL);
    for (int li = 0; li < m->NL; li++) dec_layer_args(m, li, aa[(size_t) li], fa[(size_t) li]);
    GSVK_HIP(hipMemcpy(m->d_pattn, aa.data(), aa.size() * sizeof(DecAttnArgs), hipMemcpyHostToDevice));
    GSVK_HIP(hipMemcpy(m->d_pffn, fa.data(), fa.size() * sizeof(DecFfnArgs), hipMemcpyHostToDevice));
    GSVK_HIP(hipMemsetAsync(m->d_pflags, 0, (8 * 32 + 2) * sizeof(int), m->stream));
    GSVK_HIP(hipStreamSynchronize(m->stream));
    m->persist_now = true;
    return GSVK_OK;
}

// After a run on the persistent decode: its error word. Nonzero (a barrier wait gave up: the
// workgroups were not placed 32 per XCD, or one never ran): the run's results are not valid, the
// persistent decode is not used again by this model, and the caller repeats the run.
int persist_check(gsvk_model * m, bool * failed) {
    *failed = false;
    if (!m->persist_now) return GSVK_OK;
    int err = 0;
    GSVK_HIP(hipMemcpy(&err, m->d_pflags + 8 * 32, sizeof(int), hipMemcpyDeviceToHost));
    if (err != 0) {
        fprintf(stderr, "[gsvk] persistent decode failed (code %d): using the two-launch decode from now on\n", err);
        m->persist_failed = true;
        m->persist_now = false;
        *failed = true;
    }
    return GSVK_OK;
}

int enqueue_decode_body(gsvk_model * m) {
    if (m->generic) {
        GSVK_REQUIRE(m->decode_path == GSVK_DECODE_AUTO, "decode path %d: not available for a model with F16 / "
                     "F32 projections (it has its own per-op path)", m->decode_path);
        GSVK_REQUIRE(!m->exact || m->B < DECODE_GEMM_MIN_BATCH, "exact mode decodes up to %d sequences of a model "
                     "with F16 / F32 projections (got %d)", DECODE_GEMM_MIN_BATCH - 1, m->B);
        return enqueue_decode_generic(m);
    }
    if (m->exact) {
        // the GEMV chain in groups of at most GEMV_DECODE_MAX_BATCH rows, one group after another
        // (every kernel of it computes each row on its own, so a row's arithmetic is the same in
        // any group; each launch holds at most the rows the chain is tested at)
        for (int r0 = 0; r0 < m->B; r0 += GEMV_DECODE_MAX_BATCH)
            GSVK_TRY(enqueue_decode_rows(m, r0, std::min(GEMV_DECODE_MAX_BATCH, m->B - r0), m->stream));
        return GSVK_OK;
    }
    // an explicit choice runs as asked or fails: it never falls back to another path
    switch (m->decode_path) {
    case GSVK_DECODE_GEMV:
        GSVK_REQUIRE(m->B < DECODE_GEMM_MIN_BATCH, "decode path GEMV: %d sequences (it decodes at most %d)",
                     m->B, DECODE_GEMM_MIN_BATCH - 1);
        return enqueue_decode_rows(m, 0, m->B, m->stream);
    case GSVK_DECODE_FUSED:
        GSVK_REQUIRE(fused_decode_ok(m), "decode path FUSED: not available for %d sequences (at most %d) "
                     "or for this model (it needs an F16 or F32 head)", m->B, DEC_MAX_BATCH);
        return enqueue_decode_fused(m);
    case GSVK_DECODE_PERSIST:
        GSVK_REQUIRE(m->persist_now, "decode path PERSIST: not available (%d sequences, at most %d; it needs "
                     "the 256-CU gfx950 device, an F16 or F32 head, and no earlier failure; not in exact mode or "
                     "a continuous batch)", m->B, DEC_PERSIST_MAX_BATCH);
        return enqueue_decode_persist(m);
    case GSVK_DECODE_MFMA:
        return enqueue_decode_mfma(m);
    default:
        if (m->persist_now) return enqueue_decode_persist(m);
        if (m->B <= DEC_AUTO_MAX_BATCH && fused_decode_ok(m)) return enqueue_decode_fused(m);
        break;
    }
    if (m->B >= DECODE_GEMM_MIN_BATCH) return enqueue_decode_mfma(m);
    return enqueue_decode_rows(m, 0, m->B, m->stream);
}

}  // namespace

namespace {

// ---------------------------------------------------------------------------------------
// prefill
// ---------------------------------------------------------------------------------------

int check_requests(gsvk_model * m, const gsvk_request * reqs, int B) {
    GSVK_REQUIRE(reqs && B > 0, "no requests");
    const int P = reqs[0].n_prompt;
    GSVK_REQUIRE(P >= 0 && P <= PE_MAX, "prompt length %d out of range", P);
    for (int b = 0; b < B; b++) {
        const gsvk_request & r = reqs[b];
        GSVK_REQUIRE(r.n_prompt == P, "request %d: prompt length %d differs from %d (the batch "
                     "shares one prompt length)", b, r.n_prompt, P);
        GSVK_REQUIRE(r.n_phones >= 0 && r.n_phones <= PE_MAX, "request %d: %d phones out of range",
                     b, r.n_phones);
        GSVK_REQUIRE(r.n_phones == 0 || r.phones, "request %d: null phones", b);
        GSVK_REQUIRE(P == 0 || r.prompt, "request %d: null prompt", b);
        for (int t = 0; t < r.n_phones; t++)
            GSVK_REQUIRE(r.phones[t] >= 0 && r.phones[t] < m->PH, "request %d: phone id %d out of "
                         "range", b, r.phones[t]);
        for (int t = 0; t < P; t++)
            GSVK_REQUIRE(r.prompt[t] >= 0 && r.prompt[t] < m->V, "request %d: prompt code %d out "
                         "of range", b, r.prompt[t]);
    }
    return GSVK_OK;
}

// Prefill of B requests. Default: (re)allocates the cache and decode state for this batch and
// writes the K/V of request b to cache row b, columns [0, S). Slot mode (kv_slot >= 0, one
// request, a batch that sequences join while it decodes): writes the request's K/V to cache row
// kv_slot of the existing cache at columns [col0, col0 + S) and its logits to that row of the
// model's logits, leaving the rest of the model's state as it is.
int do_prefill(gsvk_model * m, const gsvk_request * reqs, int B, int lmax_needed, float * logits_host,
               int hist_len, int max_steps, int kv_slot = -1, int col0 = 0) {
    GSVK_TRY(check_requests(m, reqs, B));
    const auto t_build = std::chrono::steady_clock::now();
    const int P = reqs[0].n_prompt;
    int max_len = 0;
    for (int b = 0; b < B; b++) max_len = std::max(max_len, reqs[b].n_phones);
    const int S = max_len + P;
    GSVK_REQUIRE(S >= 1, "empty input (no phones and no prompt)");
    const int D = m->D, F = m->FFN, BD = m->BERT;
    const bool slot_mode = kv_slot >= 0;
    if (slot_mode) {
        GSVK_REQUIRE(B == 1 && m->kc && kv_slot < m->kv_B && col0 >= 0 && col0 + S <= m->lstride,
                     "prefill into slot %d at column %d: outside the cache", kv_slot, col0);
    } else {
        GSVK_TRY(alloc_kv(m, B, std::max(lmax_needed, S + 8)));
        GSVK_TRY(ensure_state(m, B, std::max(hist_len, P + 1), std::max(max_steps, 1)));
        m->prompt_len = P;
        m->S = S;
        m->max_len = max_len;
        m->B = B;
        m->host_step = 0;
        m->prefilled = false;
    }
    const size_t slot_off = slot_mode ? (size_t) kv_slot * m->NH * m->lstride * m->HD : 0;
    hipStream_t st = m->stream;

    // host-side packing of the requests
    std::vector<int32_t> phones((size_t) B * std::max(max_len, 1), 0), pad(B), tlen(B);
    std::vector<int32_t> row_b, row_t;
    std::vector<int64_t> boff(B, -1);
    size_t bert_total = 0;
    for (int b = 0; b < B; b++) {
        const gsvk_request & r = reqs[b];
        pad[b] = max_len - r.n_phones;
        tlen[b] = r.n_phones;
        for (int t = 0; t < r.n_phones; t++) phones[(size_t) b * max_len + pad[b] + t] = r.phones[t];
        if (r.bert && r.n_phones > 0) {
            boff[b] = (int64_t) bert_total;
            bert_total += (size_t) BD * r.n_phones;
        }
    }
    // text rows (b, t): the R1 rows of requests with BERT features first (they need the projection),
    // then the rows of requests without (their projection is the bias)
    for (int pass = 0; pass < 2; pass++)
        for (int b = 0; b < B; b++)
            if ((boff[b] >= 0) == (pass == 0))
                for (int t = 0; t < reqs[b].n_phones; t++) {
                    row_b.push_back(b);
                    row_t.push_back(t);
                }
    const int R = (int) row_b.size();
    int R1 = 0;
    while (R1 < R && boff[row_b[R1]] >= 0) R1++;
    const int64_t rows = (int64_t) B * S;

    PoolArena tmp;
    tmp.base = (char *) m->pf_pool;
    tmp.cap = m->pf_cap;
    int32_t * d_phones, * d_pad, * d_prompt, * d_rowb, * d_rowt, * d_tlen;
    int64_t * d_boff;
    float * d_bert = nullptr, * feat = nullptr, * proj = nullptr;
    GSVK_TRY(tmp.alloc(d_phones, phones.size()));
    GSVK_TRY(tmp.alloc(d_pad, B));
    GSVK_TRY(tmp.alloc(d_prompt, std::max(P, 1)));
    GSVK_TRY(tmp.alloc(d_rowb, std::max(R, 1)));
    GSVK_TRY(tmp.alloc(d_rowt, std::max(R, 1)));
    GSVK_TRY(tmp.alloc(d_tlen, B));
    GSVK_TRY(tmp.alloc(d_boff, B));
    m->prof.pf_build_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_build).count();
    GSVK_HIP(hipEventRecord(m->pf_ev[0], st));
    GSVK_TRY(upload(d_phones, phones.data(), phones.size() * 4, st));
    GSVK_TRY(upload(d_pad, pad.data(), (size_t) B * 4, st));
    // the attention's sequence order: fewest padding rows (longest) first
    std::vector<int32_t> order(B);
    for (int b = 0; b < B; b++) order[b] = b;
    std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return pad[a] < pad[c]; });
    int32_t * d_order;
    GSVK_TRY(tmp.alloc(d_order, B));
    GSVK_TRY(upload(d_order, order.data(), (size_t) B * 4, st));
    if (P) GSVK_TRY(upload(d_prompt, reqs[0].prompt, (size_t) P * 4, st));
    if (R) {
        GSVK_TRY(upload(d_rowb, row_b.data(), (size_t) R * 4, st));
        GSVK_TRY(upload(d_rowt, row_t.data(), (size_t) R * 4, st));
    }
    GSVK_TRY(upload(d_tlen, tlen.data(), (size_t) B * 4, st));
    GSVK_TRY(upload(d_boff, boff.data(), (size_t) B * 8, st));
    if (bert_total) {
        GSVK_TRY(tmp.alloc(d_bert, bert_total));
        for (int b = 0; b < B; b++)
            if (boff[b] >= 0)
                GSVK_TRY(upload(d_bert + boff[b], reqs[b].bert, (size_t) BD * reqs[b].n_phones * 4, st));
    }
    // activations of the prefill rows
    Act cur, attn, n1, hq;
    float * qkv, * o, * h2, * last, * lg;
    GSVK_TRY(tmp.alloc(cur.x, rows * D));
    GSVK_TRY(tmp.alloc(cur.q, rows * D));
    GSVK_TRY(tmp.alloc(cur.d, rows * D / 32));
    GSVK_TRY(tmp.alloc(attn.x, rows * D));
    GSVK_TRY(tmp.alloc(attn.q, rows * D));
    GSVK_TRY(tmp.alloc(attn.d, rows * D / 32));
    GSVK_TRY(tmp.alloc(n1.x, rows * D));
    GSVK_TRY(tmp.alloc(n1.q, rows * D));
    GSVK_TRY(tmp.alloc(n1.d, rows * D / 32));
    GSVK_TRY(tmp.alloc(hq.q, rows * F));
    GSVK_TRY(tmp.alloc(hq.d, rows * F / 32));
    GSVK_TRY(tmp.alloc(qkv, rows * 3 * D));
    GSVK_TRY(tmp.alloc(o, rows * D));
    GSVK_TRY(tmp.alloc(h2, rows * D));
    GSVK_TRY(tmp.alloc(last, (size_t) B * D));
    GSVK_TRY(tmp.alloc(lg, (size_t) B * m->V));

    GSVK_HIP(hipEventRecord(m->pf_ev[1], st));
    // inputs: xy, then + bert_aug . [feat; 1] on the text rows
    GSVK_TRY(launch_build_xy(m->text_emb, m->audio_emb, m->pe, d_phones, d_pad, d_prompt, B, S,
                             max_len, D, m->text_alpha, m->audio_alpha, cur.x, st));
    if (R1) {
        GSVK_TRY(tmp.alloc(feat, (size_t) R1 * (BD + 1)));
        GSVK_TRY(tmp.alloc(proj, (size_t) R1 * D));
        GSVK_TRY(launch_bert_feat(d_bert, d_boff, d_rowb, d_rowt, d_tlen, BD, R1, feat, st));
        GSVK_TRY(launch_fdot(m->bert_aug, 0, D, BD + 1, feat, BD + 1, R1, proj, D, 0, st));
    }
    if (R) GSVK_TRY(launch_add_proj(cur.x, proj, m->bert_b, d_rowb, d_rowt, d_pad, S, D, R, R1, st));
    // projections on the matrix-core GEMMs from GEMM_MIN_ROWS rows on, except in exact mode (the
    // GEMV chain in ggml-cpu's order and the sequential attention at any row count)
    const bool gemm = !m->exact && !m->generic && rows >= GEMM_MIN_ROWS;
    if (gemm && m->prefill_f16) GSVK_TRY(ensure_w16(m));
    // the layer-0 QKV reads this copy: natural order for the GEMM, sliced for the GEMV
    GSVK_TRY(launch_q8_quantize(cur.x, rows, D, cur.q, cur.d, st, gemm ? Q8_NATURAL : Q8_SLICED));
    int32_t * zero = nullptr;
    GSVK_TRY(tmp.alloc(zero, 1));
    GSVK_HIP(hipMemsetAsync(zero, 0, 4, st));
    const float scale = 1.0f / std::sqrt((float) m->HD);
    float * hx = nullptr;
    if (m->generic) GSVK_TRY(tmp.alloc(hx, rows * F));
    for (int li = 0; li < m->NL && m->generic; li++) {
        // F16 / F32 projections: one launch per op (the decode's enqueue_decode_generic over the
        // B * S rows), the projections in tinyBLAS order when S >= 2 as for the head; K/V of every
        // row, padding rows included, at columns [col0, col0 + S)
        const LayerW & w = m->L[li];
        const size_t loff = (size_t) li * m->kv_B * m->NH * m->lstride * m->HD + slot_off;
        const int mode = S >= 2 ? 1 : 0;
        if (li > 0) {
            const LayerW & p = m->L[li - 1];
            GSVK_TRY(launch_layernorm(n1.x, h2, p.f2.b, p.ln2, rows, D, 1e-5f, cur.x, cur.q, cur.d, st, Q8_SLICED,
                                      nullptr, d_pad, S));
        }
        GSVK_TRY(proj_rows(w.qkv, cur.x, cur.q, cur.d, rows, qkv, mode, st));
        GSVK_TRY(launch_bias_kv(qkv, w.qkv.b, rows, D, m->kc + loff, m->vc + loff, m->NH, m->lstride, S, zero, col0,
                                st));
        if (m->exact)
            GSVK_TRY(launch_attn_exact_prefill(qkv, B, S, max_len, d_pad, m->NH, D, scale, attn.x, nullptr, nullptr,
                                               st));
        else if (attn_prefill_uses_mfma(rows))
            GSVK_TRY(launch_attn_prefill_mfma(qkv, B, S, max_len, d_pad, m->NH, D, scale, attn.x, nullptr, nullptr,
                                              st, false, d_order, true));
        else
            GSVK_TRY(launch_attn_prefill(qkv, B, S, max_len, d_pad, m->NH, D, scale, attn.x, nullptr, nullptr, st));
        if (w.out.type == GGML_Q8_0) GSVK_TRY(launch_q8_quantize(attn.x, rows, D, attn.q, attn.d, st));
        GSVK_TRY(proj_rows(w.out, attn.x, attn.q, attn.d, rows, o, mode, st));
        GSVK_TRY(launch_layernorm(cur.x, o, w.out.b, w.ln1, rows, D, 1e-5f, n1.x, n1.q, n1.d, st, Q8_SLICED, nullptr,
                                  d_pad, S));
        GSVK_TRY(proj_rows(w.f1, n1.x, n1.q, n1.d, rows, hx, mode, st));
        GSVK_TRY(launch_add_act(hx, w.f1.b, rows * F, F, 1, hx, st));
        if (w.f2.type == GGML_Q8_0) GSVK_TRY(launch_q8_quantize(hx, rows, F, hq.q, hq.d, st));
        GSVK_TRY(proj_rows(w.f2, hx, hq.q, hq.d, rows, h2, mode, st));
    }
    for (int li = 0; li < m->NL && !m->generic; li++) {
        const LayerW & w = m->L[li];
        const size_t loff = (size_t) li * m->kv_B * m->NH * m->lstride * m->HD + slot_off;
        if (gemm) {
            // LN2 of the previous layer as its own launch, then the QKV GEMM on its Q8_0 copy; the
            // left-padding rows are normalised from zeros (the LayerNorm bias: finite K/V rows that
            // no query attends)
            if (li > 0) {
                const LayerW & p = m->L[li - 1];
                GSVK_TRY(launch_layernorm(n1.x, h2, p.f2.b, p.ln2, rows, D, 1e-5f, cur.x, cur.q, cur.d, st,
                                          Q8_NATURAL, nullptr, d_pad, S));
            }
            LayerOut qo = qkv_out(m, w, loff, qkv, 3 * D, S, zero, col0);
            qo.row_pad = d_pad;   // row tiles of left padding only: zeros, no K/V (never attended)
            GSVK_TRY(prefill_gemm(m, w.qkv, rows, cur.q, cur.d, qo, st));
        } else {
            LayerIn in{};
            if (li == 0) {
                in.mode = IN_Q8;
                in.xs = cur.q;
                in.xd = cur.d;
            } else {
                const LayerW & p = m->L[li - 1];
                in.mode = IN_LN;
                in.res = n1.x;
                in.r = h2;
                in.bias = p.f2.b;
                in.wb = p.ln2;
                in.out_x = cur.x;
            }
            GSVK_TRY(launch_layer_gemv(w.qkv.qs, w.qkv.d, 3 * D, D, rows, in,
                                       qkv_out(m, w, loff, qkv, 3 * D, S, zero, col0), st));
        }
        if (m->exact)
            GSVK_TRY(launch_attn_exact_prefill(qkv, B, S, max_len, d_pad, m->NH, D, scale, attn.x, attn.q,
                                               attn.d, st));
        else if (attn_prefill_uses_mfma(rows))
            GSVK_TRY(launch_attn_prefill_mfma(qkv, B, S, max_len, d_pad, m->NH, D, scale, attn.x, attn.q,
                                              attn.d, st, gemm && m->prefill_f16, d_order, true));
        else
            GSVK_TRY(launch_attn_prefill(qkv, B, S, max_len, d_pad, m->NH, D, scale, attn.x, attn.q,
                                         attn.d, st));
        GSVK_TRY(layer_tail(m, st, w, rows, cur.x, attn, o, n1.x, hq, h2, gemm ? &n1 : nullptr,
                            Q8_NATURAL, d_pad, S, true));
    }
    GSVK_TRY(final_ln(m, st, rows, n1.x, h2, cur));
    GSVK_TRY(launch_gather_last(cur.x, B, S, D, last, st));
    Act lastq;
    lastq.x = last;
    if (m->head_type == GGML_Q8_0) {
        GSVK_TRY(tmp.alloc(lastq.q, (size_t) B * D));
        GSVK_TRY(tmp.alloc(lastq.d, (size_t) B * D / 32));
        GSVK_TRY(launch_q8_quantize(last, B, D, lastq.q, lastq.d, st));
    }
    // llamafile's tinyBLAS handles the head when the prefill has >= 2 columns
    GSVK_TRY(head_logits(m, lastq, B, S >= 2 ? 1 : 0, lg, st));
    GSVK_HIP(hipEventRecord(m->pf_ev[2], st));
    GSVK_HIP(hipMemcpyAsync(m->logits + (slot_mode ? (size_t) kv_slot * m->V : 0), lg, (size_t) B * m->V * 4,
                            hipMemcpyDeviceToDevice, st));
    if (!slot_mode) GSVK_TRY(upload(m->kv_begin, pad.data(), (size_t) B * 4, st));
    if (logits_host)
        GSVK_HIP(hipMemcpyAsync(logits_host, lg, (size_t) B * m->V * 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipEventRecord(m->pf_ev[3], st));
    GSVK_HIP(hipStreamSynchronize(st));
    {
        float t[3] = {0, 0, 0};
        for (int i = 0; i < 3; i++) GSVK_HIP(hipEventElapsedTime(&t[i], m->pf_ev[i], m->pf_ev[i + 1]));
        m->prof.pf_copy_ms = t[0];
        m->prof.pf_compute_ms = t[1];
        m->prof.pf_io_ms = t[2];
    }
    if (tmp.need > m->pf_cap) {
        // grow the workspace for the next prefill of this size (nothing of it is in use now)
        if (m->pf_pool) (void) hipFree(m->pf_pool);
        m->pf_pool = nullptr;
        m->pf_cap = 0;
        if (hipMalloc(&m->pf_pool, tmp.need) == hipSuccess)
            m->pf_cap = tmp.need;
        else
            (void) hipGetLastError();   // not an error of this call: the next one allocates apart
    }
    if (!slot_mode) m->prefilled = true;
    return GSVK_OK;
}

}  // namespace

// ===========================================================================================
// C ABI
// ===========================================================================================

extern "C" int gsvk_device_count(int * n) {
    GSVK_REQUIRE(n, "null pointer");
    int c = 0;
    if (hipGetDeviceCount(&c) != hipSuccess) {
        (void) hipGetLastError();
        c = 0;
    }
    *n = c;
    return GSVK_OK;
}

extern "C" int gsvk_parse_device(const char * s, int * device) {
    GSVK_REQUIRE(device, "null pointer");
    const std::string d = s ? s : "";
    *device = 0;
    if (d == "cpu" || d == "CPU" || d == "CPUExecutionProvider") {
        set_error("device '%s': this build runs on HIP devices only", d.c_str());
        return GSVK_ERR_NODEV;
    }
    if (d.empty()) return GSVK_OK;
    const size_t colon = d.rfind(':');
    if (colon != std::string::npos) {
        *device = std::atoi(d.c_str() + colon + 1);
        return GSVK_OK;
    }
    if (d.find_first_not_of("0123456789") == std::string::npos) {
        *device = std::atoi(d.c_str());
        return GSVK_OK;
    }
    static const char * names[] = {"gpu", "GPU", "hip", "HIP", "rocm", "ROCm", "vulkan", "Vulkan",
                                   "cuda", "CUDA"};
    for (const char * nm : names)
        if (d == nm) return GSVK_OK;
    set_error("device '%s' not recognised", d.c_str());
    return GSVK_ERR_NODEV;
}

namespace {

struct Hparams {
    int D = 512, NH = 16, NL = 24, V = 1025, PH = 732, EOS = 1024, FFN = 2048;
    bool tiled = false;   // a pre-swizzled file: layer projections in the matrix-core order
};

// Key of a pre-swizzled GGUF (gsv.cpp_amd/gguf_tiled.py): 1 = every layer's Q8_0 projection
// `X` is stored as `X.qt` (I8, its quants in the Q8_TILED order) and `X.dt` (F16, its scales in
// the Q8_TILED order), all other tensors unchanged.
constexpr const char * KEY_Q8_LAYOUT = "gsvk.q8_layout";
constexpr uint32_t Q8_LAYOUT_TILED32 = 1;

// Check the whole tensor contract of tools/export_gguf/convert_ar.py (names, types, shapes) before
// anything touches the device, so a bad file fails the same way with or without a GPU.
int validate_gguf(const GgufFile & g, Hparams & hp) {
    uint32_t v;
    if (g.get_u32("ar.hidden_dim", v)) hp.D = (int) v;
    if (g.get_u32("ar.head", v)) hp.NH = (int) v;
    if (g.get_u32("ar.n_layer", v)) hp.NL = (int) v;
    if (g.get_u32("ar.vocab_size", v)) hp.V = (int) v;
    if (g.get_u32("ar.phoneme_vocab_size", v)) hp.PH = (int) v;
    if (g.get_u32("ar.eos", v)) hp.EOS = (int) v;
    if (hp.NH <= 0 || hp.D % hp.NH != 0 || hp.D != 512 || hp.D / hp.NH != 32) {
        set_error("unsupported shape d_model=%d heads=%d (this build: 512 = 16 x 32)", hp.D, hp.NH);
        return GSVK_ERR_FORMAT;
    }
    if (hp.V <= 0 || hp.V > 2048 || hp.EOS < 0 || hp.EOS >= hp.V || hp.NL <= 0 || hp.NL > 256 ||
        hp.PH <= 0) {
        set_error("bad hparams vocab=%d eos=%d layers=%d phones=%d", hp.V, hp.EOS, hp.NL, hp.PH);
        return GSVK_ERR_FORMAT;
    }
    if (g.get_u32(KEY_Q8_LAYOUT, v)) {
        if (v != Q8_LAYOUT_TILED32) {
            set_error("%s = %u: unknown weight layout (1 = tiled)", KEY_Q8_LAYOUT, v);
            return GSVK_ERR_FORMAT;
        }
        hp.tiled = true;
    }
    auto need = [&](const std::string & name, std::initializer_list<uint32_t> types,
                    std::initializer_list<int64_t> ne) -> int {
        const GgufTensor * t = g.tensor(name);
        if (!t) { set_error("missing tensor %s", name.c_str()); return GSVK_ERR_FORMAT; }
        bool ok = false;
        for (uint32_t ty : types) ok |= t->type == ty;
        if (!ok) { set_error("%s: unsupported type %u", name.c_str(), t->type); return GSVK_ERR_FORMAT; }
        int64_t nel = 1, want = 1;
        for (int64_t x : t->ne) nel *= x;
        for (int64_t x : ne) want *= x;
        if (nel != want || (ne.size() == 2 && (t->ne.size() < 2 || t->ne[0] != *ne.begin()))) {
            set_error("%s: shape does not match the model", name.c_str());
            return GSVK_ERR_FORMAT;
        }
        return GSVK_OK;
    };
    const GgufTensor * f1 = g.tensor(hp.tiled ? "transformer.block0.ffn1_w.qt" : "transformer.block0.ffn1_w");
    if (f1 && f1->ne.size() == 2) hp.FFN = (int) f1->ne[1];
    const int D = hp.D, F = hp.FFN;
    if (F <= 0 || F % 128 != 0) { set_error("ffn size %d must be a multiple of 128", F); return GSVK_ERR_FORMAT; }
    // a Q8_0 projection [n][k]: the GGUF tensor, or its tiled pair in a pre-swizzled file
    auto need_q8 = [&](const std::string & name, int64_t k, int64_t n) -> int {
        // F16 / F32 projections too (the reference exporter's attn= / ffn= options,
        // tools/export_gguf/export.py:53-54); a pre-swizzled file holds Q8_0 only
        if (!hp.tiled) return need(name, {GGML_Q8_0, GGML_F16, GGML_F32}, {k, n});
        GSVK_TRY(need(name + ".qt", {GGML_I8}, {k, n}));
        return need(name + ".dt", {GGML_F16}, {k / 32, n});
    };
    for (int li = 0; li < hp.NL; li++) {
        const std::string p = "transformer.block" + std::to_string(li) + ".";
        GSVK_TRY(need_q8(p + "qkv_w", D, 3 * D));
        GSVK_TRY(need_q8(p + "out_w", D, D));
        GSVK_TRY(need_q8(p + "ffn1_w", D, F));
        GSVK_TRY(need_q8(p + "ffn2_w", F, D));
        GSVK_TRY(need(p + "qkv_b", {GGML_F32}, {3 * D}));
        GSVK_TRY(need(p + "out_b", {GGML_F32}, {D}));
        GSVK_TRY(need(p + "ffn1_b", {GGML_F32}, {F}));
        GSVK_TRY(need(p + "ffn2_b", {GGML_F32}, {D}));
        for (const char * n : {"norm1_w", "norm1_b", "norm2_w", "norm2_b"}) GSVK_TRY(need(p + n, {GGML_F32}, {D}));
    }
    GSVK_TRY(need("ar.predict", {GGML_F32, GGML_F16, GGML_Q8_0}, {D, hp.V}));
    // host-read tensors must be F32 (src/gsv_ar.cpp:632-637)
    GSVK_TRY(need("ar.text_emb", {GGML_F32}, {D, hp.PH}));
    GSVK_TRY(need("ar.audio_emb", {GGML_F32}, {D, hp.V}));
    GSVK_TRY(need("ar.bert_proj", {GGML_F32}, {1024, D}));
    GSVK_TRY(need("ar.bert_proj_b", {GGML_F32}, {D}));
    GSVK_TRY(need("ar.text_pe_alpha", {GGML_F32}, {1}));
    GSVK_TRY(need("ar.audio_pe_alpha", {GGML_F32}, {1}));
    return GSVK_OK;
}

}  // namespace

extern "C" int gsvk_model_load(const char * path, int device, int verbose, gsvk_model ** out) {
    GSVK_REQUIRE(path && out, "null argument");
    *out = nullptr;
    GgufFile g;
    std::string err;
    bool io_error = false;
    if (!g.open(path, err, &io_error)) {
        set_error("%s", err.c_str());
        return io_error ? GSVK_ERR_IO : GSVK_ERR_FORMAT;
    }
    Hparams hp;
    GSVK_TRY(validate_gguf(g, hp));
    int ndev = 0;
    gsvk_device_count(&ndev);
    if (device < 0 || device >= ndev) {
        set_error("HIP device %d not found (%d visible)", device, ndev);
        return GSVK_ERR_NODEV;
    }
    DeviceGuard guard(device);
    std::unique_ptr<gsvk_model> m(new gsvk_model());
    m->device = device;
    m->verbose = verbose;
    GSVK_HIP(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    if (getenv("GSVK_NO_GRAPH")) m->use_graph = false;
    m->persist_dev_ok = !getenv("GSVK_NO_PERSIST") && dec_persist_device_ok(device);
    m->D = hp.D;
    m->NH = hp.NH;
    m->NL = hp.NL;
    m->V = hp.V;
    m->PH = hp.PH;
    m->EOS = hp.EOS;
    m->FFN = hp.FFN;
    m->HD = m->D / m->NH;
    // staging buffer for the largest Q8_0 tensor
    size_t staging_bytes = 0;
    for (const auto & t : g.tensors()) staging_bytes = std::max<size_t>(staging_bytes, t.nbytes);
    DevArena stage;
    uint8_t * staging = nullptr;
    GSVK_TRY(stage.alloc(staging, staging_bytes));
    std::vector<uint8_t> host;
    m->L.resize(m->NL);
    char nm[128];
    for (int li = 0; li < m->NL; li++) {
        LayerW & w = m->L[li];
        struct { const char * suffix; Lin * lin; int expect_n, expect_k; } q8s[] = {
            {"qkv_w", &w.qkv, 3 * m->D, m->D}, {"out_w", &w.out, m->D, m->D},
            {"ffn1_w", &w.f1, -1, m->D}, {"ffn2_w", &w.f2, m->D, -1}};
        for (auto & q : q8s) {
            snprintf(nm, sizeof nm, "transformer.block%d.%s", li, q.suffix);
            if (hp.tiled) {
                const GgufTensor * tq = g.tensor(std::string(nm) + ".qt");
                const GgufTensor * td = g.tensor(std::string(nm) + ".dt");
                if (!tq || !td) { set_error("missing tensor %s.qt / .dt", nm); return GSVK_ERR_FORMAT; }
                GSVK_TRY(load_q8_tiled(m.get(), g, tq, td, *q.lin, host));
            } else {
                const GgufTensor * t = g.tensor(nm);
                if (!t) { set_error("missing tensor %s", nm); return GSVK_ERR_FORMAT; }
                if (t->type == GGML_F16 || t->type == GGML_F32) {
                    // kept as stored: ggml_mul_mat multiplies F16 / F32 rows as they are
                    if (t->ne.size() != 2) { set_error("%s: expected a 2-D tensor", nm); return GSVK_ERR_FORMAT; }
                    q.lin->type = (int) t->type;
                    q.lin->k = (int) t->ne[0];
                    q.lin->n = (int) t->ne[1];
                    host.resize(t->nbytes);
                    if (!g.read(*t, host.data())) { set_error("read of %s failed", nm); return GSVK_ERR_IO; }
                    uint8_t * d = nullptr;
                    GSVK_TRY(m->wmem.alloc(d, t->nbytes));
                    GSVK_HIP(hipMemcpy(d, host.data(), t->nbytes, hipMemcpyHostToDevice));
                    q.lin->wf = d;
                    m->generic = true;
                } else {
                    GSVK_TRY(load_q8(m.get(), g, t, *q.lin, staging, staging_bytes, host));
                }
            }
            if ((q.expect_n >= 0 && q.lin->n != q.expect_n) || (q.expect_k >= 0 && q.lin->k != q.expect_k)) {
                set_error("%s: shape [%d, %d] does not match the model", nm, q.lin->n, q.lin->k);
                return GSVK_ERR_FORMAT;
            }
        }
        if (li == 0) m->FFN = w.f1.n;
        if (w.f1.n != m->FFN || w.f2.k != m->FFN) { set_error("layer %d: inconsistent FFN size", li); return GSVK_ERR_FORMAT; }
        struct { const char * suffix; float ** dst; int64_t n; } f32s[] = {
            {"qkv_b", &w.qkv.b, 3 * m->D}, {"out_b", &w.out.b, m->D}, {"ffn1_b", &w.f1.b, m->FFN},
            {"ffn2_b", &w.f2.b, m->D}};
        for (auto & f : f32s) {
            snprintf(nm, sizeof nm, "transformer.block%d.%s", li, f.suffix);
            GSVK_TRY(load_f32(m.get(), g, nm, f.n, *f.dst));
        }
        // LayerNorm [w; b] packs (src/gsv_ar.cpp:599-626)
        std::vector<float> wv, bv, pack(2 * (size_t) m->D);
        float * tmpd = nullptr;
        for (int which = 0; which < 2; which++) {
            snprintf(nm, sizeof nm, "transformer.block%d.norm%d_w", li, which + 1);
            GSVK_TRY(load_f32(m.get(), g, nm, m->D, tmpd, &wv));
            snprintf(nm, sizeof nm, "transformer.block%d.norm%d_b", li, which + 1);
            GSVK_TRY(load_f32(m.get(), g, nm, m->D, tmpd, &bv));
            std::copy(wv.begin(), wv.end(), pack.begin());
            std::copy(bv.begin(), bv.end(), pack.begin() + m->D);
            float *& dst = which == 0 ? w.ln1 : w.ln2;
            GSVK_TRY(m->wmem.alloc(dst, pack.size()));
            GSVK_HIP(hipMemcpy(dst, pack.data(), pack.size() * 4, hipMemcpyHostToDevice));
        }
    }
    // head (any of F32 / F16 / Q8_0)
    {
        const GgufTensor * t = g.tensor("ar.predict");
        if (!t) { set_error("missing tensor ar.predict"); return GSVK_ERR_FORMAT; }
        if (t->ne.size() != 2 || t->ne[0] != m->D || t->ne[1] != m->V) {
            set_error("ar.predict: shape does not match d_model x vocab");
            return GSVK_ERR_FORMAT;
        }
        m->head_type = (int) t->type;
        if (t->type == GGML_Q8_0) {
            GSVK_TRY(load_q8(m.get(), g, t, m->head_q8, staging, staging_bytes, host));
        } else if (t->type == GGML_F16 || t->type == GGML_F32) {
            host.resize(t->nbytes);
            if (!g.read(*t, host.data())) { set_error("read of ar.predict failed"); return GSVK_ERR_IO; }
            uint8_t * d = nullptr;
            GSVK_TRY(m->wmem.alloc(d, t->nbytes));
            GSVK_HIP(hipMemcpy(d, host.data(), t->nbytes, hipMemcpyHostToDevice));
            m->head = d;
        } else {
            set_error("ar.predict: unsupported type %u", t->type);
            return GSVK_ERR_FORMAT;
        }
    }
    // embeddings and BERT projection must be F32 (src/gsv_ar.cpp:632-637)
    GSVK_TRY(load_f32(m.get(), g, "ar.text_emb", (int64_t) m->PH * m->D, m->text_emb));
    GSVK_TRY(load_f32(m.get(), g, "ar.audio_emb", (int64_t) m->V * m->D, m->audio_emb));
    {
        std::vector<float> wv, bv;
        float * tmpd = nullptr;
        GSVK_TRY(load_f32(m.get(), g, "ar.bert_proj", (int64_t) m->D * m->BERT, tmpd, &wv));
        GSVK_TRY(load_f32(m.get(), g, "ar.bert_proj_b", m->D, tmpd, &bv));
        // bert_aug [D][BERT+1] = [W | b] (src/gsv_ar.cpp:647-656)
        std::vector<float> aug((size_t) m->D * (m->BERT + 1));
        for (int d = 0; d < m->D; d++) {
            std::copy(wv.begin() + (size_t) d * m->BERT, wv.begin() + (size_t) (d + 1) * m->BERT,
                      aug.begin() + (size_t) d * (m->BERT + 1));
            aug[(size_t) d * (m->BERT + 1) + m->BERT] = bv[d];
        }
        GSVK_TRY(m->wmem.alloc(m->bert_aug, aug.size()));
        GSVK_HIP(hipMemcpy(m->bert_aug, aug.data(), aug.size() * 4, hipMemcpyHostToDevice));
        GSVK_TRY(m->wmem.alloc(m->bert_b, bv.size()));
        GSVK_HIP(hipMemcpy(m->bert_b, bv.data(), bv.size() * 4, hipMemcpyHostToDevice));
    }
    {
        std::vector<float> a1, a2;
        float * tmpd = nullptr;
        GSVK_TRY(load_f32(m.get(), g, "ar.text_pe_alpha", 1, tmpd, &a1));
        GSVK_TRY(load_f32(m.get(), g, "ar.audio_pe_alpha", 1, tmpd, &a2));
        m->text_alpha = a1[0];
        m->audio_alpha = a2[0];
    }
    // PE table (impl::mk_pe, src/gsv_ar.cpp:173-181), same float expressions, host libm
    {
        std::vector<float> pe((size_t) PE_MAX * m->D);
        for (int pos = 0; pos < PE_MAX; pos++)
            for (int i = 0; i < m->D; i += 2) {
                const float div = std::exp((float) i * -(std::log(10000.0f) / (float) m->D));
                pe[(size_t) pos * m->D + i] = std::sin((float) pos * div);
                pe[(size_t) pos * m->D + i + 1] = std::cos((float) pos * div);
            }
        GSVK_TRY(m->wmem.alloc(m->pe, pe.size()));
        GSVK_HIP(hipMemcpy(m->pe, pe.data(), pe.size() * 4, hipMemcpyHostToDevice));
    }
    // xorshift64* jump tables for this vocabulary
    {
        m->rng_chunk = (m->V + 63) / 64;
        std::vector<uint64_t> jump(RNG_JUMP_WORDS), adv(RNG_ADV_WORDS);
        rng_tables(m->V, m->rng_chunk, jump.data(), adv.data());
        GSVK_TRY(m->wmem.alloc(m->rng_jump, jump.size()));
        GSVK_TRY(m->wmem.alloc(m->rng_adv, adv.size()));
        GSVK_HIP(hipMemcpy(m->rng_jump, jump.data(), jump.size() * 8, hipMemcpyHostToDevice));
        GSVK_HIP(hipMemcpy(m->rng_adv, adv.data(), adv.size() * 8, hipMemcpyHostToDevice));
    }
    GSVK_HIP(hipHostMalloc((void **) &m->h_pinned, 64, hipHostMallocDefault));
    GSVK_HIP(hipHostMalloc((void **) &m->h_unfinished, 64, hipHostMallocMapped | hipHostMallocCoherent));
    GSVK_HIP(hipHostGetDevicePointer((void **) &m->d_unfinished_host, m->h_unfinished, 0));
    for (hipEvent_t & e : m->step_ev) GSVK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (hipEvent_t & e : m->pf_ev) GSVK_HIP(hipEventCreate(&e));
    GSVK_HIP(hipStreamSynchronize(m->stream));
    if (verbose)
        fprintf(stderr, "[gsvk] loaded %s on HIP device %d: D=%d heads=%d layers=%d vocab=%d EOS=%d "
                        "ffn=%d head=%s\n", path, device, m->D, m->NH, m->NL, m->V, m->EOS, m->FFN,
                m->head_type == 0 ? "F32" : m->head_type == 1 ? "F16" : "Q8_0");
    *out = m.release();
    return GSVK_OK;
}

extern "C" void gsvk_model_free(gsvk_model * m) {
    if (!m) return;
    DeviceGuard guard(m->device);
    (void) hipStreamSynchronize(m->stream);
    delete m;
}

extern "C" int gsvk_model_get_info(const gsvk_model * m, gsvk_model_info * info) {
    GSVK_REQUIRE(m && info, "null argument");
    info->d_model = m->D;
    info->n_head = m->NH;
    info->head_dim = m->HD;
    info->n_layer = m->NL;
    info->vocab = m->V;
    info->eos = m->EOS;
    info->phone_vocab = m->PH;
    info->bert_dim = m->BERT;
    info->ffn_dim = m->FFN;
    info->head_type = m->head_type;
    info->text_alpha = m->text_alpha;
    info->audio_alpha = m->audio_alpha;
    info->prompt_len = m->prompt_len;
    info->kv_batch = m->kv_B;
    info->kv_lmax = m->kv_lmax;
    return GSVK_OK;
}

extern "C" int gsvk_kv_alloc(gsvk_model * m, int B, int lmax) {
    GSVK_REQUIRE(m && B > 0 && lmax > 0, "bad arguments");
    DeviceGuard guard(m->device);
    return alloc_kv(m, B, lmax);
}

extern "C" int gsvk_model_set_decode_path(gsvk_model * m, int path) {
    GSVK_REQUIRE(m, "null model");
    GSVK_REQUIRE(path >= GSVK_DECODE_AUTO && path <= GSVK_DECODE_PERSIST, "bad decode path %d", path);
    DeviceGuard guard(m->device);
    cb_drop(m);
    drop_graph(m);
    m->decode_path = path;
    return GSVK_OK;
}

extern "C" int gsvk_model_set_exact(gsvk_model * m, int on) {
    GSVK_REQUIRE(m, "null model");
    DeviceGuard guard(m->device);
    cb_drop(m);
    drop_graph(m);
    m->exact = on != 0;
    return GSVK_OK;
}

extern "C" int gsvk_model_set_prefill_f16(gsvk_model * m, int on) {
    GSVK_REQUIRE(m, "null model");
    DeviceGuard guard(m->device);
    m->prefill_f16 = on != 0;   // (the prefill builds no graph; the weight copies are made at its next call)
    return GSVK_OK;
}

extern "C" int gsvk_release_cache(gsvk_model * m) {
    GSVK_REQUIRE(m, "null model");
    DeviceGuard guard(m->device);
    cb_drop(m);
    GSVK_HIP(hipStreamSynchronize(m->stream));
    drop_graph(m);
    m->smem.release();
    m->s_B = 0;
    if (m->pf_pool) (void) hipFree(m->pf_pool);
    m->pf_pool = nullptr;
    m->pf_cap = 0;
    m->kvmem.release();
    m->kc = m->vc = nullptr;
    m->kv_B = m->kv_lmax = 0;
    m->prefilled = false;
    return GSVK_OK;
}

extern "C" int gsvk_first_logits(gsvk_model * m, const gsvk_request * reqs, int B, float * logits) {
    GSVK_REQUIRE(m && logits, "null argument");
    if (B == 0) return GSVK_OK;
    DeviceGuard guard(m->device);
    cb_drop(m);
    int max_len = 0;
    for (int b = 0; b < B; b++) max_len = std::max(max_len, reqs[b].n_phones);
    return do_prefill(m, reqs, B, max_len + (B > 0 ? reqs[0].n_prompt : 0) + 8, logits, 0, 1);
}

extern "C" int gsvk_prefill(gsvk_model * m, const gsvk_request * reqs, int B, float * logits,
                            int * S_out) {
    GSVK_REQUIRE(m, "null model");
    DeviceGuard guard(m->device);
    cb_drop(m);
    int max_len = 0;
    for (int b = 0; b < B && reqs; b++) max_len = std::max(max_len, reqs[b].n_phones);
    const int S = max_len + (B > 0 && reqs ? reqs[0].n_prompt : 0);
    // keep an existing larger cache of the same batch (src/gsv_ar.cpp:95)
    const int lmax = (m->kc && m->kv_B == B) ? std::max(m->kv_lmax, S + 8) : S + 8;
    GSVK_TRY(do_prefill(m, reqs, B, lmax, logits, 0, 1));
    if (S_out) *S_out = m->S;
    return GSVK_OK;
}

extern "C" int gsvk_decode_step(gsvk_model * m, const int32_t * last_tok, float * logits) {
    GSVK_REQUIRE(m && last_tok, "null argument");
    if (!m->prefilled || m->cb_open) { set_error("decode_step before prefill"); return GSVK_ERR_STATE; }
    DeviceGuard guard(m->device);
    const int B = m->B;
    if (m->S + m->host_step >= m->kv_lmax + 1 || m->prompt_len + m->host_step >= PE_MAX) {
        set_error("decode_step: KV cache or positional table full (step %d)", m->host_step);
        return GSVK_ERR_STATE;
    }
    for (int b = 0; b < B; b++)
        GSVK_REQUIRE(last_tok[b] >= 0 && last_tok[b] < m->V, "token %d out of range", last_tok[b]);
    hipStream_t st = m->stream;
    const int32_t step1 = m->host_step + 1;
    GSVK_TRY(upload(m->last_tok, last_tok, (size_t) B * 4, st));
    GSVK_TRY(upload(m->d_step, &step1, 4, st));
    GSVK_HIP(hipStreamSynchronize(st));   // the host values above live on this stack frame
    GSVK_TRY(prepare_persist(m));
    GSVK_TRY(enqueue_decode_body(m));
    {
        GSVK_HIP(hipStreamSynchronize(st));
        bool failed = false;
        GSVK_TRY(persist_check(m, &failed));
        if (failed) GSVK_TRY(enqueue_decode_body(m));   // the same step on the two-launch decode
    }
    if (logits) GSVK_HIP(hipMemcpyAsync(logits, m->logits, (size_t) B * m->V * 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipStreamSynchronize(st));
    m->host_step++;
    return GSVK_OK;
}

// ---------------------------------------------------------------------------------------
// A batch that sequences join and leave while it decodes (continuous batching)
// ---------------------------------------------------------------------------------------
//
// The batch decodes in lockstep over a shared KV column, as generate does; a request joins at
// loop index g (the next step) by a prefill of its own, written to a free cache row left-padded
// so that it ends at the shared column (kv_begin = max_prefill + g - S); its positions, EOS-mask
// window, step limit and early-stop rule count from g. Rows without a request are finished
// (fin_step >= 0) and take no part. Per row the arithmetic is that of a batch of its own.

extern "C" int gsvk_cb_open(gsvk_model * m, int capacity, int max_prefill, int max_steps, int prompt_len,
                            const gsvk_sampler_cfg * cfg, int early_stop_num, unsigned flags) {
    GSVK_REQUIRE(m && cfg, "null argument");
    GSVK_REQUIRE(capacity > 0 && capacity <= 65535 && max_prefill >= 1 && max_steps >= 1 &&
                     prompt_len >= 0 && prompt_len <= max_prefill && max_prefill <= PE_MAX,
                 "cb_open: bad shape (capacity %d, max_prefill %d, max_steps %d, prompt %d)", capacity,
                 max_prefill, max_steps, prompt_len);
    GSVK_REQUIRE(prompt_len + max_steps <= PE_MAX, "cb_open: prompt_len + max_steps = %d exceeds the "
                 "positional table (%d)", prompt_len + max_steps, PE_MAX);
    DeviceGuard guard(m->device);
    cb_drop(m);
    drop_graph(m);   // a generate's graphs (the session captures its own)
    const int hist_len = prompt_len + max_steps;
    GSVK_TRY(alloc_kv(m, capacity, max_prefill + max_steps + 8));
    GSVK_TRY(ensure_state(m, capacity, hist_len, max_steps));
    m->B = capacity;
    m->S = max_prefill;
    m->prompt_len = prompt_len;
    m->max_len = max_prefill - prompt_len;
    m->host_step = 0;
    GSVK_TRY(m->cbmem.alloc(m->row_start, capacity));
    GSVK_TRY(m->cbmem.alloc(m->row_max, capacity));
    hipStream_t st = m->stream;
    // every row starts empty: finished, no steps, an attention range of its own fresh key only
    const std::vector<int32_t> zero(capacity, 0), none(capacity, -1), begin(capacity, max_prefill),
        ny(capacity, prompt_len);
    const std::vector<uint64_t> one(capacity, 1);
    const int32_t step0 = 0;
    GSVK_TRY(upload(m->row_start, zero.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->row_max, zero.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->fin_step, zero.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->fin_kind, none.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->kv_begin, begin.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->ny, ny.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->last_tok, zero.data(), (size_t) capacity * 4, st));
    GSVK_TRY(upload(m->rng, one.data(), (size_t) capacity * 8, st));
    GSVK_TRY(upload(m->d_step, &step0, 4, st));
    GSVK_HIP(hipMemsetAsync(m->hist, 0, (size_t) capacity * hist_len * 4, st));
    GSVK_HIP(hipMemsetAsync(m->logits, 0, (size_t) capacity * m->V * 4, st));
    GSVK_HIP(hipStreamSynchronize(st));   // the host vectors above live on this stack frame

    SampleArgs & sa = m->cb_sa;
    sa = SampleArgs{};
    sa.logits = m->logits;
    sa.V = m->V;
    sa.eos = m->EOS;
    sa.B = capacity;
    sa.P = prompt_len;
    sa.hist = m->hist;
    sa.hist_stride = hist_len;
    sa.ny = m->ny;
    sa.fin_step = m->fin_step;
    sa.fin_kind = m->fin_kind;
    sa.rng = m->rng;
    sa.jump = m->rng_jump;
    sa.adv = m->rng_adv;
    sa.chunk = m->rng_chunk;
    sa.top_k = cfg->top_k;
    sa.top_p = cfg->top_p;
    sa.temperature = cfg->temperature;
    sa.rep = cfg->repetition_penalty;
    sa.step = m->d_step;
    sa.flags = ((flags & GSVK_GEN_EOS_MASK_ALL) ? 1u : 0u) | 2u;   // early stop per row
    sa.last_tok = m->last_tok;
    sa.max_steps = max_steps;
    sa.done_counter = m->done_counter;
    sa.n_unfinished = m->n_unfinished;
    sa.early_stop = early_stop_num;
    sa.row_start = m->row_start;
    sa.row_max = m->row_max;
    m->cb_open = true;
    m->persist_now = false;
    m->cb_smax = max_prefill;
    m->cb_steps = max_steps;
    m->cb_step = 0;
    m->cb_used.assign(capacity, 0);
    m->cb_start.assign(capacity, 0);
    m->cb_max.assign(capacity, 0);
    if (m->use_graph) {
        GSVK_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        int rc = launch_sample(sa, st);
        if (rc == GSVK_OK) rc = enqueue_decode_body(m);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc != GSVK_OK) {
            if (g) (void) hipGraphDestroy(g);
            cb_drop(m);
            return rc;
        }
        if (e != hipSuccess) {
            cb_drop(m);
            GSVK_HIP(e);
        }
        m->graph = g;
        GSVK_HIP(hipGraphInstantiate(&m->gexec, g, nullptr, nullptr, 0));
    }
    m->prefilled = true;
    return GSVK_OK;
}

extern "C" int gsvk_cb_add(gsvk_model * m, const gsvk_request * req, uint64_t seed, int max_steps,
                           int * slot_out) {
    GSVK_REQUIRE(m && req && slot_out, "null argument");
    if (!m->cb_open) { set_error("cb_add: no batch session is open"); return GSVK_ERR_STATE; }
    GSVK_REQUIRE(req->n_prompt == m->prompt_len, "cb_add: prompt length %d differs from the session's %d",
                 req->n_prompt, m->prompt_len);
    const int S = req->n_phones + req->n_prompt;
    GSVK_REQUIRE(S >= 1 && S <= m->cb_smax, "cb_add: %d prefill rows exceed the session's %d", S, m->cb_smax);
    GSVK_REQUIRE(max_steps >= 1 && m->cb_step + max_steps <= m->cb_steps,
                 "cb_add: %d steps from loop index %d exceed the session's %d", max_steps, m->cb_step,
                 m->cb_steps);
    int b = 0;
    while (b < m->B && m->cb_used[b]) b++;
    if (b == m->B) { set_error("cb_add: no free row (capacity %d)", m->B); return GSVK_ERR_STATE; }
    DeviceGuard guard(m->device);
    const int col0 = m->cb_smax + m->cb_step - S;
    GSVK_TRY(do_prefill(m, req, 1, 0, nullptr, 0, 0, b, col0));
    hipStream_t st = m->stream;
    const int P = m->prompt_len;
    const int32_t fin = -1, ny = P, last = P ? req->prompt[P - 1] : 0, start = m->cb_step, mx = max_steps;
    const uint64_t rng = seed ? seed : 1;   // gsv_rng: seed 0 -> 1
    GSVK_TRY(upload(m->kv_begin + b, &col0, 4, st));
    if (P) GSVK_TRY(upload(m->hist + (size_t) b * m->cb_sa.hist_stride, req->prompt, (size_t) P * 4, st));
    GSVK_TRY(upload(m->ny + b, &ny, 4, st));
    GSVK_TRY(upload(m->fin_step + b, &fin, 4, st));
    GSVK_TRY(upload(m->fin_kind + b, &fin, 4, st));
    GSVK_TRY(upload(m->last_tok + b, &last, 4, st));
    GSVK_TRY(upload(m->rng + b, &rng, 8, st));
    GSVK_TRY(upload(m->row_start + b, &start, 4, st));
    GSVK_TRY(upload(m->row_max + b, &mx, 4, st));
    GSVK_HIP(hipStreamSynchronize(st));   // the host values above live on this stack frame
    m->cb_used[b] = 1;
    m->cb_start[b] = start;
    m->cb_max[b] = mx;
    *slot_out = b;
    return GSVK_OK;
}

extern "C" int gsvk_cb_step(gsvk_model * m, int n_steps, int * n_running) {
    GSVK_REQUIRE(m, "null model");
    if (!m->cb_open) { set_error("cb_step: no batch session is open"); return GSVK_ERR_STATE; }
    GSVK_REQUIRE(n_steps >= 0 && m->cb_step + n_steps <= m->cb_steps,
                 "cb_step: %d steps from loop index %d exceed the session's %d", n_steps, m->cb_step,
                 m->cb_steps);
    DeviceGuard guard(m->device);
    hipStream_t st = m->stream;
    for (int i = 0; i < n_steps; i++) {
        if (m->gexec) {
            GSVK_HIP(hipGraphLaunch(m->gexec, st));
        } else {
            GSVK_TRY(launch_sample(m->cb_sa, st));
            GSVK_TRY(enqueue_decode_body(m));
        }
    }
    GSVK_HIP(hipMemcpyAsync(m->h_pinned, m->n_unfinished, 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipStreamSynchronize(st));
    m->cb_step += n_steps;
    if (n_running) *n_running = n_steps > 0 ? *m->h_pinned : -1;
    return GSVK_OK;
}

extern "C" int gsvk_cb_take(gsvk_model * m, int slot, int32_t * tokens, int capacity, int * n_tokens,
                            int * len, int * finished) {
    GSVK_REQUIRE(m && n_tokens && finished, "null argument");
    if (!m->cb_open) { set_error("cb_take: no batch session is open"); return GSVK_ERR_STATE; }
    GSVK_REQUIRE(slot >= 0 && slot < m->B && m->cb_used[slot], "cb_take: row %d holds no request", slot);
    DeviceGuard guard(m->device);
    hipStream_t st = m->stream;
    int32_t fin = -1, ny = 0;
    GSVK_HIP(hipMemcpyAsync(&fin, m->fin_step + slot, 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipMemcpyAsync(&ny, m->ny + slot, 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipStreamSynchronize(st));
    const int done_steps = m->cb_step - m->cb_start[slot];
    *finished = (fin >= 0 || done_steps >= m->cb_max[slot]) ? 1 : 0;
    *n_tokens = 0;
    if (len) *len = fin >= 0 ? fin : m->cb_max[slot];
    if (!*finished) return GSVK_OK;
    // as generate's result: the history minus the stopping token (EOS or early stop), or all of it
    const int n = fin >= 0 ? ny - 1 : ny;
    GSVK_REQUIRE(n >= 0 && n <= m->cb_sa.hist_stride, "cb_take: bad history length %d", n);
    if (tokens) {
        GSVK_REQUIRE(capacity >= n, "cb_take: %d tokens do not fit in %d", n, capacity);
        GSVK_HIP(hipMemcpyAsync(tokens, m->hist + (size_t) slot * m->cb_sa.hist_stride, (size_t) n * 4,
                                hipMemcpyDeviceToHost, st));
    }
    // the row leaves the batch: finished, no steps left
    const int32_t zero = 0;
    GSVK_TRY(upload(m->fin_step + slot, &zero, 4, st));
    GSVK_TRY(upload(m->row_max + slot, &zero, 4, st));
    GSVK_HIP(hipStreamSynchronize(st));
    *n_tokens = n;
    m->cb_used[slot] = 0;
    return GSVK_OK;
}

extern "C" int gsvk_cb_close(gsvk_model * m) {
    GSVK_REQUIRE(m, "null model");
    DeviceGuard guard(m->device);
    cb_drop(m);
    return GSVK_OK;
}

extern "C" int gsvk_kv_read(gsvk_model * m, int layer, uint16_t * k_out, uint16_t * v_out) {
    GSVK_REQUIRE(m && m->kc && layer >= 0 && layer < m->NL, "bad arguments");
    DeviceGuard guard(m->device);
    const size_t per = (size_t) m->kv_B * m->NH * m->lstride * m->HD;
    if (k_out) GSVK_HIP(hipMemcpyAsync(k_out, m->kc + per * layer, per * 2, hipMemcpyDeviceToHost, m->stream));
    if (v_out) GSVK_HIP(hipMemcpyAsync(v_out, m->vc + per * layer, per * 2, hipMemcpyDeviceToHost, m->stream));
    GSVK_HIP(hipStreamSynchronize(m->stream));
    return GSVK_OK;
}


extern "C" int gsvk_generate(gsvk_model * m, const gsvk_request * reqs, int B,
                             const gsvk_sampler_cfg * cfg, uint64_t seed_base, int early_stop_num,
                             int max_steps, const int32_t * oracle, int n_oracle,
                             const uint64_t * seeds, unsigned flags, gsvk_gen_out * out) {
    GSVK_REQUIRE(m && cfg && out, "null argument");
    if (B == 0) return GSVK_OK;
    GSVK_REQUIRE(reqs && B > 0 && max_steps >= 0, "bad arguments");
    GSVK_REQUIRE(out->tokens && out->tok_len && out->lens, "null output buffers");
    DeviceGuard guard(m->device);
    cb_drop(m);
    const int P = reqs[0].n_prompt;
    GSVK_REQUIRE(out->tok_stride >= P + max_steps, "tok_stride %d < prompt + max_steps (%d)",
                 out->tok_stride, P + max_steps);
    GSVK_REQUIRE(P + max_steps <= PE_MAX, "prompt_len + max_steps = %d exceeds the positional "
                 "table (%d)", P + max_steps, PE_MAX);
    GSVK_REQUIRE(!oracle || n_oracle >= 0, "bad oracle length");
    int max_len = 0;
    for (int b = 0; b < B; b++) max_len = std::max(max_len, reqs[b].n_phones);
    const int S = max_len + P;
    const int hist_len = P + max_steps;
    const auto t_pf = std::chrono::steady_clock::now();
    GSVK_TRY(do_prefill(m, reqs, B, S + max_steps + 8, nullptr, hist_len, max_steps));
    out->prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_pf).count();
    hipStream_t st = m->stream;
    const auto t_state = std::chrono::steady_clock::now();
    std::vector<int32_t> pad(B);
    for (int b = 0; b < B; b++) pad[b] = max_len - reqs[b].n_phones;
    // host state -> device
    std::vector<int32_t> hist((size_t) B * hist_len, 0), ny(B, P), fin(B, -1), kind(B, -1), last(B, 0);
    std::vector<uint64_t> rng(B);
    for (int b = 0; b < B; b++) {
        if (P) std::copy(reqs[b].prompt, reqs[b].prompt + P, hist.begin() + (size_t) b * hist_len);
        last[b] = P ? reqs[b].prompt[P - 1] : 0;
        const uint64_t sd = seeds ? seeds[b] : seed_base + 0x9E3779B9ull * (uint64_t) b;
        rng[b] = sd ? sd : 1;   // gsv_rng: seed 0 -> 1
    }
    const int32_t zero = 0;
    GSVK_TRY(upload(m->hist, hist.data(), hist.size() * 4, st));
    GSVK_TRY(upload(m->ny, ny.data(), (size_t) B * 4, st));
    GSVK_TRY(upload(m->fin_step, fin.data(), (size_t) B * 4, st));
    GSVK_TRY(upload(m->fin_kind, kind.data(), (size_t) B * 4, st));
    GSVK_TRY(upload(m->last_tok, last.data(), (size_t) B * 4, st));
    GSVK_TRY(upload(m->rng, rng.data(), (size_t) B * 8, st));
    GSVK_TRY(upload(m->d_step, &zero, 4, st));
    GSVK_TRY(upload(m->kv_begin, pad.data(), (size_t) B * 4, st));
    if (oracle && n_oracle > 0)
        GSVK_TRY(upload(m->oracle, oracle, (size_t) std::min(n_oracle, max_steps) * 4, st));
    GSVK_HIP(hipMemsetAsync(m->sampled, 0xff, (size_t) std::max(max_steps, 1) * B * 4, st));
    GSVK_HIP(hipStreamSynchronize(st));
    const auto t_graph = std::chrono::steady_clock::now();
    m->prof.dec_copy_ms = std::chrono::duration<double, std::milli>(t_graph - t_state).count();

    // one step = sampler (loop index idx) + decode at idx; the graph is replayed max_steps times
    SampleArgs sa{};
    sa.logits = m->logits;
    sa.V = m->V;
    sa.eos = m->EOS;
    sa.B = B;
    sa.P = P;
    sa.hist = m->hist;
    sa.hist_stride = hist_len;
    sa.ny = m->ny;
    sa.fin_step = m->fin_step;
    sa.fin_kind = m->fin_kind;
    sa.rng = m->rng;
    sa.jump = m->rng_jump;
    sa.adv = m->rng_adv;
    sa.chunk = m->rng_chunk;
    sa.top_k = cfg->top_k;
    sa.top_p = cfg->top_p;
    sa.temperature = cfg->temperature;
    sa.rep = cfg->repetition_penalty;
    sa.oracle = (oracle && n_oracle > 0) ? m->oracle : nullptr;
    sa.n_oracle = std::min(n_oracle, max_steps);
    sa.step = m->d_step;
    sa.flags = (flags & GSVK_GEN_EOS_MASK_ALL) ? 1u : 0u;
    sa.last_tok = m->last_tok;
    sa.probs_dump = (flags & GSVK_GEN_PROB_DUMP) ? m->probs_dump : nullptr;
    sa.probs_per_row = 0;
    sa.tok_out = nullptr;
    sa.sampled_dump = m->sampled;
    sa.max_steps = max_steps;
    sa.done_counter = m->done_counter;
    sa.n_unfinished = m->n_unfinished;
    sa.n_unfinished_host = m->d_unfinished_host;
    sa.early_stop = early_stop_num;
    auto enqueue_step = [&]() -> int {
        GSVK_TRY(launch_sample(sa, st));
        GSVK_TRY(enqueue_decode_body(m));
        return GSVK_OK;
    };
    drop_graph(m);
    GSVK_TRY(prepare_persist(m));
    // On the persistent decode a launch holds GEN_STEPS_PER_LAUNCH steps (a graph launch after
    // another costs ~13 us of idle GPU, a kernel boundary inside a graph ~1.5 us), and the steps
    // that run after the last row finished skip the persistent kernel: each step's sampler records
    // whether any row took part (the count before it was nonzero) and the kernel reads that.
    struct GateReset {
        gsvk_model * m;
        ~GateReset() { m->persist_gate = false; }
    } gate_reset{m};
    m->persist_gate = m->persist_now;
    sa.active = m->persist_gate ? m->d_pflags + 8 * 32 + 1 : nullptr;
    const int K = (m->use_graph && m->persist_now && max_steps >= GEN_STEPS_PER_LAUNCH) ? GEN_STEPS_PER_LAUNCH : 1;
    auto capture = [&](int nsteps, hipGraph_t & graph, hipGraphExec_t & gexec) -> int {
        GSVK_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        int rc = GSVK_OK;
        for (int k = 0; k < nsteps && rc == GSVK_OK; k++) rc = enqueue_step();
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc != GSVK_OK) { if (g) (void) hipGraphDestroy(g); return rc; }
        GSVK_HIP(e);
        graph = g;
        GSVK_HIP(hipGraphInstantiate(&gexec, g, nullptr, nullptr, 0));
        return GSVK_OK;
    };
    if (m->use_graph && max_steps > 1) {
        GSVK_TRY(capture(1, m->graph, m->gexec));
        if (K > 1) GSVK_TRY(capture(K, m->graph_k, m->gexec_k));
    }
    // the count before the first step: every row
    GSVK_HIP(hipMemcpyAsync(m->n_unfinished, &B, sizeof(int32_t), hipMemcpyHostToDevice, st));
    // Completion: STEPS_IN_FLIGHT launches are queued ahead of the one whose count the host reads.
    // Before a launch the host waits for the launch STEPS_IN_FLIGHT before it to end (the GPU
    // still has the ones after it queued) and reads the unfinished count its last sampler stored
    // in pinned memory; 0 ends the loop. At most STEPS_IN_FLIGHT * K - 1 steps run after the one
    // where the last sequence finished (they sample nothing: every row is closed; on the
    // persistent decode their decoder kernel returns at once). The steps of a launch never pass
    // max_steps (the last max_steps % K go one per launch).
    constexpr int STEPS_IN_FLIGHT = 2;
    int launch_steps[STEPS_IN_FLIGHT] = {0, 0};
    *(volatile int32_t *) m->h_unfinished = B;
    int ticked = 0;   // progress callbacks so far: one per step known to have run for a sequence
    auto tick = [&]() {
        if (out->progress) out->progress(out->progress_user, ticked);
        ticked++;
    };
    GSVK_HIP(hipStreamSynchronize(st));
    const auto t_dec = std::chrono::steady_clock::now();
    m->prof.dec_build_ms = std::chrono::duration<double, std::milli>(t_dec - t_graph).count();
    for (int idx = 0, li = 0; idx < max_steps; li++) {
        hipEvent_t & ev = m->step_ev[li % STEPS_IN_FLIGHT];
        if (li >= STEPS_IN_FLIGHT) {
            GSVK_HIP(hipEventSynchronize(ev));
            if (*(volatile int32_t *) m->h_unfinished == 0) break;
            // the steps of launch li - STEPS_IN_FLIGHT ran with sequences still open
            for (int k = 0; k < launch_steps[li % STEPS_IN_FLIGHT]; k++) tick();
        }
        const int ks = (m->gexec_k && max_steps - idx >= K) ? K : 1;
        if (ks > 1) GSVK_HIP(hipGraphLaunch(m->gexec_k, st));
        else if (m->gexec) GSVK_HIP(hipGraphLaunch(m->gexec, st));
        else GSVK_TRY(enqueue_step());
        GSVK_HIP(hipEventRecord(ev, st));
        launch_steps[li % STEPS_IN_FLIGHT] = ks;
        idx += ks;
    }
    GSVK_HIP(hipStreamSynchronize(st));
    out->decode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_dec).count();
    {
        bool failed = false;
        GSVK_TRY(persist_check(m, &failed));
        if (failed)   // the run again, on the two-launch decode (prefill included: the cache was written)
            return gsvk_generate(m, reqs, B, cfg, seed_base, early_stop_num, max_steps, oracle, n_oracle, seeds,
                                 flags, out);
    }
    m->prof.dec_compute_ms = out->decode_ms;
    const auto t_res = std::chrono::steady_clock::now();
    // results
    GSVK_HIP(hipMemcpy(hist.data(), m->hist, hist.size() * 4, hipMemcpyDeviceToHost));
    GSVK_HIP(hipMemcpy(ny.data(), m->ny, (size_t) B * 4, hipMemcpyDeviceToHost));
    GSVK_HIP(hipMemcpy(fin.data(), m->fin_step, (size_t) B * 4, hipMemcpyDeviceToHost));
    GSVK_HIP(hipMemcpy(kind.data(), m->fin_kind, (size_t) B * 4, hipMemcpyDeviceToHost));
    struct Fin { int step, kind, b; };
    std::vector<Fin> order;
    int last_fin = -1;
    bool all = true;
    for (int b = 0; b < B; b++) {
        const int nb = ny[b];
        std::copy(hist.begin() + (size_t) b * hist_len, hist.begin() + (size_t) b * hist_len + nb,
                  out->tokens + (size_t) b * out->tok_stride);
        if (fin[b] >= 0) {
            out->tok_len[b] = nb - 1;   // minus the stopping token
            order.push_back({fin[b], kind[b], b});
            last_fin = std::max(last_fin, fin[b]);
        } else {
            out->tok_len[b] = nb;
            order.push_back({max_steps, 2, b});
            all = false;
        }
    }
    std::stable_sort(order.begin(), order.end(), [](const Fin & x, const Fin & y) {
        return x.step != y.step ? x.step < y.step : (x.kind != y.kind ? x.kind < y.kind : x.b < y.b);
    });
    for (int i = 0; i < B; i++) {
        out->lens[i] = order[i].step;
        if (out->finish_seq) out->finish_seq[i] = order[i].b;
    }
    out->n_steps = all ? last_fin + 1 : max_steps;
    while (ticked < out->n_steps) tick();
    if ((flags & GSVK_GEN_PROB_DUMP) && out->probs0 && out->n_steps > 0)
        GSVK_HIP(hipMemcpy(out->probs0, m->probs_dump, (size_t) out->n_steps * m->V * 4,
                           hipMemcpyDeviceToHost));
    m->prof.dec_other_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_res).count();
    m->prof.steps = out->n_steps;
    return GSVK_OK;
}

extern "C" int gsvk_model_time_decode_kernel(gsvk_model * m, int launches, float * ms_per_launch) {
    GSVK_REQUIRE(m && ms_per_launch && launches >= 1 && launches <= 100000, "bad arguments");
    if (!m->prefilled || m->cb_open) {
        set_error("time_decode_kernel: no decode state (prefill or generate first; not in a continuous batch)");
        return GSVK_ERR_STATE;
    }
    DeviceGuard guard(m->device);
    GSVK_TRY(prepare_persist(m));
    GSVK_REQUIRE(m->persist_now, "time_decode_kernel: the persistent decode does not run for this model and "
                 "batch (%d sequences) on the current decode path", m->B);
    hipStream_t st = m->stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    GSVK_HIP(hipEventCreate(&e0));
    if (hipEventCreate(&e1) != hipSuccess) {
        (void) hipEventDestroy(e0);
        set_error("time_decode_kernel: hipEventCreate failed");
        return GSVK_ERR_HIP;
    }
    DecPersistArgs pa = persist_args(m);
    int rc = hipEventRecord(e0, st) == hipSuccess ? GSVK_OK : GSVK_ERR_HIP;
    for (int i = 0; i < launches && rc == GSVK_OK; i++) {
        pa.epoch_add = i;   // flags were cleared: every launch's epoch above the last's
        rc = launch_dec_persist(pa, st);
    }
    float ms = 0.0f;
    if (rc == GSVK_OK && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                          hipEventElapsedTime(&ms, e0, e1) != hipSuccess)) {
        set_error("time_decode_kernel: event timing failed");
        rc = GSVK_ERR_HIP;
    }
    (void) hipStreamSynchronize(st);
    (void) hipEventDestroy(e0);
    (void) hipEventDestroy(e1);
    GSVK_TRY(rc);
    int err = 0;
    GSVK_HIP(hipMemcpy(&err, m->d_pflags + 8 * 32, sizeof(int), hipMemcpyDeviceToHost));
    if (err != 0) {
        set_error("time_decode_kernel: a barrier wait of the persistent decode gave up (code %d)", err);
        return GSVK_ERR_STATE;
    }
    *ms_per_launch = ms / (float) launches;
    return GSVK_OK;
}

extern "C" int gsvk_model_get_profile(gsvk_model * m, gsvk_profile * out) {
    GSVK_REQUIRE(m && out, "null argument");
    *out = m->prof;
    return GSVK_OK;
}

// Sampled-token dump of the last generate ([n_steps][B], -1 where a sequence had finished).
extern "C" int gsvk_last_sampled(gsvk_model * m, int n_steps, int32_t * out) {
    GSVK_REQUIRE(m && out && n_steps >= 0 && n_steps <= m->s_steps, "bad arguments");
    DeviceGuard guard(m->device);
    if (n_steps == 0) return GSVK_OK;
    GSVK_HIP(hipMemcpy(out, m->sampled, (size_t) n_steps * m->s_B * 4, hipMemcpyDeviceToHost));
    return GSVK_OK;
}

// BERT text encoder for gfx950: gsv_bert (src/gsv_bert.{h,cpp}), the chinese-roberta-wwm-ext-large
// encoder whose features feed the AR prefill (the `bert` input of a request).
//
// Forward (src/gsv_bert.cpp:128-155), post-LN as HF BertLayer, over the first layers_used layers:
//   x   = LN_emb(word[id] + pos[t] + type[0])
//   qkv = Wqkv . x + bqkv                         (one projection, rows q | k | v)
//   a   = softmax(q_h . k_h^T / sqrt(HD)) . v_h   per head, over the tokens of the same sequence
//   x   = LN1(x + Wo . a + bo)
//   x   = LN2(x + W2 . gelu_erf(W1 . x + b1) + b2)
// Output [hidden][T] row-major per sequence (src/gsv_bert.cpp:220-228).
//
// Design: rows of all sequences packed back to back (no padding rows); the projections are
// GEMMs on rocBLAS: F32 weights in fp32 (ggml-cpu's F32 x F32 product), F16 weights kept in fp16
// with the activations rounded to fp16 and fp32 sums (ggml-cpu converts the activations to the
// weights' F16 dot type), Q8_0 weight files widened to fp32 at load; bias,
// GELU and the residual LayerNorms are this library's kernels (norm.hip); attention is
// k_bert_attn below: one workgroup per 16 queries of one (sequence, head), four lanes per query
// (a quarter of the head dims each), keys and values staged through LDS in tiles of 64 whose 4
// chunks of 16 keys go to its 4 waves (online softmax each, merged at the end), fp32 throughout.
#include <rocblas/rocblas.h>

#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "gguf.h"
#include "gsvk.h"

namespace gsvk {

namespace {

constexpr int BA_HD = 64;   // head dim of the kernels below (BERT-large: 1024 / 16)
constexpr int BA_KT = 64;   // keys per LDS tile
constexpr int BA_CH = 16;   // keys per softmax chunk
constexpr int BA_Q = 16;    // queries per workgroup (4 lanes per query in each of its 4 waves)

// x[r] = word[id_r] + pos[t_r] + type0 (the sum order of src/gsv_bert.cpp:141-144); one
// workgroup of 256 threads per row, 4 values per thread and pass.
__global__ void __launch_bounds__(256) k_bert_embed(const float * __restrict__ word,
                                                    const float * __restrict__ pos,
                                                    const float * __restrict__ type0,
                                                    const int32_t * __restrict__ ids,
                                                    const int32_t * __restrict__ tpos, int D,
                                                    float * __restrict__ x) {
    const int64_t r = blockIdx.x;
    const float4 * w = reinterpret_cast<const float4 *>(word + (int64_t) ids[r] * D);
    const float4 * p = reinterpret_cast<const float4 *>(pos + (int64_t) tpos[r] * D);
    const float4 * t = reinterpret_cast<const float4 *>(type0);
    float4 * y = reinterpret_cast<float4 *>(x + r * D);
    for (int i = threadIdx.x; i < D / 4; i += 256) {
        const float4 a = w[i], b = p[i], c = t[i];
        y[i] = make_float4((a.x + b.x) + c.x, (a.y + b.y) + c.y, (a.z + b.z) + c.z, (a.w + b.w) + c.w);
    }
}

// Attention of one (sequence b, head h) for queries [16 * blockIdx.x, +16). Workgroup = 4 waves
// over the same 16 queries; in each wave lane = 4 * query + quarter, the quarter c holding dims
// [16c, 16c + 16) of the query and of its output (a score is the sum of the 4 quarters' partial
// dots, exchanged within the lane quad on DPP). Keys and values (plus their bias: the QKV bias
// is added here, as the projection's epilogue would) are staged through LDS in tiles of 64; wave
// w takes the chunk of 16 keys w of each tile with an online softmax in log2 units (the
// hardware exp2), and the 4 waves' (m, l, o) are merged through LDS at the end. The sequence's
// rows are [off_b, off_b + len_b) of qkv (row stride 3D: q | k | v, head h at 64h); every query
// sees every key of its sequence (the block-diagonal mask of src/gsv_bert.cpp:289-296). Output
// rows of queries past len_b are not written.
__global__ void __launch_bounds__(256) k_bert_attn(const float * __restrict__ qkv,
                                                   const float * __restrict__ qkv_b,
                                                   const int32_t * __restrict__ seq_off,
                                                   const int32_t * __restrict__ seq_len, int D,
                                                   float scale_log2, float * __restrict__ out,
                                                   _Float16 * __restrict__ out16) {
    const int h = blockIdx.y, b = blockIdx.z;
    const int len = seq_len[b];
    const int64_t off = seq_off[b];
    const int q0 = blockIdx.x * BA_Q;
    if (q0 >= len) return;   // uniform over the workgroup
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int qq = lane >> 2, c = lane & 3;
    const int64_t rs = 3 * (int64_t) D;
    const int qi = min(q0 + qq, len - 1);

    __shared__ float4 ks[BA_KT][BA_HD / 4];
    __shared__ float4 vs[BA_KT][BA_HD / 4];
    __shared__ float s_ml[4][64][2];
    __shared__ float4 s_o[4][64][4];

    float q[16];
    {
        const float4 * qp = reinterpret_cast<const float4 *>(qkv + (off + qi) * rs + h * BA_HD + 16 * c);
        const float4 * qb = reinterpret_cast<const float4 *>(qkv_b + h * BA_HD + 16 * c);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = qp[i], bb = qb[i];
            q[4 * i] = v.x + bb.x; q[4 * i + 1] = v.y + bb.y; q[4 * i + 2] = v.z + bb.z; q[4 * i + 3] = v.w + bb.w;
        }
    }
    const float4 * kbias = reinterpret_cast<const float4 *>(qkv_b + D + h * BA_HD);
    const float4 * vbias = reinterpret_cast<const float4 *>(qkv_b + 2 * D + h * BA_HD);
    float o[16];
#pragma unroll
    for (int d = 0; d < 16; d++) o[d] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    for (int k0 = 0; k0 < len; k0 += BA_KT) {
        __syncthreads();   // the previous tile has been read
        // 64 keys x 16 float4 of K and of V: 16 consecutive threads read one key's 256 bytes
#pragma unroll
        for (int r = 0; r < BA_KT * (BA_HD / 4) / 256; r++) {
            const int idx = r * 256 + tid, key = idx >> 4, part = idx & 15;
            const int kr = min(k0 + key, len - 1);   // keys past the end repeat the last (unused)
            const float * row = qkv + (off + kr) * rs + h * BA_HD + 4 * part;
            const float4 kv = *reinterpret_cast<const float4 *>(row + D), kb = kbias[part];
            const float4 vv = *reinterpret_cast<const float4 *>(row + 2 * D), vb = vbias[part];
            ks[key][part] = make_float4(kv.x + kb.x, kv.y + kb.y, kv.z + kb.z, kv.w + kb.w);
            vs[key][part] = make_float4(vv.x + vb.x, vv.y + vb.y, vv.z + vb.z, vv.w + vb.w);
        }
        __syncthreads();
        const int nk = min(BA_KT, len - k0);
        const int c0 = wave * BA_CH;   // this wave's chunk of the tile
        if (c0 < nk) {                 // uniform per wave
            float s[BA_CH];
            float cmax = -INFINITY;
#pragma unroll
            for (int j = 0; j < BA_CH; j++) {
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 kk = ks[c0 + j][4 * c + i];
                    dot = __builtin_fmaf(q[4 * i], kk.x, dot);
                    dot = __builtin_fmaf(q[4 * i + 1], kk.y, dot);
                    dot = __builtin_fmaf(q[4 * i + 2], kk.z, dot);
                    dot = __builtin_fmaf(q[4 * i + 3], kk.w, dot);
                }
                dot += dpp_f<DPP_XOR1>(dot);   // the quad's 4 quarters (lanes ^1, ^2)
                dot += dpp_f<DPP_XOR2>(dot);
                s[j] = c0 + j < nk ? dot * scale_log2 : -INFINITY;
                cmax = fmaxf(cmax, s[j]);
            }
            const float mn = fmaxf(m, cmax);                  // finite: the chunk has a key
            const float f = __builtin_amdgcn_exp2f(m - mn);   // 0 on the first chunk (m = -inf)
            l *= f;
#pragma unroll
            for (int d = 0; d < 16; d++) o[d] *= f;
            m = mn;
#pragma unroll
            for (int j = 0; j < BA_CH; j++) {
                const float p = __builtin_amdgcn_exp2f(s[j] - mn);   // masked keys: exp2(-inf) = 0
                l += p;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 vv = vs[c0 + j][4 * c + i];
                    o[4 * i] = __builtin_fmaf(p, vv.x, o[4 * i]);
                    o[4 * i + 1] = __builtin_fmaf(p, vv.y, o[4 * i + 1]);
                    o[4 * i + 2] = __builtin_fmaf(p, vv.z, o[4 * i + 2]);
                    o[4 * i + 3] = __builtin_fmaf(p, vv.w, o[4 * i + 3]);
                }
            }
        }
    }
    // merge the 4 waves (a wave that saw no key has m = -inf and weight 0)
    s_ml[wave][lane][0] = m;
    s_ml[wave][lane][1] = l;
#pragma unroll
    for (int i = 0; i < 4; i++) s_o[wave][lane][i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    __syncthreads();
    if (wave != 0 || q0 + qq >= len) return;
    float M = s_ml[0][lane][0];
#pragma unroll
    for (int w = 1; w < 4; w++) M = fmaxf(M, s_ml[w][lane][0]);
    float L = 0.0f, O[16];
#pragma unroll
    for (int d = 0; d < 16; d++) O[d] = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float mw = s_ml[w][lane][0];
        const float f = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
        L = __builtin_fmaf(s_ml[w][lane][1], f, L);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 ow = s_o[w][lane][i];
            O[4 * i] = __builtin_fmaf(ow.x, f, O[4 * i]);
            O[4 * i + 1] = __builtin_fmaf(ow.y, f, O[4 * i + 1]);
            O[4 * i + 2] = __builtin_fmaf(ow.z, f, O[4 * i + 2]);
            O[4 * i + 3] = __builtin_fmaf(ow.w, f, O[4 * i + 3]);
        }
    }
    const float inv = 1.0f / L;
    const int64_t o0 = (off + q0 + qq) * (int64_t) D + h * BA_HD + 16 * c;
    if (out16) {   // the fp16 input of an F16 out projection
#pragma unroll
        for (int d = 0; d < 16; d++) out16[o0 + d] = (_Float16) (O[d] * inv);
        return;
    }
    float4 * op = reinterpret_cast<float4 *>(out + o0);
#pragma unroll
    for (int i = 0; i < 4; i++)
        op[i] = make_float4(O[4 * i] * inv, O[4 * i + 1] * inv, O[4 * i + 2] * inv, O[4 * i + 3] * inv);
}

// h = gelu_erf(h + b[col]) (the add_act of src/gsv_bert.cpp:151-153, as norm.hip's k_add_act),
// stored in place in fp32, or to h16 in fp16 (the input of an F16 FFN2) when h16 is given
__global__ void __launch_bounds__(256) k_bias_gelu(float * __restrict__ h, const float * __restrict__ b,
                                                   int64_t rows, int F, _Float16 * __restrict__ h16) {
    const int64_t i = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= rows * F) return;   // F % 4 == 0: a thread's 4 values share a row
    const float4 v = *reinterpret_cast<const float4 *>(h + i);
    const float4 bb = *reinterpret_cast<const float4 *>(b + i % F);
    const float x[4] = {v.x + bb.x, v.y + bb.y, v.z + bb.z, v.w + bb.w};
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; k++) y[k] = 0.5f * x[k] * (1.0f + erff(x[k] * 0.70710678118654752440f));
    if (h16) {
#pragma unroll
        for (int k = 0; k < 4; k++) h16[i + k] = (_Float16) y[k];
    } else {
        *reinterpret_cast<float4 *>(h + i) = make_float4(y[0], y[1], y[2], y[3]);
    }
}

float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t) (h >> 15) << 31;
    uint32_t e = (h >> 10) & 31, f = h & 1023, u;
    if (e == 31) {
        u = s | 0x7f800000u | (f << 13);
    } else if (e == 0) {
        if (f == 0) {
            u = s;
        } else {   // subnormal: normalise
            int k = -1;
            do { f <<= 1; k++; } while (!(f & 1024));
            u = s | ((uint32_t) (127 - 15 - k) << 23) | ((f & 1023) << 13);
        }
    } else {
        u = s | ((e + 112) << 23) | (f << 13);
    }
    float x;
    memcpy(&x, &u, 4);
    return x;
}

// A projection weight [N][K]: fp16 bits when the file holds F16 (multiplied as ggml-cpu does,
// with the activations rounded to fp16 and fp32 accumulation), else fp32.
struct Proj {
    void * w = nullptr;
    bool f16 = false;
};

struct BertLayer {
    Proj qkv, ao, ff1, ff2;
    float * qkv_b = nullptr, * ao_b = nullptr, * ln1 = nullptr;
    float * ff1_b = nullptr, * ff2_b = nullptr, * ln2 = nullptr;
};

// fp32 -> fp16, round to nearest even (ggml's FP32_TO_FP16 on F16C hardware)
__global__ void __launch_bounds__(256) k_to_f16(const float * __restrict__ x, int64_t n,
                                                _Float16 * __restrict__ y) {
    const int64_t i = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (i + 3 < n) {
        const float4 v = *reinterpret_cast<const float4 *>(x + i);
        y[i] = (_Float16) v.x; y[i + 1] = (_Float16) v.y; y[i + 2] = (_Float16) v.z; y[i + 3] = (_Float16) v.w;
    } else {
        for (int64_t j = i; j < n; j++) y[j] = (_Float16) x[j];
    }
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

struct gsvk_bert {
    int device = 0;
    hipStream_t stream = nullptr;
    rocblas_handle blas = nullptr;
    gsvk_bert_info info{};
    std::vector<void *> wmem;   // weight allocations
    bool any_f16 = false;       // some projection is kept in fp16
    float * word = nullptr, * pos = nullptr, * type0 = nullptr, * emb_ln = nullptr;
    std::vector<BertLayer> L;
    // per-call workspace, grown to the largest call
    void * ws = nullptr;
    size_t ws_bytes = 0;

    ~gsvk_bert() {
        if (stream) (void) hipStreamSynchronize(stream);
        if (ws) (void) hipFree(ws);
        for (void * p : wmem) (void) hipFree(p);
        if (blas) (void) rocblas_destroy_handle(blas);
        if (stream) (void) hipStreamDestroy(stream);
    }
    template <typename T>
    int dev_alloc(T *& out, size_t count) {
        void * p = nullptr;
        const hipError_t e = hipMalloc(&p, count * sizeof(T));
        if (e != hipSuccess) {
            (void) hipGetLastError();
            set_error("hipMalloc of %zu bytes failed: %s", count * sizeof(T), hipGetErrorString(e));
            return GSVK_ERR_NOMEM;
        }
        wmem.push_back(p);
        out = (T *) p;
        return GSVK_OK;
    }
};

namespace {

struct DevGuard {
    int prev = -1;
    explicit DevGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        (void) hipSetDevice(dev);
    }
    ~DevGuard() {
        if (prev >= 0) (void) hipSetDevice(prev);
    }
};

#define GSVK_BLAS(call)                                                                          \
    do {                                                                                         \
        const rocblas_status s_ = (call);                                                        \
        if (s_ != rocblas_status_success) {                                                      \
            gsvk::set_error("%s failed: %s", #call, rocblas_status_to_string(s_));               \
            return GSVK_ERR_HIP;                                                                 \
        }                                                                                        \
    } while (0)

// Read tensor `name` of ggml shape {ne0, ne1} (ne1 = 1 for vectors) as fp32 into a new device
// buffer. F32, F16 and Q8_0 (rows of ne0 % 32 == 0) are accepted.
int load_tensor(gsvk_bert * m, const GgufFile & g, const std::string & name, int64_t ne0, int64_t ne1,
                float *& out, Proj * proj = nullptr) {
    const GgufTensor * t = g.tensor(name);
    if (!t) {
        set_error("BERT GGUF: missing tensor %s", name.c_str());
        return GSVK_ERR_FORMAT;
    }
    const int64_t got1 = t->ne.size() > 1 ? t->rows() : 1;
    if (t->ne[0] != ne0 || got1 != ne1) {
        set_error("BERT GGUF: tensor %s has shape [%lld, %lld], expected [%lld, %lld]", name.c_str(),
                  (long long) t->ne[0], (long long) got1, (long long) ne0, (long long) ne1);
        return GSVK_ERR_FORMAT;
    }
    if (t->type != GGML_F32 && t->type != GGML_F16 && t->type != GGML_Q8_0) {
        set_error("BERT GGUF: tensor %s has type %u (F32, F16 or Q8_0 supported)", name.c_str(), t->type);
        return GSVK_ERR_FORMAT;
    }
    const size_t n = (size_t) ne0 * (size_t) ne1;
    std::vector<uint8_t> raw(t->nbytes);
    if (!g.read(*t, raw.data())) {
        set_error("BERT GGUF: reading tensor %s failed", name.c_str());
        return GSVK_ERR_IO;
    }
    if (proj && t->type == GGML_F16) {   // a projection kept in fp16
        uint16_t * w16 = nullptr;
        GSVK_TRY(m->dev_alloc(w16, n));
        GSVK_HIP(hipMemcpy(w16, raw.data(), n * 2, hipMemcpyHostToDevice));
        proj->w = w16;
        proj->f16 = true;
        m->any_f16 = true;
        out = nullptr;
        return GSVK_OK;
    }
    std::vector<float> f(n);
    if (t->type == GGML_F32) {
        memcpy(f.data(), raw.data(), n * 4);
    } else if (t->type == GGML_F16) {
        const uint16_t * h = (const uint16_t *) raw.data();
        for (size_t i = 0; i < n; i++) f[i] = half_to_float(h[i]);
    } else {   // Q8_0 blocks {fp16 d; int8 q[32]}: w = fp32(d) * q
        for (size_t blk = 0; blk < n / 32; blk++) {
            const uint8_t * p = raw.data() + blk * 34;
            uint16_t dh;
            memcpy(&dh, p, 2);
            const float d = half_to_float(dh);
            for (int i = 0; i < 32; i++) f[blk * 32 + i] = d * (float) (int8_t) p[2 + i];
        }
    }
    GSVK_TRY(m->dev_alloc(out, n));
    GSVK_HIP(hipMemcpy(out, f.data(), n * 4, hipMemcpyHostToDevice));
    if (proj) {
        proj->w = out;
        proj->f16 = false;
    }
    return GSVK_OK;
}

int load_proj(gsvk_bert * m, const GgufFile & g, const std::string & name, int64_t ne0, int64_t ne1, Proj & p) {
    float * f = nullptr;
    return load_tensor(m, g, name, ne0, ne1, f, &p);
}

// [w; b] of a LayerNorm, packed as the fused LayerNorm kernel reads it
int load_ln(gsvk_bert * m, const GgufFile & g, const std::string & wn, const std::string & bn, float *& out) {
    const int D = m->info.hidden;
    float * w = nullptr, * b = nullptr;
    GSVK_TRY(load_tensor(m, g, wn, D, 1, w));
    GSVK_TRY(load_tensor(m, g, bn, D, 1, b));
    GSVK_TRY(m->dev_alloc(out, 2 * (size_t) D));
    GSVK_HIP(hipMemcpy(out, w, (size_t) D * 4, hipMemcpyDeviceToDevice));
    GSVK_HIP(hipMemcpy(out + D, b, (size_t) D * 4, hipMemcpyDeviceToDevice));
    return GSVK_OK;
}

// Y[M][N] = X[M][K] . W[N][K]^T (row-major), i.e. column-major Y^T = W^T X^T. An fp16 weight
// takes X rounded to fp16 (into x16, scratch of M*K halves) or, when X is null, the fp16 rows
// already in x16; products are summed in fp32.
int gemm(gsvk_bert * m, const Proj & W, const float * X, _Float16 * x16, float * Y, int M, int N, int K) {
    const float one = 1.0f, zero = 0.0f;
    if (!W.f16) {
        GSVK_BLAS(rocblas_sgemm(m->blas, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &one,
                                (const float *) W.w, K, X, K, &zero, Y, N));
        return GSVK_OK;
    }
    if (X) {
        const int64_t n = (int64_t) M * K;
        hipLaunchKernelGGL(k_to_f16, dim3((unsigned) ((n / 4 + 255) / 256 + 1)), dim3(256), 0, m->stream, X, n, x16);
        GSVK_LAUNCH_CHECK();
    }
    GSVK_BLAS(rocblas_gemm_ex(m->blas, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &one, W.w,
                              rocblas_datatype_f16_r, K, x16, rocblas_datatype_f16_r, K, &zero, Y,
                              rocblas_datatype_f32_r, N, Y, rocblas_datatype_f32_r, N, rocblas_datatype_f32_r,
                              rocblas_gemm_algo_standard, 0, 0));
    return GSVK_OK;
}

}  // namespace

extern "C" int gsvk_bert_load(const char * path, int device, int verbose, gsvk_bert ** out) {
    GSVK_REQUIRE(path && out, "gsvk_bert_load: null argument");
    *out = nullptr;
    GgufFile g;
    std::string err;
    bool io_error = false;
    if (!g.open(path, err, &io_error)) {
        set_error("%s", err.c_str());
        return io_error ? GSVK_ERR_IO : GSVK_ERR_FORMAT;
    }
    std::unique_ptr<gsvk_bert> m(new gsvk_bert());
    // hyperparameters (src/gsv_bert.cpp:398-405), with the reference's defaults
    uint32_t u = 0;
    auto key = [&](const char * k, int def) { return g.get_u32(k, u) ? (int) u : def; };
    gsvk_bert_info & in = m->info;
    in.layers_used = key("bert.layers_used", 22);
    in.hidden = key("bert.hidden", 1024);
    in.heads = key("bert.head", 16);
    in.inter = key("bert.inter", 4096);
    in.vocab = key("bert.vocab", 21128);
    in.max_pos = key("bert.max_pos", 512);
    float eps = 1e-12f;
    in.ln_eps = g.get_f32("bert.ln_eps", eps) ? eps : 1e-12f;
    GSVK_REQUIRE(in.heads > 0 && in.hidden == in.heads * BA_HD,
                 "BERT GGUF: hidden %d / heads %d: the kernels need head dim %d", in.hidden, in.heads, BA_HD);
    GSVK_REQUIRE(in.hidden % 32 == 0 && in.hidden <= 4096 && in.inter > 0 && in.inter % 32 == 0 &&
                     in.layers_used >= 0 && in.layers_used <= 1000 && in.vocab > 0 && in.max_pos > 0,
                 "BERT GGUF: unsupported hyperparameters (hidden %d, inter %d, layers %d)", in.hidden,
                 in.inter, in.layers_used);
    const GgufTensor * qt = g.tensor("bert.l0.qkv_w");
    in.weight_type = qt ? (int) qt->type : 0;
    int ndev = 0;
    gsvk_device_count(&ndev);
    if (device < 0 || device >= ndev) {
        set_error("HIP device %d not found (%d visible)", device, ndev);
        return GSVK_ERR_NODEV;
    }
    DevGuard guard(device);
    m->device = device;
    GSVK_HIP(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    GSVK_BLAS(rocblas_create_handle(&m->blas));
    GSVK_BLAS(rocblas_set_stream(m->blas, m->stream));
    const int D = in.hidden, F = in.inter;
    const GgufTensor * tt = g.tensor("bert.type_emb");
    GSVK_REQUIRE(tt && tt->ne[0] == D, "BERT GGUF: missing or malformed bert.type_emb");
    GSVK_TRY(load_tensor(m.get(), g, "bert.word_emb", D, in.vocab, m->word));
    GSVK_TRY(load_tensor(m.get(), g, "bert.pos_emb", D, in.max_pos, m->pos));
    GSVK_TRY(load_tensor(m.get(), g, "bert.type_emb", D, tt->rows(), m->type0));   // row 0 is used
    GSVK_TRY(load_ln(m.get(), g, "bert.emb_ln_w", "bert.emb_ln_b", m->emb_ln));
    m->L.resize(in.layers_used);
    for (int li = 0; li < in.layers_used; li++) {
        const std::string p = "bert.l" + std::to_string(li) + ".";
        BertLayer & w = m->L[li];
        GSVK_TRY(load_proj(m.get(), g, p + "qkv_w", D, 3 * D, w.qkv));
        GSVK_TRY(load_tensor(m.get(), g, p + "qkv_b", 3 * D, 1, w.qkv_b));
        GSVK_TRY(load_proj(m.get(), g, p + "attn_out_w", D, D, w.ao));
        GSVK_TRY(load_tensor(m.get(), g, p + "attn_out_b", D, 1, w.ao_b));
        GSVK_TRY(load_ln(m.get(), g, p + "attn_ln_w", p + "attn_ln_b", w.ln1));
        GSVK_TRY(load_proj(m.get(), g, p + "ff1_w", D, F, w.ff1));
        GSVK_TRY(load_tensor(m.get(), g, p + "ff1_b", F, 1, w.ff1_b));
        GSVK_TRY(load_proj(m.get(), g, p + "ff2_w", F, D, w.ff2));
        GSVK_TRY(load_tensor(m.get(), g, p + "ff2_b", D, 1, w.ff2_b));
        GSVK_TRY(load_ln(m.get(), g, p + "out_ln_w", p + "out_ln_b", w.ln2));
    }
    GSVK_HIP(hipDeviceSynchronize());
    if (verbose)
        fprintf(stderr, "[gsvk_bert] %s: hidden %d, %d heads, inter %d, %d layers used, vocab %d, weights type %d\n",
                path, D, in.heads, F, in.layers_used, in.vocab, in.weight_type);
    *out = m.release();
    return GSVK_OK;
}

extern "C" void gsvk_bert_free(gsvk_bert * m) {
    if (!m) return;
    DevGuard guard(m->device);
    delete m;
}

extern "C" int gsvk_bert_get_info(const gsvk_bert * m, gsvk_bert_info * info) {
    GSVK_REQUIRE(m && info, "gsvk_bert_get_info: null argument");
    *info = m->info;
    return GSVK_OK;
}

extern "C" int gsvk_bert_encode(gsvk_bert * m, int B, const int32_t * ids_flat, const int32_t * lens, int Tmax,
                                int n_layers, float * out) {
    GSVK_REQUIRE(m && ids_flat && lens && out, "gsvk_bert_encode: null argument");
    const gsvk_bert_info & in = m->info;
    GSVK_REQUIRE(B > 0 && Tmax > 0 && Tmax <= in.max_pos, "gsvk_bert_encode: B %d, Tmax %d (max_pos %d)", B,
                 Tmax, in.max_pos);
    if (n_layers < 0 || n_layers > in.layers_used) n_layers = in.layers_used;
    std::vector<int32_t> ids, tpos, off(B), len(B);
    int64_t rows = 0;
    for (int b = 0; b < B; b++) {
        GSVK_REQUIRE(lens[b] >= 1 && lens[b] <= Tmax, "gsvk_bert_encode: sequence %d has length %d (1..%d)", b,
                     lens[b], Tmax);
        off[b] = (int32_t) rows;
        len[b] = lens[b];
        for (int t = 0; t < lens[b]; t++) {
            const int32_t id = ids_flat[(int64_t) b * Tmax + t];
            GSVK_REQUIRE(id >= 0 && id < in.vocab, "gsvk_bert_encode: token id %d out of range (vocab %d)", id,
                         in.vocab);
            ids.push_back(id);
            tpos.push_back(t);
        }
        rows += lens[b];
    }
    const int D = in.hidden, F = in.inter;
    DevGuard guard(m->device);
    hipStream_t st = m->stream;
    // workspace: x, qkv, attention output, projection output, FFN hidden, and the small arrays
    const size_t fl = (size_t) rows * (D + 3 * D + D + D + F);
    const size_t h16 = m->any_f16 ? (size_t) rows * (F > D ? F : D) : 0;   // fp16 GEMM input
    const size_t need = fl * 4 + h16 * 2 + (size_t) rows * 8 + (size_t) B * 8 + 4096;
    if (need > m->ws_bytes) {
        if (m->ws) (void) hipFree(m->ws);
        m->ws = nullptr;
        m->ws_bytes = 0;
        const hipError_t e = hipMalloc(&m->ws, need);
        if (e != hipSuccess) {
            (void) hipGetLastError();
            set_error("hipMalloc of %zu bytes failed: %s", need, hipGetErrorString(e));
            return GSVK_ERR_NOMEM;
        }
        m->ws_bytes = need;
    }
    float * x = (float *) m->ws;
    float * qkv = x + rows * D;
    float * att = qkv + rows * 3 * D;
    float * prj = att + rows * D;
    float * h = prj + rows * D;
    _Float16 * x16 = (_Float16 *) (h + rows * F);
    int32_t * d_ids = (int32_t *) (x16 + h16 + (h16 & 1));
    int32_t * d_pos = d_ids + rows;
    int32_t * d_off = d_pos + rows;
    int32_t * d_len = d_off + B;
    GSVK_HIP(hipMemcpyAsync(d_ids, ids.data(), rows * 4, hipMemcpyHostToDevice, st));
    GSVK_HIP(hipMemcpyAsync(d_pos, tpos.data(), rows * 4, hipMemcpyHostToDevice, st));
    GSVK_HIP(hipMemcpyAsync(d_off, off.data(), (size_t) B * 4, hipMemcpyHostToDevice, st));
    GSVK_HIP(hipMemcpyAsync(d_len, len.data(), (size_t) B * 4, hipMemcpyHostToDevice, st));

    hipLaunchKernelGGL(k_bert_embed, dim3((unsigned) rows), dim3(256), 0, st, m->word, m->pos, m->type0, d_ids,
                       d_pos, D, prj);
    GSVK_LAUNCH_CHECK();
    // each LayerNorm also writes the fp16 copy its consumer takes when that is an F16 projection
    auto h16_for = [&](int li) { return li < n_layers && m->L[li].qkv.f16 ? (uint16_t *) x16 : nullptr; };
    GSVK_TRY(launch_layernorm(prj, nullptr, nullptr, m->emb_ln, rows, D, in.ln_eps, x, nullptr, nullptr, st,
                              Q8_SLICED, h16_for(0)));
    const float scale_log2 = 1.4426950408889634f / std::sqrt((float) BA_HD);
    for (int li = 0; li < n_layers; li++) {
        const BertLayer & w = m->L[li];
        // the QKV bias is added as attention reads q, k, v; the LayerNorms, attention and GELU
        // write the fp16 input of an F16 projection directly
        GSVK_TRY(gemm(m, w.qkv, w.qkv.f16 ? nullptr : x, x16, qkv, (int) rows, 3 * D, D));
        hipLaunchKernelGGL(k_bert_attn, dim3((unsigned) ((Tmax + BA_Q - 1) / BA_Q), (unsigned) in.heads, (unsigned) B),
                           dim3(256), 0, st, qkv, w.qkv_b, d_off, d_len, D, scale_log2, att,
                           w.ao.f16 ? x16 : nullptr);
        GSVK_LAUNCH_CHECK();
        GSVK_TRY(gemm(m, w.ao, w.ao.f16 ? nullptr : att, x16, prj, (int) rows, D, D));
        GSVK_TRY(launch_layernorm(x, prj, w.ao_b, w.ln1, rows, D, in.ln_eps, x, nullptr, nullptr, st, Q8_SLICED,
                                  w.ff1.f16 ? (uint16_t *) x16 : nullptr));
        GSVK_TRY(gemm(m, w.ff1, w.ff1.f16 ? nullptr : x, x16, h, (int) rows, F, D));
        hipLaunchKernelGGL(k_bias_gelu, dim3((unsigned) ((rows * F / 4 + 255) / 256)), dim3(256), 0, st, h, w.ff1_b,
                           rows, F, w.ff2.f16 ? x16 : nullptr);
        GSVK_LAUNCH_CHECK();
        GSVK_TRY(gemm(m, w.ff2, w.ff2.f16 ? nullptr : h, x16, prj, (int) rows, D, F));
        GSVK_TRY(launch_layernorm(x, prj, w.ff2_b, w.ln2, rows, D, in.ln_eps, x, nullptr, nullptr, st, Q8_SLICED,
                                  h16_for(li + 1)));
    }
    // [rows][D] -> per sequence [D][len] (src/gsv_bert.cpp:220-228)
    std::vector<float> host((size_t) rows * D);
    GSVK_HIP(hipMemcpyAsync(host.data(), x, host.size() * 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipStreamSynchronize(st));
    for (int b = 0; b < B; b++) {
        float * ob = out + (size_t) D * off[b];
        const float * hb = host.data() + (size_t) off[b] * D;
        for (int d = 0; d < D; d++)
            for (int t = 0; t < len[b]; t++) ob[(size_t) d * len[b] + t] = hb[(size_t) t * D + d];
    }
    return GSVK_OK;
}

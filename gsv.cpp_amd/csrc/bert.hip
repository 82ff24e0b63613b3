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
// Design: rows of all sequences packed back to back (no padding rows). The projections are
// k_bert_gemm below, on the matrix cores: F32 weights in fp32 (v_mfma_f32_32x32x2f32, ggml-cpu's
// F32 x F32 product), F16 weights kept in fp16 with the activations rounded to fp16 and fp32 sums
// (v_mfma_f32_32x32x16_f16; ggml-cpu converts the activations to the weights' F16 dot type),
// Q8_0 weight files widened to fp32 at load. A workgroup computes a 64-row x 32-column tile over
// a K slice, its 8 waves an eighth of the slice each, loading their operands straight into
// registers (16 bytes per lane, the next group of steps in flight while one is multiplied);
// the 8 partial tiles are summed through LDS in a fixed order. For few rows the K range is split
// over workgroups too, into partial rows that the consumer (the LayerNorm) sums in order, so
// every result is the same from run to run. The FFN1 GEMM applies bias + GELU itself.
// LayerNorm over the partial rows is k_bert_ln; attention is k_bert_attn below: one workgroup per
// 16 queries of one (sequence, head), four lanes per query (a quarter of the head dims each),
// keys and values staged through LDS in tiles of 64 whose 4 chunks of 16 keys go to its 4 waves
// (online softmax each, merged at the end), fp32 throughout.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "gguf.h"
#include "layer.h"
#include "gsvk.h"

namespace gsvk {

namespace {

constexpr int BA_HD = 64;   // head dim of the kernels below (BERT-large: 1024 / 16)
constexpr int BA_KT = 64;   // keys per LDS tile
constexpr int BA_CH = 16;   // keys per softmax chunk
constexpr int BA_Q = 16;    // queries per workgroup (4 lanes per query in each of its 4 waves)

// fp16 GEMM operands (F16 weights and the activations that meet them) are kept in the order the
// matrix cores read them: per 32-row tile and step of 16 K values a 1 KB chunk in which lane
// L = 32 g + i holds row i's values [8 g, 8 g + 8) of the step, so that a wave's operand load is
// one contiguous 1 KB. Offset (in halves) of element (r, k) of an [R][K] matrix, K % 16 == 0;
// rows are padded to a multiple of 64 (the rows of one workgroup).
__host__ __device__ inline int64_t bt_off(int64_t r, int64_t k, int64_t K) {
    return ((((r >> 5) * (K >> 4) + (k >> 4)) << 9) + (((((k >> 3) & 1) << 5) | (r & 31)) << 3)) + (k & 7);
}

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
    if (out16) {   // the fp16 input of an F16 out projection, in the operand order
        const int64_t row = off + q0 + qq;
        const int d0 = h * BA_HD + 16 * c;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                w[j] = (uint32_t) f2h(O[8 * hh + 2 * j] * inv) | ((uint32_t) f2h(O[8 * hh + 2 * j + 1] * inv) << 16);
            *reinterpret_cast<uint4 *>(out16 + bt_off(row, d0 + 8 * hh, D)) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        return;
    }
    float4 * op = reinterpret_cast<float4 *>(out + o0);
#pragma unroll
    for (int i = 0; i < 4; i++)
        op[i] = make_float4(O[4 * i] * inv, O[4 * i + 1] * inv, O[4 * i + 2] * inv, O[4 * i + 3] * inv);
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
    // Q8_0 weights: natural-order quants [N][K] and fp16 scales [N][K/32], multiplied on the int8
    // GEMM with the activations quantised as ggml-cpu quantises them (its vec_dot type for Q8_0)
    int8_t * q8 = nullptr;
    uint16_t * q8d = nullptr;
};

struct BertLayer {
    Proj qkv, ao, ff1, ff2;
    float * qkv_b = nullptr, * ao_b = nullptr, * ln1 = nullptr;
    float * ff1_b = nullptr, * ff2_b = nullptr, * ln2 = nullptr;
};

typedef _Float16 bv8h __attribute__((ext_vector_type(8)));
typedef float bv16f __attribute__((ext_vector_type(16)));

constexpr int BG_BM = 64;        // most rows per workgroup (two 32-row MFMA tiles per wave)
constexpr int BG_BN = 32;        // columns per workgroup
constexpr int BG_WAVES = 8;      // each an eighth of the workgroup's K slice
constexpr int BG_U = 4;          // MFMA steps per group of loads

// Output stage of k_bert_gemm. With a K slice per workgroup (gridDim.z > 1) only y is written:
// slice z of the sum to y + z * pstride (partial rows, summed by their consumer).
struct BgOut {
    float * y;            // [M][N] fp32, or null
    int64_t pstride;      // floats between partial slices
    const float * bias;   // added before the activation, or null
    int gelu;             // y = gelu_erf(y + bias) (the add_act of src/gsv_bert.cpp:151-153)
    _Float16 * y16;       // fp16 copy (nearest even) in the operand order (bt_off), or null
};

// K values of one MFMA step and of one 16-byte lane load, per operand type
template <typename T> struct BgStep;
template <> struct BgStep<_Float16> { static constexpr int K = 16, PER_LOAD = 8; };
template <> struct BgStep<float> { static constexpr int K = 8, PER_LOAD = 4; };

// Y[M][N] (or a K slice of it) = X[M][K] . W[N][K]^T, 8 waves each an eighth of the K slice (so
// that the loads of a few rows' GEMM are all in flight at once), RT 32-row tiles per workgroup.
// Lane (li, lg) of a wave supplies row m0 + 32 t + li of tile t (A) and column n0 + li (B) with
// the K values of slot lg of each step;
// A and B use the same slots, so each MFMA sums the step's K values once, in the hardware's order.
template <typename T, int NG, int RT>
__global__ void __launch_bounds__(BG_WAVES * 64) k_bert_gemm(const T * __restrict__ X, const T * __restrict__ W,
                                                             int M, int N, int K, int kslice, BgOut o) {
    using St = BgStep<T>;
    constexpr int BM = 32 * RT;   // rows of the workgroup: RT 32-row MFMA tiles per wave
    constexpr int HW = BG_WAVES / 2;
    __shared__ float red[HW][BM][BG_BN + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 31, lg = lane >> 5;
    const int n0 = blockIdx.x * BG_BN, m0 = blockIdx.y * BM, p = blockIdx.z;
    const int kw = kslice / BG_WAVES;
    // fp16 operands in the operand order (bt_off; rows padded to 64): a step of the wave is one
    // 1 KB chunk at stride SSTEP; fp32 operands row-major, the lane at its row and slot
    constexpr bool TL = sizeof(T) == 2;
    constexpr int64_t SSTEP = TL ? 512 : St::K;
    const T * xa[RT];
    const T * wb;
    if constexpr (TL) {
        const int64_t s0 = ((int64_t) p * kslice + (int64_t) wave * kw) / St::K, nst = K / St::K;
#pragma unroll
        for (int t = 0; t < RT; t++) xa[t] = X + (((int64_t) ((m0 >> 5) + t) * nst + s0) << 9) + lane * 8;
        wb = W + (((int64_t) (n0 >> 5) * nst + s0) << 9) + lane * 8;
    } else {
        const int64_t k0 = (int64_t) p * kslice + (int64_t) wave * kw + lg * St::PER_LOAD;
#pragma unroll
        for (int t = 0; t < RT; t++) xa[t] = X + (int64_t) min(m0 + 32 * t + li, M - 1) * K + k0;
        wb = W + (int64_t) (n0 + li) * K + k0;
    }
    bv16f acc[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) acc[t] = bv16f{};
    constexpr int GK = St::K * BG_U;   // K values per group of steps
    // two register buffers in turn: while one group is multiplied the next one (and, after it
    // is consumed, the one after) is in flight; operand t < RT: the rows of tile t, RT: the
    // weight columns
    uint4 g[2][RT + 1][BG_U];
    auto load = [&](uint4 (&gg)[RT + 1][BG_U], int kk) {
#pragma unroll
        for (int u = 0; u < BG_U; u++) {
            const int64_t off = (int64_t) (kk / St::K + u) * SSTEP;
#pragma unroll
            for (int t = 0; t < RT; t++) gg[t][u] = *reinterpret_cast<const uint4 *>(xa[t] + off);
            gg[RT][u] = *reinterpret_cast<const uint4 *>(wb + off);
        }
    };
    auto mma = [&](const uint4 (&gg)[RT + 1][BG_U]) {
#pragma unroll
        for (int u = 0; u < BG_U; u++) {
            if constexpr (sizeof(T) == 2) {
                const bv8h vb = __builtin_bit_cast(bv8h, gg[RT][u]);
#pragma unroll
                for (int t = 0; t < RT; t++)
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(bv8h, gg[t][u]), vb, acc[t], 0, 0, 0);
            } else {
                const uint32_t wv[4] = {gg[RT][u].x, gg[RT][u].y, gg[RT][u].z, gg[RT][u].w};
#pragma unroll
                for (int t = 0; t < RT; t++) {
                    const uint32_t wa[4] = {gg[t][u].x, gg[t][u].y, gg[t][u].z, gg[t][u].w};
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, wa[e]),
                                                                      __builtin_bit_cast(float, wv[e]), acc[t], 0, 0, 0);
                }
            }
        }
    };
    // NG groups per wave (kw = NG * GK), the loop unrolled at compile time: straight-line code,
    // so the wait before each group's MFMAs counts exactly the loads issued after it
    (void) kw;
    // (the scheduling barriers keep each group's loads where they are written: issued early)
    load(g[0], 0);
    if constexpr (NG > 1) load(g[1], GK);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        mma(g[gi & 1]);
        if (gi + 2 < NG) load(g[gi & 1], (gi + 2) * GK);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the eight waves' tiles summed in a fixed order, (w + (w + 4)) for w < 4 then
    // ((t0 + t1) + t2) + t3: element v of lane (li, lg) is row 8 (v / 4) + 4 lg + v % 4 of its
    // 32-row tile, column li
    if (wave >= HW) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) red[wave - HW][32 * t + 8 * (v >> 2) + 4 * lg + (v & 3)][li] = acc[t][v];
    }
    __syncthreads();
    if (wave < HW) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int r = 32 * t + 8 * (v >> 2) + 4 * lg + (v & 3);
                red[wave][r][li] = acc[t][v] + red[wave][r][li];
            }
    }
    __syncthreads();
    if (tid >= 4 * BM) return;   // 4 threads per row of the tile
    const int r = tid >> 2, c0 = (tid & 3) * 8;
    const int row = m0 + r;
    if (row >= M) return;
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
        y[j] = ((red[0][r][c0 + j] + red[1][r][c0 + j]) + red[2][r][c0 + j]) + red[3][r][c0 + j];
    const int col = n0 + c0;
    if (o.bias) {
#pragma unroll
        for (int j = 0; j < 8; j++) y[j] = y[j] + o.bias[col + j];
    }
    if (o.gelu) {
#pragma unroll
        for (int j = 0; j < 8; j++) y[j] = 0.5f * y[j] * (1.0f + erff(y[j] * 0.70710678118654752440f));
    }
    if (o.y) {
        float * yr = o.y + (int64_t) p * o.pstride + (int64_t) row * N + col;
        *reinterpret_cast<float4 *>(yr) = make_float4(y[0], y[1], y[2], y[3]);
        *reinterpret_cast<float4 *>(yr + 4) = make_float4(y[4], y[5], y[6], y[7]);
    }
    if (o.y16) {   // in the operand order of the next GEMM (K = N)
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++) h[j] = (uint32_t) f2h(y[2 * j]) | ((uint32_t) f2h(y[2 * j + 1]) << 16);
        *reinterpret_cast<uint4 *>(o.y16 + bt_off(row, col, N)) = make_uint4(h[0], h[1], h[2], h[3]);
    }
}

// LayerNorm((x + (r_0 + r_1 + ... + r_{np-1})) + bias) * w + b of one row of n = 4 x 256 values
// per workgroup (4 values per thread), r the np <= 8 partial rows of a split-K projection (np = 1:
// the projection's output; r null: x alone), every load issued before the first use. The
// LayerNorm of norm.hip otherwise: sums in double, var = E[v^2] - mean^2,
// y = fma((v - mean) * inv, w, b); y16 its fp16 copy in the operand order (bt_off).
constexpr int BL_THREADS = 256;
constexpr int BL_MAXP = 8;
__global__ void __launch_bounds__(BL_THREADS) k_bert_ln(const float * __restrict__ x, const float * __restrict__ r,
                                                        int np, int64_t pstride, const float * __restrict__ bias,
                                                        const float * __restrict__ wb, int n, float eps,
                                                        float * __restrict__ y, _Float16 * __restrict__ y16,
                                                        int8_t * __restrict__ yq, float * __restrict__ yd) {
    __shared__ double s_red[2][BL_THREADS / 64];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool act = 4 * tid < n;
    const int c = act ? 4 * tid : 0;
    const int64_t o = row * n + c;
    const float4 xv = *reinterpret_cast<const float4 *>(x + o);
    float4 pv[BL_MAXP];
#pragma unroll
    for (int q = 0; q < BL_MAXP; q++)
        if (r && q < np) pv[q] = *reinterpret_cast<const float4 *>(r + q * pstride + o);
    const float4 bv = bias ? *reinterpret_cast<const float4 *>(bias + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 wv = *reinterpret_cast<const float4 *>(wb + c);
    const float4 cv = *reinterpret_cast<const float4 *>(wb + n + c);
    float v[4] = {xv.x, xv.y, xv.z, xv.w};
    if (r) {
        float rs[4] = {pv[0].x, pv[0].y, pv[0].z, pv[0].w};
#pragma unroll
        for (int q = 1; q < BL_MAXP; q++)
            if (q < np) {
                rs[0] = rs[0] + pv[q].x; rs[1] = rs[1] + pv[q].y; rs[2] = rs[2] + pv[q].z; rs[3] = rs[3] + pv[q].w;
            }
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = v[i] + rs[i];
    }
    if (bias) {
        v[0] = v[0] + bv.x; v[1] = v[1] + bv.y; v[2] = v[2] + bv.z; v[3] = v[3] + bv.w;
    }
    double s = 0.0, s2 = 0.0;
    if (act) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s += (double) v[i];
            s2 += (double) v[i] * (double) v[i];
        }
    }
    s = wave_sum_d_uniform(s);
    s2 = wave_sum_d_uniform(s2);
    if (lane == 0) {
        s_red[0][wave] = s;
        s_red[1][wave] = s2;
    }
    __syncthreads();
    const double S = (s_red[0][0] + s_red[0][1]) + (s_red[0][2] + s_red[0][3]);
    const double S2 = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);
    const float mean = (float) (S / (double) n);
    const float var = __builtin_fmaf(-mean, mean, (float) (S2 / (double) n));
    const float inv = 1.0f / __builtin_sqrtf(var + eps);
    if (!act) return;
    const float wv4[4] = {wv.x, wv.y, wv.z, wv.w}, cv4[4] = {cv.x, cv.y, cv.z, cv.w};
    float out[4];
#pragma unroll
    for (int i = 0; i < 4; i++) out[i] = __builtin_fmaf((v[i] - mean) * inv, wv4[i], cv4[i]);
    *reinterpret_cast<float4 *>(y + o) = make_float4(out[0], out[1], out[2], out[3]);
    if (y16) {   // in the operand order of the next GEMM (K = n)
        const uint32_t h0 = (uint32_t) f2h(out[0]) | ((uint32_t) f2h(out[1]) << 16);
        const uint32_t h1 = (uint32_t) f2h(out[2]) | ((uint32_t) f2h(out[3]) << 16);
        *reinterpret_cast<uint2 *>(y16 + bt_off(row, c, n)) = make_uint2(h0, h1);
    }
    if (yq) {   // the x86 Q8_0 quantisation of the row (natural order): a block is 8 threads
        int8_t q[4];
        const float d = q8_quantize_group<4>(out, q, 8);
        *reinterpret_cast<int *>(yq + o) = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
        if ((c & 31) == 0) yd[row * (n / 32) + c / 32] = d;
    }
}

// h = gelu_erf(h) (bias already added by the FFN1 GEMM), then its x86 Q8_0 quantisation in natural
// order for a Q8_0 FFN2: 4 values per thread, a block is 8 threads
__global__ void __launch_bounds__(256) k_bert_gelu_q8(const float * __restrict__ h, int64_t n, int8_t * __restrict__ hq,
                                                      float * __restrict__ hd) {
    const int64_t i = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;   // n % 32 == 0: whole blocks leave together
    const float4 v = *reinterpret_cast<const float4 *>(h + i);
    float y[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; k++) y[k] = 0.5f * y[k] * (1.0f + erff(y[k] * 0.70710678118654752440f));
    int8_t q[4];
    const float d = q8_quantize_group<4>(y, q, 8);
    *reinterpret_cast<int *>(hq + i) = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
    if ((i & 31) == 0) hd[i / 32] = d;
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

struct gsvk_bert {
    int device = 0;
    hipStream_t stream = nullptr;
    gsvk_bert_info info{};
    std::vector<void *> wmem;   // weight allocations
    bool any_f16 = false;       // some projection is kept in fp16
    bool any_q8 = false;        // some projection is Q8_0 (int8 GEMM)
    float * word = nullptr, * pos = nullptr, * type0 = nullptr, * emb_ln = nullptr;
    std::vector<BertLayer> L;
    // per-call workspace, grown to the largest call
    void * ws = nullptr;
    size_t ws_bytes = 0;
    // pinned host staging of a call (the packed id arrays in, the features out): copies from
    // pageable memory cost tens of microseconds each
    void * pin = nullptr;
    size_t pin_bytes = 0;

    ~gsvk_bert() {
        if (stream) (void) hipStreamSynchronize(stream);
        if (ws) (void) hipFree(ws);
        if (pin) (void) hipHostFree(pin);
        for (void * p : wmem) (void) hipFree(p);
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
    if (proj && t->type == GGML_F16) {   // a projection kept in fp16, in the operand order
        if (ne0 % 16 != 0 || ne1 % 64 != 0) {
            set_error("BERT GGUF: %s: F16 projection shape [%lld, %lld] (K %% 16, N %% 64)", name.c_str(),
                      (long long) ne0, (long long) ne1);
            return GSVK_ERR_FORMAT;
        }
        std::vector<uint16_t> tiled(n);
        const uint16_t * src = (const uint16_t *) raw.data();
        for (int64_t r = 0; r < ne1; r++)
            for (int64_t k = 0; k < ne0; k++) tiled[bt_off(r, k, ne0)] = src[r * ne0 + k];
        uint16_t * w16 = nullptr;
        GSVK_TRY(m->dev_alloc(w16, n));
        GSVK_HIP(hipMemcpy(w16, tiled.data(), n * 2, hipMemcpyHostToDevice));
        proj->w = w16;
        proj->f16 = true;
        m->any_f16 = true;
        out = nullptr;
        return GSVK_OK;
    }
    if (proj && t->type == GGML_Q8_0) {   // a Q8_0 projection: quants and scales apart
        const size_t nb = n / 32;
        std::vector<int8_t> q(n);
        std::vector<uint16_t> d(nb);
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t * p = raw.data() + blk * 34;
            memcpy(&d[blk], p, 2);
            memcpy(&q[blk * 32], p + 2, 32);
        }
        GSVK_TRY(m->dev_alloc(proj->q8, n));
        GSVK_TRY(m->dev_alloc(proj->q8d, nb));
        GSVK_HIP(hipMemcpy(proj->q8, q.data(), n, hipMemcpyHostToDevice));
        GSVK_HIP(hipMemcpy(proj->q8d, d.data(), nb * 2, hipMemcpyHostToDevice));
        m->any_q8 = true;
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

// Row tiles of 32 per wave: 2 (64-row workgroups) when that still gives 256 workgroups, else 1.
int bert_row_tiles(int64_t M, int N) {
    return M > 32 && (int64_t) (N / BG_BN) * ((M + 63) / 64) >= 256 ? 2 : 1;
}

// K slices for an [M][N][K] projection: enough workgroups (row x 32-column tiles x slices) to
// cover the chip when the rows are few, each slice a multiple of the kernel's waves x steps.
int bert_kslices(int64_t M, int N, int K, int kmult, int max_slices) {
    const int bm = 32 * bert_row_tiles(M, N);
    const int64_t tiles = (int64_t) (N / BG_BN) * ((M + bm - 1) / bm);
    int p = 1;
    while (p < max_slices && tiles * p < 256 && K % (2 * p * kmult) == 0) p *= 2;
    return p;
}

// Y = X . W^T for W of the projection's type (fp16 operands when W is F16: X16 holds the
// activations already rounded by their producer; fp32 otherwise); `slices` K slices (> 1: partial
// rows at Y + z * M * N, bias / GELU / y16 not allowed).
int gemm(gsvk_bert * m, const Proj & W, const float * X, const _Float16 * X16, int64_t M, int N, int K,
         int slices, const BgOut & o) {
    const int kmult = BG_WAVES * BG_U * (W.f16 ? BgStep<_Float16>::K : BgStep<float>::K);
    GSVK_REQUIRE(M > 0 && M < (1 << 30) && N % BG_BN == 0 && slices >= 1 && K % (slices * kmult) == 0 &&
                     (slices == 1 || (!o.bias && !o.gelu && !o.y16)) && (o.y || o.y16),
                 "bert gemm: unsupported shape M=%lld N=%d K=%d slices %d", (long long) M, N, K, slices);
    const int rt = bert_row_tiles(M, N);
    const dim3 grid((unsigned) (N / BG_BN), (unsigned) ((M + 32 * rt - 1) / (32 * rt)), (unsigned) slices);
    const int ng = K / slices / kmult;   // groups of steps per wave
    GSVK_REQUIRE(ng == 1 || ng == 2 || ng == 4 || ng == 8 || ng == 16,
                 "bert gemm: K %d / %d slices gives %d groups per wave (1, 2, 4, 8 or 16)", K, slices, ng);
#define GSVK_BG(TT, NGV, XP, WP)                                                                          \
    do {                                                                                                  \
        if (rt == 2)                                                                                      \
            hipLaunchKernelGGL((k_bert_gemm<TT, NGV, 2>), grid, dim3(BG_WAVES * 64), 0, m->stream, XP, WP, \
                               (int) M, N, K, K / slices, o);                                             \
        else                                                                                              \
            hipLaunchKernelGGL((k_bert_gemm<TT, NGV, 1>), grid, dim3(BG_WAVES * 64), 0, m->stream, XP, WP, \
                               (int) M, N, K, K / slices, o);                                             \
    } while (0)
#define GSVK_BG_ALL(TT, XP, WP)                   \
    switch (ng) {                                 \
    case 1: GSVK_BG(TT, 1, XP, WP); break;        \
    case 2: GSVK_BG(TT, 2, XP, WP); break;        \
    case 4: GSVK_BG(TT, 4, XP, WP); break;        \
    case 8: GSVK_BG(TT, 8, XP, WP); break;        \
    default: GSVK_BG(TT, 16, XP, WP); break;      \
    }
    if (W.f16) {
        GSVK_REQUIRE(X16, "bert gemm: F16 weights need fp16 activations");
        GSVK_BG_ALL(_Float16, X16, (const _Float16 *) W.w);
    } else {
        GSVK_REQUIRE(X, "bert gemm: F32 weights need fp32 activations");
        GSVK_BG_ALL(float, X, (const float *) W.w);
    }
#undef GSVK_BG_ALL
#undef GSVK_BG
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

// A Q8_0 projection on the int8 GEMM of the AR path: Y = X . W^T (+ bias) with X the Q8_0 rows
// (natural order) that the producer quantised as ggml-cpu's x86 quantiser does.
int gemm_q8(gsvk_bert * m, const Proj & W, const int8_t * xq, const float * xd, int64_t M, int N, int K, float * y,
            const float * bias) {
    LayerOut lo{};
    lo.y = y;
    lo.y_stride = N;
    lo.n_store = N;
    lo.bias = bias;
    Q8Weights qw{};
    qw.qn = W.q8;
    qw.dn = W.q8d;
    return launch_q8_gemm(qw, N, K, M, xq, xd, Q8_NATURAL, lo, m->stream);
}

int bert_ln(gsvk_bert * m, const float * x, const float * r, int np, int64_t pstride, const float * bias,
            const float * wb, int64_t rows, float * y, _Float16 * y16, int8_t * yq = nullptr,
            float * yd = nullptr) {
    const int D = m->info.hidden;
    GSVK_REQUIRE(D % 4 == 0 && D <= 4 * BL_THREADS && np >= 1 && np <= BL_MAXP,
                 "bert layernorm: hidden %d (<= %d), %d partial rows", D, 4 * BL_THREADS, np);
    hipLaunchKernelGGL(k_bert_ln, dim3((unsigned) rows), dim3(BL_THREADS), 0, m->stream, x, r, np, pstride, bias,
                       wb, D, m->info.ln_eps, y, y16, yq, yd);
    GSVK_LAUNCH_CHECK();
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
    GSVK_REQUIRE(in.hidden % 512 == 0 && in.hidden <= 1024 && in.inter > 0 && in.inter % 512 == 0 &&
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
        const int nq8 = (w.qkv.q8 != nullptr) + (w.ao.q8 != nullptr) + (w.ff1.q8 != nullptr) + (w.ff2.q8 != nullptr);
        GSVK_REQUIRE(nq8 == 0 || nq8 == 4, "BERT GGUF: layer %d mixes Q8_0 and other projection types", li);
        GSVK_REQUIRE(nq8 == 0 || (D == 1024 && F == 4096),
                     "BERT GGUF: Q8_0 projections need hidden 1024 and FFN 4096 (the int8 GEMM's K)");
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
    // workspace: x, qkv, attention output, projection output (up to BERT_MAX_SLICES partial
    // rows), FFN hidden, the fp16 GEMM inputs (a D-wide row, the FFN hidden), the small arrays
    constexpr int BERT_MAX_SLICES = 8;
    const size_t fl = (size_t) rows * (D + 3 * D + D + (size_t) BERT_MAX_SLICES * D + F);
    const int64_t rows64 = (rows + BG_BM - 1) / BG_BM * BG_BM;   // fp16 operands: rows padded to 64
    const size_t n16 = m->any_f16 ? (size_t) rows64 * (D + F) : 0;
    const size_t nq = m->any_q8 ? (size_t) rows * (D + F) : 0;   // Q8_0 activations: quants
    const size_t need = fl * 4 + n16 * 2 + nq + (nq / 32) * 4 + (size_t) rows * 8 + (size_t) B * 8 + 8192;
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
    float * h = prj + (size_t) BERT_MAX_SLICES * rows * D;
    _Float16 * x16 = (_Float16 *) (h + rows * F);            // fp16 input of the D-wide projections
    _Float16 * h16 = m->any_f16 ? x16 + rows64 * D : nullptr;   // fp16 FFN hidden (FFN2's input)
    int8_t * xq = (int8_t *) (x16 + n16);                          // D-wide Q8_0 rows (+ scales)
    int8_t * hq = xq + (m->any_q8 ? rows * D : 0);                  // the FFN hidden's
    float * xqd = (float *) (((uintptr_t) (xq + nq) + 15) & ~(uintptr_t) 15);
    float * hqd = xqd + (m->any_q8 ? rows * D / 32 : 0);
    int32_t * d_ids = (int32_t *) (((uintptr_t) (xqd + nq / 32) + 15) & ~(uintptr_t) 15);
    int32_t * d_pos = d_ids + rows;
    int32_t * d_off = d_pos + rows;
    int32_t * d_len = d_off + B;
    // ids, positions, offsets and lengths packed in pinned memory, one copy (d_ids .. d_len are
    // contiguous); the same buffer takes the features back
    const size_t pin_need = std::max((size_t) (2 * rows + 2 * B) * 4, (size_t) rows * D * 4);
    if (pin_need > m->pin_bytes) {
        if (m->pin) (void) hipHostFree(m->pin);
        m->pin = nullptr;
        m->pin_bytes = 0;
        GSVK_HIP(hipHostMalloc(&m->pin, pin_need, hipHostMallocDefault));
        m->pin_bytes = pin_need;
    }
    {
        int32_t * pk = (int32_t *) m->pin;
        memcpy(pk, ids.data(), rows * 4);
        memcpy(pk + rows, tpos.data(), rows * 4);
        memcpy(pk + 2 * rows, off.data(), (size_t) B * 4);
        memcpy(pk + 2 * rows + B, len.data(), (size_t) B * 4);
    }
    GSVK_HIP(hipMemcpyAsync(d_ids, m->pin, (size_t) (2 * rows + 2 * B) * 4, hipMemcpyHostToDevice, st));

    hipLaunchKernelGGL(k_bert_embed, dim3((unsigned) rows), dim3(256), 0, st, m->word, m->pos, m->type0, d_ids,
                       d_pos, D, prj);
    GSVK_LAUNCH_CHECK();
    // each LayerNorm also writes the fp16 copy (F16 consumer) or the Q8_0 rows (Q8_0 consumer) its
    // consumer takes
    auto x16_for = [&](int li) { return li < n_layers && m->L[li].qkv.f16 ? x16 : nullptr; };
    auto xq_for = [&](int li) { return li < n_layers && m->L[li].qkv.q8 ? xq : nullptr; };
    GSVK_TRY(bert_ln(m, prj, nullptr, 1, 0, nullptr, m->emb_ln, rows, x, x16_for(0), xq_for(0), xqd));
    const float scale_log2 = 1.4426950408889634f / std::sqrt((float) BA_HD);
    auto kmult = [](const Proj & w) { return BG_WAVES * BG_U * (w.f16 ? BgStep<_Float16>::K : BgStep<float>::K); };
    const int64_t pst = rows * D;   // floats between partial rows of the D-wide projections
    for (int li = 0; li < n_layers; li++) {
        const BertLayer & w = m->L[li];
        // QKV (its bias is added as attention reads q, k, v)
        if (w.qkv.q8)
            GSVK_TRY(gemm_q8(m, w.qkv, xq, xqd, rows, 3 * D, D, qkv, nullptr));
        else
            GSVK_TRY(gemm(m, w.qkv, x, x16, rows, 3 * D, D, 1, BgOut{qkv, 0, nullptr, 0, nullptr}));
        hipLaunchKernelGGL(k_bert_attn, dim3((unsigned) ((Tmax + BA_Q - 1) / BA_Q), (unsigned) in.heads, (unsigned) B),
                           dim3(256), 0, st, qkv, w.qkv_b, d_off, d_len, D, scale_log2, att,
                           w.ao.f16 ? x16 : nullptr);
        GSVK_LAUNCH_CHECK();
        // out projection (F16 / F32: in K slices when the rows are few; LN1 sums the slices)
        int s1 = 1;
        if (w.ao.q8) {
            GSVK_TRY(launch_q8_quantize(att, rows, D, xq, xqd, st, Q8_NATURAL));
            GSVK_TRY(gemm_q8(m, w.ao, xq, xqd, rows, D, D, prj, nullptr));
        } else {
            s1 = bert_kslices(rows, D, D, kmult(w.ao), BERT_MAX_SLICES);
            GSVK_TRY(gemm(m, w.ao, att, x16, rows, D, D, s1, BgOut{prj, pst, nullptr, 0, nullptr}));
        }
        GSVK_TRY(bert_ln(m, x, prj, s1, pst, w.ao_b, w.ln1, rows, x, w.ff1.f16 ? x16 : nullptr,
                         w.ff1.q8 ? xq : nullptr, xqd));
        // FFN1 + bias + GELU, FFN2
        int s2 = 1;
        if (w.ff1.q8) {
            GSVK_TRY(gemm_q8(m, w.ff1, xq, xqd, rows, F, D, h, w.ff1_b));
            const int64_t nh = rows * F;
            hipLaunchKernelGGL(k_bert_gelu_q8, dim3((unsigned) ((nh / 4 + 255) / 256)), dim3(256), 0, st, h, nh, hq, hqd);
            GSVK_LAUNCH_CHECK();
            GSVK_TRY(gemm_q8(m, w.ff2, hq, hqd, rows, D, F, prj, nullptr));
        } else {
            // bias + GELU in the FFN1 epilogue, to fp32 (an F32 FFN2) or fp16 (an F16 FFN2)
            GSVK_TRY(gemm(m, w.ff1, x, x16, rows, F, D, 1,
                          BgOut{w.ff2.f16 ? nullptr : h, 0, w.ff1_b, 1, w.ff2.f16 ? h16 : nullptr}));
            s2 = bert_kslices(rows, D, F, kmult(w.ff2), BERT_MAX_SLICES);
            GSVK_TRY(gemm(m, w.ff2, h, h16, rows, D, F, s2, BgOut{prj, pst, nullptr, 0, nullptr}));
        }
        GSVK_TRY(bert_ln(m, x, prj, s2, pst, w.ff2_b, w.ln2, rows, x, x16_for(li + 1), xq_for(li + 1), xqd));
    }
    // [rows][D] -> per sequence [D][len] (src/gsv_bert.cpp:220-228)
    GSVK_HIP(hipMemcpyAsync(m->pin, x, (size_t) rows * D * 4, hipMemcpyDeviceToHost, st));
    GSVK_HIP(hipStreamSynchronize(st));
    const float * host = (const float *) m->pin;
    for (int b = 0; b < B; b++) {
        float * ob = out + (size_t) D * off[b];
        const float * hb = host + (size_t) off[b] * D;
        for (int d = 0; d < D; d++)
            for (int t = 0; t < len[b]; t++) ob[(size_t) d * len[b] + t] = hb[(size_t) t * D + d];
    }
    return GSVK_OK;
}

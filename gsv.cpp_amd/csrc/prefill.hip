// Prefill-only kernels for gfx950: the device-side input build of gsv_ar's impl::build_inputs
// (src/gsv_ar.cpp:186-225) and the masked self-attention of run_first (:257).
//
// Rows of the prefill are (sequence b, position s), s in [0, S), S = max_len + prompt_len, with
// left padding pad_b = max_len - T_b: text token t of sequence b sits at s = pad_b + t, prompt
// token t at s = max_len + t. The attention mask is never materialised: query s of sequence b
// sees keys k >= pad_b with k < max_len when s < max_len (text: bidirectional over text) and
// k <= s otherwise (semantic: causal over text + semantic).
#include "common.h"

namespace gsvk {

// xy[b][s] (src/gsv_ar.cpp:201-214): text_emb[ph] + text_alpha*PE[t] for text rows,
// audio_emb[prompt] + audio_alpha*PE[t] for prompt rows, 0 for padding. One wave per row.
__global__ void __launch_bounds__(64) k_build_xy(const float * __restrict__ text_emb,
                                                 const float * __restrict__ audio_emb,
                                                 const float * __restrict__ pe,
                                                 const int32_t * __restrict__ phones,   // [B][max_len], left-padded
                                                 const int32_t * __restrict__ pad,      // [B]
                                                 const int32_t * __restrict__ prompt,   // [P]
                                                 int S, int max_len, int d, float ta, float aa,
                                                 float * __restrict__ xy) {
    const int row = blockIdx.x;           // b * S + s
    const int b = row / S;
    const int s = row % S;
    const int lane = threadIdx.x;
    float * dst = xy + (int64_t) row * d;
    const int pb = pad[b];
    for (int i = lane; i < d; i += 64) {
        float v = 0.0f;
        if (s >= pb && s < max_len) {
            const int t = s - pb;
            const int ph = phones[(int64_t) b * max_len + s];
            v = __builtin_fmaf(ta, pe[(int64_t) t * d + i], text_emb[(int64_t) ph * d + i]);
        } else if (s >= max_len) {
            const int t = s - max_len;
            v = __builtin_fmaf(aa, pe[(int64_t) t * d + i], audio_emb[(int64_t) prompt[t] * d + i]);
        }
        dst[i] = v;
    }
}

// feat[r][k] for the R text rows listed in row_b/row_t: bert[b][k][t] for k < bert_dim, 1 at
// k == bert_dim (the augmented bias column of bert_aug = [W | b]); zeros for a request without BERT.
__global__ void k_bert_feat(const float * __restrict__ bert, const int64_t * __restrict__ boff,
                            const int32_t * __restrict__ row_b, const int32_t * __restrict__ row_t,
                            const int32_t * __restrict__ tlen, int bert_dim, int R,
                            float * __restrict__ feat) {
    const int r = blockIdx.x;
    if (r >= R) return;
    const int b = row_b[r], t = row_t[r], T = tlen[b];
    const float * src = boff[b] >= 0 ? bert + boff[b] : nullptr;
    float * dst = feat + (int64_t) r * (bert_dim + 1);
    for (int k = threadIdx.x; k <= bert_dim; k += blockDim.x)
        dst[k] = k == bert_dim ? 1.0f : (src ? src[(int64_t) k * T + t] : 0.0f);
}

// cur[b][pad_b + t] = xy + proj[r] (ggml_add(x, mul_mat(bert_aug, feat)), src/gsv_ar.cpp:241).
// Rows r >= R1 belong to requests without BERT features: their feat row is zeros and a trailing 1,
// so the projection is the bias column itself (the zero products add only signed zeros to it).
__global__ void k_add_proj(float * __restrict__ xy, const float * __restrict__ proj,
                           const float * __restrict__ bias, const int32_t * __restrict__ row_b,
                           const int32_t * __restrict__ row_t, const int32_t * __restrict__ pad,
                           int S, int d, int R, int R1) {
    const int r = blockIdx.x;
    if (r >= R) return;
    const int b = row_b[r];
    const int s = pad[b] + row_t[r];
    float * dst = xy + ((int64_t) b * S + s) * d;
    const float * src = r < R1 ? proj + (int64_t) r * d : bias;
    for (int i = threadIdx.x; i < d; i += blockDim.x) dst[i] = dst[i] + src[i];
}

// gather rows: out[b] = in[b * S + S - 1]
__global__ void k_gather_last(const float * __restrict__ in, int S, int d, float * __restrict__ out) {
    const int b = blockIdx.x;
    const float * src = in + ((int64_t) b * S + S - 1) * d;
    for (int i = threadIdx.x; i < d; i += blockDim.x) out[(int64_t) b * d + i] = src[i];
}

// ---------------------------------------------------------------------------------------
// Prefill attention (ggml_flash_attn_ext with F32 Q/K/V, src/gsv_ar.cpp:257).
//
// One lane per query row, 64 queries per workgroup; key tiles of 64 rows of K and V (fp32) are
// staged in LDS and read as broadcasts. Each lane runs ggml-cpu's online softmax over its valid
// keys in increasing order: s = vec_dot_f32(k, q) (GGML_F32x8_REDUCE order), s = s*scale + 0,
// on a new maximum rescale the accumulator by expf(Mold - M), otherwise weight by
// expf(s - M); acc = fma(v, w, acc); S = S*ms + vs (contracted); out = acc * (1/S).
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ float dot32_ggml(const float (&q)[32], const float * __restrict__ k) {
    // 4 accumulators x 8 lanes, one step: products, then REDUCE
    float s[4][8];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int l = 0; l < 8; l++) s[j][l] = __builtin_fmaf(k[8 * j + l], q[8 * j + l], 0.0f);
    float b8[8];
#pragma unroll
    for (int l = 0; l < 8; l++) b8[l] = (s[0][l] + s[2][l]) + (s[1][l] + s[3][l]);
    const float t0 = b8[0] + b8[4], t1 = b8[1] + b8[5], t2 = b8[2] + b8[6], t3 = b8[3] + b8[7];
    return (t0 + t1) + (t2 + t3);
}

constexpr int PA_TILE = 64;

__global__ void __launch_bounds__(64) k_attn_prefill(const float * __restrict__ qkv, int S,
                                                     int max_len, const int32_t * __restrict__ pad,
                                                     int nh, int d_model, float scale,
                                                     float * __restrict__ out,
                                                     int8_t * __restrict__ oq,
                                                     float * __restrict__ od) {
    const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    const int s = tile * PA_TILE + lane;
    const int pb = pad[b];
    const int64_t rs = 3 * (int64_t) d_model;                 // qkv row stride
    const float * base = qkv + (int64_t) b * S * rs;

    __shared__ float sk[PA_TILE][33];
    __shared__ float sv[PA_TILE][33];

    const bool valid_q = s < S;
    float q[32], acc[32];
    const float * qr = base + (int64_t) (valid_q ? s : 0) * rs + h * 32;
#pragma unroll
    for (int i = 0; i < 32; i++) { q[i] = qr[i]; acc[i] = 0.0f; }
    // key range of this query
    const int kb = pb;
    const int ke = valid_q ? (s < max_len ? max_len : s + 1) : 0;
    // key range of the tile (union over lanes)
    const int s_last = min(S - 1, tile * PA_TILE + PA_TILE - 1);
    const int tile_ke = (s_last < max_len) ? max_len : s_last + 1;

    float M = -INFINITY, Ssum = 0.0f;
    for (int k0 = kb - (kb % PA_TILE); k0 < tile_ke; k0 += PA_TILE) {
        __syncthreads();
        {
            const int kr = k0 + lane;
            if (kr < S) {
                const float * kp = base + (int64_t) kr * rs + d_model + h * 32;
                const float * vp = base + (int64_t) kr * rs + 2 * d_model + h * 32;
#pragma unroll
                for (int i = 0; i < 32; i++) { sk[lane][i] = kp[i]; sv[lane][i] = vp[i]; }
            }
        }
        __syncthreads();
        const int jb = max(kb, k0), je = min(ke, k0 + PA_TILE);
        for (int key = jb; key < je; key++) {
            const int kk = key - k0;
            float kv[32];
#pragma unroll
            for (int i = 0; i < 32; i++) kv[i] = sk[kk][i];
            float sc = dot32_ggml(q, kv);
            sc = sc * scale;
            sc = sc + 0.0f;
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            if (sc > M) {
                M = sc;
                ms = expf(Mold - M);
#pragma unroll
                for (int i = 0; i < 32; i++) acc[i] = acc[i] * ms;
            } else {
                vs = expf(sc - M);
            }
#pragma unroll
            for (int i = 0; i < 32; i++) acc[i] = __builtin_fmaf(sv[kk][i], vs, acc[i]);
            Ssum = __builtin_fmaf(Ssum, ms, vs);
        }
    }
    if (!valid_q) return;
    const float sinv = Ssum == 0.0f ? 0.0f : 1.0f / Ssum;
    float o[32];
#pragma unroll
    for (int i = 0; i < 32; i++) o[i] = acc[i] * sinv;
    const int64_t row = (int64_t) b * S + s;
    float * orow = out + row * d_model + h * 32;
#pragma unroll
    for (int i = 0; i < 32; i++) orow[i] = o[i];
    if (oq) {
        // the head's 32 outputs are one Q8_0 block (block h of the row), quantised in-lane
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(o[i]));
        const float dd = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const int nblk = d_model / 32;
        int8_t * qrow = oq + row * d_model;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int packed = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int qv = (int) __builtin_rintf(o[4 * j + t] * id);
                packed |= (qv & 0xff) << (8 * t);
            }
            *reinterpret_cast<int *>(qrow + ((int64_t) j * nblk + h) * 4) = packed;
        }
        od[row * nblk + h] = h2f(f2h(dd));
    }
}

int launch_build_xy(const float * text_emb, const float * audio_emb, const float * pe,
                    const int32_t * phones, const int32_t * pad, const int32_t * prompt, int B,
                    int S, int max_len, int d, float ta, float aa, float * xy, hipStream_t stream) {
    hipLaunchKernelGGL(k_build_xy, dim3((unsigned) (B * S)), dim3(64), 0, stream, text_emb,
                       audio_emb, pe, phones, pad, prompt, S, max_len, d, ta, aa, xy);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_bert_feat(const float * bert, const int64_t * boff, const int32_t * row_b,
                     const int32_t * row_t, const int32_t * tlen, int bert_dim, int R, float * feat,
                     hipStream_t stream) {
    if (R == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_bert_feat, dim3((unsigned) R), dim3(256), 0, stream, bert, boff, row_b,
                       row_t, tlen, bert_dim, R, feat);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_add_proj(float * xy, const float * proj, const float * bias, const int32_t * row_b,
                    const int32_t * row_t, const int32_t * pad, int S, int d, int R, int R1,
                    hipStream_t stream) {
    if (R == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_add_proj, dim3((unsigned) R), dim3(128), 0, stream, xy, proj, bias, row_b,
                       row_t, pad, S, d, R, R1);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_gather_last(const float * in, int B, int S, int d, float * out, hipStream_t stream) {
    hipLaunchKernelGGL(k_gather_last, dim3((unsigned) B), dim3(128), 0, stream, in, S, d, out);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                        int d_model, float scale, float * out, int8_t * oq, float * od,
                        hipStream_t stream) {
    GSVK_REQUIRE(d_model == nh * 32, "attn_prefill: head_dim must be 32");
    const dim3 grid((unsigned) ((S + PA_TILE - 1) / PA_TILE), (unsigned) nh, (unsigned) B);
    hipLaunchKernelGGL(k_attn_prefill, grid, dim3(PA_TILE), 0, stream, qkv, S, max_len, pad, nh,
                       d_model, scale, out, oq, od);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

// Attention rows in ggml-cpu's sequential order, bit for bit (the arithmetic of
// ggml_compute_forward_flash_attn_ext_f16_one_chunk for one query row with F32 K/V, as the oracle
// restates it): for every valid key j in order,
//     s   = dot(k_j, q) * scale            (ggml_vec_dot_f32: 4 x 8 lanes, GGML_F32x8_REDUCE)
//     if s > M: ms = expf(M - s), M = s, acc *= ms     else: vs = expf(s - M)
//     acc = fma(v_j, vs, acc);  S = fma(S, ms, vs)
// out = acc * (S == 0 ? 0 : 1 / S), expf being glibc's (expf_exact.h).
//
// One wave per (query row, head). The keys go in chunks of 256: the lanes compute the chunk's
// scores (each lane its own keys, the 32-dimension dot in ggml's order), the prefix maximum of the
// scores by a scan (max is exact in any order), then each key's ms and vs (they depend only on the
// key's score and the maximum before it); the only sequential part left is each dimension's
// chain acc = fma(v, vs, acc * ms) over the keys (lanes 0..31, one dimension each; a factor ms of
// 1 leaves acc unchanged, as skipping the multiply does) and S's chain (lane 32).
//
// This is the decode's and the prefill's attention when the model runs in exact mode
// (gsvk_model_set_exact): slower than the split kernels, used where the device must reproduce the
// oracle's tokens exactly.
#include "attn_dev.h"
#include "expf_exact.h"
#include "layer.h"

namespace gsvk {

namespace {
constexpr int AX_CH = 256;   // keys per chunk
}

__constant__ uint64_t g_exp2_tab[32] = GSVK_EXP2_TAB32;

// One row: keys [beg, end) at k_row(j), v_row(j) (KV = uint16_t: fp16 cache rows; float: fp32 rows).
template <typename KV>
__device__ __forceinline__ float attn_row_exact(const float * __restrict__ q, const KV * __restrict__ kb,
                                                const KV * __restrict__ vb, int64_t kv_stride, int beg, int end,
                                                float scale, int lane, float * s_sc, float * s_ms, float * s_vs) {
    auto ld = [](const KV * p) -> float {
        if constexpr (sizeof(KV) == 2) return h2f(*p);
        else return *p;
    };
    float qv[32];
#pragma unroll
    for (int d = 0; d < 32; d++) qv[d] = q[d];
    float M = -INFINITY;   // uniform over the wave
    float acc = 0.0f;      // lane d < 32: dimension d
    float S = 0.0f;        // lane 32
    const int dl = lane & 31;
    for (int c0 = beg; c0 < end; c0 += AX_CH) {
        const int n = min(AX_CH, end - c0);
        // scores of the chunk, each lane its own keys, ggml's dot order
        for (int t = lane; t < n; t += 64) {
            const KV * kr = kb + (int64_t) (c0 + t) * kv_stride;
            float s4[4][8];
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
#pragma unroll
                for (int l = 0; l < 8; l++) s4[jj][l] = __builtin_fmaf(ld(kr + 8 * jj + l), qv[8 * jj + l], 0.0f);
            float s0[8];
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const float a = s4[0][l] + s4[2][l];
                const float c = s4[1][l] + s4[3][l];
                s0[l] = a + c;
            }
            const float t0 = s0[0] + s0[4], t1 = s0[1] + s0[5], t2 = s0[2] + s0[6], t3 = s0[3] + s0[7];
            s_sc[t] = ((t0 + t1) + (t2 + t3)) * scale;
        }
        __builtin_amdgcn_wave_barrier();
        // the maximum before each key: lane l takes keys 4l .. 4l + 3 of the chunk
        float v4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v4[i] = 4 * lane + i < n ? s_sc[4 * lane + i] : -INFINITY;
        const float mx = fmaxf(fmaxf(v4[0], v4[1]), fmaxf(v4[2], v4[3]));
        float ex = mx;   // inclusive scan of the lane maxima, then shifted to exclusive
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(ex, off, 64);
            if (lane >= off) ex = fmaxf(ex, o);
        }
        float before = __shfl_up(ex, 1, 64);
        before = lane == 0 ? M : fmaxf(M, before);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 4 * lane + i;
            if (t < n) {
                const float s = v4[i];
                float ms = 1.0f, vs = 1.0f;
                if (s > before) ms = expf_glibc(before - s, g_exp2_tab);
                else vs = expf_glibc(s - before, g_exp2_tab);
                s_ms[t] = ms;
                s_vs[t] = vs;
                before = fmaxf(before, s);
            }
        }
        M = fmaxf(M, __shfl(ex, 63, 64));
        __builtin_amdgcn_wave_barrier();
        // the sequential chains
        if (lane < 32) {
            const KV * vr = vb + (int64_t) c0 * kv_stride + dl;
            int t = 0;
            for (; t + 8 <= n; t += 8) {
                float vv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) vv[u] = ld(vr + (int64_t) (t + u) * kv_stride);
#pragma unroll
                for (int u = 0; u < 8; u++) acc = __builtin_fmaf(vv[u], s_vs[t + u], acc * s_ms[t + u]);
            }
            for (; t < n; t++) acc = __builtin_fmaf(ld(vr + (int64_t) t * kv_stride), s_vs[t], acc * s_ms[t]);
        } else if (lane == 32) {
            for (int t = 0; t < n; t++) S = __builtin_fmaf(S, s_ms[t], s_vs[t]);
        }
        __builtin_amdgcn_wave_barrier();
    }
    S = __shfl(S, 32, 64);
    const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
    return acc * sinv;
}

// decode: workgroup (head h, sequence b); q rows of q_stride floats (q of head h at 32h)
__global__ void __launch_bounds__(64) k_attn_exact_decode(const float * __restrict__ q, int64_t q_stride,
                                                          const uint16_t * __restrict__ kc,
                                                          const uint16_t * __restrict__ vc, int nh, int64_t lstride,
                                                          const int32_t * __restrict__ kv_begin,
                                                          const int32_t * __restrict__ kv_end, float scale,
                                                          float * __restrict__ out, int8_t * __restrict__ oq,
                                                          float * __restrict__ od, int oq_layout) {
    __shared__ float s_sc[AX_CH], s_ms[AX_CH], s_vs[AX_CH];
    const int h = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x;
    int beg = kv_begin[b], end = kv_end[b];
    beg = beg < 0 ? 0 : beg;
    end = end > (int) lstride ? (int) lstride : end;
    const int64_t bh = (int64_t) b * nh + h;
    const uint16_t * kb = kc + bh * lstride * ATT_HD;
    const uint16_t * vb = vc + bh * lstride * ATT_HD;
    const float val = attn_row_exact<uint16_t>(q + (int64_t) b * q_stride + h * ATT_HD, kb, vb, ATT_HD, beg,
                                               end > beg ? end : beg, scale, lane, s_sc, s_ms, s_vs);
    attn_store_out(val, lane, bh, nh, out, nullptr, oq, od, oq_layout);
}

// prefill: workgroup (head h, query row i, sequence b); qkv rows [B][S][3 d_model]; query i of
// sequence b sees keys [pad[b], max_len) when i < max_len (text rows), else [pad[b], i]
__global__ void __launch_bounds__(64) k_attn_exact_prefill(const float * __restrict__ qkv, int S, int max_len,
                                                           const int32_t * __restrict__ pad, int nh, int d_model,
                                                           float scale, float * __restrict__ out,
                                                           int8_t * __restrict__ oq, float * __restrict__ od) {
    __shared__ float s_sc[AX_CH], s_ms[AX_CH], s_vs[AX_CH];
    const int h = blockIdx.x, i = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    int beg = pad[b];
    beg = beg < 0 ? 0 : (beg > S ? S : beg);
    int end = i < max_len ? max_len : i + 1;
    end = end > S ? S : end;
    const int64_t row3 = (int64_t) 3 * d_model;
    const float * base = qkv + (int64_t) b * S * row3;
    const float val = attn_row_exact<float>(base + (int64_t) i * row3 + h * ATT_HD, base + d_model + h * ATT_HD,
                                            base + 2 * d_model + h * ATT_HD, row3, beg, end > beg ? end : beg, scale,
                                            lane, s_sc, s_ms, s_vs);
    attn_store_out(val, lane, ((int64_t) b * S + i) * nh + h, nh, out, nullptr, oq, od, Q8_SLICED);
}

int launch_attn_exact_decode(const float * q, int64_t q_stride, const uint16_t * k, const uint16_t * v, int B,
                             int nh, int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end,
                             float scale, float * out, int8_t * oq, float * od, hipStream_t stream,
                             int oq_layout) {
    GSVK_REQUIRE(q && k && v && kv_begin && kv_end && out && B > 0 && B <= 65535 && nh > 0 && nh <= 65535 &&
                     lstride > 0 && q_stride >= (int64_t) nh * ATT_HD,
                 "attn_exact_decode: bad arguments");
    GSVK_REQUIRE((oq == nullptr) == (od == nullptr), "attn_exact_decode: oq and od go together");
    hipLaunchKernelGGL(k_attn_exact_decode, dim3((unsigned) nh, (unsigned) B), dim3(64), 0, stream, q, q_stride, k,
                       v, nh, lstride, kv_begin, kv_end, scale, out, oq, od, oq_layout);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_attn_exact_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                              int d_model, float scale, float * out, int8_t * oq, float * od, hipStream_t stream) {
    GSVK_REQUIRE(qkv && pad && out && B > 0 && B <= 65535 && S > 0 && S <= 65535 && nh > 0 && nh <= 65535 &&
                     nh * ATT_HD == d_model && max_len >= 0 && max_len <= S,
                 "attn_exact_prefill: bad arguments");
    GSVK_REQUIRE((oq == nullptr) == (od == nullptr), "attn_exact_prefill: oq and od go together");
    hipLaunchKernelGGL(k_attn_exact_prefill, dim3((unsigned) nh, (unsigned) S, (unsigned) B), dim3(64), 0, stream,
                       qkv, S, max_len, pad, nh, d_model, scale, out, oq, od);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_attn_exact(const float * q, const uint16_t * k, const uint16_t * v, int B, int nh,
                                  int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end, float scale,
                                  float * out, int8_t * oq, float * od, void * stream) {
    return gsvk::launch_attn_exact_decode(q, (int64_t) nh * gsvk::ATT_HD, k, v, B, nh, lstride, kv_begin, kv_end,
                                          scale, out, oq, od, (hipStream_t) stream, gsvk::Q8_SLICED);
}

namespace gsvk {
__global__ void k_expf_exact(const float * __restrict__ x, int64_t n, float * __restrict__ y) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = expf_glibc(x[i], g_exp2_tab);
}
}  // namespace gsvk

extern "C" int gsvk_op_expf_exact(const float * x, int64_t n, float * y, void * stream) {
    GSVK_REQUIRE(x && y && n >= 0 && n < ((int64_t) 1 << 40), "expf_exact: bad arguments");
    if (n == 0) return GSVK_OK;
    hipLaunchKernelGGL(gsvk::k_expf_exact, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, (hipStream_t) stream,
                       x, n, y);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

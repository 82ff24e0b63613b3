// This is the decode's and the prefill's attention when the model runs in exact mode
// (gsvk_model_set_exact): slower than the split kernels, used where the device must reproduce the
// oracle's tokens exactly.
//
// Per chunk (8 KB of keys: 128 fp16 rows or 64 fp32 rows) the wave loads K and V with 16-byte
// loads into registers, the next chunk's loads going out before the current chunk's chains run;
// K is stored to LDS by rows (each lane reads its keys' rows for the scores), V transposed, so
// that the lane of dimension d reads 8 consecutive keys of its dimension at once. The chain of a
// dimension is acc = fma(v, vs, acc * ms); for a key that sets no new maximum ms is exactly 1 and
// the step is one fma, acc = fma(v, vs, acc), which S's chain shares in the same instruction
// stream (lane 32: S = fma(vs, 1, S), equal to fma(S, 1, vs)). Groups of 8 keys holding a new
// maximum (a per-lane flag collected by a ballot) take the general step.
#include "attn_dev.h"
#include "expf_exact.h"
#include "layer.h"

namespace gsvk {

__constant__ uint64_t g_exp2_tab[32] = GSVK_EXP2_TAB32;

namespace {

constexpr int AX_CHUNK_BYTES = 8192;   // bytes of K (and of V) per chunk

template <typename KV>
struct AxShape {
    static constexpr int ROWB = 32 * (int) sizeof(KV);             // bytes per key row
    static constexpr int CH = AX_CHUNK_BYTES / ROWB;               // keys per chunk
    static constexpr int E16 = 16 / (int) sizeof(KV);              // elements per 16-byte load
    static constexpr int PARTS = ROWB / 16;                        // 16-byte loads per row
    static constexpr int U = AX_CHUNK_BYTES / 16 / 64;             // loads per lane per matrix
    static constexpr int KPL = CH / 64;                            // keys per lane in the scan
};

template <typename KV>
__device__ __forceinline__ float ax_val(KV x) {
    if constexpr (sizeof(KV) == 2) return h2f(x);
    else return x;
}

// word k of a uint4 (k a compile-time constant after unrolling)
__device__ __forceinline__ uint32_t u4w(const uint4 & w, int k) {
    return k == 0 ? w.x : (k == 1 ? w.y : (k == 2 ? w.z : w.w));
}

// element i of a 16-byte load of KV values, as stored (raw fp16 bits or the float)
template <typename KV>
__device__ __forceinline__ KV ax_elem(const uint4 & w, int i) {
    if constexpr (sizeof(KV) == 2) return (uint16_t) (u4w(w, i >> 1) >> (16 * (i & 1)));
    else return __builtin_bit_cast(float, u4w(w, i));
}

// LDS of one wave
template <typename KV>
struct AxLds {
    uint4 k[AX_CHUNK_BYTES / 16];                     // K rows of the chunk
    KV vt[32][AxShape<KV>::CH];                       // V transposed: [dimension][key]
    float sc[AxShape<KV>::CH], ms[AxShape<KV>::CH], vs[AxShape<KV>::CH];
};

// the 16-byte loads of the chunk's keys [c0, c0 + n), n >= 1, of one matrix: every load is
// issued, a slot past the last key reading the last key again (in bounds; never used)
template <typename KV>
__device__ __forceinline__ void ax_load(const KV * __restrict__ base, int64_t kv_stride, int c0, int n, int lane,
                                        uint4 (&r)[AxShape<KV>::U]) {
    using S = AxShape<KV>;
#pragma unroll
    for (int u = 0; u < S::U; u++) {
        const int idx = lane + 64 * u;
        const int key = min(idx / S::PARTS, n - 1), part = idx % S::PARTS;
        r[u] = *reinterpret_cast<const uint4 *>(base + (int64_t) (c0 + key) * kv_stride + part * S::E16);
    }
}

}  // namespace

// One row: keys [beg, end) at kb + j * kv_stride, vb + j * kv_stride (KV = uint16_t: fp16 cache
// rows; float: fp32 rows). Returns dimension `lane` of the output in lanes 0..31.
template <typename KV>
__device__ __forceinline__ float attn_row_exact(const float * __restrict__ q, const KV * __restrict__ kb,
                                                const KV * __restrict__ vb, int64_t kv_stride, int beg, int end,
                                                float scale, int lane, AxLds<KV> & L) {
    using S = AxShape<KV>;
    float qv[32];
#pragma unroll
    for (int d = 0; d < 32; d++) qv[d] = q[d];
    const bool is_lo = lane < 32, is_s = lane == 32;
    const int dl = lane & 31;
    float M = -INFINITY;   // uniform over the wave
    float acc = 0.0f;      // lanes 0..31: dimension lane; lane 32: S
    uint4 kr[S::U], vr[S::U];
    if (beg < end) {   // uniform
        ax_load<KV>(kb, kv_stride, beg, min(S::CH, end - beg), lane, kr);
        ax_load<KV>(vb, kv_stride, beg, min(S::CH, end - beg), lane, vr);
    } else {
#pragma unroll
        for (int u = 0; u < S::U; u++) kr[u] = vr[u] = make_uint4(0, 0, 0, 0);
    }
    for (int c0 = beg; c0 < end; c0 += S::CH) {
        const int n = min(S::CH, end - c0);
        // the chunk into LDS: K by rows, V transposed
#pragma unroll
        for (int u = 0; u < S::U; u++) {
            const int idx = lane + 64 * u;
            L.k[idx] = kr[u];
            const int key = idx / S::PARTS, d0 = (idx % S::PARTS) * S::E16;
#pragma unroll
            for (int i = 0; i < S::E16; i++) L.vt[d0 + i][key] = ax_elem<KV>(vr[u], i);
        }
        __builtin_amdgcn_wave_barrier();
        // the next chunk's loads go out now and arrive while this chunk is worked on (after the
        // last chunk: one key of this chunk again, issued unconditionally so that the registers
        // stay registers across the loop)
        {
            const bool more = c0 + S::CH < end;
            const int cn = more ? c0 + S::CH : c0;
            const int nn = more ? min(S::CH, end - cn) : 1;
            ax_load<KV>(kb, kv_stride, cn, nn, lane, kr);
            ax_load<KV>(vb, kv_stride, cn, nn, lane, vr);
        }
        // scores, each lane its own keys, ggml_vec_dot_f32's order
        for (int t = lane; t < n; t += 64) {
            const uint4 * kr4 = &L.k[t * S::PARTS];
            float kf[32];
#pragma unroll
            for (int pp = 0; pp < S::PARTS; pp++) {
                const uint4 w = kr4[pp];
#pragma unroll
                for (int i = 0; i < S::E16; i++) kf[pp * S::E16 + i] = ax_val<KV>(ax_elem<KV>(w, i));
            }
            float s4[4][8];
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
#pragma unroll
                for (int l = 0; l < 8; l++) s4[jj][l] = __builtin_fmaf(kf[8 * jj + l], qv[8 * jj + l], 0.0f);
            float s0[8];
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const float a = s4[0][l] + s4[2][l];
                const float c = s4[1][l] + s4[3][l];
                s0[l] = a + c;
            }
            const float t0 = s0[0] + s0[4], t1 = s0[1] + s0[5], t2 = s0[2] + s0[6], t3 = s0[3] + s0[7];
            L.sc[t] = ((t0 + t1) + (t2 + t3)) * scale;
        }
        __builtin_amdgcn_wave_barrier();
        // the maximum before each key (lane l: keys KPL l .. KPL l + KPL - 1), then ms and vs
        float v4[S::KPL];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < S::KPL; i++) {
            v4[i] = S::KPL * lane + i < n ? L.sc[S::KPL * lane + i] : -INFINITY;
            mx = fmaxf(mx, v4[i]);
        }
        float ex = mx;   // inclusive scan of the lane maxima, then shifted to exclusive
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(ex, off, 64);
            if (lane >= off) ex = fmaxf(ex, o);
        }
        float before = __shfl_up(ex, 1, 64);
        before = lane == 0 ? M : fmaxf(M, before);
        bool newmax = false;
#pragma unroll
        for (int i = 0; i < S::KPL; i++) {
            const int t = S::KPL * lane + i;
            if (t < n) {
                const float sv = v4[i];
                float ms = 1.0f, vs = 1.0f;
                if (sv > before) ms = expf_glibc(before - sv, g_exp2_tab);
                else vs = expf_glibc(sv - before, g_exp2_tab);
                newmax |= ms != 1.0f;
                L.ms[t] = ms;
                L.vs[t] = vs;
                before = fmaxf(before, sv);
            }
        }
        const uint64_t slow = __ballot(newmax);
        M = fmaxf(M, __shfl(ex, 63, 64));
        __builtin_amdgcn_wave_barrier();
        // the chains: lanes 0..31 acc of their dimension, lane 32 S
        int t = 0;
        for (; t + 8 <= n; t += 8) {
            float vv[8];
            if constexpr (sizeof(KV) == 2) {
                const uint4 w = *reinterpret_cast<const uint4 *>(&L.vt[dl][t]);
#pragma unroll
                for (int i = 0; i < 8; i++) vv[i] = ax_val<KV>(ax_elem<KV>(w, i));
            } else {
                const float4 a = *reinterpret_cast<const float4 *>(&L.vt[dl][t]);
                const float4 b = *reinterpret_cast<const float4 *>(&L.vt[dl][t + 4]);
                vv[0] = a.x; vv[1] = a.y; vv[2] = a.z; vv[3] = a.w;
                vv[4] = b.x; vv[5] = b.y; vv[6] = b.z; vv[7] = b.w;
            }
            const float4 vs0 = *reinterpret_cast<const float4 *>(&L.vs[t]);
            const float4 vs1 = *reinterpret_cast<const float4 *>(&L.vs[t + 4]);
            const float vsv[8] = {vs0.x, vs0.y, vs0.z, vs0.w, vs1.x, vs1.y, vs1.z, vs1.w};
            const uint64_t gbits = (slow >> (t / S::KPL)) & ((1ull << (8 / S::KPL)) - 1);
            if (gbits == 0) {   // no new maximum among the 8 keys: ms = 1
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float A = is_s ? vsv[i] : (is_lo ? vv[i] : 0.0f);
                    const float B = is_s ? 1.0f : (is_lo ? vsv[i] : 0.0f);
                    acc = __builtin_fmaf(A, B, acc);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float ms = L.ms[t + i];
                    const float lo = __builtin_fmaf(vv[i], vsv[i], acc * ms);
                    const float hs = __builtin_fmaf(acc, ms, vsv[i]);
                    acc = is_s ? hs : (is_lo ? lo : 0.0f);
                }
            }
        }
        for (; t < n; t++) {
            const float v = ax_val<KV>(L.vt[dl][t]);
            const float ms = L.ms[t], vs = L.vs[t];
            const float lo = __builtin_fmaf(v, vs, acc * ms);
            const float hs = __builtin_fmaf(acc, ms, vs);
            acc = is_s ? hs : (is_lo ? lo : 0.0f);
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float Ssum = __shfl(acc, 32, 64);
    const float sinv = Ssum == 0.0f ? 0.0f : 1.0f / Ssum;
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
    __shared__ AxLds<uint16_t> lds;
    const int h = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x;
    int beg = kv_begin[b], end = kv_end[b];
    beg = beg < 0 ? 0 : beg;
    end = end > (int) lstride ? (int) lstride : end;
    const int64_t bh = (int64_t) b * nh + h;
    const uint16_t * kb = kc + bh * lstride * ATT_HD;
    const uint16_t * vb = vc + bh * lstride * ATT_HD;
    const float val = attn_row_exact<uint16_t>(q + (int64_t) b * q_stride + h * ATT_HD, kb, vb, ATT_HD, beg,
                                               end > beg ? end : beg, scale, lane, lds);
    attn_store_out(val, lane, bh, nh, out, nullptr, oq, od, oq_layout);
}

// prefill: workgroup (head h, query row i, sequence b); qkv rows [B][S][3 d_model]; query i of
// sequence b sees keys [pad[b], max_len) when i < max_len (text rows), else [pad[b], i]
__global__ void __launch_bounds__(64) k_attn_exact_prefill(const float * __restrict__ qkv, int S, int max_len,
                                                           const int32_t * __restrict__ pad, int nh, int d_model,
                                                           float scale, float * __restrict__ out,
                                                           int8_t * __restrict__ oq, float * __restrict__ od) {
    __shared__ AxLds<float> lds;
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
                                            lane, lds);
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

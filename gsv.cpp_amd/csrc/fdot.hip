// Dot products of F16 / F32 weight rows with fp32 activation rows (the logits head and the
// prefill BERT projection), reproducing ggml-cpu's x86 summation order:
//
//  MODE 0 — ggml_vec_dot_f16 / ggml_vec_dot_f32 (decode, and any K not a multiple of 8):
//    4 accumulators of 8 lanes, sum[j][l] = fma(w[32i+8j+l], x[32i+8j+l], sum[j][l]) for every
//    full step of 32; GGML_F32x8_REDUCE: sum0+=sum2, sum1+=sum3, sum0+=sum1, then
//    t_i = s_i + s_{i+4} and ((t0+t1) + (t2+t3)); the k % 32 leftovers are fused in order.
//    GPU: 32 lanes per output row, lane p = 8j + l owns one accumulator; the reduction is the
//    xor-16, xor-8, xor-4, xor-1, xor-2 butterfly, which performs exactly those additions.
//  MODE 1 — llamafile tinyBLAS (prefill with >= 2 activation columns, K % 8 == 0):
//    one accumulator of 8 lanes, a[l] = fma(w[8i+l], x[8i+l], a[l]); hsum
//    ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) = xor-4, xor-2, xor-1 butterfly over 8 lanes.
//
// For F16 weights the activations are first rounded to fp16 (ggml's vec_dot_type for F16).
#include "common.h"
#include "layer_dev.h"

namespace gsvk {

template <typename WT>
__device__ __forceinline__ float wload(const WT * p);
template <>
__device__ __forceinline__ float wload<float>(const float * p) { return *p; }
template <>
__device__ __forceinline__ float wload<uint16_t>(const uint16_t * p) { return h2f(*p); }

__device__ __forceinline__ float xconv(float x, bool x16) { return x16 ? h2f(f2h(x)) : x; }

// MODE 0: 256 threads = 8 rows x 32 lanes; grid (ceil(n/8), ceil(m/MT))
template <typename WT, int MT>
__global__ void __launch_bounds__(256) k_fdot_ggml(const WT * __restrict__ W, int n, int k,
                                                   const float * __restrict__ X, int64_t xs, int m,
                                                   float * __restrict__ Y, int64_t ys) {
    const bool x16 = sizeof(WT) == 2;
    const int p = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int m0 = blockIdx.y * MT;
    const int rowc = row < n ? row : n - 1;
    const WT * wr = W + (int64_t) rowc * k;
    const int np = k & ~31;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;
    for (int i = 0; i < np; i += 32) {
        const float w = wload<WT>(wr + i + p);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int mm = m0 + t < m ? m0 + t : m - 1;
            acc[t] = __builtin_fmaf(w, xconv(X[(int64_t) mm * xs + i + p], x16), acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
        float v = acc[t];
        v = v + __shfl_xor(v, 16, 64);
        v = v + __shfl_xor(v, 8, 64);
        v = v + __shfl_xor(v, 4, 64);
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        acc[t] = v;
    }
    if (p != 0 || row >= n) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int mm = m0 + t;
        if (mm < m) {
            float v = acc[t];
            for (int i = np; i < k; i++)
                v = __builtin_fmaf(wload<WT>(wr + i), xconv(X[(int64_t) mm * xs + i], x16), v);
            Y[(int64_t) mm * ys + row] = v;
        }
    }
}

// MODE 0 for many activation rows (the prefill's BERT projection, m in the thousands): each
// thread keeps the same chains as k_fdot_ggml (slice lane p, fma over the steps of 32 in order,
// then the butterfly and the leftovers), for RN weight rows x MT activation rows at once, so a
// step costs RN + MT loads for RN * MT FMAs and the weights are re-read once per MT rows.
// 256 threads = 8 groups of 32 lanes; workgroup tile 8*RN weight rows x MT activation rows.
template <typename WT, int RN, int MT>
__global__ void __launch_bounds__(256) k_fdot_ggml_t(const WT * __restrict__ W, int n, int k,
                                                     const float * __restrict__ X, int64_t xs, int m,
                                                     float * __restrict__ Y, int64_t ys) {
    const bool x16 = sizeof(WT) == 2;
    const int p = threadIdx.x & 31;
    const int n0 = blockIdx.x * (8 * RN) + (threadIdx.x >> 5) * RN;
    const int m0 = blockIdx.y * MT;
    const WT * wr[RN];
    const float * xr[MT];
#pragma unroll
    for (int j = 0; j < RN; j++) wr[j] = W + (int64_t) min(n0 + j, n - 1) * k;
#pragma unroll
    for (int t = 0; t < MT; t++) xr[t] = X + (int64_t) min(m0 + t, m - 1) * xs;
    const int np = k & ~31;
    float acc[RN][MT];
#pragma unroll
    for (int j = 0; j < RN; j++)
#pragma unroll
        for (int t = 0; t < MT; t++) acc[j][t] = 0.0f;
    for (int i = 0; i < np; i += 32) {
        float w[RN], x[MT];
#pragma unroll
        for (int j = 0; j < RN; j++) w[j] = wload<WT>(wr[j] + i + p);
#pragma unroll
        for (int t = 0; t < MT; t++) x[t] = xconv(xr[t][i + p], x16);
#pragma unroll
        for (int j = 0; j < RN; j++)
#pragma unroll
            for (int t = 0; t < MT; t++) acc[j][t] = __builtin_fmaf(w[j], x[t], acc[j][t]);
    }
#pragma unroll
    for (int j = 0; j < RN; j++)
#pragma unroll
        for (int t = 0; t < MT; t++) {
            float v = acc[j][t];
            v = v + __shfl_xor(v, 16, 64);
            v = v + __shfl_xor(v, 8, 64);
            v = v + __shfl_xor(v, 4, 64);
            v = v + __shfl_xor(v, 1, 64);
            v = v + __shfl_xor(v, 2, 64);
            acc[j][t] = v;
        }
    if (p != 0) return;
#pragma unroll
    for (int j = 0; j < RN; j++)
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int row = n0 + j, mm = m0 + t;
            if (row < n && mm < m) {
                float v = acc[j][t];
                for (int i = np; i < k; i++)
                    v = __builtin_fmaf(wload<WT>(wr[j] + i), xconv(xr[t][i], x16), v);
                Y[(int64_t) mm * ys + row] = v;
            }
        }
}

// MODE 0 with K = 32 * NI known at compile time (the decode head, K = 512): the same arithmetic
// as k_fdot_ggml, with every load issued up front. The MT activation rows (rounded to fp16 for
// F16 weights) are staged once per workgroup in LDS with 16-byte loads; each lane loads its NI
// weights before the first use. 256 threads = 8 rows x 32 lanes; grid (ceil(n/8), ceil(m/MT)).
// LNIN: the MT rows are LayerNorm((res + r) + bias) * w + b of the decoder's last layer,
// computed here (one wave per row, the arithmetic of the LayerNorm kernel) instead of read from X.
struct LnSrc {
    const float * res, * r, * bias, * wb;
    // (NPARTS > 0) r = parts[0] + parts[1] + ... in that order, part g of row m at
    // parts + g * pstride + m * 512 (the FFN2 partial rows of the two-launch decode layer)
    const float * parts;
    int64_t pstride;
};

template <typename WT, int MT, int NI, bool LNIN = false, int NPARTS = 0>
__global__ void __launch_bounds__(256) k_fdot_ggml_k(const WT * __restrict__ W, int n,
                                                     const float * __restrict__ X, int64_t xs, int m,
                                                     float * __restrict__ Y, int64_t ys, LnSrc ln) {
    constexpr int K = 32 * NI;
    static_assert(!LNIN || (K == 512 && MT % 4 == 0), "LayerNorm input: rows of 512, MT / 4 rows per wave");
    const bool x16 = sizeof(WT) == 2;
    const int tid = threadIdx.x;
    const int p = tid & 31;
    const int row = blockIdx.x * 8 + (tid >> 5);
    const int m0 = blockIdx.y * MT;
    const int rowc = row < n ? row : n - 1;
    __shared__ __align__(16) float s_x[MT][K];
    constexpr int X4 = MT * K / 4;                       // float4 chunks of the MT rows
    constexpr int XN = LNIN ? 1 : (X4 + 255) / 256;
    constexpr int LR = LNIN ? MT / 4 : 1;                // LayerNorm rows per wave
    float4 xv[XN];
    LnRow lr[LR];
    const int wave = tid >> 6, lane = tid & 63;
    if constexpr (LNIN) {
#pragma unroll
        for (int u = 0; u < LR; u++) {
            const int mm = min(m0 + wave + 4 * u, m - 1);
            ln_row_load(ln.res + (int64_t) mm * K, (ln.r && NPARTS == 0) ? ln.r + (int64_t) mm * K : g_zero_row,
                        ln.bias ? ln.bias : g_zero_row, ln.wb, lane, lr[u]);
            if constexpr (NPARTS > 0) {
                float4 pa[NPARTS], pb[NPARTS];
#pragma unroll
                for (int g = 0; g < NPARTS; g++) {
                    const gf4ptr pp = as_global_f4(ln.parts + g * ln.pstride + (int64_t) mm * K + lane * 8);
                    pa[g] = ld4(pp, 0);
                    pb[g] = ld4(pp, 1);
                }
                float4 ra = pa[0], rb = pb[0];
#pragma unroll
                for (int g = 1; g < NPARTS; g++) {
                    ra.x = ra.x + pa[g].x; ra.y = ra.y + pa[g].y; ra.z = ra.z + pa[g].z; ra.w = ra.w + pa[g].w;
                    rb.x = rb.x + pb[g].x; rb.y = rb.y + pb[g].y; rb.z = rb.z + pb[g].z; rb.w = rb.w + pb[g].w;
                }
                lr[u].ra = ra;
                lr[u].rb = rb;
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < XN; u++) {
            int c = tid + u * 256;
            c = c < X4 ? c : X4 - 1;
            const int mm = min(m0 + c / (K / 4), m - 1);
            xv[u] = *reinterpret_cast<const float4 *>(X + (int64_t) mm * xs + (c % (K / 4)) * 4);
        }
    }
    const WT * wr = W + (int64_t) rowc * K;
    float w[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) w[i] = wload<WT>(wr + 32 * i + p);
    if constexpr (LNIN) {
#pragma unroll
        for (int u = 0; u < LR; u++) {
            float o[8];
            ln_row_compute(lr[u], o);
            float * dst = &s_x[wave + 4 * u][lane * 8];
#pragma unroll
            for (int i = 0; i < 8; i++) dst[i] = xconv(o[i], x16);
        }
    } else {
#pragma unroll
        for (int u = 0; u < XN; u++) {
            const int c = tid + u * 256;
            if (c < X4) {
                float4 v = xv[u];
                v.x = xconv(v.x, x16); v.y = xconv(v.y, x16); v.z = xconv(v.z, x16); v.w = xconv(v.w, x16);
                *reinterpret_cast<float4 *>(&s_x[c / (K / 4)][(c % (K / 4)) * 4]) = v;
            }
        }
    }
    __syncthreads();
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int t = 0; t < MT; t++) acc[t] = __builtin_fmaf(w[i], s_x[t][32 * i + p], acc[t]);
#pragma unroll
    for (int t = 0; t < MT; t++) {
        float v = acc[t];
        v = v + __shfl_xor(v, 16, 64);
        v = v + __shfl_xor(v, 8, 64);
        v = v + __shfl_xor(v, 4, 64);
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        acc[t] = v;
    }
    if (p != 0 || row >= n) return;
#pragma unroll
    for (int t = 0; t < MT; t++)
        if (m0 + t < m) Y[(int64_t) (m0 + t) * ys + row] = acc[t];
}

// MODE 1: 256 threads = 32 rows x 8 lanes; grid (ceil(n/32), ceil(m/MT))
template <typename WT, int MT>
__global__ void __launch_bounds__(256) k_fdot_tinyblas(const WT * __restrict__ W, int n, int k,
                                                       const float * __restrict__ X, int64_t xs,
                                                       int m, float * __restrict__ Y, int64_t ys) {
    const bool x16 = sizeof(WT) == 2;
    const int l = threadIdx.x & 7;
    const int row = blockIdx.x * 32 + (threadIdx.x >> 3);
    const int m0 = blockIdx.y * MT;
    const int rowc = row < n ? row : n - 1;
    const WT * wr = W + (int64_t) rowc * k;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;
    for (int i = 0; i < k; i += 8) {
        const float w = wload<WT>(wr + i + l);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int mm = m0 + t < m ? m0 + t : m - 1;
            acc[t] = __builtin_fmaf(w, xconv(X[(int64_t) mm * xs + i + l], x16), acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
        float v = acc[t];
        v = v + __shfl_xor(v, 4, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 1, 64);
        acc[t] = v;
    }
    if (l != 0 || row >= n) return;
#pragma unroll
    for (int t = 0; t < MT; t++)
        if (m0 + t < m) Y[(int64_t) (m0 + t) * ys + row] = acc[t];
}

// MODE 0 on the fp32 matrix cores for many activation rows of F32 weights (fdot_mfma.hip)
int launch_fdot_mfma(const float * W, int64_t n, int64_t k, const float * X, int64_t xs, int64_t m, float * Y,
                     int64_t ys, hipStream_t stream);

// wtype: 0 = F32, 1 = F16. mode: 0 = ggml vec_dot, 1 = tinyBLAS (falls back to 0 if k % 8).
int launch_fdot(const void * W, int wtype, int64_t n, int64_t k, const float * X, int64_t xs,
                int64_t m, float * Y, int64_t ys, int mode, hipStream_t stream) {
    GSVK_REQUIRE(W && X && Y && (wtype == 0 || wtype == 1), "fdot: bad arguments");
    GSVK_REQUIRE(n > 0 && k > 0 && m > 0 && n < (1 << 30) && k < (1 << 24) && m < (1 << 30) &&
                     xs >= k && ys >= n,
                 "fdot: bad shape n=%lld k=%lld m=%lld", (long long) n, (long long) k,
                 (long long) m);
    constexpr int MT = 4;
    if (mode == 1 && k % 8 == 0) {
        const dim3 grid((unsigned) ((n + 31) / 32), (unsigned) ((m + MT - 1) / MT));
        if (wtype == 1)
            hipLaunchKernelGGL((k_fdot_tinyblas<uint16_t, MT>), grid, dim3(256), 0, stream,
                               (const uint16_t *) W, (int) n, (int) k, X, xs, (int) m, Y, ys);
        else
            hipLaunchKernelGGL((k_fdot_tinyblas<float, MT>), grid, dim3(256), 0, stream,
                               (const float *) W, (int) n, (int) k, X, xs, (int) m, Y, ys);
    } else if (k == 512 && xs % 4 == 0 && ((uintptr_t) X & 15) == 0) {
        constexpr int MTK = 8;
        const dim3 grid((unsigned) ((n + 7) / 8), (unsigned) ((m + MTK - 1) / MTK));
        if (wtype == 1)
            hipLaunchKernelGGL((k_fdot_ggml_k<uint16_t, MTK, 16>), grid, dim3(256), 0, stream,
                               (const uint16_t *) W, (int) n, X, xs, (int) m, Y, ys, LnSrc{});
        else
            hipLaunchKernelGGL((k_fdot_ggml_k<float, MTK, 16>), grid, dim3(256), 0, stream,
                               (const float *) W, (int) n, X, xs, (int) m, Y, ys, LnSrc{});
    } else if (m >= 64 && wtype == 0 && n % 32 == 0 && k >= 64 && (k & ~31) % 64 == 0 &&
               (n / 32) * ((m + 31) / 32) < (1LL << 31)) {
        return launch_fdot_mfma((const float *) W, n, k, X, xs, m, Y, ys, stream);
    } else if (m >= 64) {
        constexpr int RN = 4, MTT = 16;
        const dim3 grid((unsigned) ((n + 8 * RN - 1) / (8 * RN)), (unsigned) ((m + MTT - 1) / MTT));
        if (wtype == 1)
            hipLaunchKernelGGL((k_fdot_ggml_t<uint16_t, RN, MTT>), grid, dim3(256), 0, stream,
                               (const uint16_t *) W, (int) n, (int) k, X, xs, (int) m, Y, ys);
        else
            hipLaunchKernelGGL((k_fdot_ggml_t<float, RN, MTT>), grid, dim3(256), 0, stream,
                               (const float *) W, (int) n, (int) k, X, xs, (int) m, Y, ys);
    } else {
        const dim3 grid((unsigned) ((n + 7) / 8), (unsigned) ((m + MT - 1) / MT));
        if (wtype == 1)
            hipLaunchKernelGGL((k_fdot_ggml<uint16_t, MT>), grid, dim3(256), 0, stream,
                               (const uint16_t *) W, (int) n, (int) k, X, xs, (int) m, Y, ys);
        else
            hipLaunchKernelGGL((k_fdot_ggml<float, MT>), grid, dim3(256), 0, stream,
                               (const float *) W, (int) n, (int) k, X, xs, (int) m, Y, ys);
    }
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

namespace gsvk {

// The decode head (K = 512, mode 0) with the last layer's LayerNorm as its input stage: logits
// of m rows of LayerNorm((res + r) + bias) * w + b, in the order of launch_fdot's K = 512 kernel.
int launch_head_ln(const void * W, int wtype, int64_t n, const float * res, const float * r, const float * bias,
                   const float * wb, int64_t m, float * Y, int64_t ys, hipStream_t stream) {
    GSVK_REQUIRE(W && res && wb && Y && (wtype == 0 || wtype == 1) && n > 0 && n < (1 << 30) && m > 0 &&
                     m < (1 << 30) && ys >= n,
                 "head_ln: bad arguments");
    auto al16 = [](const void * p) { return ((uintptr_t) p & 15) == 0; };
    GSVK_REQUIRE(al16(res) && al16(r) && al16(bias) && al16(wb), "head_ln: operands must be 16-byte aligned");
    constexpr int MTK = 8;
    const dim3 grid((unsigned) ((n + 7) / 8), (unsigned) ((m + MTK - 1) / MTK));
    const LnSrc ln{res, r, bias, wb};
    if (wtype == 1)
        hipLaunchKernelGGL((k_fdot_ggml_k<uint16_t, MTK, 16, true>), grid, dim3(256), 0, stream,
                           (const uint16_t *) W, (int) n, nullptr, 512, (int) m, Y, ys, ln);
    else
        hipLaunchKernelGGL((k_fdot_ggml_k<float, MTK, 16, true>), grid, dim3(256), 0, stream,
                           (const float *) W, (int) n, nullptr, 512, (int) m, Y, ys, ln);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

// The decode head after the two-launch layer: LayerNorm((res + parts[0] + ... + parts[15]) +
// bias) of each row, then the F16 / F32 head (4 rows per workgroup: one per wave).
int launch_head_ln_parts(const void * W, int wtype, int64_t n, const float * res, const float * parts,
                         int nparts, int64_t pstride, const float * bias, const float * wb, int64_t m,
                         float * Y, int64_t ys, hipStream_t stream) {
    GSVK_REQUIRE(W && res && parts && wb && Y && (wtype == 0 || wtype == 1) && n > 0 && n < (1 << 30) &&
                     m > 0 && m < (1 << 30) && ys >= n && (nparts == 16 || nparts == 32) && pstride >= m * 512,
                 "head_ln_parts: bad arguments");
    auto al16 = [](const void * p) { return ((uintptr_t) p & 15) == 0; };
    GSVK_REQUIRE(al16(res) && al16(parts) && al16(bias) && al16(wb) && pstride % 4 == 0,
                 "head_ln_parts: operands must be 16-byte aligned");
    constexpr int MTK = 4;
    const dim3 grid((unsigned) ((n + 7) / 8), (unsigned) ((m + MTK - 1) / MTK));
    const LnSrc ln{res, nullptr, bias, wb, parts, pstride};
#define GSVK_HEAD(WT, NP)                                                                           \
    hipLaunchKernelGGL((k_fdot_ggml_k<WT, MTK, 16, true, NP>), grid, dim3(256), 0, stream, (const WT *) W, (int) n, \
                       nullptr, 512, (int) m, Y, ys, ln)
    if (wtype == 1) {
        if (nparts == 32) GSVK_HEAD(uint16_t, 32); else GSVK_HEAD(uint16_t, 16);
    } else {
        if (nparts == 32) GSVK_HEAD(float, 32); else GSVK_HEAD(float, 16);
    }
#undef GSVK_HEAD
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_fdot(const void * w, int wtype, int64_t n, int64_t k, const float * x,
                            int64_t m, float * y, int mode, void * stream) {
    return gsvk::launch_fdot(w, wtype, n, k, x, k, m, y, n, mode, (hipStream_t) stream);
}

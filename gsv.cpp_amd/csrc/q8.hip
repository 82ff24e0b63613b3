// Q8_0 kernels for gfx950: dequantisation, repacking to the device layout, activation
// quantisation (ggml-cpu x86 semantics) and the GEMV/GEMM on raw int8 blocks.
//
// Q8_0 block (GGUF / ggml): { fp16 d; int8 qs[32]; } = 34 bytes, value = fp32(d) * qs[i].
//
// Device layout ("sliced"): a row of k values (nblk = k/32 blocks) is stored as
//     qs[row][j][blk][t] = q[blk*32 + 4*j + t]      j in [0,8), t in [0,4)
// plus d[row][blk] (fp16 for weights, fp32 for activations). Slice j of a row is the
// contiguous int32 sequence of the j-th 4-byte group of every block. ggml-cpu's x86 dot
// (ggml_vec_dot_q8_0_q8_0 / tinyBLAS_Q0_AVX) keeps 8 fp32 lanes, lane j accumulating
// fma(dw*dx, sum of the products of group j, acc_j) block after block, and reduces the lanes
// as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). With the sliced layout lane j of a GPU row reads
// its groups with 16-byte loads, runs the same FMA chain (one v_dot4_i32_i8 per group) and the
// 8 lanes combine with the xor-4, xor-2, xor-1 butterfly, which is that reduction order, so the
// result equals the reference's to the bit.
#include "common.h"
#include "layer.h"

namespace gsvk {

// ---------------------------------------------------------------------------------------
// dequant / repack
// ---------------------------------------------------------------------------------------

__global__ void k_q8_dequant(const uint8_t * __restrict__ blocks, int64_t nblocks,
                             float * __restrict__ out) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;   // one thread per value
    if (i >= nblocks * QK) return;
    const int64_t b = i / QK;
    const int w = (int) (i % QK);
    const uint8_t * blk = blocks + b * Q8_BLOCK_BYTES;
    const uint16_t d = (uint16_t) blk[0] | ((uint16_t) blk[1] << 8);
    out[i] = h2f(d) * (float) (int8_t) blk[2 + w];
}

// one thread per (block, group j): copies 4 quants to their slice position (and, when qn / qt
// are given, to their natural / tiled positions)
__global__ void k_q8_repack(const uint8_t * __restrict__ blocks, int64_t rows, int nblk,
                            int8_t * __restrict__ qs, uint16_t * __restrict__ d, int8_t * __restrict__ qn,
                            int8_t * __restrict__ qt, uint16_t * __restrict__ dt) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = rows * nblk * 8;
    if (i >= total) return;
    const int j = (int) (i & 7);
    const int64_t gb = i >> 3;                 // global block = row * nblk + blk
    const int64_t row = gb / nblk;
    const int blk = (int) (gb % nblk);
    const uint8_t * src = blocks + gb * Q8_BLOCK_BYTES;
    int8_t * dst = qs + ((row * 8 + j) * nblk + blk) * 4;
#pragma unroll
    for (int t = 0; t < 4; t++) dst[t] = (int8_t) src[2 + 4 * j + t];
    if (qn) {
#pragma unroll
        for (int t = 0; t < 4; t++) qn[gb * QK + 4 * j + t] = (int8_t) src[2 + 4 * j + t];
    }
    if (qt) {
#pragma unroll
        for (int t = 0; t < 4; t++) qt[q8_tiled_offset(row, nblk, blk, 4 * j + t)] = (int8_t) src[2 + 4 * j + t];
    }
    const uint16_t dv = (uint16_t) src[0] | ((uint16_t) src[1] << 8);
    if (j == 0) {
        d[gb] = dv;
        if (dt) dt[q8_tiled_scale(row, nblk, blk)] = dv;
    }
}

// The sliced (qs, d) and natural (qn) copies of a weight stored in the matrix-core operand
// order (qt, dt: the on-disk tiled layout of a pre-swizzled GGUF); one thread per 4-quant
// group, the inverse of k_q8_repack's tiled store.
__global__ void k_q8_untile(const int8_t * __restrict__ qt, const uint16_t * __restrict__ dt, int64_t rows,
                            int nblk, int8_t * __restrict__ qs, uint16_t * __restrict__ d,
                            int8_t * __restrict__ qn) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nblk * 8) return;
    const int j = (int) (i & 7);
    const int64_t gb = i >> 3;
    const int64_t row = gb / nblk;
    const int blk = (int) (gb % nblk);
    int8_t * dst = qs + ((row * 8 + j) * nblk + blk) * 4;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int8_t v = qt[q8_tiled_offset(row, nblk, blk, 4 * j + t)];
        dst[t] = v;
        qn[gb * QK + 4 * j + t] = v;
    }
    if (j == 0) d[gb] = dt[q8_tiled_scale(row, nblk, blk)];
}

// ---------------------------------------------------------------------------------------
// activation quantisation: 4 lanes per 32-block, 8 consecutive values each
// ---------------------------------------------------------------------------------------

__global__ void __launch_bounds__(64) k_q8_quantize(const float * __restrict__ x, int64_t rows,
                                                   int k, int8_t * __restrict__ xs,
                                                   float * __restrict__ xd, int layout) {
    const int nblk = k / QK;
    const int64_t gblk = (int64_t) blockIdx.x * 16 + (threadIdx.x >> 2);   // global block id
    const int sub = threadIdx.x & 3;
    if (gblk >= rows * nblk) return;
    const int64_t row = gblk / nblk;
    const int blk = (int) (gblk % nblk);
    const float * src = x + gblk * QK + sub * 8;
    float v[8];
    const float4 a = *reinterpret_cast<const float4 *>(src);
    const float4 b = *reinterpret_cast<const float4 *>(src + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    int8_t q[8];
    const float d = q8_quantize_group<8>(v, q, 4);
    q8_store_row8(xs, xd, layout, row, nblk, blk, sub, q, d, sub == 0);
}

// ---------------------------------------------------------------------------------------
// GEMV / GEMM: y[m][n] = sum_blk fp32(wd[n][blk]) * xd[m][blk] * dot_i8(w[n][blk], x[m][blk])
//
// Workgroup = one wave = 8 output rows x 8 slice lanes; grid.y splits the m rows in tiles of
// MT. A lane first issues every load it needs — its whole weight slice and the row's scales
// (from HBM), then the activation slices and scales of its MT rows (from L2) — and only then runs
// the FMA chains, so a launch costs about one memory latency. NB4 = nblk/4 is a compile-time
// constant for the model's two row lengths (512 and 2048); other lengths use the NB4 = 0 loop.
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ float q8_chain4(float a, const int4 & w, const int4 & xv, float dw0,
                                           float dw1, float dw2, float dw3, const float4 & dx) {
    a = __builtin_fmaf(dw0 * dx.x, (float) __builtin_amdgcn_sdot4(w.x, xv.x, 0, false), a);
    a = __builtin_fmaf(dw1 * dx.y, (float) __builtin_amdgcn_sdot4(w.y, xv.y, 0, false), a);
    a = __builtin_fmaf(dw2 * dx.z, (float) __builtin_amdgcn_sdot4(w.z, xv.z, 0, false), a);
    a = __builtin_fmaf(dw3 * dx.w, (float) __builtin_amdgcn_sdot4(w.w, xv.w, 0, false), a);
    return a;
}

__device__ __forceinline__ void q8_gemv_epilogue(const GemvEpilogue & epi, int row, int mm, int n,
                                                 float v, float * __restrict__ y) {
    if (epi.bias) v = v + epi.bias[row];
    if (epi.act == 1) v = v > 0.0f ? v : 0.0f;
    y[(int64_t) mm * n + row] = v;
    if (epi.kc && row >= epi.kv_row0) {
        const int rr = row - epi.kv_row0;              // [0, 2*d_model)
        const int which = rr / epi.d_model;            // 0 = K, 1 = V
        const int hd = rr % epi.d_model;
        const int h = hd >> 5, dd = hd & 31;
        const int b = mm / epi.rows_per_seq;
        const int col = *epi.col_ptr + epi.col_add + mm % epi.rows_per_seq;
        uint16_t * cache = which == 0 ? epi.kc : epi.vc;
        cache[(((int64_t) b * epi.n_head + h) * epi.lstride + col) * 32 + dd] = f2h(v);
    }
}

template <int NB4, int MT>
__global__ void __launch_bounds__(64) k_q8_gemv(const int8_t * __restrict__ ws,
                                                const uint16_t * __restrict__ wd, int n, int k,
                                                const int8_t * __restrict__ xs,
                                                const float * __restrict__ xd, int m,
                                                GemvEpilogue epi, float * __restrict__ y) {
    const int lane = threadIdx.x;
    const int r = lane >> 3;
    const int j = lane & 7;
    const int row = blockIdx.x * 8 + r;
    const int m0 = blockIdx.y * MT;
    const int nblk = NB4 > 0 ? NB4 * 4 : k >> 5;
    const bool valid = row < n;
    const int rowc = valid ? row : n - 1;
    const int4 * wsl = reinterpret_cast<const int4 *>(ws + ((int64_t) rowc * 8 + j) * nblk * 4);
    const uint2 * wdr = reinterpret_cast<const uint2 *>(wd + (int64_t) rowc * nblk);

    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;

    if constexpr (NB4 > 0) {
        int4 w[NB4];
        uint2 dh[NB4];
#pragma unroll
        for (int i = 0; i < NB4; i++) {
            w[i] = wsl[i];
            dh[i] = wdr[i];
        }
        int4 xv[MT][NB4];
        float4 dx[MT][NB4];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int mm = m0 + t < m ? m0 + t : m - 1;
            const int4 * xsl = reinterpret_cast<const int4 *>(xs + ((int64_t) mm * 8 + j) * nblk * 4);
            const float4 * xdr = reinterpret_cast<const float4 *>(xd + (int64_t) mm * nblk);
#pragma unroll
            for (int i = 0; i < NB4; i++) {
                xv[t][i] = xsl[i];
                dx[t][i] = xdr[i];
            }
        }
#pragma unroll
        for (int i = 0; i < NB4; i++) {
            const float dw0 = h2f((uint16_t) (dh[i].x & 0xffff)), dw1 = h2f((uint16_t) (dh[i].x >> 16));
            const float dw2 = h2f((uint16_t) (dh[i].y & 0xffff)), dw3 = h2f((uint16_t) (dh[i].y >> 16));
#pragma unroll
            for (int t = 0; t < MT; t++) acc[t] = q8_chain4(acc[t], w[i], xv[t][i], dw0, dw1, dw2, dw3, dx[t][i]);
        }
    } else {
        for (int i = 0; i < nblk / 4; i++) {
            const int4 w = wsl[i];
            const uint2 dh = wdr[i];
            const float dw0 = h2f((uint16_t) (dh.x & 0xffff)), dw1 = h2f((uint16_t) (dh.x >> 16));
            const float dw2 = h2f((uint16_t) (dh.y & 0xffff)), dw3 = h2f((uint16_t) (dh.y >> 16));
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int mm = m0 + t < m ? m0 + t : m - 1;
                const int4 xv = reinterpret_cast<const int4 *>(xs + ((int64_t) mm * 8 + j) * nblk * 4)[i];
                const float4 dx = reinterpret_cast<const float4 *>(xd + (int64_t) mm * nblk)[i];
                acc[t] = q8_chain4(acc[t], w, xv, dw0, dw1, dw2, dw3, dx);
            }
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
    if (!valid) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int mm = m0 + t;
        if (mm < m && (t & 7) == j) q8_gemv_epilogue(epi, row, mm, n, acc[t], y);
    }
}

int launch_q8_gemv(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, const int8_t * xs,
                   const float * xd, int64_t m, const GemvEpilogue & epi, float * y,
                   hipStream_t stream) {
    GSVK_REQUIRE(ws && wd && xs && xd && y, "q8_gemv: null pointer");
    GSVK_REQUIRE(n > 0 && k > 0 && k % 128 == 0 && m > 0 && n < (1 << 30) && m < (1 << 30) &&
                     k <= (1 << 16),
                 "q8_gemv: unsupported shape n=%lld k=%lld m=%lld (k %% 128 == 0)", (long long) n,
                 (long long) k, (long long) m);
    GSVK_REQUIRE(epi.act == 0 || epi.act == 1, "q8_gemv: act must be 0 or 1");
    if (epi.kc) {
        GSVK_REQUIRE(epi.vc && epi.col_ptr && epi.rows_per_seq > 0 && epi.d_model % 32 == 0 &&
                         epi.kv_row0 >= 0 && epi.kv_row0 + 2 * epi.d_model <= n,
                     "q8_gemv: bad KV epilogue");
    }
    const unsigned gx = (unsigned) ((n + 7) / 8);
#define GSVK_GEMV(NB4, MT)                                                                          \
    hipLaunchKernelGGL((k_q8_gemv<NB4, MT>), dim3(gx, (unsigned) ((m + MT - 1) / MT)), dim3(64), 0, \
                       stream, ws, wd, (int) n, (int) k, xs, xd, (int) m, epi, y)
    if (k == 512) {
        if (m <= 16) GSVK_GEMV(4, 2);
        else GSVK_GEMV(4, 4);
    } else if (k == 2048) {
        if (m <= 16) GSVK_GEMV(16, 1);
        else GSVK_GEMV(16, 2);
    } else {
        GSVK_GEMV(0, 4);
    }
#undef GSVK_GEMV
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_q8_quantize(const float * x, int64_t rows, int64_t k, int8_t * xs, float * xd,
                       hipStream_t stream, int layout) {
    GSVK_REQUIRE(x && xs && xd && rows >= 0 && k > 0 && k % QK == 0 && k <= (1 << 20),
                 "q8_quantize: bad arguments (k must be a multiple of 32)");
    GSVK_REQUIRE(layout >= Q8_SLICED && layout <= Q8_TILED, "q8_quantize: bad layout %d", layout);
    const int64_t nb = rows * (k / QK);
    if (nb == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_q8_quantize, dim3((unsigned) ((nb + 15) / 16)), dim3(64), 0, stream, x,
                       rows, (int) k, xs, xd, layout);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_q8_repack(const void * blocks, int64_t rows, int64_t k, int8_t * qs, uint16_t * d,
                     hipStream_t stream, int8_t * qn, int8_t * qt, uint16_t * dt) {
    GSVK_REQUIRE(blocks && qs && d && rows >= 0 && k > 0 && k % QK == 0 && k <= (1 << 20),
                 "q8_repack: bad arguments (k must be a multiple of 32)");
    GSVK_REQUIRE((qt == nullptr) == (dt == nullptr) && (!qt || rows % 32 == 0),
                 "q8_repack: the tiled copy needs quants and scales, and rows %% 32 == 0");
    const int nblk = (int) (k / QK);
    const int64_t total = rows * nblk * 8;
    if (total == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_q8_repack, dim3((unsigned) ((total + 255) / 256)), dim3(256), 0, stream,
                       (const uint8_t *) blocks, rows, nblk, qs, d, qn, qt, dt);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_q8_untile(const int8_t * qt, const uint16_t * dt, int64_t rows, int64_t k, int8_t * qs, uint16_t * d,
                     int8_t * qn, hipStream_t stream) {
    GSVK_REQUIRE(qt && dt && qs && d && qn && rows >= 0 && rows % 32 == 0 && k > 0 && k % QK == 0 &&
                     k <= (1 << 20),
                 "q8_untile: bad arguments (rows %% 32 == 0, k %% 32 == 0)");
    const int nblk = (int) (k / QK);
    const int64_t total = rows * nblk * 8;
    if (total == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_q8_untile, dim3((unsigned) ((total + 255) / 256)), dim3(256), 0, stream, qt, dt, rows,
                       nblk, qs, d, qn);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

using namespace gsvk;

extern "C" int gsvk_op_q8_dequant(const void * blocks, int64_t nblocks, float * out, void * stream) {
    GSVK_REQUIRE(blocks && out && nblocks >= 0 && nblocks < ((int64_t) 1 << 36),
                 "gsvk_op_q8_dequant: bad arguments");
    if (nblocks == 0) return GSVK_OK;
    const int64_t n = nblocks * QK;
    hipLaunchKernelGGL(k_q8_dequant, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t) stream, (const uint8_t *) blocks, nblocks, out);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

extern "C" int gsvk_op_q8_repack(const void * blocks, int64_t rows, int64_t k, int8_t * qs,
                                 uint16_t * d, void * stream) {
    return launch_q8_repack(blocks, rows, k, qs, d, (hipStream_t) stream);
}

extern "C" int gsvk_op_q8_quantize(const float * x, int64_t rows, int64_t k, int8_t * xq,
                                   float * xd, void * stream) {
    return launch_q8_quantize(x, rows, k, xq, xd, (hipStream_t) stream);
}

extern "C" int gsvk_op_q8_gemv(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k,
                               const int8_t * xq, const float * xd, int64_t m, const float * bias,
                               int act, float * y, void * stream) {
    if ((k == 512 || k == 2048) && n % 32 == 0 && wq && wd && xq && xd) {
        // the decoder's own fused kernel, input stage reading Q8_0 rows
        LayerIn in{};
        in.mode = IN_Q8;
        in.xs = xq;
        in.xd = xd;
        LayerOut out{};
        out.y = y;
        out.y_stride = n;
        out.n_store = (int) n;
        out.bias = bias;
        out.act = act;
        GSVK_REQUIRE(y, "q8_gemv: null pointer");
        GSVK_REQUIRE(act == 0 || act == 1, "q8_gemv: act must be 0 or 1");
        return launch_layer_gemv(wq, wd, n, k, m, in, out, (hipStream_t) stream);
    }
    GemvEpilogue epi{};
    epi.bias = bias;
    epi.act = act;
    return launch_q8_gemv(wq, wd, n, k, xq, xd, m, epi, y, (hipStream_t) stream);
}

extern "C" int gsvk_op_ln_gemv(const int8_t * wq, const uint16_t * wd, int64_t n, const float * res,
                               const float * r, const float * ln_bias, const float * wb, int64_t m,
                               const float * bias, int act, float * y, float * ln_out,
                               void * stream) {
    GSVK_REQUIRE(wq && wd && res && wb && y, "ln_gemv: null pointer");
    GSVK_REQUIRE(act == 0 || act == 1, "ln_gemv: act must be 0 or 1");
    LayerIn in{};
    in.mode = IN_LN;
    in.res = res;
    in.r = r;
    in.bias = ln_bias;
    in.wb = wb;
    in.out_x = ln_out;
    LayerOut out{};
    out.y = y;
    out.y_stride = n;
    out.n_store = (int) n;
    out.bias = bias;
    out.act = act;
    return launch_layer_gemv(wq, wd, n, 512, m, in, out, (hipStream_t) stream);
}

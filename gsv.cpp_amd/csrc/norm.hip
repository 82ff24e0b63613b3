// Row-wise kernels for gfx950: the fused LayerNorm(x + r + bias) * w + b with optional Q8_0
// output, the fused add + activation, and the embedding + positional-encoding gather.
//
// All of them run one wave (64 lanes) per row; each lane owns chunks of 8 consecutive floats
// (two 16-byte loads), so four neighbouring lanes hold exactly one Q8_0 block of 32.
#include "common.h"

namespace gsvk {

// ---------------------------------------------------------------------------------------
// LayerNorm (PATCH:1533-1584): v = (x + r) + bias; mean and E[v^2] accumulated in double;
// mean = float(sum / n); var = float(sum2 / n) - mean * mean; inv = 1 / sqrtf(var + eps);
// y = (v - mean) * inv * w + b. The reference's Linux build (GCC, -mfma, GNU mode) contracts
// `a - mean*mean` and `t*w + b` into single FMAs; this file is compiled without contraction and
// writes exactly those two FMAs, so every other operation rounds where the C expression does.
// ---------------------------------------------------------------------------------------

template <int MAXC, bool F16OUT>
__global__ void __launch_bounds__(256) k_layernorm(const float * __restrict__ x,
                                                  const float * __restrict__ r,
                                                  const float * __restrict__ bias,
                                                  const float * __restrict__ wb, int rows, int n,
                                                  float eps, float * __restrict__ y,
                                                  int8_t * __restrict__ yq,
                                                  float * __restrict__ yd, int layout,
                                                  uint16_t * __restrict__ y16,
                                                  const int32_t * __restrict__ row_pad, int rows_per_seq) {
    // one wave per row, up to 4 rows per workgroup (the waves are independent: no barrier)
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    // a left-padding row (prefill) is normalised from zeros instead of its stale input: its
    // output is the LayerNorm bias, finite, without reading the row (no valid row reads it, but
    // the matrix-core tiles that mix padding and valid rows multiply it)
    const bool pad_row = row_pad && row % rows_per_seq < row_pad[row / rows_per_seq];
    const int lane = threadIdx.x & 63;
    const int nchunk = n / 8;
    const float * xr = x + (int64_t) row * n;
    const float * rr = r ? r + (int64_t) row * n : nullptr;
    float v[MAXC][8];
    double s = 0.0, s2 = 0.0;
    // 16-byte loads, all issued before the first use; the branches are uniform
    // (the LayerNorm weight and bias too: they are not needed until after the reductions, but a
    // load issued then would be a second memory round trip)
    float4 xv[MAXC][2], rv[MAXC][2], bv[MAXC][2], wv[MAXC][2], cv[MAXC][2];
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const int base = (lane + 64 * c) * 8;
        const bool act = lane + 64 * c < nchunk;
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        xv[c][0] = xv[c][1] = wv[c][0] = wv[c][1] = cv[c][0] = cv[c][1] = z;
        if (act && !pad_row) {   // (an explicit branch: a select of the load would become per-word loads)
            xv[c][0] = *reinterpret_cast<const float4 *>(xr + base);
            xv[c][1] = *reinterpret_cast<const float4 *>(xr + base + 4);
        }
        if (act) {
            wv[c][0] = *reinterpret_cast<const float4 *>(wb + base);
            wv[c][1] = *reinterpret_cast<const float4 *>(wb + base + 4);
            cv[c][0] = *reinterpret_cast<const float4 *>(wb + n + base);
            cv[c][1] = *reinterpret_cast<const float4 *>(wb + n + base + 4);
        }
        rv[c][0] = rv[c][1] = bv[c][0] = bv[c][1] = z;
        if (rr && act && !pad_row) {
            rv[c][0] = *reinterpret_cast<const float4 *>(rr + base);
            rv[c][1] = *reinterpret_cast<const float4 *>(rr + base + 4);
        }
        if (bias && act && !pad_row) {
            bv[c][0] = *reinterpret_cast<const float4 *>(bias + base);
            bv[c][1] = *reinterpret_cast<const float4 *>(bias + base + 4);
        }
    }
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        if (lane + 64 * c < nchunk) {
            const float xs[8] = {xv[c][0].x, xv[c][0].y, xv[c][0].z, xv[c][0].w,
                                 xv[c][1].x, xv[c][1].y, xv[c][1].z, xv[c][1].w};
            const float rs[8] = {rv[c][0].x, rv[c][0].y, rv[c][0].z, rv[c][0].w,
                                 rv[c][1].x, rv[c][1].y, rv[c][1].z, rv[c][1].w};
            const float bs[8] = {bv[c][0].x, bv[c][0].y, bv[c][0].z, bv[c][0].w,
                                 bv[c][1].x, bv[c][1].y, bv[c][1].z, bv[c][1].w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float t = (xs[i] + rs[i]) + bs[i];   // + 0 leaves the value unchanged
                v[c][i] = t;
                s += (double) t;
                s2 += (double) t * (double) t;
            }
        }
    }
    s = wave_sum_d_uniform(s);
    s2 = wave_sum_d_uniform(s2);
    const float mean = (float) (s / (double) n);
    const float var = __builtin_fmaf(-mean, mean, (float) (s2 / (double) n));
    const float inv = 1.0f / __builtin_sqrtf(var + eps);
    float * yr = y + (int64_t) row * n;
    const int nblk = n / QK;
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const int ch = lane + 64 * c;
        const bool act = ch < nchunk;
        float o[8];
        if (act) {
            const int base = ch * 8;
            const float ws[8] = {wv[c][0].x, wv[c][0].y, wv[c][0].z, wv[c][0].w,
                                 wv[c][1].x, wv[c][1].y, wv[c][1].z, wv[c][1].w};
            const float bs[8] = {cv[c][0].x, cv[c][0].y, cv[c][0].z, cv[c][0].w,
                                 cv[c][1].x, cv[c][1].y, cv[c][1].z, cv[c][1].w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                o[i] = __builtin_fmaf((v[c][i] - mean) * inv, ws[i], bs[i]);
                if constexpr (F16OUT) y16[(int64_t) row * n + base + i] = f2h(o[i]);   // fp16 copy, nearest even
            }
            *reinterpret_cast<float4 *>(yr + base) = make_float4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<float4 *>(yr + base + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
        if (yq && (64 * c) < nchunk) {   // uniform across the wave
            if (!act) {
#pragma unroll
                for (int i = 0; i < 8; i++) o[i] = 0.0f;
            }
            int8_t q[8];
            const float d = q8_quantize_group<8>(o, q, 4);
            if (act) q8_store_row8(yq, yd, layout, row, nblk, ch >> 2, ch & 3, q, d, (ch & 3) == 0);
        }
    }
}

// ---------------------------------------------------------------------------------------
// add + activation (PATCH:1586-1620)
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 1) return v > 0.0f ? v : 0.0f;
    if (act == 2) return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
    if (act == 3) {
        const float sp = v > 20.0f ? v : log1pf(expf(v));
        return v * tanhf(sp);
    }
    return v;
}

__global__ void k_add_act(const float * __restrict__ a, const float * __restrict__ b, int64_t n,
                          int64_t ne0, int act, float * __restrict__ y) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    y[i] = apply_act(a[i] + b[i % ne0], act);
}

int launch_add_act(const float * a, const float * b, int64_t n, int64_t ne0, int act, float * y, hipStream_t stream) {
    GSVK_REQUIRE(a && b && y && n >= 0 && ne0 > 0 && act >= 0 && act <= 3, "add_act: bad arguments");
    if (n == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_add_act, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream, a, b, n, ne0, act, y);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

// ---------------------------------------------------------------------------------------
// QKV rows of an F16 / F32 projection (src/gsv_ar.cpp:244-255, :271-275, :392-399): y += bias in
// place (the ggml_add after the mul_mat), and the K and V parts, rounded to fp16, appended to the
// caches: row r belongs to sequence r / rows_per_seq and goes to column
// *col_ptr + col_add + r % rows_per_seq. One thread per element of a row of 3 * d_model.
// ---------------------------------------------------------------------------------------

__global__ void k_bias_kv(float * __restrict__ y, const float * __restrict__ bias, int64_t rows, int d_model,
                          uint16_t * __restrict__ kc, uint16_t * __restrict__ vc, int n_head, int64_t lstride,
                          int rows_per_seq, const int32_t * __restrict__ col_ptr, int col_add) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int w = 3 * d_model;
    if (i >= rows * w) return;
    const int64_t r = i / w;
    const int c = (int) (i - r * w);
    const float v = y[i] + bias[c];
    y[i] = v;
    if (c < d_model) return;
    const int which = c / d_model, j = c - which * d_model;
    const int64_t seq = r / rows_per_seq;
    const int64_t col = (int64_t) *col_ptr + col_add + r % rows_per_seq;
    if (col < 0 || col >= lstride) return;
    uint16_t * dst = which == 1 ? kc : vc;
    dst[((seq * n_head + j / 32) * lstride + col) * 32 + (j & 31)] = f2h(v);
}

int launch_bias_kv(float * y, const float * bias, int64_t rows, int d_model, uint16_t * kc, uint16_t * vc,
                   int n_head, int64_t lstride, int rows_per_seq, const int32_t * col_ptr, int col_add,
                   hipStream_t stream) {
    GSVK_REQUIRE(y && bias && kc && vc && col_ptr && rows >= 0 && rows_per_seq > 0 && n_head * 32 == d_model &&
                     lstride > 0 && rows * 3 * d_model < ((int64_t) 1 << 40),
                 "bias_kv: bad arguments");
    const int64_t n = rows * 3 * d_model;
    if (n == 0) return GSVK_OK;
    hipLaunchKernelGGL(k_bias_kv, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream, y, bias, rows, d_model,
                       kc, vc, n_head, lstride, rows_per_seq, col_ptr, col_add);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

// ---------------------------------------------------------------------------------------
// embedding + PE (src/gsv_ar.cpp:798-807): x[b] = emb[tok[b]] + alpha * pe[*pos_ptr + pos_add],
// with its Q8_0 copy (in the given layout), and kv_end[b] = *pos_ptr + kv_end_add
// when kv_end is given (the step's attention range, as the GEMV's embedding stage sets it). One
// wave per row; d_model must be 512.
// ---------------------------------------------------------------------------------------

__global__ void __launch_bounds__(64) k_embed_pe(const float * __restrict__ emb,
                                                 const float * __restrict__ pe,
                                                 const int32_t * __restrict__ tok, int vocab,
                                                 const int32_t * __restrict__ pos_ptr,
                                                 int pos_add, float alpha, int d,
                                                 float * __restrict__ x,
                                                 int8_t * __restrict__ xq,
                                                 float * __restrict__ xd,
                                                 int32_t * __restrict__ kv_end, int kv_end_add,
                                                 const int32_t * __restrict__ pos_sub, int pe_rows,
                                                 int layout) {
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    int t = tok[b];
    t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
    const int step = *pos_ptr;
    int pos = step + pos_add - (pos_sub ? pos_sub[b] : 0);
    pos = pos < 0 ? 0 : (pe_rows > 0 && pos >= pe_rows ? pe_rows - 1 : pos);
    if (kv_end && lane == 0) kv_end[b] = step + kv_end_add;
    const float * er = emb + (int64_t) t * d + lane * 8;
    const float * pr = pe + (int64_t) pos * d + lane * 8;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        o[i] = __builtin_fmaf(alpha, pr[i], er[i]);   // emb + alpha * pe, contracted
        x[(int64_t) b * d + lane * 8 + i] = o[i];
    }
    int8_t q[8];
    const float dq = q8_quantize_group<8>(o, q, 4);
    q8_store_row8(xq, xd, layout, b, d / QK, lane >> 2, lane & 3, q, dq, (lane & 3) == 0);
}

int launch_layernorm(const float * x, const float * r, const float * bias, const float * wb,
                     int64_t rows, int64_t n, float eps, float * y, int8_t * yq, float * yd,
                     hipStream_t stream, int layout, uint16_t * y16, const int32_t * row_pad, int rows_per_seq) {
    GSVK_REQUIRE(x && wb && y, "layernorm: null pointer");
    GSVK_REQUIRE(!row_pad || (rows_per_seq > 0 && rows % rows_per_seq == 0), "layernorm: bad padding rows");
    GSVK_REQUIRE(rows >= 0 && rows < (1 << 30) && n > 0 && n % 32 == 0 && n <= 4096,
                 "layernorm: unsupported shape rows=%lld n=%lld (n %% 32 == 0, n <= 4096)",
                 (long long) rows, (long long) n);
    GSVK_REQUIRE((yq == nullptr) == (yd == nullptr), "layernorm: yq and yd go together");
    GSVK_REQUIRE(layout >= Q8_SLICED && layout <= Q8_TILED, "layernorm: bad layout %d", layout);
    auto al16 = [](const void * p) { return ((uintptr_t) p & 15) == 0; };
    GSVK_REQUIRE(al16(x) && al16(r) && al16(bias) && al16(wb) && al16(y), "layernorm: operands must be 16-byte aligned");
    if (rows == 0) return GSVK_OK;
    // 4 rows (waves) per workgroup from 512 rows on: 16384 one-wave workgroups (a 16 x 1024
    // prefill) launch slower than the rows take; below, one-wave workgroups spread the rows over
    // more CUs (batch-64 decode: 63.0k -> 65.2k tokens/s)
    const int rpw = rows >= 512 ? 4 : 1;
    const dim3 grid((unsigned) ((rows + rpw - 1) / rpw)), block(64 * rpw);
    // (the fp16 copy is a separate instantiation: the kernel without it stays as it was)
#define GSVK_LN(C, H)                                                                              \
    hipLaunchKernelGGL((k_layernorm<C, H>), grid, block, 0, stream, x, r, bias, wb, (int) rows, (int) n, eps, \
                       y, yq, yd, layout, y16, row_pad, rows_per_seq)
    if (n <= 512) {
        if (y16) GSVK_LN(1, true); else GSVK_LN(1, false);
    } else if (n <= 1024) {
        if (y16) GSVK_LN(2, true); else GSVK_LN(2, false);
    } else {
        if (y16) GSVK_LN(8, true); else GSVK_LN(8, false);
    }
#undef GSVK_LN
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_embed_pe(const float * emb, const float * pe, const int32_t * tok, int vocab,
                    const int32_t * pos_ptr, int pos_add, float alpha, int d, int B, float * x,
                    int8_t * xq, float * xd, int32_t * kv_end, int kv_end_add, const int32_t * pos_sub,
                    int pe_rows, hipStream_t stream, int layout) {
    GSVK_REQUIRE(d == 512, "embed_pe: d_model must be 512");
    GSVK_REQUIRE(layout >= Q8_SLICED && layout <= Q8_TILED, "embed_pe: bad layout %d", layout);
    GSVK_REQUIRE(emb && pe && tok && pos_ptr && x && xq && xd, "embed_pe: null pointer");
    hipLaunchKernelGGL(k_embed_pe, dim3((unsigned) B), dim3(64), 0, stream, emb, pe, tok, vocab,
                       pos_ptr, pos_add, alpha, d, x, xq, xd, kv_end, kv_end_add, pos_sub, pe_rows, layout);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_layernorm(const float * x, const float * r, const float * bias,
                                 const float * wb, int64_t rows, int64_t n, float eps, float * y,
                                 int8_t * yq, float * yd, void * stream) {
    return gsvk::launch_layernorm(x, r, bias, wb, rows, n, eps, y, yq, yd, (hipStream_t) stream);
}

extern "C" int gsvk_op_add_act(const float * a, const float * b, int64_t n, int64_t ne0, int act,
                               float * y, void * stream) {
    GSVK_REQUIRE(a && b && y && n >= 0 && ne0 > 0 && act >= 0 && act <= 3,
                 "gsvk_op_add_act: bad arguments");
    if (n == 0) return GSVK_OK;
    hipLaunchKernelGGL(gsvk::k_add_act, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t) stream, a, b, n, ne0, act, y);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

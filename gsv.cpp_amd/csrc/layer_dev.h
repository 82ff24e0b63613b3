// Device helpers of the fused decoder-layer kernels (layer.hip, qkv_attn.hip).
#pragma once

#include "common.h"

namespace gsvk {

// read in place of an absent r or bias operand of the LayerNorm input stage
static __device__ __align__(16) const float g_zero_row[512] = {};

// One row of width 512 held by one wave (8 values per lane): LayerNorm as in norm.hip. The
// operands are fetched by ln_row_load with unconditional 16-byte loads (absent r or bias read a
// zero row instead of branching), so that a caller can issue them before other work and the
// stage costs one memory latency; ln_row_compute does the arithmetic.
struct LnRow {
    float4 xa, xb, ra, rb, ba, bb, wa, wbv, ca, cb;
};

__device__ __forceinline__ void ln_row_load(const float * __restrict__ res, const float * __restrict__ r,
                                            const float * __restrict__ bias, const float * __restrict__ wb,
                                            int lane, LnRow & t) {
    const int base = lane * 8;
    const float4 * x4 = reinterpret_cast<const float4 *>(res + base);
    const float4 * r4 = reinterpret_cast<const float4 *>(r + base);
    const float4 * b4 = reinterpret_cast<const float4 *>(bias + base);
    const float4 * w4 = reinterpret_cast<const float4 *>(wb + base);
    const float4 * c4 = reinterpret_cast<const float4 *>(wb + 512 + base);
    t.xa = x4[0]; t.xb = x4[1]; t.ra = r4[0]; t.rb = r4[1]; t.ba = b4[0]; t.bb = b4[1];
    t.wa = w4[0]; t.wbv = w4[1]; t.ca = c4[0]; t.cb = c4[1];
}

__device__ __forceinline__ void ln_row_compute(const LnRow & t, float (&o)[8]) {
    constexpr int n = 512;
    const float xv[8] = {t.xa.x, t.xa.y, t.xa.z, t.xa.w, t.xb.x, t.xb.y, t.xb.z, t.xb.w};
    const float rv[8] = {t.ra.x, t.ra.y, t.ra.z, t.ra.w, t.rb.x, t.rb.y, t.rb.z, t.rb.w};
    const float bv[8] = {t.ba.x, t.ba.y, t.ba.z, t.ba.w, t.bb.x, t.bb.y, t.bb.z, t.bb.w};
    const float wv[8] = {t.wa.x, t.wa.y, t.wa.z, t.wa.w, t.wbv.x, t.wbv.y, t.wbv.z, t.wbv.w};
    const float cv[8] = {t.ca.x, t.ca.y, t.ca.z, t.ca.w, t.cb.x, t.cb.y, t.cb.z, t.cb.w};
    float v[8];
    double s = 0.0, s2 = 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float x = (xv[i] + rv[i]) + bv[i];   // x + 0 and + 0 leave x unchanged
        v[i] = x;
        s += (double) x;
        s2 += (double) x * (double) x;
    }
    s = wave_sum_d_uniform(s);
    s2 = wave_sum_d_uniform(s2);
    const float mean = (float) (s / (double) n);
    const float var = __builtin_fmaf(-mean, mean, (float) (s2 / (double) n));
    const float inv = 1.0f / __builtin_sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = __builtin_fmaf((v[i] - mean) * inv, wv[i], cv[i]);
}

__device__ __forceinline__ void ln_row_wave(const float * __restrict__ res, const float * __restrict__ r,
                                            const float * __restrict__ bias,
                                            const float * __restrict__ wb, int lane, float (&o)[8]) {
    LnRow t;
    ln_row_load(res, r, bias, wb, lane, t);
    ln_row_compute(t, o);
}

}  // namespace gsvk

// Device helpers of the fused decoder-layer kernels (layer.hip, qkv_attn.hip).
#pragma once

#include "common.h"
#include "layer.h"

namespace gsvk {

// PE row of the embedding input stage for activation row `row` at loop position `step`
// (*in.pos_ptr), clamped into the table.
__device__ __forceinline__ int pe_row(const LayerIn & in, int step, int row) {
    int p = step + in.pos_add - (in.pos_sub ? in.pos_sub[row] : 0);
    p = p < 0 ? 0 : p;
    return (in.pe_rows > 0 && p >= in.pe_rows) ? in.pe_rows - 1 : p;
}

// read in place of an absent r or bias operand of the LayerNorm input stage
static __device__ __align__(16) const float g_zero_row[512] = {};

// One row of width 512 held by one wave (8 values per lane): LayerNorm as in norm.hip. The
// operands are fetched by ln_row_load with unconditional 16-byte loads (absent r or bias read a
// zero row instead of branching), so that a caller can issue them before other work and the
// stage costs one memory latency; ln_row_compute does the arithmetic.
struct LnRow {
    float4 xa, xb, ra, rb, ba, bb, wa, wbv, ca, cb;
};

// A pointer into device (global) memory, typed so that loads through it are global loads: a
// pointer chosen between a kernel argument and a __device__ array is otherwise generic, and
// generic (flat) loads make the compiler wait for every outstanding load before their use.
typedef float f4v __attribute__((ext_vector_type(4)));
typedef const f4v __attribute__((address_space(1))) * gf4ptr;
__device__ __forceinline__ gf4ptr as_global_f4(const float * p) { return (gf4ptr) p; }
__device__ __forceinline__ float4 ld4(gf4ptr p, int i) {
    const f4v v = p[i];
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void ln_row_load(const float * __restrict__ res, const float * __restrict__ r,
                                            const float * __restrict__ bias, const float * __restrict__ wb,
                                            int lane, LnRow & t) {
    const int base = lane * 8;
    const gf4ptr x4 = as_global_f4(res + base);
    const gf4ptr r4 = as_global_f4(r + base);
    const gf4ptr b4 = as_global_f4(bias + base);
    const gf4ptr w4 = as_global_f4(wb + base);
    const gf4ptr c4 = as_global_f4(wb + 512 + base);
    t.xa = ld4(x4, 0); t.xb = ld4(x4, 1); t.ra = ld4(r4, 0); t.rb = ld4(r4, 1); t.ba = ld4(b4, 0);
    t.bb = ld4(b4, 1); t.wa = ld4(w4, 0); t.wbv = ld4(w4, 1); t.ca = ld4(c4, 0); t.cb = ld4(c4, 1);
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

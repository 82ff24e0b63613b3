// Device helpers of the single-query attention kernels (attention.hip, qkv_attn.hip).
#pragma once

#include "common.h"

namespace gsvk {

constexpr int ATT_HD = 32;
constexpr int ATT_BLK = 64;            // keys per block
constexpr int ATT_PART = ATT_HD + 2;   // m, l, o[32]
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ void h8_to_f(const uint4 & u, float (&f)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = h2f((uint16_t) (w[i] & 0xffff));
        f[2 * i + 1] = h2f((uint16_t) (w[i] >> 16));
    }
}

__device__ __forceinline__ float ld_coherent(const float * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Final output of one (seq, head): lanes 0..31 of the calling wave hold one dimension each.
// The Q8_0 copy of a row of nh*32 values is written in the given layout (Q8Layout: sliced for
// the GEMV, natural or tiled for the GEMMs); head h is block h.
__device__ __forceinline__ void attn_store_out(float val, int lane, int64_t bh, int nh,
                                               float * __restrict__ out,
                                               uint16_t * __restrict__ out16,
                                               int8_t * __restrict__ oq,
                                               float * __restrict__ od, int layout = Q8_SLICED) {
    if (lane < ATT_HD) {
        out[bh * ATT_HD + lane] = val;
        if (out16) out16[bh * ATT_HD + lane] = f2h(val);
    }
    if (oq) {
        float v1[1] = {lane < ATT_HD ? val : 0.0f};
        int8_t q1[1];
        const float d = q8_quantize_group<1>(v1, q1, 32);
        if (lane < ATT_HD) {
            const int64_t b = bh / nh;
            const int h = (int) (bh % nh);
            if (layout == Q8_TILED) {
                oq[q8_tiled_offset(b, nh, h, lane)] = q1[0];
                if (lane == 0) od[q8_tiled_scale(b, nh, h)] = d;
            } else {
                oq[b * nh * ATT_HD + (layout == Q8_NATURAL ? (int64_t) h * ATT_HD + lane
                                                            : q8_sliced_offset(nh, h, lane))] = q1[0];
                if (lane == 0) od[bh] = d;   // block index == b*nh + h
            }
        }
    }
}

struct KV8 {
    uint4 k[4], v[4];
};

// Loads of one block: lane (ks, qd) reads the quarter qd of keys key0 + 16p + ks, p < 4. Every
// load is issued (no branch, so all 8 are in flight together); a key past `last` reads key
// `last` instead (an index inside the buffer, on the same cache lines), and the caller masks
// such keys at use: score -inf and V replaced by zero (a select, so whatever the slot holds
// cannot reach the result). NT: non-temporal (streaming) loads, for a cache whose step reads far
// exceed the 256 MB MALL, where keeping the rows only evicts what is reused (the weights).
template <bool NT = false>
__device__ __forceinline__ void load_block(const uint16_t * __restrict__ kb,
                                           const uint16_t * __restrict__ vb, int key0, int last,
                                           int ks, KV8 & r) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int p = 0; p < 4; p++) {
        int key = key0 + p * 16 + ks;
        key = key < last ? key : last;
        if constexpr (NT) {
            const u4v kk = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(kb + (int64_t) key * ATT_HD));
            const u4v vv = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(vb + (int64_t) key * ATT_HD));
            r.k[p] = make_uint4(kk.x, kk.y, kk.z, kk.w);
            r.v[p] = make_uint4(vv.x, vv.y, vv.z, vv.w);
        } else {
            r.k[p] = *reinterpret_cast<const uint4 *>(kb + (int64_t) key * ATT_HD);
            r.v[p] = *reinterpret_cast<const uint4 *>(vb + (int64_t) key * ATT_HD);
        }
    }
}

// Sum over the 4 quarter lanes of a key (lane ^ 1, lane ^ 2), the same in each of them.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    return v;
}

// Sum over the 16 key slots (lane bits 2..5), butterfly order lane ^ 4, ^ 8, ^ 16, ^ 32.
__device__ __forceinline__ float slot_sum(float v) {
    v += swz_xor4(v);
    v += dpp_f<DPP_ROR8>(v);
    v += swz_xor16(v);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// One block of 64 keys of a wave's online softmax: scores q.k (scale in log2 units; keys at or
// past `end` get -inf and a zero V), the running max m, sum l and output o[8] (this lane's
// quarter of the 32 dimensions, per key slot). SUBST: the key at column `col` is taken from
// knew / vnew instead of the loaded registers.
template <bool SUBST>
__device__ __forceinline__ void attn_block_step(KV8 cur, int key0, int end, int ks, const float (&qv)[8],
                                                float scale_log2, int col, const uint4 & knew,
                                                const uint4 & vnew, float & m, float & l, float (&o)[8]) {
    if constexpr (SUBST) {
#pragma unroll
        for (int p = 0; p < 4; p++)
            if (key0 + p * 16 + ks == col) {
                cur.k[p] = knew;
                cur.v[p] = vnew;
            }
    }
    float s[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        float kf[8];
        h8_to_f(cur.k[p], kf);
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) dot = __builtin_fmaf(qv[i], kf[i], dot);
        dot = quad_sum(dot);
        s[p] = (key0 + p * 16 + ks < end) ? dot * scale_log2 : -INFINITY;
    }
    const float bm = wave_max_uniform(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
    const float mn = fmaxf(m, bm);                    // finite: each block has a valid key
    const float f = __builtin_amdgcn_exp2f(m - mn);   // 0 on the first block (m = -inf)
    l *= f;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] *= f;
    m = mn;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const float pr = __builtin_amdgcn_exp2f(s[p] - m);   // masked keys: exp2(-inf) = 0
        const bool valid = key0 + p * 16 + ks < end;
        float vf[8];
        h8_to_f(valid ? cur.v[p] : make_uint4(0, 0, 0, 0), vf);
        l += pr;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = __builtin_fmaf(pr, vf[i], o[i]);
    }
}

// waves per workgroup and splits per (seq, head) of the decode attention (attention.hip)
int attn_waves(int B, int nh, int64_t max_keys);
// Split of the rows: nsplit runs per (seq, head), of `chunk` blocks each when chunk > 0 (merged by
// a second launch), else of ceil(blocks / nsplit) blocks (merged by the last workgroup).
struct AttnPlan {
    int nsplit;
    int chunk;
};
AttnPlan attn_plan(int B, int nh, int64_t max_keys);
int attn_nsplit(int B, int nh, int64_t max_keys);

}  // namespace gsvk

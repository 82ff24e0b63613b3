// Single-query (decode) attention over a per-sequence fp16 KV cache, for gfx950.
//
// Work decomposition: split-K over the key axis. Workgroup (chunk, head, seq) owns up to
// ATT_CHUNK consecutive valid keys of one (seq, head). Inside a workgroup each wave takes 64
// keys as 4 passes of 16: lane = (key slot ks = lane/4, quarter qd = lane%4); a lane loads the
// 16-byte quarter [8qd, 8qd+8) of a 64-byte fp16 K row, so one wave-wide load reads 1 KiB of
// contiguous cache. Scores are completed with two lane shuffles, the chunk's softmax is local
// (max, then exp and V accumulation in fp32), and chunks are merged by the last workgroup of
// each (seq, head) to finish (a device-scope counter), so one launch does the whole op.
//
// Numerics follow ggml_flash_attn_ext on one query row: s = (q . k) * scale over the valid keys,
// softmax, times V, output divided by the sum (multiplied by its reciprocal), fp32 throughout.
#include "common.h"

namespace gsvk {

constexpr int ATT_CHUNK = 256;
constexpr int ATT_HD = 32;
constexpr int ATT_PART = ATT_HD + 2;   // m, l, o[32]

__device__ __forceinline__ void load_h8(const uint16_t * p, float (&f)[8]) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
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
// The Q8_0 copy is written in the sliced layout of a row of nh*32 values: head h is block h.
__device__ __forceinline__ void attn_store_out(float val, int lane, int64_t bh, int nh,
                                               float * __restrict__ out,
                                               uint16_t * __restrict__ out16,
                                               int8_t * __restrict__ oq,
                                               float * __restrict__ od) {
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
            oq[b * nh * ATT_HD + q8_sliced_offset(nh, h, lane)] = q1[0];
            if (lane == 0) od[bh] = d;   // block index == b*nh + h
        }
    }
}

__global__ void __launch_bounds__(256) k_attn_decode(
    const float * __restrict__ q, int64_t q_stride, const uint16_t * __restrict__ kc,
    const uint16_t * __restrict__ vc, int nh, int64_t lstride, const int32_t * __restrict__ kv_begin,
    const int32_t * __restrict__ kv_end, int maxch, float scale, float * __restrict__ out,
    uint16_t * __restrict__ out16, int8_t * __restrict__ oq, float * __restrict__ od,
    float * __restrict__ part, int32_t * __restrict__ counters) {
    const int chunk = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    // clamp to the buffer so that a bad range can never read outside the cache
    int beg = kv_begin[b];
    int end = kv_end[b];
    beg = beg < 0 ? 0 : beg;
    end = end > (int) lstride ? (int) lstride : end;
    if (end - beg > maxch * ATT_CHUNK) end = beg + maxch * ATT_CHUNK;
    const int nkeys = end > beg ? end - beg : 0;
    const int nch = (nkeys + ATT_CHUNK - 1) / ATT_CHUNK;
    if (chunk >= (nch > 0 ? nch : 1)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ks = lane >> 2;
    const int qd = lane & 3;
    const int64_t bh = (int64_t) b * nh + h;

    __shared__ float s_max[4];
    __shared__ float s_l[4];
    __shared__ float s_o[4][ATT_HD];

    if (nkeys == 0) {   // no valid key: ggml returns 0 (S == 0 -> S_inv = 0)
        if (wave == 0) attn_store_out(0.0f, lane, bh, nh, out, out16, oq, od);
        return;
    }

    float qv[8];
    {
        const float * qp = q + (int64_t) b * q_stride + h * ATT_HD + qd * 8;
        const float4 a = *reinterpret_cast<const float4 *>(qp);
        const float4 c = *reinterpret_cast<const float4 *>(qp + 4);
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w;
        qv[4] = c.x; qv[5] = c.y; qv[6] = c.z; qv[7] = c.w;
    }
    const uint16_t * kb = kc + bh * lstride * ATT_HD + qd * 8;
    const uint16_t * vb = vc + bh * lstride * ATT_HD + qd * 8;
    const int c0 = beg + chunk * ATT_CHUNK + wave * 64;

    float s[4];
    bool ok[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int key = c0 + p * 16 + ks;
        ok[p] = key < end;
        float dot = 0.0f;
        if (ok[p]) {
            float kf[8];
            load_h8(kb + (int64_t) key * ATT_HD, kf);
#pragma unroll
            for (int i = 0; i < 8; i++) dot = __builtin_fmaf(qv[i], kf[i], dot);
        }
        dot += __shfl_xor(dot, 1, 64);
        dot += __shfl_xor(dot, 2, 64);
        s[p] = ok[p] ? dot * scale : -INFINITY;
    }
    float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mx = warp_max(mx);
    if (lane == 0) s_max[wave] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));

    float l = 0.0f;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        if (ok[p]) {
            const int key = c0 + p * 16 + ks;
            const float pr = expf(s[p] - m);
            float vf[8];
            load_h8(vb + (int64_t) key * ATT_HD, vf);
            l += pr;
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = __builtin_fmaf(pr, vf[i], o[i]);
        }
    }
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] += __shfl_xor(o[i], off, 64);
    }
    if (lane < 4) {
#pragma unroll
        for (int i = 0; i < 8; i++) s_o[wave][lane * 8 + i] = o[i];
        if (lane == 0) s_l[wave] = l;
    }
    __syncthreads();
    if (wave != 0) return;

    float od_ = 0.0f, lt = 0.0f;
    if (lane < ATT_HD) od_ = ((s_o[0][lane] + s_o[1][lane]) + s_o[2][lane]) + s_o[3][lane];
    lt = ((s_l[0] + s_l[1]) + s_l[2]) + s_l[3];

    if (nch == 1) {
        const float inv = 1.0f / lt;
        attn_store_out(od_ * inv, lane, bh, nh, out, out16, oq, od);
        return;
    }

    // multi-chunk: publish the partial, the last workgroup of this (seq, head) merges
    float * pp = part + (bh * maxch + chunk) * ATT_PART;
    if (lane < ATT_HD) st_coherent(pp + 2 + lane, od_);
    if (lane == 0) {
        st_coherent(pp + 0, m);
        st_coherent(pp + 1, lt);
    }
    __threadfence();
    int lastflag = 0;
    if (lane == 0) {
        const int prev = __hip_atomic_fetch_add(counters + bh, 1, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT);
        lastflag = (prev == nch - 1);
    }
    const int last = __shfl(lastflag, 0, 64);
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

    float M = -INFINITY;
    for (int c = 0; c < nch; c++) M = fmaxf(M, ld_coherent(part + (bh * maxch + c) * ATT_PART));
    float L = 0.0f, O = 0.0f;
    for (int c = 0; c < nch; c++) {
        const float * pc = part + (bh * maxch + c) * ATT_PART;
        const float w = expf(ld_coherent(pc) - M);
        L = __builtin_fmaf(ld_coherent(pc + 1), w, L);
        if (lane < ATT_HD) O = __builtin_fmaf(ld_coherent(pc + 2 + lane), w, O);
    }
    attn_store_out(O * (1.0f / L), lane, bh, nh, out, out16, oq, od);
    if (lane == 0)
        __hip_atomic_store(counters + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t attn_workspace_bytes(int B, int nh, int64_t max_keys) {
    const int64_t maxch = (max_keys + ATT_CHUNK - 1) / ATT_CHUNK;
    const size_t part = (size_t) B * nh * (maxch > 0 ? maxch : 1) * ATT_PART * sizeof(float);
    const size_t cnt = (size_t) B * nh * sizeof(int32_t);
    return ((part + 255) / 256) * 256 + cnt;
}

// The counter area (the tail of ws) must be zero before the first call; every call leaves it
// zero again.
int launch_attn_decode(const float * q, int64_t q_stride, const uint16_t * k, const uint16_t * v,
                       int B, int nh, int hd, int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end,
                       int64_t max_keys, float scale, float * out, uint16_t * out16, int8_t * oq,
                       float * od, void * ws, hipStream_t stream) {
    GSVK_REQUIRE(q && k && v && kv_begin && kv_end && out && ws, "attn_decode: null pointer");
    GSVK_REQUIRE(hd == ATT_HD, "attn_decode: head_dim must be 32 (got %d)", hd);
    GSVK_REQUIRE(q_stride >= (int64_t) nh * hd && q_stride % 4 == 0, "attn_decode: bad q stride");
    GSVK_REQUIRE(B > 0 && B <= 65535 && nh > 0 && nh <= 65535 && lstride > 0 && max_keys >= 0 &&
                     max_keys <= lstride,
                 "attn_decode: bad shape B=%d nh=%d lstride=%lld max_keys=%lld", B, nh,
                 (long long) lstride, (long long) max_keys);
    GSVK_REQUIRE((oq == nullptr) == (od == nullptr), "attn_decode: oq and od go together");
    const int64_t maxch64 = (max_keys + ATT_CHUNK - 1) / ATT_CHUNK;
    const int maxch = (int) (maxch64 > 0 ? maxch64 : 1);
    const size_t part_bytes = (size_t) B * nh * maxch * ATT_PART * sizeof(float);
    float * part = (float *) ws;
    int32_t * counters = (int32_t *) ((char *) ws + ((part_bytes + 255) / 256) * 256);
    hipLaunchKernelGGL(k_attn_decode, dim3((unsigned) maxch, (unsigned) nh, (unsigned) B), dim3(256),
                       0, stream, q, q_stride, k, v, nh, lstride, kv_begin, kv_end, maxch, scale, out, out16,
                       oq, od, part, counters);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" size_t gsvk_attn_workspace_bytes(int B, int nh, int64_t max_keys) {
    return gsvk::attn_workspace_bytes(B, nh, max_keys);
}

extern "C" int gsvk_op_attn_decode(const float * q, const uint16_t * k, const uint16_t * v, int B,
                                   int nh, int hd, int64_t lstride, const int32_t * kv_begin,
                                   const int32_t * kv_end, int64_t max_keys, float scale,
                                   float * out, uint16_t * out_f16, int8_t * oq, float * od,
                                   void * ws, void * stream) {
    return gsvk::launch_attn_decode(q, (int64_t) nh * hd, k, v, B, nh, hd, lstride, kv_begin, kv_end, max_keys, scale,
                                    out, out_f16, oq, od, ws, (hipStream_t) stream);
}

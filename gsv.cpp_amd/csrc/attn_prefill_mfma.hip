// Prefill self-attention on the gfx950 matrix cores (the flash_attn_ext of src/gsv_ar.cpp:257
// over all B*S rows), for long prompts; the lane-per-query kernel of prefill.hip covers short
// ones.
//
// Masks as the reference builds them (src/gsv_ar.cpp:215-223): query s of sequence b sees the
// keys [pad_b, max_len) when it is a text row (s < max_len, bidirectional over the text) and the
// keys [pad_b, s] when it is a semantic row (causal); no valid key gives 0.
//
// Work: workgroup = (128 queries, head, sequence), 4 waves of 32 queries. Key tiles of 32 are
// staged through LDS (double buffered) as fp16 pairs hi + lo (x = hi + lo to ~2^-22 relative),
// and every product is formed as hi*lo + lo*hi + hi*hi in three v_mfma_f32_32x32x16_f16 with
// fp32 accumulation, so the scores and the weighted sum carry about fp32 accuracy (the reference
// computes in fp32; plain fp16 operands would cost ~1e-3 relative).
//
//   scores, transposed: S^T[key][query] = K[key] . Q[query]   (A = K tile, B = Q^T)
//     -> lane l holds query l%32 and 16 keys (rows 8*(v/4) + 4*(l/32) + v%4 of the tile), so the
//        online softmax of a query is in-lane plus one exchange with lane l^32;
//   output, transposed: O^T[dim][query] += V^T[dim][key] . P^T[key][query]
//     -> the P^T operand is taken straight from those registers (keys in their native order:
//        4h..4h+3, 8+4h..8+4h+3 for the first 16, +16 for the second), and the V^T operand is
//        read from LDS in the same key order, so the product sums over the right keys.
// The online softmax runs in log2 units (exp2); the output is divided by the final sum. Key tiles
// start at the sequence's first valid key, so left padding changes no result bit.
#include "common.h"
#include "layer.h"

namespace gsvk {

// the lane-per-query kernel (prefill.hip)
int launch_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                        int d_model, float scale, float * out, int8_t * oq, float * od,
                        hipStream_t stream);

namespace {
constexpr int PM_Q = 32;                 // queries per wave
constexpr int PM_WAVES = 4;
constexpr int PM_KT = 32;                // keys per tile
constexpr int PM_KROW = 32 * 2 + 16;     // LDS bytes per key row of K (32 fp16, padded)
constexpr int PM_VROW = PM_KT * 2 + 16;  // LDS bytes per dim row of V^T (32 keys fp16, padded)

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct PmTile {
    int8_t khi[PM_KT * PM_KROW];
    int8_t klo[PM_KT * PM_KROW];
    int8_t vhi[32 * PM_VROW];   // V^T [dim][key]
    int8_t vlo[32 * PM_VROW];
};

__device__ __forceinline__ void split_h(float x, _Float16 & hi, _Float16 & lo) {
    hi = (_Float16) x;
    lo = (_Float16) (x - (float) hi);
}
}  // namespace

// One thread's share of a key tile: 4 dims of K and of V of one key (256 threads: 32 keys x 8).
struct PmRegs {
    float4 k, v;
};

// fetch key tile [k0, k0 + 32) of head h (keys past S read key S - 1; they are masked later)
__device__ __forceinline__ PmRegs pm_fetch(const float * __restrict__ base, int64_t rs, int d_model, int h,
                                           int S, int k0, int tid) {
    const int key = tid >> 3, dq = (tid & 7) * 4;
    const float * kp = base + (int64_t) min(k0 + key, S - 1) * rs + d_model + h * 32 + dq;
    PmRegs r;
    r.k = *reinterpret_cast<const float4 *>(kp);
    r.v = *reinterpret_cast<const float4 *>(kp + d_model);
    return r;
}

// split the fetched values into fp16 hi + lo and store them: K as [key][dim], V as V^T [dim][key]
__device__ __forceinline__ void pm_store(const PmRegs & r, int tid, PmTile & t) {
    const int key = tid >> 3, dq = (tid & 7) * 4;
    const float kx[4] = {r.k.x, r.k.y, r.k.z, r.k.w};
    const float vx[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
    v4h kh, kl;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        _Float16 hi, lo;
        split_h(kx[i], hi, lo);
        kh[i] = hi;
        kl[i] = lo;
        split_h(vx[i], hi, lo);
        *reinterpret_cast<_Float16 *>(&t.vhi[(dq + i) * PM_VROW + key * 2]) = hi;
        *reinterpret_cast<_Float16 *>(&t.vlo[(dq + i) * PM_VROW + key * 2]) = lo;
    }
    *reinterpret_cast<v4h *>(&t.khi[key * PM_KROW + dq * 2]) = kh;
    *reinterpret_cast<v4h *>(&t.klo[key * PM_KROW + dq * 2]) = kl;
}

__global__ void __launch_bounds__(PM_WAVES * 64) k_attn_prefill_mfma(
    const float * __restrict__ qkv, int S, int max_len, const int32_t * __restrict__ pad, int nh, int d_model,
    float scale_log2, float * __restrict__ out, int8_t * __restrict__ oq, float * __restrict__ od) {
    const int h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int q0w = blockIdx.x * (PM_Q * PM_WAVES);      // first query of the workgroup
    const int qw = q0w + wave * PM_Q;                     // first query of this wave
    const int q = qw + li;                                // this lane's query
    const int pb = pad[b];
    const int64_t rs = 3 * (int64_t) d_model;
    const float * base = qkv + (int64_t) b * S * rs;

    __shared__ __align__(16) PmTile tiles[2];

    // key range of this lane's query, of the wave and of the workgroup
    const auto key_end = [&](int s) { return s < max_len ? max_len : s + 1; };
    const int qc = min(q, S - 1);
    const int ke = min(key_end(qc), S);
    const int qlast_w = min(qw + PM_Q - 1, S - 1);
    const int ke_w = min(key_end(qlast_w), S);            // the wave's last query sees the most keys
    const int qlast_g = min(q0w + PM_Q * PM_WAVES - 1, S - 1);
    const int ke_g = min(key_end(qlast_g), S);
    // tiles start at the first valid key: a sequence's arithmetic does not depend on its left pad
    const int kt0 = pb;

    // Q^T operand (B): query q, dims 16c + 8*lh + [0, 8), split hi + lo
    v8h qh[2], ql[2];
    {
        const float * qp = base + (int64_t) qc * rs + h * 32;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const float4 a = *reinterpret_cast<const float4 *>(qp + 16 * c + 8 * lh);
            const float4 d = *reinterpret_cast<const float4 *>(qp + 16 * c + 8 * lh + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, d.x, d.y, d.z, d.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                _Float16 hi, lo;
                split_h(x[i], hi, lo);
                qh[c][i] = hi;
                ql[c][i] = lo;
            }
        }
    }

    v16f o = {};               // O^T: this lane's query, dims 8*(v/4) + 4*lh + v%4
    float m = -INFINITY, l = 0.0f;

    if (kt0 < ke_g) pm_store(pm_fetch(base, rs, d_model, h, S, kt0, tid), tid, tiles[0]);
    __syncthreads();
    int buf = 0;
    for (int k0 = kt0; k0 < ke_g; k0 += PM_KT, buf ^= 1) {
        // the next tile is fetched into registers before this one is used, and stored after
        const bool more = k0 + PM_KT < ke_g;   // uniform over the workgroup
        PmRegs nxt{};
        if (more) nxt = pm_fetch(base, rs, d_model, h, S, k0 + PM_KT, tid);
        if (k0 < ke_w) {   // uniform per wave
            const PmTile & t = tiles[buf];
            // S^T = K . Q^T over the 32 dims (2 chunks of 16)
            v16f sc = {};
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const v8h kh = *reinterpret_cast<const v8h *>(&t.khi[li * PM_KROW + (16 * c + 8 * lh) * 2]);
                const v8h kl = *reinterpret_cast<const v8h *>(&t.klo[li * PM_KROW + (16 * c + 8 * lh) * 2]);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[c], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[c], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[c], sc, 0, 0, 0);
            }
            // mask, scale, running max of this query (own 16 keys + lane l^32's 16)
            float s[16];
            float rmax = -INFINITY;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int key = k0 + 8 * (v >> 2) + 4 * lh + (v & 3);
                const bool valid = key >= pb && key < ke;
                s[v] = valid ? sc[v] * scale_log2 : -INFINITY;
                rmax = fmaxf(rmax, s[v]);
            }
            rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
            const float mn = fmaxf(m, rmax);
            // all keys so far masked: keep zeros (exp2(-inf - -inf) would be NaN)
            const float f = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
            float psum = 0.0f;
            float p[16];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                p[v] = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[v] - mn);
                psum += p[v];
            }
            psum += __shfl_xor(psum, 32, 64);
            l = l * f + psum;
            m = mn;
#pragma unroll
            for (int v = 0; v < 16; v++) o[v] *= f;
            // O^T += V^T . P^T, keys in the register order (two chunks of 16)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                v8h ph, pl;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    _Float16 hi, lo;
                    split_h(p[8 * c + i], hi, lo);
                    ph[i] = hi;
                    pl[i] = lo;
                }
                // V^T rows: dim li, keys 16c + 4*lh + [0,4) and 16c + 8 + 4*lh + [0,4)
                const int kA = 16 * c + 4 * lh, kB = 16 * c + 8 + 4 * lh;
                const v4h a0 = *reinterpret_cast<const v4h *>(&t.vhi[li * PM_VROW + kA * 2]);
                const v4h a1 = *reinterpret_cast<const v4h *>(&t.vhi[li * PM_VROW + kB * 2]);
                const v4h b0 = *reinterpret_cast<const v4h *>(&t.vlo[li * PM_VROW + kA * 2]);
                const v4h b1 = *reinterpret_cast<const v4h *>(&t.vlo[li * PM_VROW + kB * 2]);
                v8h vh, vl;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    vh[i] = a0[i]; vh[4 + i] = a1[i];
                    vl[i] = b0[i]; vl[4 + i] = b1[i];
                }
                o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pl, o, 0, 0, 0);
                o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, ph, o, 0, 0, 0);
                o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, ph, o, 0, 0, 0);
            }
        }
        if (more) pm_store(nxt, tid, tiles[buf ^ 1]);
        __syncthreads();
    }

    // output: query q, dims 8*(v/4) + 4*lh + v%4; the head's 32 values are one Q8_0 block,
    // split between this lane and lane l^32
    if (q >= S) return;   // (the exchanges below pair lanes of the same query)
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float y[16];
    float amax = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        y[v] = o[v] * inv;
        amax = fmaxf(amax, fabsf(y[v]));
    }
    const int64_t row = (int64_t) b * S + q;
    float * orow = out + row * d_model + h * 32;
#pragma unroll
    for (int g = 0; g < 4; g++)
        *reinterpret_cast<float4 *>(orow + 8 * g + 4 * lh) = make_float4(y[4 * g], y[4 * g + 1], y[4 * g + 2], y[4 * g + 3]);
    if (oq) {
        // natural order (the out projection's GEMM reads it)
        amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
        const float dd = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const int nblk = d_model / 32;
        int8_t * qrow = oq + row * d_model + h * 32;
#pragma unroll
        for (int v = 0; v < 16; v += 4) {
            // dims 8*(v/4) + 4*lh + [0,4) of block h
            int packed = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) packed |= (((int) __builtin_rintf(y[v + t] * id)) & 0xff) << (8 * t);
            *reinterpret_cast<int *>(qrow + 8 * (v >> 2) + 4 * lh) = packed;
        }
        if (lh == 0) od[row * nblk + h] = h2f(f2h(dd));
    }
}

int launch_attn_prefill_mfma(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                             int d_model, float scale, float * out, int8_t * oq, float * od, hipStream_t stream) {
    GSVK_REQUIRE(qkv && pad && out && B > 0 && S > 0 && nh * 32 == d_model && max_len <= S,
                 "attn_prefill_mfma: bad arguments");
    GSVK_REQUIRE((oq == nullptr) == (od == nullptr), "attn_prefill_mfma: oq and od go together");
    GSVK_REQUIRE(((uintptr_t) qkv & 15) == 0 && ((uintptr_t) out & 15) == 0,
                 "attn_prefill_mfma: qkv and out must be 16-byte aligned");
    const dim3 grid((unsigned) ((S + PM_Q * PM_WAVES - 1) / (PM_Q * PM_WAVES)), (unsigned) nh, (unsigned) B);
    hipLaunchKernelGGL(k_attn_prefill_mfma, grid, dim3(PM_WAVES * 64), 0, stream, qkv, S, max_len, pad, nh,
                       d_model, scale * 1.4426950408889634f, out, oq, od);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                                    int hd, float scale, int path, float * out, int8_t * oq, float * od,
                                    void * stream) {
    GSVK_REQUIRE(hd == 32, "attn_prefill: head_dim must be 32");
    GSVK_REQUIRE(path >= 0 && path <= 2, "attn_prefill: path must be 0 (auto), 1 or 2");
    const bool mfma = path == 2 || (path == 0 && gsvk::attn_prefill_uses_mfma((int64_t) B * S));
    if (mfma)
        return gsvk::launch_attn_prefill_mfma(qkv, B, S, max_len, pad, nh, nh * hd, scale, out, oq, od,
                                              (hipStream_t) stream);
    return gsvk::launch_attn_prefill(qkv, B, S, max_len, pad, nh, nh * hd, scale, out, oq, od,
                                     (hipStream_t) stream);
}

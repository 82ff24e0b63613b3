// Prefill self-attention on the gfx950 matrix cores (the flash_attn_ext of src/gsv_ar.cpp:257
// over all B*S rows), for long prompts; the lane-per-query kernel of prefill.hip covers short
// ones.
//
// Masks as the reference builds them (src/gsv_ar.cpp:215-223): query s of sequence b sees the
// keys [pad_b, max_len) when it is a text row (s < max_len, bidirectional over the text) and the
// keys [pad_b, s] when it is a semantic row (causal); no valid key gives 0.
//
// Work: workgroup = (256 queries, head, sequence), 8 waves of 32 queries. Key tiles of 64 are
// staged through LDS (double buffered; one fetch and barrier per 64 keys, the 8 waves sharing
// it), each wave consuming a tile as two halves of 32 keys, as fp16 pairs hi + lo (x = hi + lo
// to ~2^-22 relative),
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
// In the prefill's fp16 mode (PV_HILO false) the weighted sum is one product of fp16(P) and
// fp16(V) (about 2^-11 relative, 5e-4 of the output's scale): V's remainder is neither split nor
// staged and P is rounded instead of split; the scores keep their three products (their error
// would pass through the exponential).
#include <algorithm>
#include <vector>

#include "common.h"
#include "layer.h"

namespace gsvk {

// the lane-per-query kernel (prefill.hip)
int launch_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                        int d_model, float scale, float * out, int8_t * oq, float * od,
                        hipStream_t stream);

namespace {
constexpr int PM_Q = 32;                 // queries per wave
constexpr int PM_WAVES = 8;
constexpr int PM_KT = 64;                // keys per LDS tile (two halves of 32 for the MFMAs)
constexpr int PM_KROW = 32 * 2 + 16;     // LDS bytes per key row of K (32 fp16, padded)
constexpr int PM_VROW = PM_KT * 2 + 16;  // LDS bytes per dim row of V^T (64 keys fp16, padded)

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct PmTile {
    int8_t khi[PM_KT * PM_KROW];
    int8_t klo[PM_KT * PM_KROW];
    int8_t vhi[32 * PM_VROW];   // V^T [dim][key]
    int8_t vlo[32 * PM_VROW];
};

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split_h(float x, _Float16 & hi, _Float16 & lo) {
    hi = (_Float16) x;
    lo = (_Float16) (x - (float) hi);
}

// The same split for a pair: hi = fp16(x) (nearest), lo = fp16(x - hi), where x - hi (exact in
// fp32) comes from one v_fma_mix per value (the fp16 hi times -1 plus the fp32 x, rounded to
// fp16) instead of a conversion back to fp32 and a subtraction.
__device__ __forceinline__ void split_pair(float x0, float x1, v2h & hi, v2h & lo) {
    hi = v2h{(_Float16) x0, (_Float16) x1};
    uint32_t h = __builtin_bit_cast(uint32_t, hi), r;
    asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(r)
        : "v"(h), "v"(x0), "v"(x1));
    lo = __builtin_bit_cast(v2h, r);
}
}  // namespace

// One thread's share of a key tile (256 threads): 4 dims of K of one key (thread = 32 keys x 8
// groups of 4 dims) and 1 dim of V of 4 keys (thread = 32 dims x 8 groups of 4 keys), so that
// both land in LDS with 8-byte stores: K as [key][dim], V transposed as [dim][key].
struct PmRegs {
    float4 k;
    float v[4];
};

// fetch key tile [k0, k0 + 32) of head h (keys past S read key S - 1; they are masked later)
__device__ __forceinline__ PmRegs pm_fetch(const float * __restrict__ base, int64_t rs, int d_model, int h,
                                           int S, int k0, int tid) {
    const int key = tid >> 3, dq = (tid & 7) * 4;
    const int vd = tid & 31, vk = (tid >> 5) * 4;
    PmRegs r;
    r.k = *reinterpret_cast<const float4 *>(base + (int64_t) min(k0 + key, S - 1) * rs + d_model + h * 32 + dq);
#pragma unroll
    for (int i = 0; i < 4; i++) r.v[i] = base[(int64_t) min(k0 + vk + i, S - 1) * rs + 2 * d_model + h * 32 + vd];
    return r;
}

// split the fetched values into fp16 hi + lo and store them (V: hi only without PV_HILO)
template <bool PV_HILO>
__device__ __forceinline__ void pm_store(const PmRegs & r, int tid, PmTile & t) {
    const int key = tid >> 3, dq = (tid & 7) * 4;
    const int vd = tid & 31, vk = (tid >> 5) * 4;
    v2h k0h, k0l, k1h, k1l;
    split_pair(r.k.x, r.k.y, k0h, k0l);
    split_pair(r.k.z, r.k.w, k1h, k1l);
    const v4h kh = {k0h[0], k0h[1], k1h[0], k1h[1]}, kl = {k0l[0], k0l[1], k1l[0], k1l[1]};
    *reinterpret_cast<v4h *>(&t.khi[key * PM_KROW + dq * 2]) = kh;
    *reinterpret_cast<v4h *>(&t.klo[key * PM_KROW + dq * 2]) = kl;
    if constexpr (PV_HILO) {
        v2h v0h, v0l, v1h, v1l;
        split_pair(r.v[0], r.v[1], v0h, v0l);
        split_pair(r.v[2], r.v[3], v1h, v1l);
        const v4h vh = {v0h[0], v0h[1], v1h[0], v1h[1]}, vl = {v0l[0], v0l[1], v1l[0], v1l[1]};
        *reinterpret_cast<v4h *>(&t.vhi[vd * PM_VROW + vk * 2]) = vh;
        *reinterpret_cast<v4h *>(&t.vlo[vd * PM_VROW + vk * 2]) = vl;
    } else {
        const v4h vh = {(_Float16) r.v[0], (_Float16) r.v[1], (_Float16) r.v[2], (_Float16) r.v[3]};
        *reinterpret_cast<v4h *>(&t.vhi[vd * PM_VROW + vk * 2]) = vh;
    }
}

template <bool PV_HILO>
__global__ void __launch_bounds__(PM_WAVES * 64) k_attn_prefill_mfma(
    const float * __restrict__ qkv, int S, int max_len, const int32_t * __restrict__ pad, int nh, int d_model,
    float scale_log2, float * __restrict__ out, int8_t * __restrict__ oq, float * __restrict__ od,
    const int32_t * __restrict__ seq_order, int skip_pad) {
    // seq_order (or null): the sequences in dispatch order, and each sequence's query blocks from
    // the last (the most keys) down, so that the longest workgroups start first
    const int h = blockIdx.y;
    const int b = seq_order ? seq_order[blockIdx.z] : blockIdx.z;
    const int qb = seq_order ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int q0w = qb * (PM_Q * PM_WAVES);             // first query of the workgroup
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
    const int ke_min_w = min(key_end(min(qw, S - 1)), S);   // the wave's first query sees the fewest keys
    const int ke_w = min(key_end(qlast_w), S);            // the wave's last query sees the most keys
    const int qlast_g = min(q0w + PM_Q * PM_WAVES - 1, S - 1);
    const int ke_g = min(key_end(qlast_g), S);
    // tiles start at the first valid key: a sequence's arithmetic does not depend on its left pad
    const int kt0 = pb;
    // skip_pad: a wave whose 32 queries are all left-padding rows computes nothing (those rows
    // get zeros); it only helps stage the tiles, and a workgroup of such waves stages none
    // (uniform). Padding queries in a wave with valid ones are computed as the masks give them.
    const bool idle = skip_pad && qw + PM_Q <= pb;
    const int kend = skip_pad && q0w + PM_Q * PM_WAVES <= pb ? kt0 : ke_g;

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

    if (kt0 < kend) pm_store<PV_HILO>(pm_fetch(base, rs, d_model, h, S, kt0, tid), tid, tiles[0]);
    __syncthreads();
    int buf = 0;
    for (int k0 = kt0; k0 < kend; k0 += PM_KT, buf ^= 1) {
        // the next tile is fetched into registers before this one is used, and stored after
        const bool more = k0 + PM_KT < kend;   // uniform over the workgroup
        PmRegs nxt{};
        if (more) nxt = pm_fetch(base, rs, d_model, h, S, k0 + PM_KT, tid);
        const PmTile & t = tiles[buf];
#pragma unroll
        for (int hf = 0; hf < PM_KT / 32; hf++) {
            const int kk = k0 + 32 * hf;   // the half's first key
            if (kk >= ke_w || idle) break; // uniform per wave
            // S^T = K . Q^T over the 32 dims (2 chunks of 16)
            v16f sc = {};
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const v8h kh = *reinterpret_cast<const v8h *>(&t.khi[(32 * hf + li) * PM_KROW + (16 * c + 8 * lh) * 2]);
                const v8h kl = *reinterpret_cast<const v8h *>(&t.klo[(32 * hf + li) * PM_KROW + (16 * c + 8 * lh) * 2]);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[c], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[c], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[c], sc, 0, 0, 0);
            }
            // Softmax step in log2 units. A tile that every query of the wave sees whole (the
            // usual case: all but the last tile or two of a row) skips the masks; otherwise
            // invisible keys get -inf.
            const bool full = kk + 32 <= ke_min_w;   // uniform per wave (tiles start at pb)
            float p[16];
            float f, psum = 0.0f;
            if (full) {
                float rmax = sc[0];
#pragma unroll
                for (int v = 1; v < 16; v++) rmax = fmaxf(rmax, sc[v]);
                rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
                const float mn = fmaxf(m, rmax * scale_log2);
                f = __builtin_amdgcn_exp2f(m - mn);   // m = -inf before the first tile: f = 0
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[v], scale_log2, -mn));
                    psum += p[v];
                }
                m = mn;
            } else {
                float rmax = -INFINITY;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int key = kk + 8 * (v >> 2) + 4 * lh + (v & 3);
                    if (!(key >= pb && key < ke)) sc[v] = -INFINITY;
                    rmax = fmaxf(rmax, sc[v]);
                }
                rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
                const float mn = fmaxf(m, rmax * scale_log2);
                // all keys so far masked: keep zeros (exp2(-inf - -inf) would be NaN)
                const bool dead = mn == -INFINITY;
                f = dead ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    p[v] = dead ? 0.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(sc[v], scale_log2, -mn));
                    psum += p[v];
                }
                m = mn;
            }
            psum += __shfl_xor(psum, 32, 64);
            l = l * f + psum;
            if (__any(f != 1.0f)) {   // no running max of the wave moved: nothing to rescale
#pragma unroll
                for (int v = 0; v < 16; v++) o[v] *= f;
            }
            // O^T += V^T . P^T, keys in the register order (two chunks of 16)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                // V^T rows: dim li, keys 16c + 4*lh + [0,4) and 16c + 8 + 4*lh + [0,4)
                const int kA = 32 * hf + 16 * c + 4 * lh, kB = 32 * hf + 16 * c + 8 + 4 * lh;
                const v4h a0 = *reinterpret_cast<const v4h *>(&t.vhi[li * PM_VROW + kA * 2]);
                const v4h a1 = *reinterpret_cast<const v4h *>(&t.vhi[li * PM_VROW + kB * 2]);
                v8h vh;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    vh[i] = a0[i]; vh[4 + i] = a1[i];
                }
                v8h ph;
                if constexpr (PV_HILO) {
                    v8h pl;
#pragma unroll
                    for (int i = 0; i < 8; i += 2) {
                        v2h hi, lo;
                        split_pair(p[8 * c + i], p[8 * c + i + 1], hi, lo);
                        ph[i] = hi[0]; ph[i + 1] = hi[1];
                        pl[i] = lo[0]; pl[i + 1] = lo[1];
                    }
                    const v4h b0 = *reinterpret_cast<const v4h *>(&t.vlo[li * PM_VROW + kA * 2]);
                    const v4h b1 = *reinterpret_cast<const v4h *>(&t.vlo[li * PM_VROW + kB * 2]);
                    v8h vl;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        vl[i] = b0[i]; vl[4 + i] = b1[i];
                    }
                    o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pl, o, 0, 0, 0);
                    o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, ph, o, 0, 0, 0);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) ph[i] = (_Float16) p[8 * c + i];
                }
                o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, ph, o, 0, 0, 0);
            }
        }
        if (more) pm_store<PV_HILO>(nxt, tid, tiles[buf ^ 1]);
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
                             int d_model, float scale, float * out, int8_t * oq, float * od, hipStream_t stream,
                             bool pv_f16, const int32_t * seq_order, bool skip_pad) {
    GSVK_REQUIRE(qkv && pad && out && B > 0 && S > 0 && nh * 32 == d_model && max_len <= S,
                 "attn_prefill_mfma: bad arguments");
    GSVK_REQUIRE((oq == nullptr) == (od == nullptr), "attn_prefill_mfma: oq and od go together");
    GSVK_REQUIRE(((uintptr_t) qkv & 15) == 0 && ((uintptr_t) out & 15) == 0,
                 "attn_prefill_mfma: qkv and out must be 16-byte aligned");
    const dim3 grid((unsigned) ((S + PM_Q * PM_WAVES - 1) / (PM_Q * PM_WAVES)), (unsigned) nh, (unsigned) B);
    if (pv_f16)
        hipLaunchKernelGGL(k_attn_prefill_mfma<false>, grid, dim3(PM_WAVES * 64), 0, stream, qkv, S, max_len, pad,
                           nh, d_model, scale * 1.4426950408889634f, out, oq, od, seq_order, (int) skip_pad);
    else
        hipLaunchKernelGGL(k_attn_prefill_mfma<true>, grid, dim3(PM_WAVES * 64), 0, stream, qkv, S, max_len, pad,
                           nh, d_model, scale * 1.4426950408889634f, out, oq, od, seq_order, (int) skip_pad);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                                    int hd, float scale, int path, float * out, int8_t * oq, float * od,
                                    void * stream) {
    GSVK_REQUIRE(hd == 32, "attn_prefill: head_dim must be 32");
    GSVK_REQUIRE(path >= 0 && path <= 4, "attn_prefill: path must be 0 (auto), 1, 2, 3 or 4");
    if (path == 4) {
        // the decoder prefill's dispatch: sequences longest first (the fewest padding rows; equal
        // pads in index order), each sequence's query blocks from the last, waves of padding
        // queries skipped. The order is built on the host from pad and lives in a temporary
        // device array; the stream is synchronised before it is freed.
        GSVK_REQUIRE(B > 0 && pad, "attn_prefill: bad arguments");
        hipStream_t st = (hipStream_t) stream;
        std::vector<int32_t> hp((size_t) B), order((size_t) B);
        GSVK_HIP(hipMemcpyAsync(hp.data(), pad, (size_t) B * 4, hipMemcpyDeviceToHost, st));
        GSVK_HIP(hipStreamSynchronize(st));
        for (int b = 0; b < B; b++) order[(size_t) b] = b;
        std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return hp[(size_t) a] < hp[(size_t) c]; });
        int32_t * d_order = nullptr;
        GSVK_HIP(hipMalloc(&d_order, (size_t) B * 4));
        int rc = hipMemcpyAsync(d_order, order.data(), (size_t) B * 4, hipMemcpyHostToDevice, st) == hipSuccess
                     ? gsvk::launch_attn_prefill_mfma(qkv, B, S, max_len, pad, nh, nh * hd, scale, out, oq, od, st,
                                                      false, d_order, true)
                     : GSVK_ERR_HIP;
        if (hipStreamSynchronize(st) != hipSuccess && rc == GSVK_OK) rc = GSVK_ERR_HIP;
        (void) hipFree(d_order);
        return rc;
    }
    const bool mfma = path >= 2 || (path == 0 && gsvk::attn_prefill_uses_mfma((int64_t) B * S));
    if (mfma)
        return gsvk::launch_attn_prefill_mfma(qkv, B, S, max_len, pad, nh, nh * hd, scale, out, oq, od,
                                              (hipStream_t) stream, path == 3);
    return gsvk::launch_attn_prefill(qkv, B, S, max_len, pad, nh, nh * hd, scale, out, oq, od,
                                     (hipStream_t) stream);
}

// QKV projection + single-query attention of one decoder layer in one launch, for gfx950.
//
// Workgroup (seq b, head h), NW waves (the same NW as the standalone attention, attn_waves):
//   1. every wave issues the loads of its first block of cached keys [begin, col) (they do not
//      depend on this step) together with its share of head h's QKV weight rows;
//   2. wave 0 builds the Q8_0 input row in LDS: LayerNorm((res + r) + bias) (layers > 0) or
//      emb[tok] + alpha * PE[pos] (layer 0), as the input stages of layer.hip;
//   3. the 96 rows of head h (q, k, v; rows 32h.., 512+32h.., 1024+32h..) are computed in the
//      Q8_0 x86 dot order of q8.hip (8 rows per wave, 8 slice lanes per row); q goes to LDS, the
//      new k and v are rounded to fp16, appended to the cache at column col and kept in LDS;
//   4. the attention of attention.hip over keys [begin, col] with the preloaded first block;
//      the key at column col is taken from LDS (the preloaded registers hold the slot's old
//      contents).
// The result equals the separate QKV GEMV + k_attn_decode<NW> bit for bit: the same input row,
// the same per-row dot, the same blocks per wave and the same merge order.
//
// head h's workgroups are blockIdx.x = b * nh + h: with nh a multiple of 8 they all run on one
// XCD, so the 52 KB of weights of head h are read from HBM once per XCD L2.
//
// Exact mode (EXACT): step 4 is flash_attn_ext's sequential online softmax in ggml-cpu's order
// (src/gsv_ar.cpp:404; the oracle's orc_attn_row), bit for bit, in chunks of 384 keys, 7 waves:
//   a. producer thread p of the 6 producer waves takes key c0 + p: its score q.k in
//      ggml_vec_dot_f32's order times the scale, and its V row into LDS as fp32, transposed; the
//      next chunk's K/V rows are loaded now;
//   b. the maximum before each key (an exclusive prefix max over the chunk, seeded with the
//      running maximum) gives each key's ms and vs (glibc's expf): ms = expf(before - s), vs = 1
//      for a new maximum, else ms = 1, vs = expf(s - before);
//   c. the chain wave runs the chains over the chunk before (a and b fill one of two LDS buffers
//      while c reads the other), one dependent fma per key: lanes 0..31 acc_d = fma(v_d, vs,
//      acc_d * ms), lane 32 S = fma(S, ms, vs); with ms = 1 (no new maximum among 16 keys, a
//      ballot per key) both are fma(x, vs, acc) with x = v_d or 1.
#include "attn_dev.h"
#include "expf_exact.h"
#include "layer.h"
#include "layer_dev.h"
#include "qkv_attn.h"

namespace gsvk {

namespace {
constexpr int QA_K = 512;                // d_model
constexpr int QA_NBLK = QA_K / 32;
constexpr int QA_NB4 = QA_K / 128;       // int4 weight loads per slice lane
constexpr int QA_ROWS = 3 * ATT_HD;      // rows of one head: q, k, v

constexpr int QX_C = 384;    // keys per chunk of the exact attention: one per producer thread
constexpr int QX_NP = QX_C / 64;   // producer waves
constexpr int QX_CW = 3;     // the chain's wave: with 7 waves dealt to a CU's 4 SIMDs in turn, the
                             // only one with a SIMD of its own
constexpr int QX_G = 16;     // keys per group of the chain (one bit of the new-maximum mask)
constexpr int QX_RA = 3 * QX_G;   // entries past the chunk that the chain reads ahead (never used)
constexpr int QX_TS = 452;   // floats per dimension row of the transposed V: >= QX_C + QX_RA, and
                             // 4 more than a multiple of 32 so that 8 lanes' 16-byte reads of
                             // consecutive rows fall in distinct banks

struct QxLds {
    // V transposed: row d < 32 holds dimension d of the chunk's keys, row 32 holds 1.0 (S's chain;
    // written once); keys past the chunk's end hold -0.0 (a product of -0.0 added to any value
    // leaves it) and weight 0 (S + 1 * 0 is S)
    // (two of each: the chunk the producers fill, the chunk the chain reads)
    float xt[2][ATT_HD + 1][QX_TS];
    float vs[2][QX_C + QX_RA];   // the key's weight exp(s - max before it); 0 past the chunk's end
    float ms[2][QX_C];
    float wmax[QX_C / 64];
    uint8_t gm[2][8];            // per producer wave, one bit per group of QX_G keys that holds a new maximum
    uint64_t etab[32];           // the exponential's table
};

__constant__ uint64_t qx_exp2_tab[32] = GSVK_EXP2_TAB32;

// v moved across lanes by the DPP control CTRL; lanes with no source lane, or outside the rows
// of ROW_MASK, read -inf
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float qx_dpp_ninf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp((int) 0xff800000u, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// inclusive maximum scan over the 64 lanes: row shifts by 1, 2, 4 and 8 within each row of 16,
// then row 0's last lane into row 1 (and row 2's into row 3), then lane 31 into rows 2 and 3
__device__ __forceinline__ float qx_wave_incl_max(float v) {
    v = fmaxf(v, qx_dpp_ninf<0x111, 0xf>(v));
    v = fmaxf(v, qx_dpp_ninf<0x112, 0xf>(v));
    v = fmaxf(v, qx_dpp_ninf<0x114, 0xf>(v));
    v = fmaxf(v, qx_dpp_ninf<0x118, 0xf>(v));
    v = fmaxf(v, qx_dpp_ninf<0x142, 0xa>(v));
    v = fmaxf(v, qx_dpp_ninf<0x143, 0xc>(v));
    return v;
}

// the K and V rows (64 bytes each) of key j of one (sequence, head); a key past `last` reads key
// `last` (in the buffer; not used)
__device__ __forceinline__ void qx_load(const uint16_t * __restrict__ kb, const uint16_t * __restrict__ vb, int j,
                                        int last, KV8 & r) {
    const int key = j < last ? j : last;
    const uint4 * kp = reinterpret_cast<const uint4 *>(kb + (int64_t) key * ATT_HD);
    const uint4 * vp = reinterpret_cast<const uint4 *>(vb + (int64_t) key * ATT_HD);
#pragma unroll
    for (int p = 0; p < 4; p++) {
        r.k[p] = kp[p];
        r.v[p] = vp[p];
    }
}

// producer index of a thread of the exact attention's producer waves (every wave but QX_CW)
__device__ __forceinline__ int qx_ptid(int wave, int lane) { return (wave < QX_CW ? wave : wave - 1) * 64 + lane; }

// Exact attention of one (sequence, head) over keys [beg, end), end - 1 == col (the new key, in
// s_kv); (QX_NP + 1) * 64 threads. The producer waves (producer thread p holding key c0 + p of a
// chunk of QX_C) compute each chunk's scores, maxima and weights into one of two LDS buffers; wave
// QX_CW runs the sequential chain over the chunk before, from the other buffer, in two parts
// around the producers' barrier. `first` holds the rows of key beg + p on entry (producers);
// etab_v: entry lane % 32 of the exponential's table. Returns dimension `lane` of the output in
// wave QX_CW's lanes 0..31.
__device__ __forceinline__ float qx_attend(const KV8 & first, const uint16_t * __restrict__ kb,
                                           const uint16_t * __restrict__ vb, int beg, int end, int col,
                                           int last_old, const float * s_q, const uint16_t (*s_kv)[ATT_HD],
                                           uint64_t etab_v, float scale, int tid) {
    __shared__ __align__(16) QxLds L;
    const int lane = tid & 63, wave = tid >> 6;
    const bool prod = wave != QX_CW;             // uniform per wave
    const int pwave = wave < QX_CW ? wave : wave - 1, ptid = qx_ptid(wave, lane);   // producers
    if (tid < 32) L.etab[tid] = etab_v;   // (read after the first chunk's first barrier)
    for (int i = tid; i < 2 * (QX_C + QX_RA); i += (QX_NP + 1) * 64)   // S's rows (read after a barrier too)
        L.xt[i / (QX_C + QX_RA)][ATT_HD][i % (QX_C + QX_RA)] = 1.0f;
    const int dl = lane < 32 ? lane : 32;
    float M = -INFINITY;   // producers: running maximum (uniform)
    float acc = 0.0f;      // wave 0: lanes 0..31 the output dimensions, lane 32 (and above) S
    uint4 rk0 = first.k[0], rk1 = first.k[1], rk2 = first.k[2], rk3 = first.k[3];
    uint4 rv0 = first.v[0], rv1 = first.v[1], rv2 = first.v[2], rv3 = first.v[3];
    float s = -INFINITY, excl = -INFINITY;   // producers: the key's score, the maximum before it in the wave

    // the chain over groups [g0, g1) of the chunk in buffer `bf` (wave 0): groups of QX_G keys,
    // the last one completed by keys of weight 0 and value -0.0 (acc * 1 + -0.0 * 0 is acc, and so
    // is fma(-0.0, 0, acc)); each group's LDS reads are issued three groups ahead into a ring of
    // four register sets (four groups per iteration, so that no copy between the sets is needed)
    auto chain_range = [&](int bf, int g0, int g1) {
        if (g0 >= g1) return;   // (uniform)
        constexpr int G = QX_G, GPW = 64 / QX_G;
        // group g's bit is bit g % GPW of byte g / GPW (uniform, a scalar register)
        const uint32_t glo = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t *>(&L.gm[bf][0]));
        const uint32_t ghi = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t *>(&L.gm[bf][4]));
        const uint64_t gmask = (uint64_t) glo | ((uint64_t) ghi << 32);
        float x0[G], v0[G], x1[G], v1[G], x2[G], v2[G], x3[G], v3[G];
        auto group = [&](int g, float (&xs)[G], float (&vs8)[G]) {
#pragma unroll
            for (int i = 0; i < G / 4; i++) {
                const float4 a = *reinterpret_cast<const float4 *>(&L.xt[bf][dl][G * g + 4 * i]);
                const float4 c = *reinterpret_cast<const float4 *>(&L.vs[bf][G * g + 4 * i]);
                xs[4 * i] = a.x; xs[4 * i + 1] = a.y; xs[4 * i + 2] = a.z; xs[4 * i + 3] = a.w;
                vs8[4 * i] = c.x; vs8[4 * i + 1] = c.y; vs8[4 * i + 2] = c.z; vs8[4 * i + 3] = c.w;
            }
        };
        auto chain = [&](const float (&xs)[G], const float (&vs8)[G], int g) {
            const int bit = 8 * (g / GPW) + g % GPW;
            if (__builtin_expect(((gmask >> bit) & 1ull) == 0, 1)) {   // no new maximum: ms = 1 (the
                                                                      // fall-through path)
#pragma unroll
                for (int i = 0; i < G; i++) acc = __builtin_fmaf(xs[i], vs8[i], acc);
            } else {
#pragma unroll
                for (int i4 = 0; i4 < G / 4; i4++) {
                    const float4 m4 = *reinterpret_cast<const float4 *>(&L.ms[bf][G * g + 4 * i4]);
                    const float m[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float lo = __builtin_fmaf(xs[4 * i4 + i], vs8[4 * i4 + i], acc * m[i]);
                        const float hs = __builtin_fmaf(acc, m[i], vs8[4 * i4 + i]);
                        acc = lane >= 32 ? hs : lo;
                    }
                }
            }
        };
        // (groups up to g1 + 2 <= QX_C / G + 2 are read: entries up to QX_C + QX_RA - 1)
        group(g0, x0, v0);
        group(g0 + 1, x1, v1);
        group(g0 + 2, x2, v2);
        int g = g0;
        for (; g + 4 <= g1; g += 4) {
            group(g + 3, x3, v3);
            chain(x0, v0, g);
            group(g + 4, x0, v0);
            chain(x1, v1, g + 1);
            group(g + 5, x1, v1);
            chain(x2, v2, g + 2);
            group(g + 6, x2, v2);
            chain(x3, v3, g + 3);
        }
        if (g < g1) chain(x0, v0, g);
        if (g + 1 < g1) chain(x1, v1, g + 1);
        if (g + 2 < g1) chain(x2, v2, g + 2);
    };

    const int nchunks = (end - beg + QX_C - 1) / QX_C;
    for (int it = 0; it <= nchunks; it++) {   // uniform: chunk it's scan, chunk it - 1's chain
        const int bf = it & 1;
        const int c0 = beg + it * QX_C;
        const int n = min(QX_C, end - c0);   // (<= 0 in the last iteration)
        const int np = min(QX_C, end - (c0 - QX_C));   // keys of chunk it - 1
        const int ngp = (np + QX_G - 1) / QX_G;
        // the chain's part before the producers' barrier (all of it when no chunk is being scanned)
        const int gsplit = it == nchunks ? ngp : (ngp * 5 + 4) / 8;
        if (prod && it < nchunks) {
            const int j = c0 + ptid;
            // the new key from LDS (the loaded slot holds the old contents)
            uint4 kw[4] = {rk0, rk1, rk2, rk3}, vw[4] = {rv0, rv1, rv2, rv3};
            if (j == col) {   // (one thread)
                const uint4 * nk = reinterpret_cast<const uint4 *>(&s_kv[0][0]);
                const uint4 * nv = reinterpret_cast<const uint4 *>(&s_kv[1][0]);
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    kw[p] = nk[p];
                    vw[p] = nv[p];
                }
            }
            if (c0 + QX_C < end) {   // the next chunk's rows (uniform)
                const int key = j + QX_C < last_old ? j + QX_C : last_old;
                const uint4 * kp = reinterpret_cast<const uint4 *>(kb + (int64_t) key * ATT_HD);
                const uint4 * vp = reinterpret_cast<const uint4 *>(vb + (int64_t) key * ATT_HD);
                rk0 = kp[0]; rk1 = kp[1]; rk2 = kp[2]; rk3 = kp[3];
                rv0 = vp[0]; rv1 = vp[1]; rv2 = vp[2]; rv3 = vp[3];
            }
            s = -INFINITY;
            if (ptid < n) {
                float qv[32];
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const float4 q4 = *reinterpret_cast<const float4 *>(&s_q[4 * c]);
                    qv[4 * c] = q4.x; qv[4 * c + 1] = q4.y; qv[4 * c + 2] = q4.z; qv[4 * c + 3] = q4.w;
                }
                float kf[32], vf[32];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    float t8[8];
                    h8_to_f(kw[p], t8);
#pragma unroll
                    for (int i = 0; i < 8; i++) kf[8 * p + i] = t8[i];
                    h8_to_f(vw[p], t8);
#pragma unroll
                    for (int i = 0; i < 8; i++) vf[8 * p + i] = t8[i];
                }
                // ggml_vec_dot_f32 (32 elements): 4 x 8 partial products, (0 + 2) + (1 + 3), hsum
                float s0[8];
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    const float p0 = __builtin_fmaf(kf[l], qv[l], 0.0f), p1 = __builtin_fmaf(kf[8 + l], qv[8 + l], 0.0f);
                    const float p2 = __builtin_fmaf(kf[16 + l], qv[16 + l], 0.0f), p3 = __builtin_fmaf(kf[24 + l], qv[24 + l], 0.0f);
                    s0[l] = (p0 + p2) + (p1 + p3);
                }
                const float t0 = s0[0] + s0[4], t1 = s0[1] + s0[5], t2 = s0[2] + s0[6], t3 = s0[3] + s0[7];
                s = ((t0 + t1) + (t2 + t3)) * scale;
#pragma unroll
                for (int d = 0; d < ATT_HD; d++) L.xt[bf][d][ptid] = vf[d];
            } else {
#pragma unroll
                for (int d = 0; d < ATT_HD; d++) L.xt[bf][d][ptid] = -0.0f;
            }
            // the maximum before each key: inclusive scan within the wave, the waves' maxima,
            // seeded with the running maximum (max is exact in any order)
            const float incl = qx_wave_incl_max(s);
            excl = qx_dpp_ninf<0x138, 0xf>(incl);   // wave_shr:1 (lane 0: -inf)
            if (lane == 63) L.wmax[pwave] = incl;
        }
        if (!prod && it >= 1) chain_range(bf ^ 1, 0, gsplit);
        if (it < nchunks) __syncthreads();   // (uniform)
        if (prod && it < nchunks) {
            float before = M, mn = M;
#pragma unroll
            for (int w = 0; w < QX_C / 64; w++) {
                const float wm = L.wmax[w];
                if (w < pwave) before = fmaxf(before, wm);
                mn = fmaxf(mn, wm);
            }
            before = fmaxf(before, excl);
            float ms = 1.0f, vs = 0.0f;   // past the chunk's end: weight 0, maximum unchanged
            if (ptid < n) {
                vs = 1.0f;
                if (s > before) ms = expf_glibc(before - s, L.etab);
                else vs = expf_glibc(s - before, L.etab);
            }
            L.ms[bf][ptid] = ms;
            L.vs[bf][ptid] = vs;
            const uint64_t nm = __ballot(ms != 1.0f);
            const uint64_t gz = __ballot(lane < 64 / QX_G && ((nm >> (QX_G * lane)) & ((1ull << QX_G) - 1)) != 0);
            if (lane == 0) L.gm[bf][pwave] = (uint8_t) gz;
            M = mn;
        }
        if (!prod && it >= 1) chain_range(bf ^ 1, gsplit, ngp);
        __syncthreads();
    }
    const float S = __shfl(acc, 32, 64);
    return acc * (S == 0.0f ? 0.0f : 1.0f / S);
}
}  // namespace

template <int NW, int MODE, bool EXACT>
__global__ void __launch_bounds__(NW * 64) k_qkv_attn(QkvAttnArgs a) {
    static_assert(!EXACT || (NW - 1) * 64 == QX_C, "exact mode: one key of a chunk per producer thread");
    constexpr int PASSES = (QA_ROWS / 8 + NW - 1) / NW;   // 8 rows per wave and pass
    const int nh = a.n_head;
    const int bh = blockIdx.x;
    const int b = __builtin_amdgcn_readfirstlane(bh / nh);   // uniform: scalar registers
    const int h = bh - b * nh;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ks = lane >> 2;
    const int qd = lane & 3;
    const int rsub = lane >> 3;   // GEMV: row within the wave's 8
    const int j = lane & 7;       // GEMV: slice lane

    constexpr int SLICE_B = QA_NBLK * 4 + 16;   // slices padded by 16 bytes: conflict-free reads
    __shared__ __align__(16) int8_t s_x[8 * SLICE_B];
    __shared__ __align__(16) float s_d[QA_NBLK];
    __shared__ __align__(16) float s_q[ATT_HD];
    __shared__ __align__(16) uint16_t s_kv[2][ATT_HD];
    __shared__ float s_m[NW];
    __shared__ float s_l[NW];
    __shared__ float s_o[NW][ATT_HD];

    // Order of work, chosen so that no wave-dependent branch separates a load from its use (the
    // compiler then waits exactly; a wait on a load also completes every load issued before it):
    // the scalars; the input row's operands (every wave); every wave's weight rows; wave 0's input
    // stage arithmetic; every wave's first block of keys. The key blocks (the bulk of the bytes)
    // go last so that the weights and the input row are not queued behind them.
    const LayerIn & in = a.in;
    const int col = *a.col_ptr + a.col_add;   // column of this step's key
    int beg = a.kv_begin[b];

    // the input row's operands first, in every wave (the same loads in every wave keep the waits
    // exact; only wave 0 uses them), so that they are not queued behind the weights and keys
    LnRow lnr;
    if constexpr (MODE == IN_LN)
        ln_row_load(in.res + (int64_t) b * QA_K, in.r ? in.r + (int64_t) b * QA_K : g_zero_row,
                    in.bias ? in.bias : g_zero_row, in.wb, lane, lnr);
    int4 w[PASSES][QA_NB4];
    uint2 dh[PASSES][QA_NB4];
    float rbias[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int rl = (p * NW + wave) * 8 + rsub;
        const int rlc = rl < QA_ROWS ? rl : QA_ROWS - 1;
        const int row = (rlc >> 5) * QA_K + h * ATT_HD + (rlc & 31);
        const int4 * wsl = reinterpret_cast<const int4 *>(a.ws + ((int64_t) row * 8 + j) * QA_NBLK * 4);
        const uint2 * wdr = reinterpret_cast<const uint2 *>(a.wd + (int64_t) row * QA_NBLK);
#pragma unroll
        for (int i = 0; i < QA_NB4; i++) {
            w[p][i] = wsl[i];
            dh[p][i] = wdr[i];
        }
        rbias[p] = a.bias[row];
    }

    // 2. the input row, quantised into LDS
    if (wave == 0) {
        float o[8];
        if constexpr (MODE == IN_LN) {
            ln_row_compute(lnr, o);
        } else {
            const int pos = *in.pos_ptr;
            int tk = in.tok[b];
            tk = tk < 0 ? 0 : (tk >= in.vocab ? in.vocab - 1 : tk);
            const float4 * er = reinterpret_cast<const float4 *>(in.emb + (int64_t) tk * QA_K + lane * 8);
            const float4 * pr = reinterpret_cast<const float4 *>(in.pe + (int64_t) pe_row(in, pos, b) * QA_K +
                                                                 lane * 8);
            const float4 e0 = er[0], e1 = er[1], p0 = pr[0], p1 = pr[1];
            const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
            const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = __builtin_fmaf(in.alpha, pv[i], ev[i]);
            if (h == 0 && in.kv_end && lane == 0) in.kv_end[b] = pos + in.kv_end_add;
        }
        if (h == 0 && in.out_x) {
            float4 * dst = reinterpret_cast<float4 *>(in.out_x + (int64_t) b * QA_K + lane * 8);
            dst[0] = make_float4(o[0], o[1], o[2], o[3]);
            dst[1] = make_float4(o[4], o[5], o[6], o[7]);
        }
        int8_t q[8];
        const float d = q8_quantize_group<8>(o, q, 4);
        q8_store_sliced_s(s_x, SLICE_B, lane >> 2, lane & 3, q);
        if ((lane & 3) == 0) s_d[lane >> 2] = d;
    }

    // 1b. the first block of cached keys, keys < col (the new key is substituted later); a wave
    // past the last block loads that block again and does not use it
    const bool col_ok = col >= 0 && col < a.lstride;
    beg = beg < 0 ? 0 : (beg < a.lstride ? beg : (int) a.lstride - 1);
    const int end = col + 1;
    const int nkeys = (col_ok && end > beg) ? end - beg : 0;
    const int nblk = (nkeys + ATT_BLK - 1) / ATT_BLK;
    const int64_t pair = (int64_t) b * nh + h;
    const uint16_t * kb = a.kc + pair * a.lstride * ATT_HD + qd * 8;
    const uint16_t * vb = a.vc + pair * a.lstride * ATT_HD + qd * 8;
    int last_old = col > beg ? col - 1 : beg;          // keys past it read this one
    last_old = last_old < a.lstride ? last_old : (int) a.lstride - 1;
    int blk = nblk > 0 ? (wave < nblk ? wave : nblk - 1) : 0;
    KV8 cur;
    if constexpr (EXACT)   // producer p: the rows of key beg + p (the first chunk); the chain's wave: unused
        qx_load(a.kc + pair * a.lstride * ATT_HD, a.vc + pair * a.lstride * ATT_HD,
                wave != QX_CW ? beg + qx_ptid(wave, lane) : beg, last_old, cur);
    // exact mode: the exponential's table, for LDS (a lookup in constant memory per lane would be a
    // memory round trip inside each chunk's scan); loaded after the first chunk's keys, which the
    // scan waits for first
    uint64_t etab_v = 0;
    if constexpr (EXACT) etab_v = qx_exp2_tab[lane & 31];
    else
        load_block(kb, vb, beg + blk * ATT_BLK, last_old, ks, cur);
    __syncthreads();
    if (!col_ok) {   // the new key is outside the cache: write nothing to it, output 0
        if (wave == 0) attn_store_out(0.0f, lane, pair, nh, a.out, nullptr, a.oq, a.od);
        return;
    }

    // 3. the 96 rows of head h
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int rl = (p * NW + wave) * 8 + rsub;
        if ((p * NW + wave) * 8 >= QA_ROWS) break;   // uniform per wave
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < QA_NB4; i++) {
            const float dw0 = h2f((uint16_t) (dh[p][i].x & 0xffff)), dw1 = h2f((uint16_t) (dh[p][i].x >> 16));
            const float dw2 = h2f((uint16_t) (dh[p][i].y & 0xffff)), dw3 = h2f((uint16_t) (dh[p][i].y >> 16));
            const int4 xv = *reinterpret_cast<const int4 *>(&s_x[j * SLICE_B + 16 * i]);
            const float4 dx = *reinterpret_cast<const float4 *>(&s_d[4 * i]);
            acc = __builtin_fmaf(dw0 * dx.x, (float) __builtin_amdgcn_sdot4(w[p][i].x, xv.x, 0, false), acc);
            acc = __builtin_fmaf(dw1 * dx.y, (float) __builtin_amdgcn_sdot4(w[p][i].y, xv.y, 0, false), acc);
            acc = __builtin_fmaf(dw2 * dx.z, (float) __builtin_amdgcn_sdot4(w[p][i].z, xv.z, 0, false), acc);
            acc = __builtin_fmaf(dw3 * dx.w, (float) __builtin_amdgcn_sdot4(w[p][i].w, xv.w, 0, false), acc);
        }
        acc = acc + __shfl_xor(acc, 4, 64);
        acc = acc + __shfl_xor(acc, 2, 64);
        acc = acc + __shfl_xor(acc, 1, 64);
        if (j == 0 && rl < QA_ROWS) {
            const int which = rl >> 5, dd = rl & 31;
            const float v = acc + rbias[p];
            if (which == 0) {
                s_q[dd] = v;
            } else {
                const uint16_t hv = f2h(v);
                s_kv[which - 1][dd] = hv;
                (which == 1 ? a.kc : a.vc)[(pair * a.lstride + col) * ATT_HD + dd] = hv;
            }
        }
    }
    __syncthreads();

    // 4. attention over [beg, col]
    if (nkeys == 0) {   // (col < beg: nothing valid; ggml returns 0)
        if (wave == 0) attn_store_out(0.0f, lane, pair, nh, a.out, nullptr, a.oq, a.od);
        return;
    }
    if constexpr (EXACT) {
        const float val = qx_attend(cur, a.kc + pair * a.lstride * ATT_HD, a.vc + pair * a.lstride * ATT_HD, beg,
                                    end, col, last_old, s_q, s_kv, etab_v, a.scale, tid);
        if (wave == QX_CW) attn_store_out(val, lane, pair, nh, a.out, nullptr, a.oq, a.od);
        return;
    }
    float qv[8];
    {
        const float4 q0 = *reinterpret_cast<const float4 *>(&s_q[qd * 8]);
        const float4 q1 = *reinterpret_cast<const float4 *>(&s_q[qd * 8 + 4]);
        qv[0] = q0.x; qv[1] = q0.y; qv[2] = q0.z; qv[3] = q0.w;
        qv[4] = q1.x; qv[5] = q1.y; qv[6] = q1.z; qv[7] = q1.w;
    }
    const uint4 knew = *reinterpret_cast<const uint4 *>(&s_kv[0][qd * 8]);
    const uint4 vnew = *reinterpret_cast<const uint4 *>(&s_kv[1][qd * 8]);
    const float scale_log2 = a.scale_log2;

    float m = -INFINITY, l = 0.0f;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;
    if (wave < nblk) {
        while (blk + NW < nblk) {
            KV8 pre;
            load_block(kb, vb, beg + (blk + NW) * ATT_BLK, last_old, ks, pre);
            attn_block_step<true>(cur, beg + blk * ATT_BLK, end, ks, qv, scale_log2, col, knew, vnew, m, l, o);
            cur = pre;
            blk += NW;
        }
        attn_block_step<true>(cur, beg + blk * ATT_BLK, end, ks, qv, scale_log2, col, knew, vnew, m, l, o);
    }
    l = slot_sum(l);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = slot_sum(o[i]);
    if (lane < 4) {
#pragma unroll
        for (int i = 0; i < 8; i++) s_o[wave][lane * 8 + i] = o[i];
        if (lane == 0) {
            s_l[wave] = l;
            s_m[wave] = m;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    float M = s_m[0];
#pragma unroll
    for (int w2 = 1; w2 < NW; w2++) M = fmaxf(M, s_m[w2]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < NW; w2++) {
        const float f = s_m[w2] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w2] - M);
        L = __builtin_fmaf(s_l[w2], f, L);
        if (lane < ATT_HD) O = __builtin_fmaf(s_o[w2][lane], f, O);
    }
    attn_store_out(O * (1.0f / L), lane, pair, nh, a.out, nullptr, a.oq, a.od);
}

bool qkv_attn_supported(int B, int nh, int64_t max_keys) {
    return attn_nsplit(B, nh, max_keys) == 1;
}

// The decode's GEMV chain runs below DECODE_GEMM_MIN_BATCH sequences only (from there the
// matrix-core path takes over), so the fused kernel is used below it as well.
bool qkv_attn_preferred(int B, int nh, int64_t max_keys) {
    return B < DECODE_GEMM_MIN_BATCH && qkv_attn_supported(B, nh, max_keys);
}

int launch_qkv_attn(const QkvAttnArgs & a, int B, int64_t max_keys, hipStream_t stream, bool exact) {
    GSVK_REQUIRE(a.ws && a.wd && a.bias && a.kc && a.vc && a.kv_begin && a.col_ptr && a.out,
                 "qkv_attn: null pointer");
    GSVK_REQUIRE(a.n_head * ATT_HD == QA_K && B > 0 && a.lstride > 0 && max_keys <= a.lstride,
                 "qkv_attn: needs 16 heads of 32 (d_model 512)");
    GSVK_REQUIRE(a.in.mode == IN_LN ? (a.in.res && a.in.wb) : (a.in.mode == IN_EMB && a.in.emb && a.in.pe &&
                                                                a.in.tok && a.in.pos_ptr),
                 "qkv_attn: bad input stage");
    GSVK_REQUIRE((a.oq == nullptr) == (a.od == nullptr), "qkv_attn: oq and od go together");
    const dim3 grid((unsigned) ((int64_t) B * a.n_head));
    if (exact) {   // any row length: the chunks cover it
        GSVK_REQUIRE(B <= 65535 * 16 && a.scale > 0.0f, "qkv_attn: bad exact-mode arguments");
        if (a.in.mode == IN_LN)
            hipLaunchKernelGGL((k_qkv_attn<QX_NP + 1, IN_LN, true>), grid, dim3((QX_NP + 1) * 64), 0, stream, a);
        else
            hipLaunchKernelGGL((k_qkv_attn<QX_NP + 1, IN_EMB, true>), grid, dim3((QX_NP + 1) * 64), 0, stream, a);
        GSVK_LAUNCH_CHECK();
        return GSVK_OK;
    }
    GSVK_REQUIRE(qkv_attn_supported(B, a.n_head, max_keys), "qkv_attn: rows this long need the split path");
    const int nw = attn_waves(B, a.n_head, max_keys);
#define GSVK_QA(W, MODE) hipLaunchKernelGGL((k_qkv_attn<W, MODE, false>), grid, dim3(W * 64), 0, stream, a)
    if (a.in.mode == IN_LN) {
        if (nw == 8) GSVK_QA(8, IN_LN);
        else GSVK_QA(4, IN_LN);
    } else {
        if (nw == 8) GSVK_QA(8, IN_EMB);
        else GSVK_QA(4, IN_EMB);
    }
#undef GSVK_QA
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

namespace {
int op_qkv_attn(const int8_t * wq, const uint16_t * wd, const float * bias, const float * res, const float * r,
                const float * ln_bias, const float * wb, int B, int nh, uint16_t * k, uint16_t * v, int64_t lstride,
                const int32_t * kv_begin, const int32_t * col, float scale, float * out, int8_t * oq, float * od,
                float * ln_out, void * stream, bool exact) {
    using namespace gsvk;
    GSVK_REQUIRE(res && wb, "qkv_attn: null pointer");
    QkvAttnArgs a{};
    a.ws = wq;
    a.wd = wd;
    a.bias = bias;
    a.in.mode = IN_LN;
    a.in.res = res;
    a.in.r = r;
    a.in.bias = ln_bias;
    a.in.wb = wb;
    a.in.out_x = ln_out;
    a.kc = k;
    a.vc = v;
    a.lstride = lstride;
    a.kv_begin = kv_begin;
    a.col_ptr = col;
    a.col_add = 0;
    a.n_head = nh;
    a.scale_log2 = scale * LOG2E;
    a.scale = scale;
    a.out = out;
    a.oq = oq;
    a.od = od;
    return launch_qkv_attn(a, B, lstride, (hipStream_t) stream, exact);
}
}  // namespace

extern "C" int gsvk_op_qkv_attn(const int8_t * wq, const uint16_t * wd, const float * bias, const float * res,
                                const float * r, const float * ln_bias, const float * wb, int B, int nh,
                                uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                                const int32_t * col, float scale, float * out, int8_t * oq, float * od,
                                float * ln_out, void * stream) {
    return op_qkv_attn(wq, wd, bias, res, r, ln_bias, wb, B, nh, k, v, lstride, kv_begin, col, scale, out, oq, od,
                       ln_out, stream, false);
}

extern "C" int gsvk_op_qkv_attn_exact(const int8_t * wq, const uint16_t * wd, const float * bias, const float * res,
                                      const float * r, const float * ln_bias, const float * wb, int B, int nh,
                                      uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                                      const int32_t * col, float scale, float * out, int8_t * oq, float * od,
                                      float * ln_out, void * stream) {
    return op_qkv_attn(wq, wd, bias, res, r, ln_bias, wb, B, nh, k, v, lstride, kv_begin, col, scale, out, oq, od,
                       ln_out, stream, true);
}

extern "C" int gsvk_qkv_attn_supported(int B, int nh, int64_t max_keys) {
    return gsvk::qkv_attn_supported(B, nh, max_keys) ? 1 : 0;
}

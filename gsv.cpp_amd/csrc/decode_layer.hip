// Decode step at small batch (up to DEC_MAX_BATCH = 64 sequences) in two launches per decoder layer,
// for gfx950.
//
// The decoder layer of src/gsv_ar.cpp:392-413 (QKV, K/V append, flash_attn_ext, out projection,
// LN1, FFN1 + ReLU, FFN2, LN2) has three all-to-all dependencies inside a sequence's row: the out
// projection needs every head, LN1 and FFN1 need every output of the out projection, FFN2 needs
// every hidden unit. The layer runs as two launches by splitting the two K-reductions that cross
// workgroups into partial rows that the next launch sums in a fixed order:
//
//   k_dec_attn, workgroup (head h, sequence b), 8 waves:
//     every thread loads element `tid` of the input row's operands (the previous layer's LN1
//     output, its 16 or 32 FFN2 partial rows, b_2, LN2's w and b), every wave its share of
//     head h's 96 QKV weight rows and of the 512 x 32 out-projection slice of head h, and its
//     first block of cached keys, all before any of them is used;
//     LN2 over the workgroup (double sums, one value per thread), the x86 Q8_0 quantisation of
//     the row into LDS (layer 0: the embedding + alpha * PE);
//     head h's q, k, v (the x86 8-lane Q8_0 dot of q8.hip), the fp16 K/V append and the attention
//     of attention.hip over [kv_begin, col];
//     the head's 32 outputs quantised to one Q8_0 block (the block the out projection's activation
//     quantisation gives them: head h is block h of the row) and multiplied by the slice: for
//     output n, (d_w d_a) * (exact int32 block dot), the partial row p1[h][b].
//   k_dec_ffn, workgroup (hidden group g of 128 or 64 units, sequence b), 8 waves:
//     LN1((x + sum_h p1[h]) + b_o), quantised; FFN1 + b_1 + ReLU for the group's 128 units (the
//     8-lane dot), quantised to 4 Q8_0 blocks (those of FFN2's activation row), and the 512 x 128
//     slice of FFN2: p2[g][b][n] = sum over the 4 blocks of (d_w d_h) * (int32 block dot).
//
// The sums over heads and groups change only fp32 summation orders against ggml's single 8-lane
// chain over all blocks (each block's int32 dot is exact either way). The out-projection and
// FFN2 weights are read in the matrix-core operand order (Q8_TILED): one 16-byte load per lane
// covers a whole 32-row x 32-column tile in 8 full 128-byte lines.
#include "attn_dev.h"
#include "decode_layer.h"
#include "layer_dev.h"

namespace gsvk {

namespace {
constexpr int DL_K = 512;                // d_model
constexpr int DL_NBLK = DL_K / 32;       // Q8_0 blocks of a row
constexpr int DL_NH = 16;                // heads
constexpr int DL_FFN = 2048;
constexpr int DL_THREADS = 512;          // one row element per thread
constexpr int DL_WAVES = DL_THREADS / 64;
constexpr int DL_SLICE_B = DL_NBLK * 4 + 16;   // LDS row slices padded by 16 bytes
constexpr int DL_QKV_ROWS = 3 * ATT_HD;

// Row LayerNorm over the workgroup, one value per thread: the LayerNorm of norm.hip and
// layer_dev.h (sums of the values and their squares in double, var = E[v^2] - mean^2 in float).
__device__ __forceinline__ float wg_layernorm(float v, float w, float c, int lane, int wave,
                                              double (*s_red)[DL_WAVES]) {
    double s = wave_sum_d_uniform((double) v);
    double s2 = wave_sum_d_uniform((double) v * (double) v);
    if (lane == 0) {
        s_red[0][wave] = s;
        s_red[1][wave] = s2;
    }
    __syncthreads();
    double S = 0.0, S2 = 0.0;
#pragma unroll
    for (int w2 = 0; w2 < DL_WAVES; w2++) {
        S += s_red[0][w2];
        S2 += s_red[1][w2];
    }
    const float mean = (float) (S / (double) DL_K);
    const float var = __builtin_fmaf(-mean, mean, (float) (S2 / (double) DL_K));
    const float inv = 1.0f / __builtin_sqrtf(var + 1e-5f);
    return __builtin_fmaf((v - mean) * inv, w, c);
}

// Maximum of |v| over the 32 lanes of each half wave, in every lane (DPP within rows of 16,
// then a swizzle across the two rows of the half; max is exact in any order).
__device__ __forceinline__ float half_wave_amax(float v) {
    float a = fabsf(v);
    a = fmaxf(a, dpp_f<DPP_XOR1>(a));
    a = fmaxf(a, dpp_f<DPP_XOR2>(a));
    a = fmaxf(a, dpp_f<DPP_ROR4>(a));
    a = fmaxf(a, dpp_f<DPP_ROR8>(a));
    return fmaxf(a, swz_xor16(a));
}

// The x86 Q8_0 quantisation of one value per lane, a block being the 32 lanes of a half wave
// (q8_quantize_group's arithmetic). Returns fp32(fp16(d)).
__device__ __forceinline__ float half_wave_quantize(float v, int8_t & q) {
    const float amax = half_wave_amax(v);
    const float d = amax / 127.0f;
    const float id = (amax != 0.0f) ? 127.0f / amax : 0.0f;
    q = (int8_t) (int) __builtin_rintf(v * id);
    return h2f(f2h(d));
}

// The x86 Q8_0 quantisation of element tid of a row of 512 held one per thread (a block is the
// 32 threads of a half wave), stored into the sliced LDS row (s_x, s_d) that the 8-lane dot reads.
__device__ __forceinline__ void wg_quantize_row(float y, int tid, int8_t * s_x, float * s_d) {
    const float amax = half_wave_amax(y);
    const float d = amax / 127.0f;
    const float id = (amax != 0.0f) ? 127.0f / amax : 0.0f;
    const int8_t q = (int8_t) (int) __builtin_rintf(y * id);
    const int blk = tid >> 5, c = tid & 31;
    s_x[(c >> 2) * DL_SLICE_B + blk * 4 + (c & 3)] = q;
    if (c == 0) s_d[blk] = h2f(f2h(d));
}

// One 8-lane x86 Q8_0 dot of a weight row (sliced, 4 int4 of quants + their 16 fp16 scales
// held by this lane) with the LDS row: lane j's chain over the 16 blocks, then the 3-step
// butterfly over the 8 lanes (the order of q8.hip).
__device__ __forceinline__ float row_dot8(const int4 (&w)[4], const uint2 (&dh)[4], const int8_t * s_x,
                                          const float * s_d, int j) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float dw0 = h2f((uint16_t) (dh[i].x & 0xffff)), dw1 = h2f((uint16_t) (dh[i].x >> 16));
        const float dw2 = h2f((uint16_t) (dh[i].y & 0xffff)), dw3 = h2f((uint16_t) (dh[i].y >> 16));
        const int4 xv = *reinterpret_cast<const int4 *>(&s_x[j * DL_SLICE_B + 16 * i]);
        const float4 dx = *reinterpret_cast<const float4 *>(&s_d[4 * i]);
        acc = __builtin_fmaf(dw0 * dx.x, (float) __builtin_amdgcn_sdot4(w[i].x, xv.x, 0, false), acc);
        acc = __builtin_fmaf(dw1 * dx.y, (float) __builtin_amdgcn_sdot4(w[i].y, xv.y, 0, false), acc);
        acc = __builtin_fmaf(dw2 * dx.z, (float) __builtin_amdgcn_sdot4(w[i].z, xv.z, 0, false), acc);
        acc = __builtin_fmaf(dw3 * dx.w, (float) __builtin_amdgcn_sdot4(w[i].w, xv.w, 0, false), acc);
    }
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) in lane j = 0 of each 8-lane row (the other lanes
    // hold partial values): rotating a 16-lane DPP row by 12 brings lane j + 4 to lanes j < 4 of
    // either 8-lane half
    acc = acc + dpp_f<DPP_ROR12>(acc);
    acc = acc + dpp_f<DPP_XOR2>(acc);
    acc = acc + dpp_f<DPP_XOR1>(acc);
    return acc;
}

// The exact int32 dot of one tiled 32 x 32 weight tile-block row with a Q8_0 activation block in
// LDS: lane 32 hh + i holds quants [16 hh, 16 hh + 16) of row i; lane i < 32 ends with the sum.
__device__ __forceinline__ int tile_dot(const int4 & w, const int8_t * a_blk, int lane) {
    const int4 av = *reinterpret_cast<const int4 *>(a_blk + 16 * (lane >> 5));
    int s = __builtin_amdgcn_sdot4(w.x, av.x, 0, false);
    s = __builtin_amdgcn_sdot4(w.y, av.y, s, false);
    s = __builtin_amdgcn_sdot4(w.z, av.z, s, false);
    s = __builtin_amdgcn_sdot4(w.w, av.w, s, false);
    // lanes i < 32 add lane i + 32 (the other lanes' results are not used)
    const auto sw = __builtin_amdgcn_permlane32_swap(s, s, false, false);
    return s + (int) sw[1];
}

// ---- the persistent decode's barrier among the 32 workgroups of one XCD ----
// Each workgroup owns one flag word and stores into it, after its stores of a phase are complete,
// the count of phases it has finished (an epoch from the step counter plus the phase); a workgroup
// that needs the results of a phase waits until all 32 words have reached it. The words and the
// rows the phases exchange are written with plain stores (performed at the XCD's L2) and read
// with device-scope loads (which bypass the CU's L1), so the L2 shared by the XCD carries them;
// no atomic read-modify-write is involved. Every wait is bounded: a workgroup that gives up (or
// finds the error word set) sets the error word and the kernel ends, the host then falls back.
constexpr int XBAR_SPIN_MAX = 1 << 18;     // polls (each a round trip to L2): about 0.2 s
struct XBar {
    int * flags;    // the XCD's 32 flag words
    int * err;      // error word (0: none)
    int target;     // wait until every word >= target (0: no wait)
    int li = -1;    // the persistent decode's layer (its phase stamps); -1 outside it
};

// Phase stamps of the persistent decode, in a library built with GSVK_PHASE_STAMPS only (build.py
// --phase-stamps): thread 0 of every workgroup records s_memrealtime (100 MHz) at each step of
// each layer's two phases into slot [workgroup][layer * 16 + event] (the last launch's values
// remain): 0 barrier seen, 1 input row quantised, 2 QKV and K/V append done, 3 attention merged,
// 4 out-projection partial row stored, 5 flag stored; 8 barrier seen, 9 LN1 row quantised, 10
// FFN1 blocks quantised, 11 FFN2 partial row stored, 12 flag stored; slot 63 * 16: the launch's
// start, 63 * 16 + 1: the workgroup's XCD. gsvk_phase_stamps reads them.
constexpr int DL_STAMP_SLOTS = 64 * 16;
#if defined(GSVK_PHASE_STAMPS)
__device__ long long g_phase_stamps[DEC_PERSIST_WGS][DL_STAMP_SLOTS];
#define DL_STAMP_AT(li, ev, v)                                                                         \
    do {                                                                                               \
        if ((li) >= 0 && threadIdx.x == 0 && blockIdx.x < DEC_PERSIST_WGS)                              \
            g_phase_stamps[blockIdx.x][((li) & 63) * 16 + (ev)] = (long long) (v);                     \
    } while (0)
#else
#define DL_STAMP_AT(li, ev, v) \
    do {                      \
    } while (0)
#endif
#define DL_STAMP(li, ev) DL_STAMP_AT(li, ev, __builtin_amdgcn_s_memrealtime())

// PW: the wave that polls (its loads issued before the poll return ahead of the poll's)
template <int PW = 0>
__device__ __forceinline__ bool xbar_wait(const XBar & x, int tid, int * s_ok) {
    if (x.target == 0) return true;
    if ((tid >> 6) == PW) {
        const int ln = tid & 63;
        bool ok = false;
        for (int spins = 0; spins < XBAR_SPIN_MAX; spins++) {
            const int v = ln < 32 ? __hip_atomic_load(&x.flags[ln], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : x.target;
            if (__all(v >= x.target)) {
                ok = true;
                break;
            }
            if ((spins & 255) == 255 &&
                __hip_atomic_load(x.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
                break;
        }
        if (ln == 0) {
            *s_ok = ok;
            if (!ok) __hip_atomic_store(x.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    return *s_ok != 0;
}

__device__ __forceinline__ void xbar_signal(int * flag, int value, int tid) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);   // this thread's stores are performed
    __syncthreads();
    if (tid == 0) __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// a row element another workgroup of the XCD wrote in this kernel (PERSIST) or before it
template <bool PERSIST>
__device__ __forceinline__ float ld_row(const float * p) {
    if constexpr (PERSIST) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

}  // namespace

// Launch 1's work for (head h, sequence b). PERSIST (the persistent decode): the loads that do not
// depend on the previous phase go out first, then the wait on `bar`, then the input row's
// operands, read with device-scope loads; returns false when the wait gave up. OPAQUE: the thread
// index is made opaque to the compiler per call, so that the indexing derived from it is
// recomputed for each item instead of being hoisted out of the persistent decode's layer loop and
// kept live across it (which the loop form spilled: 28 VGPRs; without spills it is 0.60 instead of
// 0.67 ms per step at batch 17-24; the one-item form is faster without it).
template <int MODE, int NP, bool PERSIST, bool OPAQUE = false, bool NT = false>
__device__ __forceinline__ bool dec_attn_body(const DecAttnArgs & a, const int h, const int b, const XBar & bar,
                                              const int col_pre = 0, const int beg_pre = 0) {
    constexpr int NW = DL_WAVES;
    constexpr int PASSES = (DL_QKV_ROWS / 8 + NW - 1) / NW;   // 8 rows per wave and pass
    constexpr int WO_T = DL_NBLK / NW;                        // out-projection tiles per wave
    const int B = a.B;
    int tid_v = threadIdx.x;
    if constexpr (OPAQUE) asm volatile("" : "+v"(tid_v));
    const int tid = tid_v;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ks = lane >> 2;
    const int qd = lane & 3;
    const int rsub = lane >> 3;
    const int j = lane & 7;

    __shared__ __align__(16) int8_t s_x[8 * DL_SLICE_B];
    __shared__ __align__(16) float s_d[DL_NBLK];
    __shared__ double s_red[2][DL_WAVES];
    __shared__ __align__(16) float s_q[ATT_HD];
    __shared__ __align__(16) uint16_t s_kv[2][ATT_HD];
    __shared__ float s_m[NW];
    __shared__ float s_l[NW];
    __shared__ float s_o[NW][ATT_HD];
    __shared__ __align__(16) int8_t s_a[DL_WAVES][ATT_HD];
    __shared__ int s_ok;
    if constexpr (PERSIST) __syncthreads();   // the previous item's LDS reads are done

    // ---- loads, in the order their data is needed, with no branch between them ----
    // The key range first, as vector loads (an index the compiler cannot see to be zero): a
    // scalar load's value would be consumed right after it (the compiler places its wait there),
    // holding back every load below; a vector load's wait is placed at its first use, after the
    // scheduling barrier below.
    // (PERSIST: *col_ptr and kv_begin[b] come in as col_pre, beg_pre, read once per launch)
    int col_ld = col_pre, beg_ld = beg_pre;
    if constexpr (!PERSIST) {
        int vz;
        asm volatile("v_mov_b32 %0, 0" : "=v"(vz));
        col_ld = a.col_ptr[vz];
        beg_ld = a.kv_begin[b + vz];
    }
    float xr = 0.0f, xb = 0.0f, xw = 0.0f, xc = 0.0f, xe = 0.0f, xpe = 0.0f;
    float xp[NP];
    int pos = 0;
    auto load_ln_rows = [&]() {
        xr = ld_row<PERSIST>(a.res + (int64_t) b * DL_K + tid);
#pragma unroll
        for (int g = 0; g < NP; g++) xp[g] = ld_row<PERSIST>(a.parts + ((int64_t) g * B + b) * DL_K + tid);
    };
    auto load_ln_params = [&]() {
        xb = a.bias[tid];
        xw = a.wb[tid];
        xc = a.wb[DL_K + tid];
    };
    if constexpr (MODE == IN_LN) {
        if constexpr (!PERSIST) {
            load_ln_rows();
            load_ln_params();
        }
    } else {
        pos = *a.pos_ptr;
        int tk = a.tok[b];
        tk = tk < 0 ? 0 : (tk >= a.vocab ? a.vocab - 1 : tk);
        int pr = pos + a.pos_add - (a.pos_sub ? a.pos_sub[b] : 0);
        pr = pr < 0 ? 0 : pr;
        pr = (a.pe_rows > 0 && pr >= a.pe_rows) ? a.pe_rows - 1 : pr;
        xe = a.emb[(int64_t) tk * DL_K + tid];
        xpe = a.pe[(int64_t) pr * DL_K + tid];
    }
    int4 w[PASSES][4];
    uint2 dh[PASSES][4];
    float rbias[PASSES];
    int4 wo[WO_T];
    uint16_t wos[WO_T];
    auto load_qkv_weights = [&]() {
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            // (the persistent decode: waves past the 96 rows in the second pass load nothing)
            if (PERSIST && (p * NW + wave) * 8 >= DL_QKV_ROWS) break;   // (uniform per wave)
            const int rl = (p * NW + wave) * 8 + rsub;
            const int rlc = rl < DL_QKV_ROWS ? rl : DL_QKV_ROWS - 1;
            const int row = (rlc >> 5) * DL_K + h * ATT_HD + (rlc & 31);
            const int4 * wsl = reinterpret_cast<const int4 *>(a.wq + ((int64_t) row * 8 + j) * DL_NBLK * 4);
            const uint2 * wdr = reinterpret_cast<const uint2 *>(a.wd + (int64_t) row * DL_NBLK);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                w[p][i] = wsl[i];
                dh[p][i] = wdr[i];
            }
            rbias[p] = a.bqkv[row];
        }
    };
    auto load_out_weights = [&]() {
#pragma unroll
        for (int u = 0; u < WO_T; u++) {
            const int t = wave + NW * u;    // 32-row tile of the out projection's 512 outputs
            wo[u] = *reinterpret_cast<const int4 *>(a.woq + (((int64_t) t * DL_NBLK + h) << 10) + lane * 16);
            wos[u] = a.wod[(((int64_t) t * DL_NBLK + h) << 5) + (lane & 31)];
        }
    };
    // PERSIST: the QKV weights go out ahead of the barrier's poll, the cached keys after the input
    // row's, behind the wait, and the out projection's once the input row is quantised (issued
    // with the row's loads, they delayed the LayerNorm: batch 16 0.332 -> 0.325 ms per step over
    // 20 steps, 0.348 -> 0.342 over 500)
    load_qkv_weights();
    if constexpr (!PERSIST) load_out_weights();
    // (the key range arrived first: its loads were issued first and retire in order)
    __builtin_amdgcn_sched_barrier(0);
    const int col = __builtin_amdgcn_readfirstlane(col_ld) + a.col_add;   // column of this step's key
    int beg = __builtin_amdgcn_readfirstlane(beg_ld);
    // the first block of cached keys [beg, col) (the new key is substituted later); a wave past
    // the last block loads that block again and does not use it
    const bool col_ok = col >= 0 && col < a.lstride;
    beg = beg < 0 ? 0 : (beg < a.lstride ? beg : (int) a.lstride - 1);
    const int end = col + 1;
    const int nkeys = (col_ok && end > beg) ? end - beg : 0;
    const int nblk = (nkeys + ATT_BLK - 1) / ATT_BLK;
    const int64_t pair = (int64_t) b * DL_NH + h;
    const uint16_t * kb = a.kc + pair * a.lstride * ATT_HD + qd * 8;
    const uint16_t * vb = a.vc + pair * a.lstride * ATT_HD + qd * 8;
    int last_old = col > beg ? col - 1 : beg;
    last_old = last_old < a.lstride ? last_old : (int) a.lstride - 1;
    int blk = nblk > 0 ? (wave < nblk ? wave : nblk - 1) : 0;
    KV8 cur;
    if constexpr (!PERSIST) {
        load_block<NT>(kb, vb, beg + blk * ATT_BLK, last_old, ks, cur);
    } else {
        // polled by wave 4 with 32 FFN groups (batch <= 8), one pass of QKV weights ahead of its
        // poll instead of wave 0's two (batch 1 0.309 -> 0.306 ms per step; at batch 16 no gain)
        // the LayerNorm's weights (constant) ahead of the poll as well: batch 1 0.2847 -> 0.2808 ms
        // per step, batch 16 unchanged
        if constexpr (MODE == IN_LN) load_ln_params();
        if (!xbar_wait<NP == 32 ? 4 : 0>(bar, tid, &s_ok)) return false;
        DL_STAMP(bar.li, 0);
        if constexpr (MODE == IN_LN) load_ln_rows();
        load_block<NT>(kb, vb, beg + blk * ATT_BLK, last_old, ks, cur);
    }

    // ---- the input row: LN2 of the previous layer (or the embedding), quantised into LDS ----
    float x;
    if constexpr (MODE == IN_LN) {
        float r = xp[0];
#pragma unroll
        for (int g = 1; g < NP; g++) r = r + xp[g];
        x = wg_layernorm((xr + r) + xb, xw, xc, lane, wave, s_red);
    } else {
        x = __builtin_fmaf(a.alpha, xpe, xe);
        if (h == 0 && tid == 0 && a.kv_end) a.kv_end[b] = pos + a.kv_end_add;
    }
    if (h == 0 && a.x_out) a.x_out[(int64_t) b * DL_K + tid] = x;
    wg_quantize_row(x, tid, s_x, s_d);
    if constexpr (PERSIST) load_out_weights();
    __syncthreads();
    DL_STAMP(bar.li, 1);

    // ---- q, k, v of head h; the new K/V appended at column col ----
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int rl = (p * NW + wave) * 8 + rsub;
        if ((p * NW + wave) * 8 >= DL_QKV_ROWS) break;   // uniform per wave
        const float acc = row_dot8(w[p], dh[p], s_x, s_d, j);
        if (j == 0 && rl < DL_QKV_ROWS) {
            const int which = rl >> 5, dd = rl & 31;
            const float v = acc + rbias[p];
            if (which == 0) {
                s_q[dd] = v;
            } else {
                const uint16_t hv = f2h(v);
                s_kv[which - 1][dd] = hv;
                if (col_ok) (which == 1 ? a.kc : a.vc)[(pair * a.lstride + col) * ATT_HD + dd] = hv;
            }
        }
    }
    __syncthreads();
    DL_STAMP(bar.li, 2);

    // ---- attention over [beg, col] (the block loop of attention.hip) ----
    float m = -INFINITY, l = 0.0f;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;
    if (nkeys > 0) {   // uniform over the workgroup
        float qv[8];
        const float4 q0 = *reinterpret_cast<const float4 *>(&s_q[qd * 8]);
        const float4 q1 = *reinterpret_cast<const float4 *>(&s_q[qd * 8 + 4]);
        qv[0] = q0.x; qv[1] = q0.y; qv[2] = q0.z; qv[3] = q0.w;
        qv[4] = q1.x; qv[5] = q1.y; qv[6] = q1.z; qv[7] = q1.w;
        const uint4 knew = *reinterpret_cast<const uint4 *>(&s_kv[0][qd * 8]);
        const uint4 vnew = *reinterpret_cast<const uint4 *>(&s_kv[1][qd * 8]);
        if (wave < nblk) {
            while (blk + NW < nblk) {
                KV8 pre;
                load_block<NT>(kb, vb, beg + (blk + NW) * ATT_BLK, last_old, ks, pre);
                attn_block_step<true>(cur, beg + blk * ATT_BLK, end, ks, qv, a.scale_log2, col, knew, vnew, m, l, o);
                cur = pre;
                blk += NW;
            }
            attn_block_step<true>(cur, beg + blk * ATT_BLK, end, ks, qv, a.scale_log2, col, knew, vnew, m, l, o);
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
    }
    __syncthreads();
    DL_STAMP(bar.li, 3);
    // every wave merges the waves' partials (the same arithmetic in each) into the head's output,
    // lane d < 32 holding dimension d, quantised to one Q8_0 block (no valid key: 0, as ggml) and
    // kept in the wave's own LDS slot: no further barrier
    float val = 0.0f;
    if (nkeys > 0) {
        float M = s_m[0];
#pragma unroll
        for (int w2 = 1; w2 < NW; w2++) M = fmaxf(M, s_m[w2]);
        float L = 0.0f, O = 0.0f;
        const int dl = lane & (ATT_HD - 1);
#pragma unroll
        for (int w2 = 0; w2 < NW; w2++) {
            const float f = s_m[w2] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w2] - M);
            L = __builtin_fmaf(s_l[w2], f, L);
            O = __builtin_fmaf(s_o[w2][dl], f, O);
        }
        val = O * (1.0f / L);
    }
    int8_t qa;
    const float da = half_wave_quantize(lane < ATT_HD ? val : 0.0f, qa);
    if (lane < ATT_HD) s_a[wave][lane] = qa;
    __builtin_amdgcn_wave_barrier();

    // ---- out projection of head h: partial row p1[h][b] ----
    float * prow = a.p1 + ((int64_t) h * B + b) * DL_K;
#pragma unroll
    for (int u = 0; u < WO_T; u++) {
        const int t = wave + NW * u;
        const int isum = tile_dot(wo[u], s_a[wave], lane);
        const float y = (h2f(wos[u]) * da) * (float) isum;
        if (lane < 32) prow[t * 32 + lane] = y;
    }
    DL_STAMP(bar.li, 4);
    return true;
}

template <int MODE, int NP>   // NP: the FFN2 partial rows of the input stage (IN_LN)
__global__ void __launch_bounds__(DL_THREADS) k_dec_attn(DecAttnArgs a) {
    dec_attn_body<MODE, NP, false>(a, blockIdx.x, blockIdx.y, XBar{});
}

// Launch 2's work for (hidden group g, sequence b); PERSIST and OPAQUE as for dec_attn_body.
template <int G, bool PERSIST, bool OPAQUE = false>
__device__ __forceinline__ bool dec_ffn_body(const DecFfnArgs & a, const int g, const int b, const XBar & bar) {
    constexpr int NW = DL_WAVES;
    constexpr int U = DL_FFN / G;              // hidden units of the group
    constexpr int UB = U / 32;                 // their Q8_0 blocks
    constexpr int PASSES = U / (8 * NW);       // FFN1 rows: 8 per wave and pass
    constexpr int W2_T = (DL_K / 32) / NW;     // FFN2 output tiles per wave
    constexpr int K2_NBLK = DL_FFN / 32;       // blocks of an FFN2 weight row
    static_assert(U % (8 * NW) == 0 && UB * 32 == U && W2_T * NW * 32 == DL_K, "group shape");
    const int B = a.B;
    int tid_v = threadIdx.x;
    if constexpr (OPAQUE) asm volatile("" : "+v"(tid_v));
    const int tid = tid_v;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int rsub = lane >> 3;
    const int j = lane & 7;

    __shared__ __align__(16) int8_t s_x[8 * DL_SLICE_B];
    __shared__ __align__(16) float s_d[DL_NBLK];
    __shared__ double s_red[2][DL_WAVES];
    __shared__ float s_h[U];
    __shared__ __align__(16) int8_t s_hq[U];
    __shared__ float s_hd[UB];
    __shared__ int s_ok;
    if constexpr (PERSIST) __syncthreads();   // the previous item's LDS reads are done

    // ---- loads: the LN1 operands of element tid, then the group's weights ----
    float xr = 0.0f;
    float xp[DL_NH];
    auto load_ln_rows = [&]() {
        xr = ld_row<PERSIST>(a.res + (int64_t) b * DL_K + tid);
#pragma unroll
        for (int hh = 0; hh < DL_NH; hh++) xp[hh] = ld_row<PERSIST>(a.p1 + ((int64_t) hh * B + b) * DL_K + tid);
    };
    float xb = 0.0f, xw = 0.0f, xc = 0.0f;
    auto load_ln_params = [&]() {
        xb = a.bo[tid];
        xw = a.wb1[tid];
        xc = a.wb1[DL_K + tid];
    };
    if constexpr (!PERSIST) {
        load_ln_rows();
        load_ln_params();
    }
    int4 w1[PASSES][4];
    uint2 d1[PASSES][4];
    float rb1[PASSES];
    int4 w2[W2_T][UB];
    uint16_t d2[W2_T][UB];
    auto load_ffn1_weights = [&]() {
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const int row = g * U + (p * NW + wave) * 8 + rsub;
            const int4 * wsl = reinterpret_cast<const int4 *>(a.w1q + ((int64_t) row * 8 + j) * DL_NBLK * 4);
            const uint2 * wdr = reinterpret_cast<const uint2 *>(a.w1d + (int64_t) row * DL_NBLK);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                w1[p][i] = wsl[i];
                d1[p][i] = wdr[i];
            }
            rb1[p] = a.b1[row];
        }
    };
    auto load_ffn2_weights = [&](int u0 = 0, int u1 = W2_T) {
#pragma unroll
        for (int u = 0; u < W2_T; u++) {
            if (u < u0 || u >= u1) continue;
            const int t = wave + NW * u;
#pragma unroll
            for (int k = 0; k < UB; k++) {
                const int64_t tb = (int64_t) t * K2_NBLK + g * UB + k;
                w2[u][k] = *reinterpret_cast<const int4 *>(a.w2q + (tb << 10) + lane * 16);
                d2[u][k] = a.w2d[(tb << 5) + (lane & 31)];
            }
        }
    };
    // PERSIST: FFN1's weights ahead of the barrier's poll; FFN2's once LN1 is quantised with 32
    // groups (batch <= 8: batch 1 0.293 -> 0.283 ms per step, against after the input row's), with
    // 16 groups (twice the FFN2 bytes per workgroup) half after the input row's and half after LN1
    // (batch 16 0.3158 -> 0.3124; all after LN1: 0.3169 -> 0.3208)
    load_ffn1_weights();
    if constexpr (!PERSIST) {
        load_ffn2_weights();
    } else {
        load_ln_params();
        if (!xbar_wait(bar, tid, &s_ok)) return false;
        DL_STAMP(bar.li, 8);
        load_ln_rows();
        if constexpr (G != 32) load_ffn2_weights(0, 1);
    }

    // ---- n1 = LN1((x + o) + b_o), quantised into LDS ----
    float r = xp[0];
#pragma unroll
    for (int hh = 1; hh < DL_NH; hh++) r = r + xp[hh];
    const float y = wg_layernorm((xr + r) + xb, xw, xc, lane, wave, s_red);
    if (g == 0) a.n1_out[(int64_t) b * DL_K + tid] = y;
    wg_quantize_row(y, tid, s_x, s_d);
    if constexpr (PERSIST && G == 32) load_ffn2_weights();
    if constexpr (PERSIST && G != 32) load_ffn2_weights(1, W2_T);
    __syncthreads();
    DL_STAMP(bar.li, 9);

    // ---- FFN1 + b_1 + ReLU of the group's units ----
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const float acc = row_dot8(w1[p], d1[p], s_x, s_d, j);
        if (j == 0) {
            float v = acc + rb1[p];
            v = v > 0.0f ? v : 0.0f;
            s_h[(p * NW + wave) * 8 + rsub] = v;
        }
    }
    __syncthreads();
    // their Q8_0 blocks: wave k quantises block k
    if (wave < UB) {
        int8_t q1;
        const float d = half_wave_quantize(lane < 32 ? s_h[wave * 32 + lane] : 0.0f, q1);
        if (lane < 32) s_hq[wave * 32 + lane] = q1;
        if (lane == 0) s_hd[wave] = d;
    }
    __syncthreads();
    DL_STAMP(bar.li, 10);

    // ---- FFN2 over the group's blocks: partial row p2[g][b] ----
    float * prow = a.p2 + ((int64_t) g * B + b) * DL_K;
#pragma unroll
    for (int u = 0; u < W2_T; u++) {
        const int t = wave + NW * u;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < UB; k++) {
            const int isum = tile_dot(w2[u][k], s_hq + k * 32, lane);
            acc = __builtin_fmaf(h2f(d2[u][k]) * s_hd[k], (float) isum, acc);
        }
        if (lane < 32) prow[t * 32 + lane] = acc;
    }
    DL_STAMP(bar.li, 11);
    return true;
}

template <int G>
__global__ void __launch_bounds__(DL_THREADS) k_dec_ffn(DecFfnArgs a) {
    dec_ffn_body<G, false>(a, blockIdx.x, blockIdx.y, XBar{});
}

// one layer's two phases of the persistent decode on this workgroup (MODE: layer 0's embedding
// input or a LayerNorm of the previous layer's rows); false when a wait gave up
// A layer's arguments, read through the constant address space (scalar loads into SGPRs: they do
// not change during the launch) with every pointer in it declared a global-memory one, so that the
// loads through them are global loads (counted by vmcnt alone) and not flat ones, whose completion
// an LDS wait would also have to wait for.
#define GSVK_GLOBAL_PTR(ptr) \
    __builtin_assume(!__builtin_amdgcn_is_shared((const void *) (ptr)) && !__builtin_amdgcn_is_private((const void *) (ptr)))
// (device pass only: the host pass sees a plain copy it never runs)
__device__ __forceinline__ DecAttnArgs persist_attn_args(const DecAttnArgs * all, int li) {
#if !defined(__HIP_DEVICE_COMPILE__)
    return all[li];
#else
    DecAttnArgs a = ((const __attribute__((address_space(4))) DecAttnArgs *) all)[li];
    GSVK_GLOBAL_PTR(a.res); GSVK_GLOBAL_PTR(a.parts); GSVK_GLOBAL_PTR(a.bias); GSVK_GLOBAL_PTR(a.wb);
    GSVK_GLOBAL_PTR(a.emb); GSVK_GLOBAL_PTR(a.pe); GSVK_GLOBAL_PTR(a.tok); GSVK_GLOBAL_PTR(a.pos_ptr);
    GSVK_GLOBAL_PTR(a.pos_sub); GSVK_GLOBAL_PTR(a.kv_end); GSVK_GLOBAL_PTR(a.x_out); GSVK_GLOBAL_PTR(a.wq);
    GSVK_GLOBAL_PTR(a.wd); GSVK_GLOBAL_PTR(a.bqkv); GSVK_GLOBAL_PTR(a.kc); GSVK_GLOBAL_PTR(a.vc);
    GSVK_GLOBAL_PTR(a.kv_begin); GSVK_GLOBAL_PTR(a.col_ptr); GSVK_GLOBAL_PTR(a.woq); GSVK_GLOBAL_PTR(a.wod);
    GSVK_GLOBAL_PTR(a.p1);
    return a;
#endif
}
__device__ __forceinline__ DecFfnArgs persist_ffn_args(const DecFfnArgs * all, int li) {
#if !defined(__HIP_DEVICE_COMPILE__)
    return all[li];
#else
    DecFfnArgs a = ((const __attribute__((address_space(4))) DecFfnArgs *) all)[li];
    GSVK_GLOBAL_PTR(a.res); GSVK_GLOBAL_PTR(a.p1); GSVK_GLOBAL_PTR(a.bo); GSVK_GLOBAL_PTR(a.wb1);
    GSVK_GLOBAL_PTR(a.n1_out); GSVK_GLOBAL_PTR(a.w1q); GSVK_GLOBAL_PTR(a.w1d); GSVK_GLOBAL_PTR(a.b1);
    GSVK_GLOBAL_PTR(a.w2q); GSVK_GLOBAL_PTR(a.w2d); GSVK_GLOBAL_PTR(a.p2);
    return a;
#endif
}

// The workgroup's attention items are (head it % 16, sequence x + 8 (it / 16)) for it = w, w + 32:
// at most 2 (4 sequences per XCD), the same in every layer; col (the new key's column before
// col_add) and beg[k] (item k's first key) were read at the launch's start. ONE: at most one
// attention item and one FFN item per workgroup (up to 2 sequences per XCD, batch <= 16), written
// without the item loops; the loop form (batch 17-32) runs its bodies OPAQUE.
static_assert(DEC_PERSIST_MAX_BATCH / 8 * DL_NH <= 2 * 32, "two attention items per workgroup at most");

template <int MODE, int G, bool ONE, bool NT>
__device__ __forceinline__ bool dec_persist_layer(const DecPersistArgs & p, int li, int x, int w, int ns, int epoch,
                                                  const XBar & bar, int * my, int tid, int col, const int (&beg)[2]) {
    const DecAttnArgs aa = persist_attn_args(p.attn, li);
    if constexpr (ONE) {
        if (w < ns * DL_NH) {   // uniform over the workgroup
            XBar bw = bar;
            bw.target = MODE == IN_LN ? epoch + 2 * li : 0;
            bw.li = li;
            if (!dec_attn_body<MODE, MODE == IN_LN ? G : 16, true, false, NT>(aa, w % DL_NH, x + 8 * (w / DL_NH), bw, col,
                                                                               beg[0]))
                return false;
        }
    } else {
        for (int it = w, k = 0; it < ns * DL_NH; it += 32, k++) {
            XBar bw = bar;
            bw.target = (MODE == IN_LN && k == 0) ? epoch + 2 * li : 0;
            bw.li = li;
            if (!dec_attn_body<MODE, MODE == IN_LN ? G : 16, true, true, NT>(aa, it % DL_NH, x + 8 * (it / DL_NH), bw,
                                                                          col, k == 0 ? beg[0] : beg[1]))
                return false;
        }
    }
    xbar_signal(my, epoch + 2 * li + 1, tid);
    DL_STAMP(li, 5);
    const DecFfnArgs fa = persist_ffn_args(p.ffn, li);
    if constexpr (ONE) {
        if (w < ns * G) {
            XBar bw = bar;
            bw.target = epoch + 2 * li + 1;
            bw.li = li;
            if (!dec_ffn_body<G, true>(fa, w % G, x + 8 * (w / G), bw)) return false;
        }
    } else {
        for (int it = w; it < ns * G; it += 32) {
            XBar bw = bar;
            bw.target = it == w ? epoch + 2 * li + 1 : 0;
            bw.li = li;
            if (!dec_ffn_body<G, true, true>(fa, it % G, x + 8 * (it / G), bw)) return false;
        }
    }
    xbar_signal(my, epoch + 2 * li + 2, tid);
    DL_STAMP(li, 12);
    return true;
}

// Placement: the dispatcher hands consecutive workgroups to the 8 XCDs in turn, starting where the
// previous dispatch stopped, so the workgroups on one XCD are 32 consecutive multiples of 8 apart:
// (the XCD, blockIdx / 8) numbers them 0..31 within it. The XCD comes from the hardware (XCC_ID),
// so the workgroups that exchange a sequence's rows share an L2 whatever the placement; a
// placement other than 32 per XCD leaves some flag word unwritten and the waits give up.
template <int G, bool ONE, bool NT>
__global__ void __launch_bounds__(DL_THREADS) k_dec_persist(DecPersistArgs p) {
    const int tid = threadIdx.x;
    int xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const int x = xcc & 7, w = blockIdx.x >> 3;
    __shared__ int s_go;
    if (tid == 0) {
        const bool placed = (xcc & 0xf) < 8;
        if (!placed) __hip_atomic_store(p.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool active = !p.active || __hip_atomic_load(p.active, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
        s_go = placed && __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0 && active;
    }
    __syncthreads();
    if (!s_go) return;
    DL_STAMP(63, 0);
    DL_STAMP_AT(63, 1, x);
    const int ns = x < p.B ? (p.B - 1 - x) / 8 + 1 : 0;   // sequences x, x + 8, ...
    const int epoch = (__builtin_amdgcn_readfirstlane(*p.step) + p.epoch_add) * 64;   // 2 phases per layer, < 64
    const XBar bar{p.flags + x * 32, p.err, 0};
    int * my = p.flags + x * 32 + w;
    const DecAttnArgs a0 = persist_attn_args(p.attn, 0);
    const int col = __builtin_amdgcn_readfirstlane(*a0.col_ptr);
    int beg[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int it = w + 32 * k;
        if (it < ns * DL_NH) beg[k] = __builtin_amdgcn_readfirstlane(a0.kv_begin[x + 8 * (it / DL_NH)]);
    }
    if (!dec_persist_layer<IN_EMB, G, ONE, NT>(p, 0, x, w, ns, epoch, bar, my, tid, col, beg)) return;
    for (int li = 1; li < p.n_layer; li++)
        if (!dec_persist_layer<IN_LN, G, ONE, NT>(p, li, x, w, ns, epoch, bar, my, tid, col, beg)) return;
}

int launch_dec_persist(const DecPersistArgs & a, hipStream_t stream) {
    GSVK_REQUIRE(a.B >= 1 && a.B <= DEC_PERSIST_MAX_BATCH && a.groups == dec_ffn_groups(a.B) && a.n_layer >= 1 &&
                     a.attn && a.ffn && a.flags && a.err && a.step,
                 "dec_persist: bad arguments (batch %d, %d layers)", a.B, a.n_layer);
    // one item per workgroup and phase while the XCD holds at most 2 sequences (32 groups: 1)
#define GSVK_DP(G, ONE)                                                                                     \
    do {                                                                                                    \
        if (a.nt) hipLaunchKernelGGL((k_dec_persist<G, ONE, true>), dim3(DEC_PERSIST_WGS), dim3(DL_THREADS), 0, \
                                     stream, a);                                                            \
        else hipLaunchKernelGGL((k_dec_persist<G, ONE, false>), dim3(DEC_PERSIST_WGS), dim3(DL_THREADS), 0,    \
                                stream, a);                                                                 \
    } while (0)
    if (a.groups == 32) GSVK_DP(32, true);
    else if (a.B <= 16) GSVK_DP(16, true);
    else GSVK_DP(16, false);
#undef GSVK_DP
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

bool dec_persist_device_ok(int device) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return false;
    int occ[6] = {};
    const void * kern[6] = {(const void *) k_dec_persist<16, true, false>, (const void *) k_dec_persist<16, false, false>,
                            (const void *) k_dec_persist<32, true, false>, (const void *) k_dec_persist<16, true, true>,
                            (const void *) k_dec_persist<16, false, true>, (const void *) k_dec_persist<32, true, true>};
    for (int i = 0; i < 6; i++) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ[i], kern[i], DL_THREADS, 0) != hipSuccess || occ[i] < 1) {
            (void) hipGetLastError();
            return false;
        }
    }
    return prop.multiProcessorCount == DEC_PERSIST_WGS && std::string(prop.gcnArchName).rfind("gfx950", 0) == 0;
}

bool dec_layer_supported(int B, int nh, int d_model, int ffn, int64_t max_keys) {
    return B >= 1 && B <= DEC_MAX_BATCH && nh == DL_NH && d_model == DL_K && ffn == DL_FFN &&
           attn_nsplit(B, nh, max_keys) == 1;
}

int launch_dec_attn(const DecAttnArgs & a, hipStream_t stream) {
    GSVK_REQUIRE(a.B >= 1 && a.B <= DEC_MAX_BATCH, "dec_attn: batch %d out of range (1..%d)", a.B, DEC_MAX_BATCH);
    GSVK_REQUIRE(a.wq && a.wd && a.bqkv && a.kc && a.vc && a.kv_begin && a.col_ptr && a.woq && a.wod && a.p1,
                 "dec_attn: null pointer");
    GSVK_REQUIRE(a.lstride > 0, "dec_attn: bad cache stride");
    GSVK_REQUIRE(a.mode == IN_LN ? (a.res && a.parts && a.bias && a.wb)
                                 : (a.mode == IN_EMB && a.emb && a.pe && a.tok && a.pos_ptr),
                 "dec_attn: bad input stage");
    GSVK_REQUIRE(a.mode != IN_LN || a.nparts == 16 || a.nparts == 32, "dec_attn: %d partial rows (16 or 32)",
                 a.nparts);
    const dim3 grid(DL_NH, (unsigned) a.B);
    if (a.mode == IN_LN && a.nparts == 32)
        hipLaunchKernelGGL((k_dec_attn<IN_LN, 32>), grid, dim3(DL_THREADS), 0, stream, a);
    else if (a.mode == IN_LN)
        hipLaunchKernelGGL((k_dec_attn<IN_LN, 16>), grid, dim3(DL_THREADS), 0, stream, a);
    else
        hipLaunchKernelGGL((k_dec_attn<IN_EMB, 16>), grid, dim3(DL_THREADS), 0, stream, a);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_dec_ffn(const DecFfnArgs & a, hipStream_t stream) {
    GSVK_REQUIRE(a.B >= 1 && a.B <= DEC_MAX_BATCH, "dec_ffn: batch %d out of range (1..%d)", a.B, DEC_MAX_BATCH);
    GSVK_REQUIRE(a.res && a.p1 && a.bo && a.wb1 && a.n1_out && a.w1q && a.w1d && a.b1 && a.w2q && a.w2d && a.p2,
                 "dec_ffn: null pointer");
    GSVK_REQUIRE(a.groups == 16 || a.groups == 32, "dec_ffn: %d hidden groups (16 or 32)", a.groups);
    if (a.groups == 32)
        hipLaunchKernelGGL(k_dec_ffn<32>, dim3(32, (unsigned) a.B), dim3(DL_THREADS), 0, stream, a);
    else
        hipLaunchKernelGGL(k_dec_ffn<16>, dim3(16, (unsigned) a.B), dim3(DL_THREADS), 0, stream, a);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_phase_stamps(int64_t * out, size_t n) {
    using namespace gsvk;
    GSVK_REQUIRE(out && n >= (size_t) DEC_PERSIST_WGS * DL_STAMP_SLOTS, "phase_stamps: need %d values",
                 DEC_PERSIST_WGS * DL_STAMP_SLOTS);
#if defined(GSVK_PHASE_STAMPS)
    GSVK_HIP(hipMemcpyFromSymbol(out, HIP_SYMBOL(g_phase_stamps), sizeof(g_phase_stamps), 0, hipMemcpyDeviceToHost));
    return GSVK_OK;
#else
    set_error("phase_stamps: this library was built without phase stamps (build.py --phase-stamps)");
    return GSVK_ERR_STATE;
#endif
}

extern "C" int gsvk_op_dec_attn(int B, const float * res, const float * parts, const float * ln_bias,
                                const float * ln_wb, const float * emb, const float * pe, const int32_t * tok,
                                const int32_t * pos, int pos_add, float alpha, int vocab, int pe_rows,
                                float * x_out, const int8_t * wq, const uint16_t * wd, const float * bqkv,
                                uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                                const int32_t * col, float scale, const int8_t * woq, const uint16_t * wod,
                                float * p1, void * stream) {
    using namespace gsvk;
    DecAttnArgs a{};
    a.mode = res ? IN_LN : IN_EMB;
    a.res = res;
    a.parts = parts;
    a.nparts = DEC_FFN_GROUPS;
    a.bias = ln_bias;
    a.wb = ln_wb;
    a.emb = emb;
    a.pe = pe;
    a.tok = tok;
    a.pos_ptr = pos;
    a.pos_add = pos_add;
    a.pe_rows = pe_rows;
    a.alpha = alpha;
    a.vocab = vocab;
    a.x_out = x_out;
    a.wq = wq;
    a.wd = wd;
    a.bqkv = bqkv;
    a.kc = k;
    a.vc = v;
    a.lstride = lstride;
    a.kv_begin = kv_begin;
    a.col_ptr = col;
    a.col_add = 0;
    a.scale_log2 = scale * LOG2E;
    a.woq = woq;
    a.wod = wod;
    a.p1 = p1;
    a.B = B;
    return launch_dec_attn(a, (hipStream_t) stream);
}

extern "C" int gsvk_op_dec_ffn(int B, const float * res, const float * p1, const float * bo, const float * ln1_wb,
                               float * n1_out, const int8_t * w1q, const uint16_t * w1d, const float * b1,
                               const int8_t * w2q, const uint16_t * w2d, float * p2, void * stream) {
    using namespace gsvk;
    DecFfnArgs a{};
    a.res = res;
    a.p1 = p1;
    a.bo = bo;
    a.wb1 = ln1_wb;
    a.n1_out = n1_out;
    a.w1q = w1q;
    a.w1d = w1d;
    a.b1 = b1;
    a.w2q = w2q;
    a.w2d = w2d;
    a.p2 = p2;
    a.groups = DEC_FFN_GROUPS;
    a.B = B;
    return launch_dec_ffn(a, (hipStream_t) stream);
}

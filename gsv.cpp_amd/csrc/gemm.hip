// Q8_0 x Q8_0 GEMM on the gfx950 matrix cores, for the projections once the batch makes them
// dense contractions (prefill over B*S rows, decode at large batch):
//
//   Y[m][n] = sum_blk  dx[m][blk] * dw[n][blk] * (sum_{k in blk} qx[m][k] * qw[n][k])
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-value Q8_0 block of a 32x32 output tile, so
// every block's integer sum is exact. The scale products dx * dw of the tile come from a second
// MFMA (an fp16 outer product: both scales are fp16 values, so the fp32 products are exact), and
// the vector ALUs do the rest, acc += float(C) * (dx * dw): two instructions per output and
// block, which bound the kernel. The fp32 accumulation order (block by block) differs from the
// ggml-cpu x86 order (8 lanes, then hsum), so results agree with it to fp32 rounding, not bit
// for bit; the decode path keeps the bit-exact GEMV.
//
// Tiling: workgroup 256 threads = 4 waves, output tile 128 (rows m) x 128 (columns n); wave w
// owns rows 64*(w/2).. and columns 64*(w%2).., i.e. 2 x 2 MFMA tiles. K is staged through LDS in
// chunks of 4 blocks (128 values) by direct global -> LDS loads, double buffered: the next
// chunk streams in while the current one is multiplied, with no staging registers (70 KB of LDS
// and <= 256 VGPRs: 2 workgroups per CU, 2 waves per SIMD). Operands arrive with their quants in
// natural order (q[row][k]; scales apart). A lane's MFMA operand is one half (16 values) of a
// block of one row; A and B use the same halves, so the product sums over the block whatever
// order the hardware assigns to the bytes. Per block a wave issues the MFMA pair of a tile two
// tiles ahead of the vector work that consumes it, so that the matrix cores and the vector ALUs
// run side by side.
//
// Epilogue (the options of the decoder's GEMV, layer.h LayerOut): bias, ReLU, fp32 store of
// columns < n_store, the fp16 K/V append, or the Q8_0 quantisation of each 32-column block (in
// natural order: the next GEMM reads it).
#include "common.h"
#include "layer.h"

namespace gsvk {

namespace {
constexpr int GM_THREADS = 256;
constexpr int GM_BM = 128;                 // rows (m) per workgroup
constexpr int GM_BN = 128;                 // columns (n) per workgroup
constexpr int GM_KC = 4;                   // blocks per K chunk
constexpr int GM_NBUF = 2;                 // chunk buffers (a chunk streams in while one is used)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;
}  // namespace

// K chunk buffers, filled by direct global -> LDS loads (no staging registers), block-major:
// a[buf][block][row] is the row's 32 quants of that block. Half h (16 bytes) of row r sits in
// slot h ^ gemm_swz(r), so that the 16-byte operand reads of a wave (lane (i, g) reads half g of
// row i) cover every bank once per 8 and per 16 lanes, and every operand address of a wave is
// one base register plus a constant.
struct GemmLds {
    int8_t a[GM_NBUF][GM_KC][GM_BM][32];
    int8_t b[GM_NBUF][GM_KC][GM_BN][32];
    float da[GM_NBUF][GM_BM * GM_KC];      // activation scales [row][block]
    uint16_t db[GM_NBUF][GM_BN * GM_KC];   // weight scales (fp16) [col][block]
};

__device__ __forceinline__ int gemm_swz(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

// The chunk buffers during the K loop; half of the fp32 output tile (64 rows, padded by 4 floats)
// in the epilogue.
union GemmSmem {
    GemmLds k;
    float y[GM_BM / 2][GM_BN + 4];
};

__device__ __forceinline__ void lds_dma16(const void * g, void * lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *) lds, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void * g, void * lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *) lds, 4, 0, 0);
}
// (a direct load places lane L's data at 4 * L for the 1-, 2- and 4-byte forms: the fp16 weight
// scales travel in pairs)

// Per-lane offsets of a wave's direct loads, fixed over the K loop (32-bit: m * k < 2^31 is
// checked at launch). Wave w loads rows [32 w, 32 w + 32) of the tile: lane L the half of row
// 32 w + L / 2 that belongs in its 16-byte LDS slot.
struct GemmIssue {
    uint32_t xo, wo;          // quants: row offset + half
    uint32_t xdo[GM_KC / 2];  // activation scales: 256 (row, block) pairs per instruction
    uint32_t wdo;             // weight scales: a pair of blocks of one column per lane
};

template <int NBLK>
__device__ __forceinline__ GemmIssue gemm_issue_offsets(int m, int m0, int n0, int wave, int lane) {
    GemmIssue o;
    const int r = 32 * wave + lane / 2;
    const uint32_t half = (uint32_t) ((lane & 1) ^ gemm_swz(r));
    o.xo = (uint32_t) min(m0 + r, m - 1) * (NBLK * 32) + half * 16;
    o.wo = (uint32_t) (n0 + r) * (NBLK * 32) + half * 16;
#pragma unroll
    for (int u = 0; u < GM_KC / 2; u++) {
        const int i = u * 256 + wave * 64 + lane;
        o.xdo[u] = (uint32_t) min(m0 + i / GM_KC, m - 1) * NBLK + i % GM_KC;
    }
    const int i = wave * 64 + lane;
    o.wdo = (uint32_t) (n0 + i / (GM_KC / 2)) * NBLK + 2 * (i % (GM_KC / 2));
    return o;
}

// Issue the direct loads of one K chunk into buffer buf. A wave's load instruction writes 64
// consecutive 16-byte (or 4-byte) LDS slots, lane L the L-th.
template <int NBLK>
__device__ __forceinline__ void gemm_issue(const int8_t * __restrict__ xs, const float * __restrict__ xd,
                                           const int8_t * __restrict__ ws, const uint16_t * __restrict__ wd,
                                           const GemmIssue & o, int chunk, int wave, GemmLds & s, int buf) {
    const int blk0 = chunk * GM_KC;
#pragma unroll
    for (int u = 0; u < GM_KC; u++) {
        lds_dma16(xs + (blk0 + u) * 32 + o.xo, &s.a[buf][u][32 * wave][0]);
        lds_dma16(ws + (blk0 + u) * 32 + o.wo, &s.b[buf][u][32 * wave][0]);
    }
#pragma unroll
    for (int u = 0; u < GM_KC / 2; u++) lds_dma4(xd + blk0 + o.xdo[u], &s.da[buf][u * 256 + wave * 64]);
    // 128 columns x GM_KC fp16 scales, two per 4-byte lane: 64 * GM_KC lanes
    static_assert(GM_BN * GM_KC / 2 == 256, "one weight-scale load per wave");
    lds_dma4(wd + blk0 + o.wdo, &s.db[buf][2 * (wave * 64)]);
}

// One block's MFMA operands for a wave: 16 quants of each of its two row groups (A) and
// column groups (B), and the raw scales of those rows and columns (see gemm_scales).
struct GemmOps {
    v4i fa[2], fb[2];
    float dx[2];
    uint32_t dw[2];   // fp16 bits
};

__device__ __forceinline__ GemmOps gemm_ops(const GemmLds & s, int buf, int bb, int wm, int wn, int li, int lg) {
    GemmOps o;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int ra = wm + 32 * h + li, rb = wn + 32 * h + li;
        o.fa[h] = *reinterpret_cast<const v4i *>(&s.a[buf][bb][ra][16 * (lg ^ gemm_swz(li))]);
        o.fb[h] = *reinterpret_cast<const v4i *>(&s.b[buf][bb][rb][16 * (lg ^ gemm_swz(li))]);
        o.dx[h] = s.da[buf][ra * GM_KC + bb];
        o.dw[h] = s.db[buf][rb * GM_KC + bb];
    }
    return o;
}

// The scales as fp16 MFMA operands holding dx (A) or dw (B) in their first K slot and zeros
// elsewhere (the caller keeps the zeros; only slot 0 is written). Every lane carries its row's or
// column's scale, so the K sum holds two equal terms (one per lane half) and the fp16 MFMA
// returns 2 * dx * dw, exactly (both are fp16 values, so dx * dw is exact in fp32 and doubling
// it is too). The accumulators thus hold exactly twice the sum; the epilogue halves them, which
// is exact as well.
__device__ __forceinline__ void gemm_scales(const GemmOps & o, v8h (&adx)[2], v8h (&bdw)[2]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
        adx[h][0] = (_Float16) o.dx[h];
        bdw[h][0] = __builtin_bit_cast(_Float16, (uint16_t) o.dw[h]);
    }
}

// acc += float(c) * sc over a tile's 16 values per lane (c: exact integer sums of one block; sc:
// twice the scale products)
__device__ __forceinline__ void gemm_fold(float (&acc)[16], const v16i & c, const v16f & sc) {
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = __builtin_fmaf((float) c[v], sc[v], acc[v]);
}

// The maximum over each aligned group of 8 lanes, by DPP: quad swaps (1 0 3 2) and (2 3 0 1),
// then the half-row mirror (lane i <-> 7 - i of the 8), which pairs the two quads.
__device__ __forceinline__ float max8_lanes(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    return v;
}

// The tile of this workgroup. The hardware deals workgroup ids round-robin to the 8 XCDs.
// Renumbered so that each XCD takes a contiguous run of tiles (column tiles fastest), the column
// tiles of a row tile run on one XCD and share its L2 copy of the activation rows.
__device__ __forceinline__ void gemm_tile_origin(int n, int & n0, int & m0) {
    const int total = (int) gridDim.x, b = (int) blockIdx.x;
    const int per = (total + 7) / 8, tall = total % 8 == 0 ? 8 : total % 8;
    const int xcd = b % 8, loc = b / 8;
    const int t = xcd < tall ? xcd * per + loc : tall * per + (xcd - tall) * (per - 1) + loc;
    const int nx = n / GM_BN;
    n0 = (t % nx) * GM_BN;
    m0 = (t / nx) * GM_BM;
}

// A tile of left-padding rows only (out.row_pad): zeros out, no products; returns whether the
// tile was one (the same answer in every thread).
__device__ __forceinline__ bool gemm_pad_tile(const LayerOut & out, int n, int m, int n0, int m0, int tid) {
    bool all_pad = true;
    const int S = out.rows_per_seq;
    const int mend = min(m0 + GM_BM, m);
    for (int r0 = m0; r0 < mend && all_pad;) {
        const int b = r0 / S;
        const int e = min((b + 1) * S, mend);
        if (e - b * S > out.row_pad[b]) all_pad = false;
        r0 = e;
    }
    if (!all_pad) return false;
    const int nblk_out = n / 32;
    for (int i = tid; i < (mend - m0) * (GM_BN / 4); i += GM_THREADS) {
        const int row = m0 + i / (GM_BN / 4), c4 = n0 + 4 * (i % (GM_BN / 4));
        if (out.y && c4 < out.n_store)
            *reinterpret_cast<float4 *>(out.y + (int64_t) row * out.y_stride + c4) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (out.yq) {
            *reinterpret_cast<int *>(out.yq + (int64_t) row * n + c4) = 0;   // natural order
            if ((c4 & 31) == 0) out.yd[(int64_t) row * nblk_out + (c4 >> 5)] = 0.0f;
        }
    }
    return true;
}

// The epilogue of the 128 x 128 GEMMs: acc (a wave's 2 x 2 tiles of 32 x 32) times f is the
// output tile; yl is the LDS space of half the tile (64 rows, padded by 4 floats).
__device__ __forceinline__ void gemm_epilogue(float (*yl)[GM_BN + 4], const float (&acc)[4][16], float f,
                                              const LayerOut & out, int n, int m, int n0, int m0, int wave,
                                              int lane) {
    const int wm = (wave >> 1) * 64;
    const int wn = (wave & 1) * 64;
    const int li = lane & 31;
    const int lg = lane >> 5;
    // Each half of the 128 x 128 tile goes through LDS; then a wave takes 16 of its rows, two per
    // step, lane l the 4 columns 4 (l % 32).. of row 2 i + l / 32, so that every store instruction
    // writes whole rows (fp32: 512 bytes, Q8_0: 128 bytes, K/V: 64 bytes per head) and a Q8_0
    // block is 8 lanes (its absmax: three exchanges).
    int kvcol0 = 0;
    if (out.kc) kvcol0 = *out.col_ptr + out.col_add;
    const int nblk_out = n / 32;
    const int c4 = lane & 31;
    const int col = n0 + 4 * c4;
    float4 b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (out.bias) b4 = *reinterpret_cast<const float4 *>(out.bias + col);
    const bool store_y = out.y && col < out.n_store;
    const bool q8_only = out.yq && !out.y && !out.kc;
    const int colq = n0 + 16 * (lane & 7);
    float bq[16];
#pragma unroll
    for (int k = 0; k < 16; k++) bq[k] = 0.0f;
    if (q8_only && out.bias) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 f = *reinterpret_cast<const float4 *>(out.bias + colq + 4 * j);
            bq[4 * j] = f.x; bq[4 * j + 1] = f.y; bq[4 * j + 2] = f.z; bq[4 * j + 3] = f.w;
        }
    }
    // K/V append: the 32-column block of this lane's columns is one head of K or V
    uint16_t * kv_head = nullptr;
    if (out.kc && (col & ~31) >= out.kv_row0) {
        const int rr = (col & ~31) - out.kv_row0;
        kv_head = (rr / out.d_model == 0 ? out.kc : out.vc) + ((rr % out.d_model) >> 5) * out.lstride * 32 + (col & 31);
    }
#pragma unroll 1
    for (int half = 0; half < 2; half++) {
        if (half) __syncthreads();       // the first half has been read
        if (wm == 64 * half) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int ta = t >> 1, tb = t & 1;
#pragma unroll
                for (int v = 0; v < 16; v++)
                    yl[32 * ta + 8 * (v >> 2) + 4 * lg + (v & 3)][wn + 32 * tb + li] = f * acc[t][v];
            }
        }
        __syncthreads();
        if (q8_only) {
            // Q8_0 output alone: lane l takes the 16 columns 16 (l % 8).. of row l / 8 of a group
            // of 8 rows, so a block is a lane pair (one exchange for its absmax) and its quants are
            // one 16-byte store per lane
#pragma unroll
            for (int it = 0; it < 2; it++) {
                const int r = 16 * wave + 8 * it + (lane >> 3);
                const int row = m0 + 64 * half + r;
                float y[16];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 f = *reinterpret_cast<const float4 *>(&yl[r][16 * (lane & 7) + 4 * j]);
                    y[4 * j] = f.x; y[4 * j + 1] = f.y; y[4 * j + 2] = f.z; y[4 * j + 3] = f.w;
                }
                if (out.bias) {
#pragma unroll
                    for (int k = 0; k < 16; k++) y[k] = y[k] + bq[k];
                }
                if (out.act == 1) {
#pragma unroll
                    for (int k = 0; k < 16; k++) y[k] = y[k] > 0.0f ? y[k] : 0.0f;
                }
                float amax = 0.0f;
#pragma unroll
                for (int k = 0; k < 16; k++) amax = fmaxf(amax, fabsf(y[k]));
                amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
                const float d = amax / 127.0f;
                const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
                int w[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    w[j] = 0;
#pragma unroll
                    for (int t = 0; t < 4; t++) w[j] |= (((int) __builtin_rintf(y[4 * j + t] * id)) & 0xff) << (8 * t);
                }
                if (row < m) {
                    *reinterpret_cast<int4 *>(out.yq + (int64_t) row * n + colq) = make_int4(w[0], w[1], w[2], w[3]);
                    if ((lane & 1) == 0) out.yd[(int64_t) row * nblk_out + (colq >> 5)] = h2f(f2h(d));
                }
            }
            continue;
        }
        float4 yv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) yv[i] = *reinterpret_cast<const float4 *>(&yl[16 * wave + 2 * i + (lane >> 5)][4 * c4]);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int row = m0 + 64 * half + 16 * wave + 2 * i + (lane >> 5);
            float4 y = yv[i];
            if (out.bias) { y.x = y.x + b4.x; y.y = y.y + b4.y; y.z = y.z + b4.z; y.w = y.w + b4.w; }
            if (out.act == 1) {
                y.x = y.x > 0.0f ? y.x : 0.0f; y.y = y.y > 0.0f ? y.y : 0.0f;
                y.z = y.z > 0.0f ? y.z : 0.0f; y.w = y.w > 0.0f ? y.w : 0.0f;
            }
            const bool valid = row < m;
            if (valid && store_y) *reinterpret_cast<float4 *>(out.y + (int64_t) row * out.y_stride + col) = y;
            if (out.yq) {
                const float amax = max8_lanes(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
                const float d = amax / 127.0f;
                const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
                const int w = (((int) __builtin_rintf(y.x * id)) & 0xff) | ((((int) __builtin_rintf(y.y * id)) & 0xff) << 8) |
                              ((((int) __builtin_rintf(y.z * id)) & 0xff) << 16) | ((((int) __builtin_rintf(y.w * id)) & 0xff) << 24);
                if (valid) {
                    *reinterpret_cast<int *>(out.yq + (int64_t) row * n + col) = w;   // natural order
                    if ((lane & 7) == 0) out.yd[(int64_t) row * nblk_out + (col >> 5)] = h2f(f2h(d));
                }
            }
            if (kv_head && valid) {
                const int b = row / out.rows_per_seq;
                const int kcol = kvcol0 + row % out.rows_per_seq;
                uint2 w;
                w.x = (uint32_t) f2h(y.x) | ((uint32_t) f2h(y.y) << 16);
                w.y = (uint32_t) f2h(y.z) | ((uint32_t) f2h(y.w) << 16);
                *reinterpret_cast<uint2 *>(kv_head + ((int64_t) b * out.n_head * out.lstride + kcol) * 32) = w;
            }
        }
    }
}

template <int NBLK>
__global__ void __launch_bounds__(GM_THREADS) __attribute__((amdgpu_waves_per_eu(2))) k_q8_gemm(const int8_t * __restrict__ ws,
                                                           const uint16_t * __restrict__ wd, int n, int m,
                                                           const int8_t * __restrict__ xs,
                                                           const float * __restrict__ xd, LayerOut out) {
    constexpr int NCH = NBLK / GM_KC;
    __shared__ __align__(16) GemmSmem sm;
    GemmLds & s = sm.k;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int n0, m0;
    gemm_tile_origin(n, n0, m0);
    if (out.row_pad && gemm_pad_tile(out, n, m, n0, m0, tid)) return;   // (uniform)
    const int wm = (wave >> 1) * 64;   // this wave's rows within the tile
    const int wn = (wave & 1) * 64;    // and columns
    const int li = lane & 31;          // MFMA: row of A / column of B held by this lane
    const int lg = lane >> 5;          // MFMA: which half of the block

    float acc[4][16];                  // tile t = 2 * ta + tb; twice the output (see gemm_ops)
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    const GemmIssue io = gemm_issue_offsets<NBLK>(m, m0, n0, wave, lane);
#pragma unroll
    for (int c = 0; c < GM_NBUF - 1; c++)
        if (c < NCH) gemm_issue<NBLK>(xs, xd, ws, wd, io, c, wave, s, c);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

#pragma unroll 1
    for (int ch = 0; ch < NCH; ch++) {
        const int buf = ch % GM_NBUF;
        // the chunk GM_NBUF - 1 ahead streams into the buffer read before the previous barrier
        if (ch + GM_NBUF - 1 < NCH)
            gemm_issue<NBLK>(xs, xd, ws, wd, io, ch + GM_NBUF - 1, wave, s, (ch + GM_NBUF - 1) % GM_NBUF);
        GemmOps op = gemm_ops(s, buf, 0, wm, wn, li, lg);
        v8h adx[2] = {v8h{}, v8h{}}, bdw[2] = {v8h{}, v8h{}};
        // Per block: the four tiles' MFMA pairs are issued two tiles ahead of the vector work that
        // consumes them, so that the matrix cores run while the vector ALUs fold the previous
        // tile; the next block's operands are read from LDS under the last two folds. The
        // scheduling barriers keep the compiler from regrouping the pairs (it would otherwise
        // serialise every tile on one result register set).
#pragma unroll
        for (int bb = 0; bb < GM_KC; bb++) {
            gemm_scales(op, adx, bdw);
            const v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(op.fa[0], op.fb[0], v16i{}, 0, 0, 0);
            const v16f s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(adx[0], bdw[0], v16f{}, 0, 0, 0);
            const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(op.fa[0], op.fb[1], v16i{}, 0, 0, 0);
            const v16f s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(adx[0], bdw[1], v16f{}, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            gemm_fold(acc[0], c0, s0);
            __builtin_amdgcn_sched_barrier(0);
            const v16i c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(op.fa[1], op.fb[0], v16i{}, 0, 0, 0);
            const v16f s2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(adx[1], bdw[0], v16f{}, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            gemm_fold(acc[1], c1, s1);
            __builtin_amdgcn_sched_barrier(0);
            const v16i c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(op.fa[1], op.fb[1], v16i{}, 0, 0, 0);
            const v16f s3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(adx[1], bdw[1], v16f{}, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (bb + 1 < GM_KC) op = gemm_ops(s, buf, bb + 1, wm, wn, li, lg);
            __builtin_amdgcn_sched_barrier(0);
            gemm_fold(acc[2], c2, s2);
            gemm_fold(acc[3], c3, s3);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(0);   // the chunks issued so far have landed
        __syncthreads();                 // and every wave is done with this one
    }

    gemm_epilogue(sm.y, acc, 0.5f, out, n, m, n0, m0, wave, lane);   // (acc holds twice the output)
}

// ---- Q8_0 activations x fp16 weights on the fp16 matrix cores (the prefill's fp16 mode) ----
// The tiling, staging and epilogue of k_q8_gemm, for weights dequantised once to fp16
// (w16[n][k] = fp16(d * q), nearest even) and activations still in Q8_0: each wave turns its A
// operand (16 quants of a row and the row's block scale) into fp16(dx * q) in registers and
// issues plain v_mfma_f32_32x32x16_f16, two per 32-value block and tile, whose fp32 accumulators
// take the products directly (no per-block fold). Both operands are rounded to fp16 (at most
// 2^-11 relative each), so an output differs from ggml's by about 1e-4 of its row's scale
// instead of by fp32 rounding.
namespace {
// s_waitcnt operand that waits until at most n vector-memory operations are outstanding (gfx9
// encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at their maxima, i.e. not waited on)
#define GSVK_VMCNT(n) ((((n) & 0xF) | ((((n) >> 4) & 3) << 14)) | (0x7 << 4) | (0xF << 8))
constexpr int GH_KC = 2;     // blocks per K chunk
constexpr int GH_NBUF = 2;   // chunk buffers: the next chunk streams in while one is used
// direct loads a wave issues per chunk: GH_KC of activation quants, 1 of their scales, 4 of weights
constexpr int GH_LOADS = GH_KC + 1 + 4;
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
}  // namespace

// K chunk buffers: activation quants and scales as GemmLds; weights b[buf][block][col] = the 32
// fp16 values of that column's block (64 bytes, four 16-byte slots, slot s at s ^ gemm_swz_h(col)
// so that 8 consecutive columns read by a half wave hit distinct banks).
struct GemmLdsH {
    int8_t a[GH_NBUF][GH_KC][GM_BM][32];
    uint8_t b[GH_NBUF][GH_KC][GM_BN][64];
    float da[GH_NBUF][GM_BM * GH_KC];
};

union GemmSmemH {
    GemmLdsH k;
    float y[GM_BM / 2][GM_BN + 4];
};

__device__ __forceinline__ int gemm_swz_h(int c) { return (c >> 1) & 3; }

// The workgroup barrier of the fp16 GEMM's K loop, without the release fence of __syncthreads
// (which waits for every outstanding direct load, the chunk streaming ahead included): each
// wave has waited for its own loads of the next chunk before it arrives, the LDS is one memory
// for the workgroup, and the operands read from the current chunk are in registers (their uses
// waited for them). The memory clobber keeps the compiler's LDS accesses on their side of it.
__device__ __forceinline__ void gemm_barrier() { asm volatile("s_barrier" ::: "memory"); }

struct GemmIssueH {
    uint32_t xo;       // activation quants: row offset + half (as GemmIssue)
    uint32_t xdo;      // activation scales: one (row, block) pair per lane
    uint32_t wo[4];    // weights: byte offset of this lane's 16-byte piece, per instruction
};

// Wave w issues activation rows [32 w, 32 w + 32) (as k_q8_gemm) and weight instructions
// g = 4 w + j, j < 4, of the chunk's 16: instruction g covers block g / 8 of the columns
// 16 (g % 8) .., lane L the slot L % 4 of column 16 (g % 8) + L / 4.
template <int NBLK>
__device__ __forceinline__ GemmIssueH gemm_issue_offsets_h(int m, int m0, int n0, int wave, int lane) {
    GemmIssueH o;
    const int r = 32 * wave + lane / 2;
    const uint32_t half = (uint32_t) ((lane & 1) ^ gemm_swz(r));
    o.xo = (uint32_t) min(m0 + r, m - 1) * (NBLK * 32) + half * 16;
    const int i = wave * 64 + lane;   // (row, block) = (i / GH_KC, i % GH_KC)
    o.xdo = (uint32_t) min(m0 + i / GH_KC, m - 1) * NBLK + i % GH_KC;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int g = 4 * wave + j;
        const int c = 16 * (g % 8) + lane / 4;
        const int piece = (lane & 3) ^ gemm_swz_h(c);
        o.wo[j] = (uint32_t) (n0 + c) * (NBLK * 64) + (uint32_t) (g / 8) * 64 + (uint32_t) piece * 16;
    }
    return o;
}

template <int NBLK>
__device__ __forceinline__ void gemm_issue_h(const int8_t * __restrict__ xs, const float * __restrict__ xd,
                                             const uint8_t * __restrict__ w16, const GemmIssueH & o, int chunk,
                                             int wave, GemmLdsH & s, int buf) {
    const int blk0 = chunk * GH_KC;
#pragma unroll
    for (int u = 0; u < GH_KC; u++) lds_dma16(xs + (blk0 + u) * 32 + o.xo, &s.a[buf][u][32 * wave][0]);
    static_assert(GM_BM * GH_KC == 256, "one activation-scale load per wave");
    lds_dma4(xd + blk0 + o.xdo, &s.da[buf][wave * 64]);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int g = 4 * wave + j;
        lds_dma16(w16 + (uint32_t) blk0 * 64 + o.wo[j], &s.b[buf][g / 8][16 * (g % 8)][0]);
    }
}

struct GemmOpsH {
    v4i fa[2];       // 16 activation quants (k = 16 lg ..) of the two row groups
    float dx[2];
    v8h fb[2][2];    // fp16 weights of the two column groups: k = 16 lg .. + 8, 16 lg + 8 .. + 8
};

__device__ __forceinline__ GemmOpsH gemm_ops_h(const GemmLdsH & s, int buf, int bb, int wm, int wn, int li, int lg) {
    GemmOpsH o;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int ra = wm + 32 * h + li, rb = wn + 32 * h + li;
        o.fa[h] = *reinterpret_cast<const v4i *>(&s.a[buf][bb][ra][16 * (lg ^ gemm_swz(li))]);
        o.dx[h] = s.da[buf][ra * GH_KC + bb];
        const int sw = gemm_swz_h(rb);
        o.fb[h][0] = *reinterpret_cast<const v8h *>(&s.b[buf][bb][rb][16 * ((2 * lg) ^ sw)]);
        o.fb[h][1] = *reinterpret_cast<const v8h *>(&s.b[buf][bb][rb][16 * ((2 * lg + 1) ^ sw)]);
    }
    return o;
}

// fp16(d * q) of 16 quants, in k order, as two 8-value MFMA operands. The fp16 with bits
// 0x6400 | (q ^ 0x80) is 1024 + q + 128 exactly; less 1152 it is q, and the product with d
// (an fp16 value) rounds once, to nearest even, as fp16(d * q) computed in fp32 does.
__device__ __forceinline__ void q8_to_h16(const v4i & q, float d, v8h & lo, v8h & hi) {
    const _Float16 dh = (_Float16) d;
    const v2h dd = {dh, dh};
    const v2h off = {(_Float16) 1152.0f, (_Float16) 1152.0f};
    v2h r[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t x = (uint32_t) q[w] ^ 0x80808080u;
        const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);   // bytes 0, 1
        const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);   // bytes 2, 3
        r[2 * w] = (__builtin_bit_cast(v2h, p01) - off) * dd;
        r[2 * w + 1] = (__builtin_bit_cast(v2h, p23) - off) * dd;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        lo[2 * i] = r[i][0];
        lo[2 * i + 1] = r[i][1];
        hi[2 * i] = r[4 + i][0];
        hi[2 * i + 1] = r[4 + i][1];
    }
}

template <int NBLK>
__global__ void __launch_bounds__(GM_THREADS) __attribute__((amdgpu_waves_per_eu(2))) k_q8h_gemm(const uint8_t * __restrict__ w16,
                                                           int n, int m, const int8_t * __restrict__ xs,
                                                           const float * __restrict__ xd, LayerOut out) {
    constexpr int NCH = NBLK / GH_KC;
    __shared__ __align__(16) GemmSmemH sm;
    GemmLdsH & s = sm.k;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int n0, m0;
    gemm_tile_origin(n, n0, m0);
    if (out.row_pad && gemm_pad_tile(out, n, m, n0, m0, tid)) return;   // (uniform)
    const int wm = (wave >> 1) * 64;
    const int wn = (wave & 1) * 64;
    const int li = lane & 31;
    const int lg = lane >> 5;

    v16f acc[4] = {v16f{}, v16f{}, v16f{}, v16f{}};
    const GemmIssueH io = gemm_issue_offsets_h<NBLK>(m, m0, n0, wave, lane);
    static_assert(NCH >= GH_NBUF - 1, "the chunks in flight exist");
#pragma unroll
    for (int c = 0; c < GH_NBUF - 1; c++) gemm_issue_h<NBLK>(xs, xd, w16, io, c, wave, s, c);
    // chunk 0 has landed (the loads retire in order)
    __builtin_amdgcn_s_waitcnt(GSVK_VMCNT((GH_NBUF - 2) * GH_LOADS));
    gemm_barrier();

#pragma unroll 1
    for (int ch = 0; ch < NCH; ch++) {
        const int buf = ch % GH_NBUF;
        // chunk ch + GH_NBUF - 1 streams into the buffer that every wave finished reading before
        // the last barrier
        const int ahead = ch + GH_NBUF - 1;
        if (ahead < NCH) gemm_issue_h<NBLK>(xs, xd, w16, io, ahead, wave, s, ahead % GH_NBUF);
#pragma unroll
        for (int bb = 0; bb < GH_KC; bb++) {
            const GemmOpsH op = gemm_ops_h(s, buf, bb, wm, wn, li, lg);
            v8h a[2][2];
            q8_to_h16(op.fa[0], op.dx[0], a[0][0], a[0][1]);
            q8_to_h16(op.fa[1], op.dx[1], a[1][0], a[1][1]);
            // the first k half of all four tiles, then the second: dependent products 4 apart
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[t >> 1][kh], op.fb[t & 1][kh], acc[t], 0, 0, 0);
        }
        // chunk ch + 1 has landed (only the later chunks' loads may still be in flight), and
        // every wave is done with chunk ch
        if constexpr (GH_NBUF == 3) {
            if (ahead < NCH)
                __builtin_amdgcn_s_waitcnt(GSVK_VMCNT(GH_LOADS));
            else
                __builtin_amdgcn_s_waitcnt(GSVK_VMCNT(0));
        } else {
            static_assert(GH_NBUF == 2, "two or three chunk buffers");
            __builtin_amdgcn_s_waitcnt(GSVK_VMCNT(0));
        }
        gemm_barrier();
    }
    float accf[4][16];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) accf[t][v] = acc[t][v];
    gemm_epilogue(sm.y, accf, 1.0f, out, n, m, n0, m0, wave, lane);
}

// w16[n][k] = fp16(d[n][k/32] * q[n][k]) (nearest even): each thread 16 values
__global__ void __launch_bounds__(256) k_q8_dequant_f16(const int8_t * __restrict__ q, const uint16_t * __restrict__ d,
                                                       int64_t n16, uint16_t * __restrict__ w16) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;   // 16-value piece
    if (i >= n16) return;
    const int4 qv = *reinterpret_cast<const int4 *>(q + 16 * i);
    const float dv = h2f(d[i >> 1]);
    const int w[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int b0 = (int) (int8_t) ((w[j >> 1] >> (16 * (j & 1))) & 0xff);
        const int b1 = (int) (int8_t) ((w[j >> 1] >> (16 * (j & 1) + 8)) & 0xff);
        o[j] = (uint32_t) f2h(dv * (float) b0) | ((uint32_t) f2h(dv * (float) b1) << 16);
    }
    uint4 * dst = reinterpret_cast<uint4 *>(w16 + 16 * i);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

int launch_q8_dequant_f16(const int8_t * q, const uint16_t * d, int64_t n, int64_t k, uint16_t * w16,
                          hipStream_t stream) {
    GSVK_REQUIRE(q && d && w16 && n > 0 && k > 0 && k % 32 == 0, "q8_dequant_f16: bad arguments");
    GSVK_REQUIRE(((uintptr_t) q & 15) == 0 && ((uintptr_t) w16 & 15) == 0,
                 "q8_dequant_f16: q and w16 must be 16-byte aligned");
    const int64_t n16 = n * k / 16;
    hipLaunchKernelGGL(k_q8_dequant_f16, dim3((unsigned) ((n16 + 255) / 256)), dim3(256), 0, stream, q, d, n16, w16);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_q8h_gemm(const uint16_t * w16, int64_t n, int64_t k, int64_t m, const int8_t * xs, const float * xd,
                    const LayerOut & out, hipStream_t stream) {
    GSVK_REQUIRE(w16 && xs && xd, "q8h_gemm: null pointer");
    GSVK_REQUIRE(n > 0 && n % GM_BN == 0 && m > 0 && (k == 512 || k == 2048),
                 "q8h_gemm: n must be a multiple of %d and k 512 or 2048 (n=%lld k=%lld m=%lld)", GM_BN,
                 (long long) n, (long long) k, (long long) m);
    GSVK_REQUIRE(m * k < ((int64_t) 1 << 31) && n * k * 2 < ((int64_t) 1 << 31),
                 "q8h_gemm: operands above 2 GiB (m=%lld n=%lld k=%lld)", (long long) m, (long long) n, (long long) k);
    GSVK_REQUIRE(!out.yq || (out.yd && out.yq_layout == Q8_NATURAL), "q8h_gemm: bad quantised output");
    GSVK_REQUIRE(!out.kc || (out.vc && out.col_ptr && out.rows_per_seq > 0 && out.kv_row0 + 2 * out.d_model <= n),
                 "q8h_gemm: bad KV epilogue");
    GSVK_REQUIRE(!out.row_pad || out.rows_per_seq > 0, "q8h_gemm: padding rows need rows_per_seq");
    GSVK_REQUIRE(out.act == 0 || out.act == 1, "q8h_gemm: act must be 0 or 1");
    GSVK_REQUIRE(((uintptr_t) w16 & 15) == 0 && ((uintptr_t) out.bias & 15) == 0 && ((uintptr_t) out.y & 15) == 0 &&
                     out.y_stride % 4 == 0 && ((uintptr_t) out.kc & 15) == 0 && ((uintptr_t) out.vc & 15) == 0,
                 "q8h_gemm: w16, bias, y (and its row stride) and the K/V caches must be 16-byte aligned");
    const dim3 grid((unsigned) (n / GM_BN * ((m + GM_BM - 1) / GM_BM)));
    const uint8_t * wb = reinterpret_cast<const uint8_t *>(w16);
    if (k == 512)
        hipLaunchKernelGGL(k_q8h_gemm<16>, grid, dim3(GM_THREADS), 0, stream, wb, (int) n, (int) m, xs, xd, out);
    else
        hipLaunchKernelGGL(k_q8h_gemm<64>, grid, dim3(GM_THREADS), 0, stream, wb, (int) n, (int) m, xs, xd, out);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

// ---- small batches (decode at 64-256 rows): tiles of 32 columns x 32*MT rows ----
// A 128 x 128 tile leaves most of the chip idle at these sizes (a 512-column projection would
// be 4 workgroups). Here a workgroup of 4 waves owns 32 columns and 32*MT rows, and the K range
// is split over its waves (wave w takes blocks [w*NBLK/4, (w+1)*NBLK/4)): each wave computes the
// whole tile over its quarter with operands loaded from global memory straight into registers
// (lane (li, lg): 16 values of row/column li, half lg of the block), a group of blocks ahead of
// its use. The four partial tiles are summed through LDS in wave order, so the result does not
// depend on timing. Same arithmetic per block as k_q8_gemm.
constexpr int64_t GS_MAX_ROWS = 256;      // launch_q8_gemm takes this kernel up to this many rows

template <int NBLK, int MT, int W = 4>   // W waves, each a W-th of K
__global__ void __launch_bounds__(W * 64) k_q8_gemm_small(Q8Weights w, int n, int m,
                                                                const int8_t * __restrict__ xs,
                                                                const float * __restrict__ xd,
                                                                bool x_tiled, LayerOut out) {
    constexpr int NBW = NBLK / W;                                  // blocks per wave
    // blocks per load group: every load at once for one row tile (16 blocks = 128 VGPRs of
    // operands), two or eight groups for more rows
    constexpr int G = (NBW <= 4 || MT == 1) ? NBW : (MT == 2 ? NBW / 2 : 2);
    constexpr int NG = NBW / G;
    static_assert(NBW % G == 0, "load groups must tile the wave's blocks");
    __shared__ float red[W][32 * MT][33];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 31;
    const int lg = lane >> 5;
    const int n0 = blockIdx.x * 32;
    const int m0 = blockIdx.y * 32 * MT;
    const int kb0 = wave * NBW;
    // the epilogue's own operands first: their round trip overlaps the K loop
    const int cg = tid & 7;
    const int col = n0 + 4 * cg;
    float4 bias4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (out.bias) bias4 = *reinterpret_cast<const float4 *>(out.bias + col);
    int kvcol0 = 0;
    if (out.kc) kvcol0 = *out.col_ptr + out.col_add;
    // operand of block kb: quants at base + kb * step (16 bytes), scale at dbase[kb * dstep]. Tiled:
    // the (tile, block) kilobyte in lane order (one whole-line wave load); natural: 16 bytes of
    // row li.
    const bool w_tiled = w.qt != nullptr;
    const int8_t * wrow;
    const uint16_t * wdr;
    if (w_tiled) {
        wrow = w.qt + ((int64_t) (n0 >> 5) * NBLK << 10) + lane * 16;
        wdr = w.dt + ((int64_t) (n0 >> 5) * NBLK << 5) + li;
    } else {
        wrow = w.qn + (int64_t) (n0 + li) * NBLK * 32 + lg * 16;
        wdr = w.dn + (int64_t) (n0 + li) * NBLK;
    }
    const int wstep = w_tiled ? 1024 : 32, wdstep = w_tiled ? 32 : 1;
    const int8_t * xrow[MT];
    const float * xdr[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        if (x_tiled) {                                  // rows are padded to the tile
            const int64_t tile = (m0 >> 5) + t;
            xrow[t] = xs + ((tile * NBLK) << 10) + lane * 16;
            xdr[t] = xd + ((tile * NBLK) << 5) + li;
        } else {
            const int mm = min(m0 + 32 * t + li, m - 1);   // rows past m repeat the last one (unused)
            xrow[t] = xs + (int64_t) mm * NBLK * 32 + lg * 16;
            xdr[t] = xd + (int64_t) mm * NBLK;
        }
    }
    const int xstep = x_tiled ? 1024 : 32, xdstep = x_tiled ? 32 : 1;

    v4i a[2][G][MT], b[2][G];
    float dx[2][G][MT];
    uint16_t dw[2][G];
    auto load = [&](int g, int s) {
#pragma unroll
        for (int u = 0; u < G; u++) {
            const int kb = kb0 + g * G + u;
            b[s][u] = *reinterpret_cast<const v4i *>(wrow + (int64_t) kb * wstep);
#pragma unroll
            for (int t = 0; t < MT; t++) a[s][u][t] = *reinterpret_cast<const v4i *>(xrow[t] + (int64_t) kb * xstep);
            dw[s][u] = wdr[kb * wdstep];
#pragma unroll
            for (int t = 0; t < MT; t++) dx[s][u][t] = xdr[t][kb * xdstep];
        }
    };

    float acc[MT][16];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;
    load(0, 0);
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const int s = g & 1;
        if (g + 1 < NG) load(g + 1, s ^ 1);
#pragma unroll
        for (int u = 0; u < G; u++) {
            v8h bdw = v8h{};
            if (lg == 0) bdw[0] = __builtin_bit_cast(_Float16, dw[s][u]);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                v8h adx = v8h{};
                if (lg == 0) adx[0] = (_Float16) dx[s][u][t];
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][u][t], b[s][u], v16i{}, 0, 0, 0);
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(adx, bdw, v16f{}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) acc[t][v] = __builtin_fmaf((float) c[v], sc[v], acc[t][v]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) red[wave][32 * t + 8 * (v >> 2) + 4 * lg + (v & 3)][li] = acc[t][v];
    __syncthreads();

    // epilogue: thread -> row (tid / 8) + 8 W i, columns 4 * (tid % 8) .. + 4 of the tile
    constexpr int RPP = 8 * W;   // rows per pass
#pragma unroll
    for (int i = 0; i < (32 * MT + RPP - 1) / RPP; i++) {
        const int r = (tid >> 3) + RPP * i;
        if (RPP > 32 * MT && r >= 32 * MT) break;
        const int row = m0 + r;
        const bool valid = row < m;
        float y[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float t = red[0][r][4 * cg + c];   // the waves' partials in wave order
#pragma unroll
            for (int q = 1; q < W; q++) t = t + red[q][r][4 * cg + c];
            y[c] = t;
        }
        if (out.bias) {
            y[0] = y[0] + bias4.x; y[1] = y[1] + bias4.y; y[2] = y[2] + bias4.z; y[3] = y[3] + bias4.w;
        }
        if (out.act == 1) {
#pragma unroll
            for (int c = 0; c < 4; c++) y[c] = y[c] > 0.0f ? y[c] : 0.0f;
        }
        if (out.y && n0 < out.n_store && valid)
            *reinterpret_cast<float4 *>(out.y + (int64_t) row * out.y_stride + col) = make_float4(y[0], y[1], y[2], y[3]);
        if (out.yq) {
            // the 32 columns of the tile are one Q8_0 block of the row, spread over 8 lanes
            int8_t q[4];
            const float d = q8_quantize_group<4>(y, q, 8);
            if (valid) {
                const int qw = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
                const int nb = n / 32;
                if (out.yq_layout == Q8_TILED) {
                    *reinterpret_cast<int *>(out.yq + q8_tiled_offset(row, nb, blockIdx.x, 4 * cg)) = qw;
                    if (cg == 0) out.yd[q8_tiled_scale(row, nb, blockIdx.x)] = d;
                } else {
                    *reinterpret_cast<int *>(out.yq + (int64_t) row * n + col) = qw;
                    if (cg == 0) out.yd[(int64_t) row * nb + blockIdx.x] = d;
                }
            }
        }
        if (out.kc && n0 >= out.kv_row0 && valid) {
            // one 32-column tile = one head of K or V
            const int rr = n0 - out.kv_row0;
            const int which = rr / out.d_model;
            const int h = (rr % out.d_model) >> 5;
            const int b = row / out.rows_per_seq;
            const int kcol = kvcol0 + row % out.rows_per_seq;
            uint16_t * cache = (which == 0 ? out.kc : out.vc) +
                               (((int64_t) b * out.n_head + h) * out.lstride + kcol) * 32 + 4 * cg;
            uint2 w;
            w.x = (uint32_t) f2h(y[0]) | ((uint32_t) f2h(y[1]) << 16);
            w.y = (uint32_t) f2h(y[2]) | ((uint32_t) f2h(y[3]) << 16);
            *reinterpret_cast<uint2 *>(cache) = w;
        }
    }
}

// Rows per workgroup of the small-tile kernel (mt = 1, 2 or 4 tiles of 32; 0 picks one).
int launch_q8_gemm_small(const Q8Weights & w, int64_t n, int64_t k, int64_t m, const int8_t * xs,
                         const float * xd, bool x_tiled, const LayerOut & out, int mt,
                         hipStream_t stream) {
    if (mt == 0) mt = m <= 64 ? 1 : 2;
    GSVK_REQUIRE(mt == 1 || mt == 2 || mt == 4, "q8_gemm: row tiles per workgroup must be 1, 2 or 4");
    const dim3 grid((unsigned) (n / 32), (unsigned) ((m + 32 * mt - 1) / (32 * mt)));
#define GSVK_GS(NB, MT, W) \
    hipLaunchKernelGGL((k_q8_gemm_small<NB, MT, W>), grid, dim3(W * 64), 0, stream, w, (int) n, (int) m, xs, xd, \
                       x_tiled, out)
    // a 512-column projection has only 16 column tiles: 8 waves per workgroup (each an eighth
    // of K) put twice the waves on the chip and halve each wave's chain
    // (for every row tiling alike, so that the tiling does not change a bit of the result)
    const bool wide = n == 512;
    if (k == 512) {
        if (mt == 1) { if (wide) GSVK_GS(16, 1, 8); else GSVK_GS(16, 1, 4); }
        else if (mt == 2) { if (wide) GSVK_GS(16, 2, 8); else GSVK_GS(16, 2, 4); }
        else { if (wide) GSVK_GS(16, 4, 8); else GSVK_GS(16, 4, 4); }
    } else if (k == 1024) {   // (the BERT encoder's Q8_0 files)
        if (mt == 1) GSVK_GS(32, 1, 4);
        else if (mt == 2) GSVK_GS(32, 2, 4);
        else GSVK_GS(32, 4, 4);
    } else if (k == 2048) {
        if (mt == 1) { if (wide) GSVK_GS(64, 1, 8); else GSVK_GS(64, 1, 4); }
        else if (mt == 2) { if (wide) GSVK_GS(64, 2, 8); else GSVK_GS(64, 2, 4); }
        else { if (wide) GSVK_GS(64, 4, 8); else GSVK_GS(64, 4, 4); }
    } else {   // k == 4096: 8 waves, so that a wave's blocks (16) fit its registers
        if (mt == 1) GSVK_GS(128, 1, 8);
        else if (mt == 2) GSVK_GS(128, 2, 8);
        else GSVK_GS(128, 4, 8);
    }
#undef GSVK_GS
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

int launch_q8_gemm(const Q8Weights & w, int64_t n, int64_t k, int64_t m, const int8_t * xs,
                   const float * xd, int x_layout, const LayerOut & out, hipStream_t stream,
                   int tile_rows) {
    GSVK_REQUIRE(((w.qn && w.dn) || (w.qt && w.dt)) && xs && xd, "q8_gemm: null pointer");
    GSVK_REQUIRE(x_layout == Q8_NATURAL || x_layout == Q8_TILED, "q8_gemm: bad activation layout %d", x_layout);
    GSVK_REQUIRE(!out.yq || out.yq_layout == Q8_NATURAL || out.yq_layout == Q8_TILED,
                 "q8_gemm: bad output layout %d", out.yq_layout);
    GSVK_REQUIRE(n > 0 && n % 32 == 0 && n < (1 << 30) && m > 0 && m < (1 << 30),
                 "q8_gemm: n must be a multiple of 32 (n=%lld m=%lld)", (long long) n, (long long) m);
    GSVK_REQUIRE(k == 512 || k == 1024 || k == 2048 || k == 4096,
                 "q8_gemm: k must be 512, 1024, 2048 or 4096 (got %lld)", (long long) k);
    GSVK_REQUIRE(!out.yq || out.yd, "q8_gemm: bad quantised output");
    GSVK_REQUIRE(!out.kc || (out.vc && out.col_ptr && out.rows_per_seq > 0 && out.kv_row0 + 2 * out.d_model <= n),
                 "q8_gemm: bad KV epilogue");
    GSVK_REQUIRE(out.act == 0 || out.act == 1, "q8_gemm: act must be 0 or 1");
    GSVK_REQUIRE(((uintptr_t) out.bias & 15) == 0 && ((uintptr_t) out.y & 15) == 0 && out.y_stride % 4 == 0 &&
                     ((uintptr_t) out.kc & 15) == 0 && ((uintptr_t) out.vc & 15) == 0,
                 "q8_gemm: bias, y (and its row stride) and the K/V caches must be 16-byte aligned");
    if (m <= GS_MAX_ROWS || n % GM_BN != 0 || !w.qn || x_layout == Q8_TILED)
        return launch_q8_gemm_small(w, n, k, m, xs, xd, x_layout == Q8_TILED, out, tile_rows, stream);
    GSVK_REQUIRE(tile_rows == 0, "q8_gemm: row tiles are a choice of the small-batch kernel (m <= %lld)",
                 (long long) GS_MAX_ROWS);
    GSVK_REQUIRE(!out.row_pad || out.rows_per_seq > 0, "q8_gemm: padding rows need rows_per_seq");
    GSVK_REQUIRE(m * k < ((int64_t) 1 << 31) && n * k < ((int64_t) 1 << 31),
                 "q8_gemm: operands above 2 GiB (m=%lld n=%lld k=%lld)", (long long) m, (long long) n, (long long) k);
    GSVK_REQUIRE(x_layout == Q8_NATURAL && (!out.yq || out.yq_layout == Q8_NATURAL),
                 "q8_gemm: above %lld rows the operands are in natural order", (long long) GS_MAX_ROWS);
    const int8_t * ws = w.qn;
    const uint16_t * wd = w.dn;
    const dim3 grid((unsigned) (n / GM_BN * ((m + GM_BM - 1) / GM_BM)));
    if (k == 512)
        hipLaunchKernelGGL(k_q8_gemm<16>, grid, dim3(GM_THREADS), 0, stream, ws, wd, (int) n, (int) m, xs, xd, out);
    else if (k == 1024)
        hipLaunchKernelGGL(k_q8_gemm<32>, grid, dim3(GM_THREADS), 0, stream, ws, wd, (int) n, (int) m, xs, xd, out);
    else if (k == 2048)
        hipLaunchKernelGGL(k_q8_gemm<64>, grid, dim3(GM_THREADS), 0, stream, ws, wd, (int) n, (int) m, xs, xd, out);
    else
        hipLaunchKernelGGL(k_q8_gemm<128>, grid, dim3(GM_THREADS), 0, stream, ws, wd, (int) n, (int) m, xs, xd, out);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_q8_gemm(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k, const int8_t * xq,
                               const float * xd, int64_t m, const float * bias, int act, float * y,
                               void * stream) {
    return gsvk_op_q8_gemm_ex(wq, wd, n, k, xq, xd, m, bias, act, y, nullptr, nullptr, 0, 0, stream);
}

extern "C" int gsvk_op_q8_gemm_ex(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k,
                                  const int8_t * xq, const float * xd, int64_t m, const float * bias,
                                  int act, float * y, int8_t * yq, float * yd, int tile_rows,
                                  int tiled, void * stream) {
    gsvk::LayerOut out{};
    out.y = y;
    out.y_stride = n;
    out.n_store = (int) n;
    out.bias = bias;
    out.act = act;
    out.yq = yq;
    out.yd = yd;
    out.yq_layout = tiled ? gsvk::Q8_TILED : gsvk::Q8_NATURAL;
    GSVK_REQUIRE(y || yq, "q8_gemm: null pointer");
    gsvk::Q8Weights w{};
    if (tiled) {
        w.qt = wq;
        w.dt = wd;
    } else {
        w.qn = wq;
        w.dn = wd;
    }
    return gsvk::launch_q8_gemm(w, n, k, m, xq, xd, tiled ? gsvk::Q8_TILED : gsvk::Q8_NATURAL, out,
                                (hipStream_t) stream, tile_rows);
}

extern "C" int gsvk_op_q8_dequant_f16(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k, uint16_t * w16,
                                      void * stream) {
    return gsvk::launch_q8_dequant_f16(wq, wd, n, k, w16, (hipStream_t) stream);
}

extern "C" int gsvk_op_q8h_gemm(const uint16_t * w16, int64_t n, int64_t k, const int8_t * xq, const float * xd,
                                int64_t m, const float * bias, int act, float * y, int8_t * yq, float * yd,
                                void * stream) {
    GSVK_REQUIRE(y || yq, "q8h_gemm: null pointer");
    gsvk::LayerOut out{};
    out.y = y;
    out.y_stride = n;
    out.n_store = (int) n;
    out.bias = bias;
    out.act = act;
    out.yq = yq;
    out.yd = yd;
    out.yq_layout = gsvk::Q8_NATURAL;
    return gsvk::launch_q8h_gemm(w16, n, k, m, xq, xd, out, (hipStream_t) stream);
}

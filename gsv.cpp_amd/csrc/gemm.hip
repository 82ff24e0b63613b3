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
// chunks of 2 blocks (64 values) by direct global -> LDS loads, double buffered: the next
// chunk streams in while the current one is multiplied, with no staging registers, and the
// 35 KB of LDS and <= 168 VGPRs let 3 workgroups share a CU. Operands arrive with their quants
// in natural order (q[row][k]; scales apart), so a chunk of a row is half a 128-byte line. A
// lane's MFMA operand is one half (16 values) of a block of one row; A and B use the same halves,
// so the product sums over the block whatever order the hardware assigns to the bytes.
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
constexpr int GM_KC = 2;                   // blocks per K chunk
constexpr int GM_NBUF = 2;                 // chunk buffers (a chunk streams in while one is used)
constexpr int GM_ROWB = GM_KC * 32;        // LDS bytes per row and chunk
constexpr int GM_SLOTS = GM_ROWB / 16;     // 16-byte slots per row and chunk
constexpr int GM_SWZ = GM_SLOTS - 1;       // slot swizzle mask

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;
}  // namespace

// K chunk buffers, filled by direct global -> LDS loads (no staging registers). A row's chunk is
// 64 bytes = 4 slots of 16 bytes; piece p of row r sits in slot p ^ (r & 3), so that the 16-byte
// operand reads of consecutive rows fall in different banks.
struct GemmLds {
    int8_t a[GM_NBUF][GM_BM * GM_ROWB];
    int8_t b[GM_NBUF][GM_BN * GM_ROWB];
    float da[GM_NBUF][GM_BM * GM_KC];      // activation scales [row][block]
    uint16_t db[GM_NBUF][GM_BN * GM_KC];   // weight scales (fp16) [col][block]
};

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

// Issue the direct loads of one K chunk into buffer buf. A wave's load instruction writes 64
// consecutive 16-byte (or 4-byte) LDS slots, lane L the L-th; the global address of each lane is
// chosen so that the slot receives what the layout above puts there.
template <int NBLK>
__device__ __forceinline__ void gemm_issue(const int8_t * __restrict__ xs, const float * __restrict__ xd,
                                           const int8_t * __restrict__ ws, const uint16_t * __restrict__ wd,
                                           int m, int m0, int n0, int chunk, int wave, int lane, GemmLds & s,
                                           int buf) {
    const int blk0 = chunk * GM_KC;
    constexpr int ROWS_PER_SEG = 64 / GM_SLOTS;   // rows covered by one wave instruction (1 KB)
#pragma unroll
    for (int u = 0; u < GM_KC; u++) {
        const int seg = u * 4 + wave;
        const int r = seg * ROWS_PER_SEG + lane / GM_SLOTS;
        const int p = (lane % GM_SLOTS) ^ (r & GM_SWZ);   // the piece that belongs in this slot
        const int mm = min(m0 + r, m - 1);
        lds_dma16(xs + (int64_t) mm * NBLK * 32 + blk0 * 32 + p * 16, &s.a[buf][seg * 1024]);
        lds_dma16(ws + (int64_t) (n0 + r) * NBLK * 32 + blk0 * 32 + p * 16, &s.b[buf][seg * 1024]);
    }
#pragma unroll
    for (int u = 0; u < GM_KC / 2; u++) {          // 128 rows x GM_KC scales, 256 per instruction
        const int i = u * 256 + wave * 64 + lane;
        const int mm = min(m0 + i / GM_KC, m - 1);
        lds_dma4(xd + (int64_t) mm * NBLK + blk0 + i % GM_KC, &s.da[buf][u * 256 + wave * 64]);
    }
    // 128 columns x GM_KC fp16 scales, two per 4-byte lane
    constexpr int DB_LANES = GM_BN * GM_KC / 2;
    if (wave * 64 < DB_LANES) {
        const int i = wave * 64 + lane;
        const int col = i / (GM_KC / 2), pair = i % (GM_KC / 2);
        lds_dma4(wd + (int64_t) (n0 + col) * NBLK + blk0 + 2 * pair, &s.db[buf][2 * (wave * 64)]);
    }
}

template <int NBLK>
__global__ void __launch_bounds__(GM_THREADS) k_q8_gemm(const int8_t * __restrict__ ws,
                                                           const uint16_t * __restrict__ wd, int n, int m,
                                                           const int8_t * __restrict__ xs,
                                                           const float * __restrict__ xd, LayerOut out) {
    constexpr int NCH = NBLK / GM_KC;
    __shared__ __align__(16) GemmSmem sm;
    GemmLds & s = sm.k;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n0 = blockIdx.x * GM_BN;
    const int m0 = blockIdx.y * GM_BM;
    if (out.row_pad) {   // a tile of padding rows only: zeros out, no products (uniform branch)
        bool all_pad = true;
        const int S = out.rows_per_seq;
        const int mend = min(m0 + GM_BM, m);
        for (int r0 = m0; r0 < mend && all_pad;) {
            const int b = r0 / S;
            const int e = min((b + 1) * S, mend);
            if (e - b * S > out.row_pad[b]) all_pad = false;
            r0 = e;
        }
        if (all_pad) {
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
            return;
        }
    }
    const int wm = (wave >> 1) * 64;   // this wave's rows within the tile
    const int wn = (wave & 1) * 64;    // and columns
    const int li = lane & 31;          // MFMA: row of A / column of B held by this lane
    const int lg = lane >> 5;          // MFMA: which half of the block

    float acc[4][16];                  // tile t = 2 * ta + tb
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

#pragma unroll
    for (int c = 0; c < GM_NBUF - 1; c++)
        if (c < NCH) gemm_issue<NBLK>(xs, xd, ws, wd, m, m0, n0, c, wave, lane, s, c);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int ch = 0; ch < NCH; ch++) {
        const int buf = ch % GM_NBUF;
        // the chunk GM_NBUF - 1 ahead streams into the buffer read before the previous barrier
        if (ch + GM_NBUF - 1 < NCH)
            gemm_issue<NBLK>(xs, xd, ws, wd, m, m0, n0, ch + GM_NBUF - 1, wave, lane, s, (ch + GM_NBUF - 1) % GM_NBUF);
#pragma unroll 1
        for (int bb = 0; bb < GM_KC; bb++) {
            // operands: piece 2 * bb + lg (16 values) of the wave's rows / columns
            v4i fa[2], fb[2];
            v8h adx[2], bdw[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int ra = wm + 32 * h + li, rb = wn + 32 * h + li;
                fa[h] = *reinterpret_cast<const v4i *>(&s.a[buf][ra * GM_ROWB + (((2 * bb + lg) ^ (ra & GM_SWZ)) << 4)]);
                fb[h] = *reinterpret_cast<const v4i *>(&s.b[buf][rb * GM_ROWB + (((2 * bb + lg) ^ (rb & GM_SWZ)) << 4)]);
                // the scale-product MFMA: A = dx of the tile's rows, B = dw of its columns, in one
                // K slot of lanes 0-31, every other slot zero. Both scales are fp16 values (the
                // activation scale is rounded to fp16 when it is made), so their product is exact
                // in the fp16 MFMA's fp32 result, as in a vector multiply.
                adx[h] = v8h{};
                bdw[h] = v8h{};
                if (lg == 0) {
                    adx[h][0] = (_Float16) s.da[buf][ra * GM_KC + bb];
                    bdw[h][0] = __builtin_bit_cast(_Float16, s.db[buf][rb * GM_KC + bb]);
                }
            }
            // per tile: the exact integer sum of the block, the products dx * dw, then
            // acc += float(C) * (dx * dw) on the vector ALUs
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[t >> 1], fb[t & 1], v16i{}, 0, 0, 0);
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(adx[t >> 1], bdw[t & 1], v16f{}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) acc[t][v] = __builtin_fmaf((float) c[v], sc[v], acc[t][v]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);   // the chunks issued so far have landed
        __syncthreads();                 // and every wave is done with this one
    }

    // ---- epilogue: each half of the 128 x 128 tile goes through LDS so that each thread then
    // owns a 32-column block of a row: coalesced stores and an in-register Q8_0 quantisation ----
    int kvcol0 = 0;
    if (out.kc) kvcol0 = *out.col_ptr + out.col_add;
    const int nblk_out = n / 32;
#pragma unroll 1
    for (int half = 0; half < 2; half++) {
        if (half) __syncthreads();       // the first half has been read
        if (wm == 64 * half) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int ta = t >> 1, tb = t & 1;
#pragma unroll
                for (int v = 0; v < 16; v++)
                    sm.y[32 * ta + 8 * (v >> 2) + 4 * lg + (v & 3)][wn + 32 * tb + li] = acc[t][v];
            }
        }
        __syncthreads();
        const int r = tid >> 2, cb = tid & 3;      // 64 rows x 4 blocks of 32 columns
        const int row = m0 + 64 * half + r;
        if (row >= m) continue;
        const int col0 = n0 + 32 * cb;
        float y[32];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 f = *reinterpret_cast<const float4 *>(&sm.y[r][32 * cb + 4 * j]);
            y[4 * j] = f.x; y[4 * j + 1] = f.y; y[4 * j + 2] = f.z; y[4 * j + 3] = f.w;
        }
        if (out.bias) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 b4 = *reinterpret_cast<const float4 *>(out.bias + col0 + 4 * j);
                y[4 * j] = y[4 * j] + b4.x; y[4 * j + 1] = y[4 * j + 1] + b4.y;
                y[4 * j + 2] = y[4 * j + 2] + b4.z; y[4 * j + 3] = y[4 * j + 3] + b4.w;
            }
        }
        if (out.act == 1) {
#pragma unroll
            for (int k = 0; k < 32; k++) y[k] = y[k] > 0.0f ? y[k] : 0.0f;
        }
        if (out.y && col0 < out.n_store) {
            float * yr = out.y + (int64_t) row * out.y_stride + col0;
#pragma unroll
            for (int j = 0; j < 8; j++)
                *reinterpret_cast<float4 *>(yr + 4 * j) = make_float4(y[4 * j], y[4 * j + 1], y[4 * j + 2], y[4 * j + 3]);
        }
        if (out.yq) {
            float amax = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(y[k]));
            const float d = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            const int blk = col0 >> 5;
            int w[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                w[j] = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) w[j] |= (((int) __builtin_rintf(y[4 * j + t] * id)) & 0xff) << (8 * t);
            }
            int4 * qr = reinterpret_cast<int4 *>(out.yq + (int64_t) row * n + col0);   // natural order
            qr[0] = make_int4(w[0], w[1], w[2], w[3]);
            qr[1] = make_int4(w[4], w[5], w[6], w[7]);
            out.yd[(int64_t) row * nblk_out + blk] = h2f(f2h(d));
        }
        if (out.kc && col0 >= out.kv_row0) {
            // one 32-column block = one head of K or V
            const int rr = col0 - out.kv_row0;
            const int which = rr / out.d_model;
            const int h = (rr % out.d_model) >> 5;
            const int b = row / out.rows_per_seq;
            const int kcol = kvcol0 + row % out.rows_per_seq;
            uint16_t * cache = (which == 0 ? out.kc : out.vc) + (((int64_t) b * out.n_head + h) * out.lstride + kcol) * 32;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint4 w;
                w.x = (uint32_t) f2h(y[8 * j + 0]) | ((uint32_t) f2h(y[8 * j + 1]) << 16);
                w.y = (uint32_t) f2h(y[8 * j + 2]) | ((uint32_t) f2h(y[8 * j + 3]) << 16);
                w.z = (uint32_t) f2h(y[8 * j + 4]) | ((uint32_t) f2h(y[8 * j + 5]) << 16);
                w.w = (uint32_t) f2h(y[8 * j + 6]) | ((uint32_t) f2h(y[8 * j + 7]) << 16);
                *reinterpret_cast<uint4 *>(cache + 8 * j) = w;
            }
        }
    }
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
    GSVK_REQUIRE(x_layout == Q8_NATURAL && (!out.yq || out.yq_layout == Q8_NATURAL),
                 "q8_gemm: above %lld rows the operands are in natural order", (long long) GS_MAX_ROWS);
    const int8_t * ws = w.qn;
    const uint16_t * wd = w.dn;
    const dim3 grid((unsigned) (n / GM_BN), (unsigned) ((m + GM_BM - 1) / GM_BM));
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

// Q8_0 x Q8_0 GEMM on the gfx950 matrix cores, for the projections once the batch makes them
// dense contractions (prefill over B*S rows, decode at large batch):
//
//   Y[m][n] = sum_blk  dx[m][blk] * dw[n][blk] * (sum_{k in blk} qx[m][k] * qw[n][k])
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-value Q8_0 block of a 32x32 output tile, so
// every block's integer sum is exact; the per-block fp32 scaling is done on the vector ALUs
// (acc += float(C) * (dx * dw), three operations per output and block: this kernel is bound by
// them, not by the matrix cores). The fp32 accumulation order (block by block) differs from the
// ggml-cpu x86 order (8 lanes, then hsum), so results agree with it to fp32 rounding, not bit
// for bit; the decode path keeps the bit-exact GEMV.
//
// Tiling: workgroup 256 threads = 4 waves, output tile 128 (rows m) x 128 (columns n); wave w
// owns rows 64*(w/2).. and columns 64*(w%2).., i.e. 2 x 2 MFMA tiles. K is staged through LDS in
// chunks of 4 blocks (128 values), double buffered: the next chunk's global loads are in flight
// while the current one is multiplied. Operands arrive in the sliced Q8_0 layout (slice j of a
// row = bytes 4j..4j+3 of every block); LDS holds them as [row][block][32 bytes in value order],
// rows padded by 16 bytes so that a wave's 16-byte reads are bank-conflict free. A lane's MFMA
// operand is one half (16 values) of a block of one row; A and B use the same halves, so the
// product sums over the block whatever order the hardware assigns to the bytes.
//
// Epilogue (the options of the decoder's GEMV, layer.h LayerOut): bias, ReLU, fp32 store of
// columns < n_store, the fp16 K/V append, or the Q8_0 quantisation of each 32-column block.
#include "common.h"
#include "layer.h"

namespace gsvk {

namespace {
constexpr int GM_THREADS = 256;
constexpr int GM_BM = 128;                 // rows (m) per workgroup
constexpr int GM_BN = 128;                 // columns (n) per workgroup
constexpr int GM_KC = 4;                   // blocks per K chunk
constexpr int GM_ROWB = GM_KC * 32 + 16;   // LDS bytes per row and chunk (padded)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
}  // namespace

struct GemmLds {
    int8_t a[2][GM_BM * GM_ROWB];
    int8_t b[2][GM_BN * GM_ROWB];
    float da[2][GM_KC][GM_BM];   // activation scales [block][row]
    float db[2][GM_KC][GM_BN];   // weight scales (fp16 -> fp32) [block][col]
};

// Global -> registers for one K chunk: each thread loads 4 x 16 bytes of A and of B (one slice
// of 4 consecutive blocks of one row each) and its share of the scales.
struct GemmStage {
    int4 a[4], b[4];
    float da[2];
    uint16_t db[2];
};

template <int NBLK>
__device__ __forceinline__ void gemm_load(const int8_t * __restrict__ xs, const float * __restrict__ xd,
                                          const int8_t * __restrict__ ws, const uint16_t * __restrict__ wd,
                                          int m, int m0, int n0, int chunk, int tid, GemmStage & g) {
    const int blk0 = chunk * GM_KC;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = tid + u * GM_THREADS;   // 0..1023 = 128 rows x 8 slices
        const int row = idx >> 3, j = idx & 7;
        const int mm = min(m0 + row, m - 1);
        g.a[u] = *reinterpret_cast<const int4 *>(xs + ((int64_t) mm * 8 + j) * NBLK * 4 + blk0 * 4);
        g.b[u] = *reinterpret_cast<const int4 *>(ws + ((int64_t) (n0 + row) * 8 + j) * NBLK * 4 + blk0 * 4);
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = tid + u * GM_THREADS;   // 0..511 = 128 rows x 4 blocks
        const int row = idx >> 2, bb = idx & 3;
        const int mm = min(m0 + row, m - 1);
        g.da[u] = xd[(int64_t) mm * NBLK + blk0 + bb];
        g.db[u] = wd[(int64_t) (n0 + row) * NBLK + blk0 + bb];
    }
}

__device__ __forceinline__ void gemm_store(GemmLds & s, int buf, int tid, const GemmStage & g) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = tid + u * GM_THREADS;
        const int row = idx >> 3, j = idx & 7;
        // g.a[u] holds slice j of blocks 0..3: word q -> block q, bytes 4j..4j+3
        int * pa = reinterpret_cast<int *>(&s.a[buf][row * GM_ROWB + j * 4]);
        int * pb = reinterpret_cast<int *>(&s.b[buf][row * GM_ROWB + j * 4]);
        pa[0] = g.a[u].x; pa[8] = g.a[u].y; pa[16] = g.a[u].z; pa[24] = g.a[u].w;
        pb[0] = g.b[u].x; pb[8] = g.b[u].y; pb[16] = g.b[u].z; pb[24] = g.b[u].w;
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = tid + u * GM_THREADS;
        const int row = idx >> 2, bb = idx & 3;
        s.da[buf][bb][row] = g.da[u];
        s.db[buf][bb][row] = h2f(g.db[u]);
    }
}

template <int NBLK>
__global__ void __launch_bounds__(GM_THREADS) k_q8_gemm(const int8_t * __restrict__ ws,
                                                        const uint16_t * __restrict__ wd, int n, int m,
                                                        const int8_t * __restrict__ xs,
                                                        const float * __restrict__ xd, LayerOut out) {
    constexpr int NCH = NBLK / GM_KC;
    __shared__ __align__(16) GemmLds s;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n0 = blockIdx.x * GM_BN;
    const int m0 = blockIdx.y * GM_BM;
    const int wm = (wave >> 1) * 64;   // this wave's rows within the tile
    const int wn = (wave & 1) * 64;    // and columns
    const int li = lane & 31;          // MFMA: row of A / column of B held by this lane
    const int lg = lane >> 5;          // MFMA: which half of the block

    float acc[2][2][16];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;

    GemmStage g;
    gemm_load<NBLK>(xs, xd, ws, wd, m, m0, n0, 0, tid, g);
    gemm_store(s, 0, tid, g);
    __syncthreads();

    for (int ch = 0; ch < NCH; ch++) {
        const int buf = ch & 1;
        if (ch + 1 < NCH) gemm_load<NBLK>(xs, xd, ws, wd, m, m0, n0, ch + 1, tid, g);
#pragma unroll 1
        for (int bb = 0; bb < GM_KC; bb++) {
            v4i fa[2], fb[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                fa[t] = *reinterpret_cast<const v4i *>(&s.a[buf][(wm + 32 * t + li) * GM_ROWB + bb * 32 + lg * 16]);
                fb[t] = *reinterpret_cast<const v4i *>(&s.b[buf][(wn + 32 * t + li) * GM_ROWB + bb * 32 + lg * 16]);
            }
            float dwv[2];
#pragma unroll
            for (int t = 0; t < 2; t++) dwv[t] = s.db[buf][bb][wn + 32 * t + li];
#pragma unroll
            for (int ta = 0; ta < 2; ta++) {
                // activation scales of the 16 rows this lane's outputs belong to:
                // row = 8 * (v / 4) + 4 * lg + v % 4 within the 32-row tile
                float dxv[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 d4 = *reinterpret_cast<const float4 *>(&s.da[buf][bb][wm + 32 * ta + 8 * q + 4 * lg]);
                    dxv[4 * q + 0] = d4.x; dxv[4 * q + 1] = d4.y; dxv[4 * q + 2] = d4.z; dxv[4 * q + 3] = d4.w;
                }
#pragma unroll
                for (int tb = 0; tb < 2; tb++) {
                    v16i c = {};
                    c = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ta], fb[tb], c, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        acc[ta][tb][v] = __builtin_fmaf((float) c[v], dxv[v] * dwv[tb], acc[ta][tb][v]);
                }
            }
        }
        if (ch + 1 < NCH) {
            gemm_store(s, buf ^ 1, tid, g);   // the other buffer: last read before the previous barrier
        }
        __syncthreads();
    }

    // ---- epilogue: lane holds column li of each 32x32 tile, rows 8*(v/4) + 4*lg + v%4 ----
    int kvcol0 = 0;
    if (out.kc) kvcol0 = *out.col_ptr + out.col_add;
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
        const int col = n0 + wn + 32 * tb + li;
        const float bias = out.bias ? out.bias[col] : 0.0f;
#pragma unroll
        for (int ta = 0; ta < 2; ta++) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm + 32 * ta + 8 * (v >> 2) + 4 * lg + (v & 3);
                float y = acc[ta][tb][v];
                if (out.bias) y = y + bias;
                if (out.act == 1) y = y > 0.0f ? y : 0.0f;
                if (out.yq) {
                    // the 32 columns of this block of row `row` are the 32 lanes of this half
                    float v1[1] = {y};
                    int8_t q1[1];
                    const float d = q8_quantize_group<1>(v1, q1, 32);
                    if (row < m) {
                        const int nblk_out = n / 32;
                        const int blk = col >> 5;
                        out.yq[(int64_t) row * n + q8_sliced_offset(nblk_out, blk, li)] = q1[0];
                        if (li == 0) out.yd[(int64_t) row * nblk_out + blk] = d;
                    }
                }
                if (row >= m) continue;
                if (out.y && col < out.n_store) out.y[(int64_t) row * out.y_stride + col] = y;
                if (out.kc && col >= out.kv_row0) {
                    const int rr = col - out.kv_row0;
                    const int which = rr / out.d_model;
                    const int hd = rr % out.d_model;
                    const int h = hd >> 5, dd = hd & 31;
                    const int b = row / out.rows_per_seq;
                    const int kcol = kvcol0 + row % out.rows_per_seq;
                    uint16_t * cache = which == 0 ? out.kc : out.vc;
                    cache[(((int64_t) b * out.n_head + h) * out.lstride + kcol) * 32 + dd] = f2h(y);
                }
            }
        }
    }
}

int launch_q8_gemm(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, int64_t m,
                   const int8_t * xs, const float * xd, const LayerOut & out, hipStream_t stream) {
    GSVK_REQUIRE(ws && wd && xs && xd, "q8_gemm: null pointer");
    GSVK_REQUIRE(n > 0 && n % GM_BN == 0 && n < (1 << 30) && m > 0 && m < (1 << 30),
                 "q8_gemm: n must be a multiple of %d (n=%lld m=%lld)", GM_BN, (long long) n, (long long) m);
    GSVK_REQUIRE(k == 512 || k == 2048, "q8_gemm: k must be 512 or 2048 (got %lld)", (long long) k);
    GSVK_REQUIRE(!out.yq || out.yd, "q8_gemm: bad quantised output");
    GSVK_REQUIRE(!out.kc || (out.vc && out.col_ptr && out.rows_per_seq > 0 && out.kv_row0 + 2 * out.d_model <= n),
                 "q8_gemm: bad KV epilogue");
    GSVK_REQUIRE(out.act == 0 || out.act == 1, "q8_gemm: act must be 0 or 1");
    const dim3 grid((unsigned) (n / GM_BN), (unsigned) ((m + GM_BM - 1) / GM_BM));
    if (k == 512)
        hipLaunchKernelGGL(k_q8_gemm<16>, grid, dim3(GM_THREADS), 0, stream, ws, wd, (int) n, (int) m, xs, xd, out);
    else
        hipLaunchKernelGGL(k_q8_gemm<64>, grid, dim3(GM_THREADS), 0, stream, ws, wd, (int) n, (int) m, xs, xd, out);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

extern "C" int gsvk_op_q8_gemm(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k, const int8_t * xq,
                               const float * xd, int64_t m, const float * bias, int act, float * y,
                               void * stream) {
    gsvk::LayerOut out{};
    out.y = y;
    out.y_stride = n;
    out.n_store = (int) n;
    out.bias = bias;
    out.act = act;
    GSVK_REQUIRE(y, "q8_gemm: null pointer");
    return gsvk::launch_q8_gemm(wq, wd, n, k, m, xq, xd, out, (hipStream_t) stream);
}

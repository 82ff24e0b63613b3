// Fused decoder-layer GEMV for gfx950: one launch computes the Q8_0 input of a projection and
// the projection itself.
//
//   input stage (per workgroup, for its MT activation rows, into LDS):
//     IN_Q8  : the rows are already Q8_0 (attention output, FFN1 output)
//     IN_LN  : v = (res + r) + bias; LayerNorm(v) * w + b (PATCH:1533-1584), then the ggml-cpu
//              x86 Q8_0 quantisation; workgroups of column 0 also store the fp32 LayerNorm output
//              (the next residual). Every workgroup computes identical values (same code, same
//              inputs), so this replaces the separate LayerNorm + quantise launches bit-exactly.
//     IN_EMB : x = emb[tok] + alpha * PE[pos] (src/gsv_ar.cpp:798-807), quantised likewise;
//              column-0 workgroups store x and set kv_end for the step.
//   GEMV stage: the sliced Q8_0 dot in ggml-cpu's x86 order (see q8.hip), 32 output rows per
//   workgroup (4 waves x 8 rows x 8 slice lanes); the weight loads are issued before the input
//   stage so their HBM latency overlaps it.
//   output stage: bias, ReLU, fp32 store of rows < n_store, the K/V append to the fp16 cache, or
//   (OUT_Q8) the Q8_0 quantisation of each 32-row output block, written sliced.
#include "common.h"
#include "layer.h"
#include "layer_dev.h"

namespace gsvk {

constexpr int LG_THREADS = 256;
constexpr int LG_ROWS = 32;   // output rows per workgroup

template <int NB4, int MT, int MODE, int WAVES = 4>
__global__ void __launch_bounds__(WAVES * 64) k_layer_gemv(const int8_t * __restrict__ ws,
                                                           const uint16_t * __restrict__ wd, int n,
                                                           int m, LayerIn in, LayerOut out) {
    constexpr int NT = WAVES * 64;     // threads
    constexpr int ROWS = WAVES * 8;    // output rows of the workgroup
    static_assert(MODE == IN_Q8 || MT <= WAVES, "one wave per LayerNorm / embedding row");
    constexpr int K = NB4 * 128;
    constexpr int NBLK = K / 32;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane >> 3;
    const int j = lane & 7;
    const int row = blockIdx.x * ROWS + wave * 8 + r;
    const int m0 = blockIdx.y * MT;
    const bool valid = row < n;
    const int rowc = valid ? row : n - 1;

    // LDS copy of the sliced input rows, each slice padded by 16 bytes (bank-conflict free reads)
    constexpr int SLICE_B = NBLK * 4 + 16;
    __shared__ __align__(16) int8_t s_x[MT][8 * SLICE_B];
    __shared__ __align__(16) float s_d[MT][NBLK];
    __shared__ float s_out[MT][ROWS];

    // Loads go out in the order their data is needed, each thread issuing a fixed number of them
    // (indices clamped rather than skipped, so that no wave-dependent branch separates a load
    // from its use and every wait is exact): the input rows first, then the weights. Waiting for
    // the input then does not wait for the weights, whose HBM latency overlaps the input stage.
    constexpr int CH = K / 16;                                      // 16-byte chunks per row
    constexpr int QN = (MT * CH + NT - 1) / NT;     // chunks per thread
    constexpr int DN = (MT * NBLK + NT - 1) / NT;   // scales per thread
    constexpr int CPS = NBLK / 4;                                   // 16-byte chunks per slice
    int4 xq[MODE == IN_Q8 ? QN : 1];
    float xdv[MODE == IN_Q8 ? DN : 1];
    LnRow lnr;
    float4 e0, e1, p0, p1;
    const int tr = wave < MT ? wave : MT - 1;   // LN / embedding: this wave's row (waves past MT
    const int mmr = min(m0 + tr, m - 1);        // repeat the last one and discard it)
    int pos = 0;
    if constexpr (MODE == IN_Q8) {
#pragma unroll
        for (int u = 0; u < QN; u++) {
            int c = tid + u * NT;
            c = c < MT * CH ? c : MT * CH - 1;
            const int mm = min(m0 + c / CH, m - 1);
            xq[u] = *reinterpret_cast<const int4 *>(in.xs + (int64_t) mm * K + (c % CH) * 16);
        }
#pragma unroll
        for (int u = 0; u < DN; u++) {
            int c = tid + u * NT;
            c = c < MT * NBLK ? c : MT * NBLK - 1;
            const int mm = min(m0 + c / NBLK, m - 1);
            xdv[u] = in.xd[(int64_t) mm * NBLK + c % NBLK];
        }
    } else if constexpr (MODE == IN_LN) {
        ln_row_load(in.res + (int64_t) mmr * 512, in.r ? in.r + (int64_t) mmr * 512 : g_zero_row,
                    in.bias ? in.bias : g_zero_row, in.wb, lane, lnr);
    } else {   // IN_EMB
        int tk = in.tok[mmr];
        tk = tk < 0 ? 0 : (tk >= in.vocab ? in.vocab - 1 : tk);
        pos = *in.pos_ptr;
        const float4 * er = reinterpret_cast<const float4 *>(in.emb + (int64_t) tk * 512 + lane * 8);
        const float4 * pr = reinterpret_cast<const float4 *>(in.pe + (int64_t) pe_row(in, pos, mmr) * 512 + lane * 8);
        e0 = er[0]; e1 = er[1]; p0 = pr[0]; p1 = pr[1];
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the input loads ahead of the weight loads
    int4 w[NB4];
    uint2 dh[NB4];
    {
        const int4 * wsl = reinterpret_cast<const int4 *>(ws + ((int64_t) rowc * 8 + j) * NBLK * 4);
        const uint2 * wdr = reinterpret_cast<const uint2 *>(wd + (int64_t) rowc * NBLK);
#pragma unroll
        for (int i = 0; i < NB4; i++) {
            w[i] = wsl[i];
            dh[i] = wdr[i];
        }
    }

    // ---- input stage: LayerNorm / embedding arithmetic, the Q8_0 rows into LDS ----
    if constexpr (MODE == IN_Q8) {
#pragma unroll
        for (int u = 0; u < QN; u++) {
            const int c = tid + u * NT;
            if (c < MT * CH) {
                const int t = c / CH, cc = c % CH;
                *reinterpret_cast<int4 *>(&s_x[t][(cc / CPS) * SLICE_B + (cc % CPS) * 16]) = xq[u];
            }
        }
#pragma unroll
        for (int u = 0; u < DN; u++) {
            const int c = tid + u * NT;
            if (c < MT * NBLK) s_d[c / NBLK][c % NBLK] = xdv[u];
        }
    } else {
        float o[8];
        if constexpr (MODE == IN_LN) {
            ln_row_compute(lnr, o);
        } else {
            const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
            const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = __builtin_fmaf(in.alpha, pv[i], ev[i]);
        }
        if (wave < MT) {
            if (blockIdx.x == 0 && m0 + tr < m) {
                if (in.out_x) {
                    float4 * dst = reinterpret_cast<float4 *>(in.out_x + (int64_t) mmr * 512 + lane * 8);
                    dst[0] = make_float4(o[0], o[1], o[2], o[3]);
                    dst[1] = make_float4(o[4], o[5], o[6], o[7]);
                }
                if constexpr (MODE == IN_EMB)
                    if (in.kv_end && lane == 0) in.kv_end[mmr] = pos + in.kv_end_add;
            }
            int8_t q[8];
            const float d = q8_quantize_group<8>(o, q, 4);
            q8_store_sliced_s(&s_x[tr][0], SLICE_B, lane >> 2, lane & 3, q);
            if ((lane & 3) == 0) s_d[tr][lane >> 2] = d;
        }
    }
    __syncthreads();

    // ---- GEMV stage ----
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < NB4; i++) {
        const float dw0 = h2f((uint16_t) (dh[i].x & 0xffff)), dw1 = h2f((uint16_t) (dh[i].x >> 16));
        const float dw2 = h2f((uint16_t) (dh[i].y & 0xffff)), dw3 = h2f((uint16_t) (dh[i].y >> 16));
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int4 xv = *reinterpret_cast<const int4 *>(&s_x[t][j * SLICE_B + 16 * i]);
            const float4 dx = *reinterpret_cast<const float4 *>(&s_d[t][4 * i]);
            float a = acc[t];
            a = __builtin_fmaf(dw0 * dx.x, (float) __builtin_amdgcn_sdot4(w[i].x, xv.x, 0, false), a);
            a = __builtin_fmaf(dw1 * dx.y, (float) __builtin_amdgcn_sdot4(w[i].y, xv.y, 0, false), a);
            a = __builtin_fmaf(dw2 * dx.z, (float) __builtin_amdgcn_sdot4(w[i].z, xv.z, 0, false), a);
            a = __builtin_fmaf(dw3 * dx.w, (float) __builtin_amdgcn_sdot4(w[i].w, xv.w, 0, false), a);
            acc[t] = a;
        }
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
        float v = acc[t];
        v = v + __shfl_xor(v, 4, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 1, 64);
        acc[t] = v;
    }

    // ---- output stage ----
    const float bias = (out.bias && valid) ? out.bias[row] : 0.0f;
    int kvcol0 = 0;
    if (out.kc) kvcol0 = *out.col_ptr + out.col_add;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int mm = m0 + t;
        if ((t & 7) != j) continue;
        float v = acc[t];
        if (out.bias) v = v + bias;
        if (out.act == 1) v = v > 0.0f ? v : 0.0f;
        if (out.yq) s_out[t][wave * 8 + r] = v;
        if (!valid || mm >= m) continue;
        if (out.y && row < out.n_store) out.y[(int64_t) mm * out.y_stride + row] = v;
        if (out.kc && row >= out.kv_row0) {
            const int rr = row - out.kv_row0;
            const int which = rr / out.d_model;
            const int hd = rr % out.d_model;
            const int h = hd >> 5, dd = hd & 31;
            const int b = mm / out.rows_per_seq;
            const int col = kvcol0 + mm % out.rows_per_seq;
            uint16_t * cache = which == 0 ? out.kc : out.vc;
            cache[(((int64_t) b * out.n_head + h) * out.lstride + col) * 32 + dd] = f2h(v);
        }
    }
    if (out.yq) {
        __syncthreads();
        // one 32-value block per activation row: block index blockIdx.x of a row of n values
        for (int t = wave; t < MT; t += NT / 64) {
            const int mm = m0 + t;
            float v1[1] = {lane < ROWS ? s_out[t][lane] : 0.0f};
            int8_t q1[1];
            const float d = q8_quantize_group<1>(v1, q1, 32);
            if (mm < m && lane < ROWS) {
                const int nblk_out = n / 32;
                out.yq[(int64_t) mm * n + q8_sliced_offset(nblk_out, blockIdx.x, lane)] = q1[0];
                if (lane == 0) out.yd[(int64_t) mm * nblk_out + blockIdx.x] = d;
            }
        }
    }
}

int launch_layer_gemv(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, int64_t m,
                      const LayerIn & in, const LayerOut & out, hipStream_t stream) {
    GSVK_REQUIRE(ws && wd && n > 0 && m > 0 && n % LG_ROWS == 0 && n < (1 << 30) && m < (1 << 30),
                 "layer_gemv: bad shape n=%lld m=%lld", (long long) n, (long long) m);
    GSVK_REQUIRE(k == 512 || k == 2048, "layer_gemv: k must be 512 or 2048 (got %lld)", (long long) k);
    GSVK_REQUIRE(in.mode == IN_Q8 ? (in.xs && in.xd) : (k == 512), "layer_gemv: bad input mode");
    GSVK_REQUIRE(in.mode != IN_LN || (in.res && in.wb), "layer_gemv: LayerNorm input needs res and wb");
    auto al16 = [](const void * p) { return ((uintptr_t) p & 15) == 0; };
    GSVK_REQUIRE(in.mode != IN_LN || (al16(in.res) && al16(in.r) && al16(in.bias) && al16(in.wb)),
                 "layer_gemv: LayerNorm operands must be 16-byte aligned");
    GSVK_REQUIRE(in.mode != IN_EMB || (al16(in.emb) && al16(in.pe)),
                 "layer_gemv: embedding tables must be 16-byte aligned");
    GSVK_REQUIRE(in.mode != IN_EMB || (in.emb && in.pe && in.tok && in.pos_ptr), "layer_gemv: bad embedding input");
    GSVK_REQUIRE(!out.yq || (out.yd && n % 32 == 0), "layer_gemv: bad quantised output");
    GSVK_REQUIRE(!out.kc || (out.vc && out.col_ptr && out.rows_per_seq > 0 &&
                             out.kv_row0 + 2 * out.d_model <= n), "layer_gemv: bad KV epilogue");
    // activation rows per workgroup: the latency of a wave's dot chain grows with the rows it
    // carries, the weight re-reads (from L2) with the number of row tiles
    const unsigned gx = (unsigned) (n / LG_ROWS);
#define GSVK_LG(NB4, MT, MODE)                                                                      \
    hipLaunchKernelGGL((k_layer_gemv<NB4, MT, MODE>), dim3(gx, (unsigned) ((m + MT - 1) / MT)),     \
                       dim3(LG_THREADS), 0, stream, ws, wd, (int) n, (int) m, in, out)
    if (k == 512) {
        if (in.mode == IN_Q8) {
            if (m <= 16 && !out.yq) {
                // one wave (8 output rows) per workgroup: the out projection's 512 rows over 64
                // workgroups per activation row instead of 16 (2.24 -> 2.10 us at batch 16)
                hipLaunchKernelGGL((k_layer_gemv<4, 1, IN_Q8, 1>), dim3((unsigned) (n / 8), (unsigned) m), dim3(64),
                                   0, stream, ws, wd, (int) n, (int) m, in, out);
            } else if (m <= 16) GSVK_LG(4, 1, IN_Q8);
            else if (m <= 64) GSVK_LG(4, 2, IN_Q8);
            else GSVK_LG(4, 4, IN_Q8);
        } else if (in.mode == IN_LN) {
            if (m <= 2) GSVK_LG(4, 2, IN_LN);
            else GSVK_LG(4, 4, IN_LN);
        } else {
            if (m <= 32) GSVK_LG(4, 2, IN_EMB);
            else GSVK_LG(4, 4, IN_EMB);
        }
    } else {
        if (m <= 32) GSVK_LG(16, 1, IN_Q8);
        else GSVK_LG(16, 2, IN_Q8);
    }
#undef GSVK_LG
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

// Fused decoder-layer GEMV (layer.hip): input-stage and output-stage options.
#pragma once

#include "common.h"

namespace gsvk {

enum LayerInMode { IN_Q8 = 0, IN_LN = 1, IN_EMB = 2 };

struct LayerIn {
    int mode;
    // IN_Q8: rows already quantised (sliced quants [m][k], fp32 scales [m][k/32])
    const int8_t * xs;
    const float * xd;
    // IN_LN: LayerNorm((res + r) + bias) * wb[0:512] + wb[512:1024]; r and bias may be null.
    // All rows are 16-byte aligned.
    const float * res;
    const float * r;
    const float * bias;
    const float * wb;
    // IN_EMB: emb[tok[m]] + alpha * pe[*pos_ptr + pos_add]
    const float * emb;
    const float * pe;
    const int32_t * tok;
    const int32_t * pos_ptr;
    int pos_add;
    float alpha;
    int vocab;
    // IN_LN / IN_EMB: fp32 input rows stored by the column-0 workgroups (may be null)
    float * out_x;
    // IN_EMB: kv_end[m] = *pos_ptr + kv_end_add, stored by the column-0 workgroups (may be null)
    int32_t * kv_end;
    int kv_end_add;
    // IN_EMB: the PE row of row m is *pos_ptr + pos_add - pos_sub[m] (pos_sub may be null: 0; a
    // batch that sequences join while it decodes), clamped into the table's pe_rows rows
    const int32_t * pos_sub;
    int pe_rows;
};

struct LayerOut {
    float * y;          // fp32 output rows < n_store, row stride y_stride (may be null)
    int64_t y_stride;
    int n_store;
    const float * bias;
    int act;            // 0 none, 1 relu
    int8_t * yq;        // Q8_0 output (quants + scales [m][n/32]) or null, in yq_layout
    float * yd;
    int yq_layout;      // Q8Layout: the GEMV writes Q8_SLICED, the GEMMs Q8_NATURAL or Q8_TILED
    // K/V append of rows [kv_row0, kv_row0 + 2*d_model) to fp16 caches [B][n_head][lstride][32]
    // at column *col_ptr + col_add + m % rows_per_seq of sequence m / rows_per_seq
    uint16_t * kc;
    uint16_t * vc;
    int kv_row0;
    int d_model;
    int n_head;
    int64_t lstride;
    int rows_per_seq;
    const int32_t * col_ptr;
    int col_add;
    // (128 x 128 GEMM only) left-padding rows per sequence of rows_per_seq rows: a row tile that
    // holds only padding rows writes zeros to y / yq / yd and skips its products and K/V (no
    // query attends a padding key), or null
    const int32_t * row_pad;
};

// A Q8_0 weight matrix [n][k] as the GEMMs read it: quants in natural order with the fp16 scales
// apart (qn [n][k] as in the GGUF blocks, dn [n][k/32]), and/or the same in the Q8_TILED order
// (qt, dt), which the small-batch kernel loads with whole-line reads.
struct Q8Weights {
    const int8_t * qn;
    const uint16_t * dn;
    const int8_t * qt;
    const uint16_t * dt;
};

// Q8_0 x Q8_0 GEMM on the matrix cores (gemm.hip) with the same epilogue options: n % 32 == 0,
// k in {512, 1024, 2048, 4096} (1024 and 4096: the BERT encoder's Q8_0 projections). Activations
// xs [m][k] with fp32 scales xd [m][k/32] (fp16 values) in x_layout: Q8_NATURAL, or Q8_TILED (rows padded to 32; small-batch kernel only); a Q8_0 output
// is written in out.yq_layout (Q8_NATURAL or Q8_TILED). Up to 256 rows (or n % 128 != 0) a kernel
// of 32-column tiles runs (tiled weights if given), tile_rows (1, 2 or 4 row tiles of 32 per
// workgroup, 0 = its own choice) selecting its row tiling; above, the 128 x 128 kernel (natural
// operands only).
int launch_q8_gemm(const Q8Weights & w, int64_t n, int64_t k, int64_t m, const int8_t * xs,
                   const float * xd, int x_layout, const LayerOut & out, hipStream_t stream,
                   int tile_rows = 0);

// w16[n][k] = fp16(d * q) (nearest even) of a natural-order Q8_0 matrix (gemm.hip).
int launch_q8_dequant_f16(const int8_t * q, const uint16_t * d, int64_t n, int64_t k, uint16_t * w16,
                          hipStream_t stream);

// The same projection on the fp16 matrix cores (gemm.hip): the Q8_0 activations (natural order)
// taken as fp16(d * q) times the fp16 weights w16 [n][k] of launch_q8_dequant_f16, fp32
// accumulation, the epilogue of launch_q8_gemm's 128 x 128 kernel (natural-order Q8_0 output);
// n % 128 == 0, k 512 or 2048.
int launch_q8h_gemm(const uint16_t * w16, int64_t n, int64_t k, int64_t m, const int8_t * xs, const float * xd,
                    const LayerOut & out, hipStream_t stream);

// Row count from which the prefill projections run on launch_q8_gemm rather than the GEMV.
constexpr int64_t GEMM_MIN_ROWS = 64;

// The decode's GEMV chain (the fused QKV + attention and the layer GEMVs, one activation row per
// sequence) runs up to 16 sequences: one batch-32 decode run of it ended in a GPU memory fault
// whose cause has not been found, so the decode refuses it above (a constant, not a build
// option; the kernels themselves are tested at up to 64 rows one launch at a time). From
// DECODE_GEMM_MIN_BATCH the matrix-core path takes the projections when the two-launch layer
// does not run.
constexpr int GEMV_DECODE_MAX_BATCH = 16;
constexpr int DECODE_GEMM_MIN_BATCH = GEMV_DECODE_MAX_BATCH + 1;

// Prefill self-attention on the matrix cores (attn_prefill_mfma.hip): qkv rows [B][S][3*d_model],
// head_dim 32, 16-byte aligned qkv and out; used from GEMM_MIN_ROWS rows on, like the GEMM.
// pv_f16: the weighted sum as one fp16 product (the prefill's fp16 mode) instead of hi/lo pairs.
// seq_order: a permutation of the B sequences, dispatched in that order (longest first), or null
// (index order); the order changes only the dispatch, not a value. skip_pad: a wave whose 32 queries
// are all left-padding rows computes nothing and those rows get zeros (the decoder's prefill, where
// no valid row reads them); padding queries sharing a wave with valid ones are computed.
int launch_attn_prefill_mfma(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                             int d_model, float scale, float * out, int8_t * oq, float * od, hipStream_t stream,
                             bool pv_f16 = false, const int32_t * seq_order = nullptr, bool skip_pad = false);
inline bool attn_prefill_uses_mfma(int64_t rows) { return rows >= GEMM_MIN_ROWS; }

// n % 32 == 0, k in {512, 2048}; IN_LN and IN_EMB need k == 512.
int launch_layer_gemv(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, int64_t m,
                      const LayerIn & in, const LayerOut & out, hipStream_t stream);

}  // namespace gsvk

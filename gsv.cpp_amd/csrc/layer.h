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
};

struct LayerOut {
    float * y;          // fp32 output rows < n_store, row stride y_stride (may be null)
    int64_t y_stride;
    int n_store;
    const float * bias;
    int act;            // 0 none, 1 relu
    int8_t * yq;        // Q8_0 output (sliced [m][n] + scales [m][n/32]) or null
    float * yd;
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
};

// Q8_0 x Q8_0 GEMM on the matrix cores (gemm.hip) with the same epilogue options: n % 128 == 0,
// k in {512, 2048}. Both operands have their quants in natural order (ws [n][k] as in the GGUF
// blocks, xs [m][k]) with the scales apart (fp16 wd [n][k/32], fp32 xd [m][k/32]); a Q8_0 output
// (yq) is written in natural order too.
int launch_q8_gemm(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, int64_t m,
                   const int8_t * xs, const float * xd, const LayerOut & out, hipStream_t stream);

// Row count from which the projections run on launch_q8_gemm rather than the GEMV.
constexpr int64_t GEMM_MIN_ROWS = 64;

// Prefill self-attention on the matrix cores (attn_prefill_mfma.hip): qkv rows [B][S][3*d_model],
// head_dim 32, 16-byte aligned qkv and out; used from GEMM_MIN_ROWS rows on, like the GEMM.
int launch_attn_prefill_mfma(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                             int d_model, float scale, float * out, int8_t * oq, float * od, hipStream_t stream);
inline bool attn_prefill_uses_mfma(int64_t rows) { return rows >= GEMM_MIN_ROWS; }

// n % 32 == 0, k in {512, 2048}; IN_LN and IN_EMB need k == 512.
int launch_layer_gemv(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, int64_t m,
                      const LayerIn & in, const LayerOut & out, hipStream_t stream);

}  // namespace gsvk

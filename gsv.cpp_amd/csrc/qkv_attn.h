// Fused QKV projection + decode attention of one layer (qkv_attn.hip).
#pragma once

#include "common.h"
#include "layer.h"

namespace gsvk {

struct QkvAttnArgs {
    const int8_t * ws;         // sliced Q8_0 QKV weights [3 * 512][512]
    const uint16_t * wd;       // their fp16 scales [3 * 512][16]
    const float * bias;        // [3 * 512]
    LayerIn in;                // IN_LN or IN_EMB input row per sequence
    uint16_t * kc;             // this layer's fp16 caches [B][n_head][lstride][32]
    uint16_t * vc;
    int64_t lstride;
    const int32_t * kv_begin;  // [B] first valid key
    const int32_t * col_ptr;   // the new key's column is *col_ptr + col_add (same for all rows)
    int col_add;
    int n_head;
    float scale_log2;          // softmax scale * log2(e)
    float scale;               // softmax scale (exact mode's scores: q.k * scale, as ggml)
    float * out;               // attention output fp32 [B][512]
    int8_t * oq;               // and its Q8_0 copy (sliced) + scales [B][16], or null
    float * od;
};

// One workgroup per (sequence, head) covers rows up to the longest: false when the standalone
// attention would split the rows (few sequences, long rows), which the fused kernel does not.
bool qkv_attn_supported(int B, int nh, int64_t max_keys);
// what the decode's GEMV chain uses: supported, and fewer than DECODE_GEMM_MIN_BATCH sequences
bool qkv_attn_preferred(int B, int nh, int64_t max_keys);
// exact: the attention in ggml-cpu's order (flash_attn_ext's sequential online softmax with
// glibc's expf), bit for bit with the oracle; any row length (no split needed)
int launch_qkv_attn(const QkvAttnArgs & a, int B, int64_t max_keys, hipStream_t stream, bool exact = false);

}  // namespace gsvk

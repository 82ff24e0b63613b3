// Decode step at small batch in two launches per decoder layer (decode_layer.hip).
#pragma once

#include "common.h"
#include "layer.h"

namespace gsvk {

// Hidden-unit groups of the FFN launch: each workgroup computes FFN1 for 2048 / groups hidden
// units of one sequence and their share of FFN2, written as one partial row of 512 that the next
// launch sums. 32 groups of 64 units while the 32 x B workgroups fit the 256 CUs (up to batch 8:
// half the weight bytes per workgroup, twice the partial rows for the next LayerNorm), 16 groups
// of 128 above. Whole step, 24 layers, 16 / 32 groups: batch 1 0.340 / 0.313 ms, batch 2 0.347 /
// 0.322, batch 4 0.352 / 0.329, batch 8 0.371 / 0.349, batch 10 0.384 / 0.402, batch 16 0.406 /
// 0.436.
constexpr int DEC_FFN_GROUPS = 16;       // the C-ABI ops (gsvk_op_dec_attn / _ffn) and above batch 8
constexpr int DEC_FFN_GROUPS_MAX = 32;
inline int dec_ffn_groups(int B) { return B <= 8 ? DEC_FFN_GROUPS_MAX : DEC_FFN_GROUPS; }

// Largest batch the two-launch layer takes (its grids are 16 x B workgroups; nothing else in it
// depends on the batch).
constexpr int DEC_MAX_BATCH = 64;

// Largest batch the library's default choice runs on the two-launch layer; above, the matrix-core
// GEMMs are faster. Whole step, 24 layers, the batch-16 request shape, two-launch against
// matrix-core: batch 24 0.68 / 0.82 ms, batch 32 0.71 / 0.84, batch 36 0.93 / 0.90, batch 48
// 0.97 / 0.91, batch 64 1.24 / 0.95. (16 x 32 workgroups are two per CU; from batch 33 a launch
// takes a third round.)
constexpr int DEC_AUTO_MAX_BATCH = 32;

// Launch 1 of a layer, workgroup (head h, sequence b):
//   input row  x = LN2((res + parts[0] + ... + parts[NP-1]) + bias) (the previous layer's LN1
//              output, FFN2 partials and b_2), or emb[tok] + alpha * PE[pos] for layer 0;
//   QKV of head h (the x86 Q8_0 dot of the GEMV), K/V append, attention over [kv_begin, col];
//   the head's attention output quantised to one Q8_0 block and multiplied by the 512 x 32
//   slice of the out projection: partial row p1[h][b][0:512].
struct DecAttnArgs {
    int mode;                 // IN_LN or IN_EMB
    const float * res;        // IN_LN: [B][512]
    const float * parts;      // IN_LN: [nparts][B][512]
    int nparts;               // IN_LN: the previous FFN launch's groups (16 or 32)
    const float * bias;       // IN_LN: [512]
    const float * wb;         // IN_LN: [w; b], 1024
    const float * emb;        // IN_EMB: embedding table [vocab][512]
    const float * pe;         // IN_EMB: positional table [pe_rows][512]
    const int32_t * tok;      // IN_EMB: [B]
    const int32_t * pos_ptr;  // IN_EMB: the PE row of sequence b is *pos_ptr + pos_add - pos_sub[b]
    int pos_add;
    const int32_t * pos_sub;  // (may be null)
    int pe_rows;
    float alpha;
    int vocab;
    int32_t * kv_end;         // IN_EMB: kv_end[b] = *pos_ptr + kv_end_add (may be null)
    int kv_end_add;
    float * x_out;            // the input row x [B][512], stored by the head-0 workgroups
    const int8_t * wq;        // QKV weights, sliced Q8_0 [1536][512], fp16 scales, bias
    const uint16_t * wd;
    const float * bqkv;
    uint16_t * kc;            // this layer's fp16 caches [B][16][lstride][32]
    uint16_t * vc;
    int64_t lstride;
    const int32_t * kv_begin; // [B]
    const int32_t * col_ptr;  // the new key's column: *col_ptr + col_add
    int col_add;
    float scale_log2;
    const int8_t * woq;       // out projection [512][512] in the Q8_TILED order
    const uint16_t * wod;
    float * p1;               // [16][B][512]
    int B;
};

// Launch 2 of a layer, workgroup (hidden group g, sequence b):
//   n1 = LN1((res + p1[0] + ... + p1[15]) + bo), stored by the group-0 workgroups;
//   the group's 2048 / groups hidden units h = relu(W1 . n1 + b1) (x86 Q8_0 dot),
//   quantised to Q8_0 blocks, times the matching columns of W2: partial row p2[g][b][0:512].
struct DecFfnArgs {
    const float * res;        // [B][512] (x_out of launch 1)
    const float * p1;         // [16][B][512]
    const float * bo;         // [512]
    const float * wb1;        // LN1 [w; b]
    float * n1_out;           // [B][512]
    const int8_t * w1q;       // FFN1 sliced Q8_0 [2048][512], fp16 scales, bias
    const uint16_t * w1d;
    const float * b1;
    const int8_t * w2q;       // FFN2 [512][2048] in the Q8_TILED order
    const uint16_t * w2d;
    float * p2;               // [groups][B][512]
    int groups;               // 16 or 32 (dec_ffn_groups)
    int B;
};

// ---- the persistent decode: all layers of a step in one launch ----
// 256 workgroups, 32 on each XCD (the dispatcher's round-robin; the hardware's XCC id names the
// XCD a workgroup runs on); XCD x owns the sequences b = x, x + 8, ... and runs, per layer, launch 1's
// work (head h of each of its sequences), a barrier among its 32 workgroups, launch 2's work
// (group g of each), a barrier. The arithmetic is the two launches' to the bit. Each layer's
// arguments are those of its two launches, kept in device memory (attn[n_layer], ffn[n_layer]).
struct DecPersistArgs {
    const DecAttnArgs * attn;   // [n_layer]: layer 0 IN_EMB, the others IN_LN with nparts = groups
    const DecFfnArgs * ffn;     // [n_layer]
    int n_layer;
    int B;
    int groups;                 // dec_ffn_groups(B)
    const int32_t * step;       // the device step counter: the barrier's epoch
    int epoch_add;              // added to *step for the epoch (0; 0, 1, ... when the kernel of
                                // one step is launched repeatedly, every launch's words above the last)
    int * flags;                // [8][32] barrier words (zero before the first step of a run)
    int * err;                  // 0, or 1 (a wait gave up) / 2 (an XCC id outside 0..7)
    const int * active;         // or null: 0 there (no row took part in this step, as the step's
                                // sampler records) makes the launch return at once
    int nt;                     // 1: the cached keys by non-temporal (streaming) loads, for a cache
                                // whose per-step reads far exceed the 256 MB MALL
};
constexpr int DEC_PERSIST_WGS = 256;
constexpr int DEC_PERSIST_MAX_BATCH = 32;   // 4 sequences per XCD
// Largest batch the library's default choice runs on the persistent decode (above 16 a workgroup
// takes two items of a phase in turn). Whole step, 24 layers, the batch-16 request shape (batch 1:
// 128 phones), two-launch against persistent: batch 1 0.310 / 0.297 ms, 2 0.319 / 0.307, 4 0.326 /
// 0.308, 8 0.346 / 0.341, 12 0.385 / 0.319, 16 0.406 / 0.333, 17 0.621 / 0.561, 20 0.638 / 0.572,
// 24 0.666 / 0.615, 32 0.689 / 0.597.
constexpr int DEC_PERSIST_AUTO_MAX_BATCH = 32;
int launch_dec_persist(const DecPersistArgs & a, hipStream_t stream);
// The device has the 256 CUs in 8 XCDs the kernel assumes, and one workgroup of it fits a CU.
bool dec_persist_device_ok(int device);

// 1 when the two-launch layer covers this shape: d_model 512, 16 heads of 32, FFN 2048, at most
// DEC_MAX_BATCH (64) sequences (the library's default choice up to DEC_AUTO_MAX_BATCH, 32), and rows
// the attention takes in one workgroup per (sequence, head).
bool dec_layer_supported(int B, int nh, int d_model, int ffn, int64_t max_keys);
int launch_dec_attn(const DecAttnArgs & a, hipStream_t stream);
int launch_dec_ffn(const DecFfnArgs & a, hipStream_t stream);

}  // namespace gsvk

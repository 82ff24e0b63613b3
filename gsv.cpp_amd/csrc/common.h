// Internal helpers shared by the gfx950 kernels and the host runtime.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "gsvk.h"

namespace gsvk {

// Thread-local last error (gsvk_last_error()).
void set_error(const char * fmt, ...) __attribute__((format(printf, 1, 2)));
const char * get_error();

}  // namespace gsvk

// Return GSVK_ERR_HIP from the enclosing function when a HIP call fails.
#define GSVK_HIP(call)                                                                        \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess) {                                                               \
            gsvk::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__,  \
                            __LINE__);                                                        \
            return GSVK_ERR_HIP;                                                              \
        }                                                                                     \
    } while (0)

// Return GSVK_ERR_ARG with a message when a condition does not hold.
#define GSVK_REQUIRE(cond, ...)                                                               \
    do {                                                                                      \
        if (!(cond)) {                                                                        \
            gsvk::set_error(__VA_ARGS__);                                                     \
            return GSVK_ERR_ARG;                                                              \
        }                                                                                     \
    } while (0)

// Propagate a non-zero status.
#define GSVK_TRY(call)                                                                        \
    do {                                                                                      \
        int s_ = (call);                                                                      \
        if (s_ != GSVK_OK) return s_;                                                         \
    } while (0)

#define GSVK_LAUNCH_CHECK()                                                                   \
    do {                                                                                      \
        hipError_t e_ = hipGetLastError();                                                    \
        if (e_ != hipSuccess) {                                                               \
            gsvk::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(e_),        \
                            __FILE__, __LINE__);                                              \
            return GSVK_ERR_HIP;                                                              \
        }                                                                                     \
    } while (0)

namespace gsvk {

constexpr int QK = 32;           // Q8_0 block length
constexpr int Q8_BLOCK_BYTES = 34;

// ---- device helpers -------------------------------------------------------------------

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, h);
    return (float) v;
}

// fp32 -> fp16, round to nearest even (the F16C conversion ggml-cpu uses), of the fp32 value f.
// The empty asm makes f opaque: without it the compiler may fuse the FMA or multiply that
// produced f with the conversion (v_fma_mixlo_f16), rounding the exact result once to fp16
// instead of first to fp32, which differs where the fp32 value is an fp16 tie.
__device__ __forceinline__ uint16_t f2h(float f) {
    __asm__("" : "+v"(f));
    _Float16 v = (_Float16) f;
    return __builtin_bit_cast(uint16_t, v);
}

// ---- cross-lane exchanges without LDS traffic (gfx9 DPP and ds_swizzle) ----
constexpr int DPP_XOR1 = 0xB1;    // quad_perm [1,0,3,2]: lane i <- lane i ^ 1
constexpr int DPP_XOR2 = 0x4E;    // quad_perm [2,3,0,1]: lane i <- lane i ^ 2
constexpr int DPP_ROR1 = 0x121;   // row_ror within 16-lane rows
constexpr int DPP_ROR2 = 0x122;
constexpr int DPP_ROR4 = 0x124;
constexpr int DPP_ROR8 = 0x128;   // rotation by 8 of 16 = lane i <- lane i ^ 8
constexpr int DPP_ROR12 = 0x12C;  // lane i <- lane (i + 4) mod 16 within 16-lane rows

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xf, 0xf, false);
    return __hiloint2double(hi, lo);
}
// lane i <- lane i ^ 4 / i ^ 16 (ds_swizzle bit mode, within 32 lanes)
__device__ __forceinline__ float swz_xor4(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));
}
__device__ __forceinline__ float swz_xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), l),
                            __builtin_amdgcn_readlane(__double2loint(v), l));
}

// Maximum over the 64 lanes, the same value in every lane (max is exact: order does not matter).
__device__ __forceinline__ float wave_max_uniform(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_ROR8>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Sum over the 64 lanes, the same value in every lane: each 16-lane row is summed by rotations
// (8, 4, 2, 1), then the four row totals of lanes 0, 16, 32, 48 as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ double wave_sum_d_uniform(double v) {
    v += dpp_d<DPP_ROR8>(v);
    v += dpp_d<DPP_ROR4>(v);
    v += dpp_d<DPP_ROR2>(v);
    v += dpp_d<DPP_ROR1>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double warp_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Q8_0 activation quantisation of one 32-block held as 32 values spread over `lanes` lanes
// (each lane holds 32/lanes values in v[]). Mirrors ggml-cpu's x86 quantiser: the scale stored
// is fp16(amax / 127) and the quants are round-half-even(x * (127 / amax)).
// Returns the fp32 value of the stored fp16 scale.
template <int PER_LANE>
__device__ __forceinline__ float q8_quantize_group(const float (&v)[PER_LANE], int8_t (&q)[PER_LANE],
                                                   int lanes) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_LANE; i++) amax = fmaxf(amax, fabsf(v[i]));
    if (lanes == 4) {
        amax = fmaxf(amax, dpp_f<DPP_XOR1>(amax));
        amax = fmaxf(amax, dpp_f<DPP_XOR2>(amax));
    } else {
        for (int o = 1; o < lanes; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    }
    const float d = amax / 127.0f;
    const float id = (amax != 0.0f) ? 127.0f / amax : 0.0f;
#pragma unroll
    for (int i = 0; i < PER_LANE; i++) q[i] = (int8_t) (int) __builtin_rintf(v[i] * id);
    return h2f(f2h(d));
}

// Store the 8 quants of values [8*sub, 8*sub+8) of block blk of one row in the sliced layout
// (qs[j][blk][t] = q[blk*32 + 4j + t]): they are groups j = 2*sub and 2*sub + 1.
__device__ __forceinline__ void q8_store_sliced(int8_t * row, int nblk, int blk, int sub,
                                                const int8_t (&q)[8]) {
    const int lo = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
    const int hi = (q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) | ((q[7] & 0xff) << 24);
    *reinterpret_cast<int *>(row + ((int64_t) (2 * sub) * nblk + blk) * 4) = lo;
    *reinterpret_cast<int *>(row + ((int64_t) (2 * sub + 1) * nblk + blk) * 4) = hi;
}

// Store the same 8 quants in natural order (q[blk*32 + 8*sub + i]), the layout of the operands
// of the matrix-core GEMM (one 4-block chunk of a row = one 128-byte line).
__device__ __forceinline__ void q8_store_natural(int8_t * row, int blk, int sub, const int8_t (&q)[8]) {
    const int lo = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
    const int hi = (q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) | ((q[7] & 0xff) << 24);
    *reinterpret_cast<int2 *>(row + blk * 32 + sub * 8) = make_int2(lo, hi);
}

// Layouts of a Q8_0 matrix [rows][k] whose scales are stored apart from the quants:
//   Q8_SLICED  quants of row r: group j of every block together, qs[r][j][blk][4] (the GEMV's
//              operand), scales [r][k/32];
//   Q8_NATURAL quants [r][k] in order, scales [r][k/32] (the 128 x 128 GEMM's operand);
//   Q8_TILED   the matrix-core operand order of the small-batch GEMM: for each 32-row tile and
//              block, 1 KB in which lane L = 32*h + i holds the 16 quants [16h, 16h+16) of
//              row i of the tile at bytes [16L, 16L+16); scales per (tile, block) as 32
//              consecutive values (row i at i). Rows are padded to a multiple of 32.
enum Q8Layout { Q8_SLICED = 0, Q8_NATURAL = 1, Q8_TILED = 2 };

// Byte offset of quant c (0..31) of block blk of row r in a Q8_TILED matrix of nblk blocks per row.
__device__ __host__ __forceinline__ int64_t q8_tiled_offset(int64_t r, int nblk, int blk, int c) {
    return (((r >> 5) * nblk + blk) << 10) + ((((c >> 4) << 5) | (int) (r & 31)) << 4) + (c & 15);
}
// Index of the scale of block blk of row r in a Q8_TILED matrix.
__device__ __host__ __forceinline__ int64_t q8_tiled_scale(int64_t r, int nblk, int blk) {
    return (((r >> 5) * nblk + blk) << 5) + (r & 31);
}

// Store the 8 quants [8*sub, 8*sub+8) of block blk of row r of a Q8_TILED matrix.
__device__ __forceinline__ void q8_store_tiled(int8_t * base, int64_t r, int nblk, int blk, int sub,
                                               const int8_t (&q)[8]) {
    const int lo = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
    const int hi = (q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) | ((q[7] & 0xff) << 24);
    *reinterpret_cast<int2 *>(base + q8_tiled_offset(r, nblk, blk, 8 * sub)) = make_int2(lo, hi);
}

// Store the 8 quants of values [8*sub, 8*sub+8) of block blk of row r (and the block's scale
// when store_d) in the given layout (matrix of nblk blocks per row).
__device__ __forceinline__ void q8_store_row8(int8_t * q, float * qd, int layout, int64_t r, int nblk,
                                              int blk, int sub, const int8_t (&v)[8], float d,
                                              bool store_d) {
    if (layout == Q8_TILED) {
        q8_store_tiled(q, r, nblk, blk, sub, v);
        if (store_d) qd[q8_tiled_scale(r, nblk, blk)] = d;
        return;
    }
    if (layout == Q8_NATURAL)
        q8_store_natural(q + r * nblk * 32, blk, sub, v);
    else
        q8_store_sliced(q + r * nblk * 32, nblk, blk, sub, v);
    if (store_d) qd[r * nblk + blk] = d;
}

// The same with an explicit byte distance between slices (LDS copies of a row pad each slice by
// 16 bytes, so that the 8 slices a wave reads at once fall in different banks).
__device__ __forceinline__ void q8_store_sliced_s(int8_t * row, int slice_bytes, int blk, int sub,
                                                  const int8_t (&q)[8]) {
    const int lo = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
    const int hi = (q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) | ((q[7] & 0xff) << 24);
    *reinterpret_cast<int *>(row + (2 * sub) * slice_bytes + blk * 4) = lo;
    *reinterpret_cast<int *>(row + (2 * sub + 1) * slice_bytes + blk * 4) = hi;
}

// Byte offset of value w (0..31) of block blk in a sliced row.
__device__ __forceinline__ int64_t q8_sliced_offset(int nblk, int blk, int w) {
    return ((int64_t) (w >> 2) * nblk + blk) * 4 + (w & 3);
}

// Epilogue of the Q8_0 GEMV: bias, activation, and optionally the KV-cache append of the K and
// V rows (rows [kv_row0, kv_row0 + 2*d_model)) as fp16 into caches laid out
// [B][n_head][lstride][32]; output row m belongs to sequence m / rows_per_seq at cache column
// *col_ptr + col_add + m % rows_per_seq.
struct GemvEpilogue {
    const float * bias;
    int act;
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

int launch_q8_gemv(const int8_t * ws, const uint16_t * wd, int64_t n, int64_t k, const int8_t * xs,
                   const float * xd, int64_t m, const GemvEpilogue & epi, float * y,
                   hipStream_t stream);
// Q8_0 outputs go to the given layout (Q8Layout; the GEMV reads Q8_SLICED, the GEMMs
// Q8_NATURAL / Q8_TILED).
int launch_q8_quantize(const float * x, int64_t rows, int64_t k, int8_t * xs, float * xd,
                       hipStream_t stream, int layout = Q8_SLICED);
// qn (may be null): the quants in natural order as well; qt/dt (may be null; rows % 32 == 0):
// quants and scales in the Q8_TILED order
int launch_q8_repack(const void * blocks, int64_t rows, int64_t k, int8_t * qs, uint16_t * d,
                     hipStream_t stream, int8_t * qn = nullptr, int8_t * qt = nullptr,
                     uint16_t * dt = nullptr);
// The sliced (qs, d) and natural (qn) copies of a weight given in the Q8_TILED order (qt, dt;
// rows % 32 == 0): the load of a pre-swizzled GGUF
int launch_q8_untile(const int8_t * qt, const uint16_t * dt, int64_t rows, int64_t k, int8_t * qs, uint16_t * d,
                     int8_t * qn, hipStream_t stream);
// (y16: optional fp16 copy of y, rounded to nearest even; row_pad: left-padding rows per sequence
// of rows_per_seq rows, or null: padding rows are neither read nor written, their outputs keep
// what they held)
int launch_layernorm(const float * x, const float * r, const float * bias, const float * wb,
                     int64_t rows, int64_t n, float eps, float * y, int8_t * yq, float * yd,
                     hipStream_t stream, int layout = Q8_SLICED, uint16_t * y16 = nullptr,
                     const int32_t * row_pad = nullptr, int rows_per_seq = 0);
int launch_embed_pe(const float * emb, const float * pe, const int32_t * tok, int vocab,
                    const int32_t * pos_ptr, int pos_add, float alpha, int d, int B, float * x,
                    int8_t * xq, float * xd, int32_t * kv_end, int kv_end_add, const int32_t * pos_sub,
                    int pe_rows, hipStream_t stream, int layout = Q8_SLICED);
int launch_add_act(const float * a, const float * b, int64_t n, int64_t ne0, int act, float * y, hipStream_t stream);
// QKV rows [rows][3 * d_model] of an F16 / F32 projection: + bias in place, K and V (fp16) appended
// at column *col_ptr + col_add + r % rows_per_seq of sequence r / rows_per_seq
int launch_bias_kv(float * y, const float * bias, int64_t rows, int d_model, uint16_t * kc, uint16_t * vc,
                   int n_head, int64_t lstride, int rows_per_seq, const int32_t * col_ptr, int col_add,
                   hipStream_t stream);
size_t attn_workspace_bytes(int B, int nh, int64_t max_keys);
int launch_attn_decode(const float * q, int64_t q_stride, const uint16_t * k, const uint16_t * v,
                       int B, int nh, int hd, int64_t lstride, const int32_t * kv_begin,
                       const int32_t * kv_end, int64_t max_keys, float scale, float * out,
                       uint16_t * out16, int8_t * oq, float * od, void * ws, hipStream_t stream,
                       int oq_layout = Q8_SLICED);

}  // namespace gsvk

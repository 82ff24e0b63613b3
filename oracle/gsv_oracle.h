/*
 * gsv_oracle.h — CPU restatement of gsv.cpp's AR (text-to-semantic) decoder path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP implementation and the
 * timed host-CPU baseline. Product code must never link, load or call it.
 *
 * It restates, in plain C (with AVX2 intrinsics where ggml-cpu's x86 build uses them):
 *   - src/gsv_ar.cpp            build_inputs, prefill (run_first), decode (run_decode), the
 *                               generate loop (EOS rule, early stop, oracle tokens, seeds)
 *   - src/gsv_sampler.{h,cpp}   repetition penalty, top-p, temperature, top-k, softmax,
 *                               xorshift64* sampling
 *   - PATCH:1533-1620           ggml_compute_forward_layernorm_affine / add_act
 *   - ggml-cpu (llama.cpp f0c41e01, not vendored): the x86 AVX2 arithmetic of mul_mat
 *     (Q8_0 activation quantisation + int8 block dot, F16/F32 dots) and of flash_attn_ext.
 *
 * Floating-point convention: the reference's Linux build is GCC -O3 -mavx2 -mfma in GNU mode,
 * which contracts a*b + c into one FMA; this file is compiled with -ffp-contract=off and writes
 * those FMAs explicitly (fmaf) where the reference source has an a*b + c expression.
 *
 * What pins each function (tests/test_oracle_pins.py), i.e. what checks it against something
 * other than its own formula:
 *   orc_q8_quantize_ref, orc_q8_dequant   known-answer blocks (zero block, +-127 extremes,
 *                                         negative zero); closed form of the 34-byte block
 *   orc_q8_quantize_x86                   known answers incl. exact ties (half to even), fp16 d
 *   orc_q8_dot, orc_q8_matmul             exact integer block sums, fp64 within 1e-6, and the
 *                                         lane-by-lane scalar restatement
 *   orc_f16_matmul, orc_f32_matmul        fp64 within the bound of fp32 summation
 *   orc_layernorm                         closed forms (constant row -> b, arithmetic ramp)
 *   orc_add_act                           the reference's fixture (tests/test_add_act.cpp:66-98)
 *   orc_attn_row, orc_attn_decode_f16     fp64 brute force; one key -> that V row; constant V
 *   orc_logits_to_probs, orc_rng_*,       golden vectors written by the reference's own
 *   orc_sample, orc_argmax_probs_over_q   src/gsv_sampler.cpp compiled from source
 *   orc_pe_table                          fp64 closed form
 *   orc_generate, orc_prefill_kv,         known-answer models (tests/test_oracle_composition.py):
 *   orc_first_logits                      zero / exact-identity projections give float64 closed
 *                                         forms of the input rows (BERT projection, PE positions,
 *                                         alphas, padding), the LayerNorm chain with b_o and b_2,
 *                                         the head over the last row, the prefill attention masks,
 *                                         the decode embedding position and K/V cache column, the
 *                                         decode attention's key range [pad, len] (new key
 *                                         included) and 1/sqrt(32) scale, and the ReLU between
 *                                         FFN1 and FFN2 (exactly quantisable activations); plus
 *                                         left-padding invariance and EOS / early-stop traces
 * Parity unpinned: the ORDER of ggml-cpu's floating-point arithmetic (the x86 activation
 * rounding mode, the 8-lane Q8_0 and F16 dot orders, flash_attn_ext's online-softmax order and
 * expf) lives in llama.cpp f0c41e01, which is not under the reference tree, and no reference
 * test or fixture holds its outputs. The values above are pinned to fp64; the exact rounding
 * sequence follows the published ggml-cpu source as restated here and is unpinned.
 */
#ifndef GSV_ORACLE_H
#define GSV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (F16C, round to nearest even) ---- */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);

/* ---- Q8_0: 34-byte blocks {fp16 d; int8 q[32]} ---- */
/* ggml quantize_row_q8_0_ref (weights, gguf export): d = amax/127, id = d ? 1/d : 0, roundf */
void  orc_q8_quantize_ref(const float * x, int64_t n, uint8_t * blocks);
/* ggml-cpu x86 quantize_row_q8_0 (activations): id = 127/amax, round half even */
void  orc_q8_quantize_x86(const float * x, int64_t n, uint8_t * blocks);
void  orc_q8_dequant(const uint8_t * blocks, int64_t nblocks, float * out);
/* ggml_vec_dot_q8_0_q8_0, x86 AVX2 arithmetic (8 fp32 lanes, FMA per block, hsum) */
float orc_q8_dot(const uint8_t * w, const uint8_t * x, int64_t nblocks);
/* the same arithmetic written lane by lane in scalar C (pins the intrinsic version) */
float orc_q8_dot_scalar(const uint8_t * w, const uint8_t * x, int64_t nblocks);
/* Y[m][n] = W[n] . X[m]: X rows quantised with orc_q8_quantize_x86 first (ggml mul_mat) */
void  orc_q8_matmul(const uint8_t * W, int64_t N, int64_t K, const float * X, int64_t M,
                    float * Y, int nthreads);

/* ---- F16 / F32 weight dots (the head) ----
 * mode 0: ggml_vec_dot_f16/_f32 (decode: 4 accumulators of 8 lanes + GGML_F32x8_REDUCE)
 * mode 1: llamafile tinyBLAS (prefill with >= 2 columns: 1 accumulator of 8 lanes + hsum)
 * F16: X is rounded to fp16 first (vec_dot_type F16). */
void orc_f16_matmul(const uint16_t * W, int64_t N, int64_t K, const float * X, int64_t M,
                    float * Y, int mode, int nthreads);
void orc_f32_matmul(const float * W, int64_t N, int64_t K, const float * X, int64_t M, float * Y,
                    int mode, int nthreads);

/* ---- fused ops of the patch ---- */
void orc_layernorm(const float * x, const float * r, const float * bias, const float * wb,
                   int64_t rows, int64_t n, float eps, float * y);
void orc_add_act(const float * a, const float * b, int64_t n, int64_t ne0, int act, float * y);

/* ---- attention, one query row (ggml flash_attn_ext CPU online softmax) ----
 * q[hd]; keys j in [0, L) at k + j*kstride (fp32); mask_skip[j] != 0 skips key j (mask -inf).
 * out[hd]. */
void orc_attn_row(const float * q, const float * k, const float * v, int64_t kstride, int hd,
                  int64_t L, const uint8_t * mask_skip, float scale, float * out);
/* y[i] = expf(x[i]) with this host's libm (glibc: the exponential of flash_attn_ext's online
 * softmax above and in ggml-cpu) */
void orc_expf_n(const float * x, int64_t n, float * y);
/* decode attention over an fp16 cache laid out [B][nh][lstride][hd] (the device layout), keys
 * [kv_begin[b], kv_end[b]) valid: out [B][nh*hd]. */
void orc_attn_decode_f16(const float * q, const uint16_t * k, const uint16_t * v, int B, int nh,
                         int hd, int64_t lstride, const int32_t * kv_begin,
                         const int32_t * kv_end, float scale, float * out, int nthreads);

/* prefill self-attention over fp32 qkv rows [B][S][3*nh*hd] with the reference's masks
 * (src/gsv_ar.cpp:215-223): query qi of sequence b sees keys [pad[b], max_len) when
 * qi < max_len (text rows), else [pad[b], qi] (causal semantic rows). out [B][S][nh*hd]. */
void orc_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                      int hd, float scale, float * out, int nthreads);

/* ---- sampler (src/gsv_sampler.cpp) ---- */
void     orc_logits_to_probs(int top_k, float top_p, float temperature, float rep, float * logits,
                             int V, const int32_t * prev, int n_prev, float * probs);
uint64_t orc_rng_next(uint64_t * state);
float    orc_rng_exponential(uint64_t * state);
void     orc_rng_exponential_n(uint64_t * state, int64_t n, float * out);
int      orc_argmax_probs_over_q(const float * probs, const float * q, int V);
int      orc_sample(const float * probs, int V, uint64_t * state);

/* ---- positional encoding (src/gsv_ar.cpp:173-181) ---- */
void orc_pe_table(int D, int npos, float * out);

/* ---- model ---- */
typedef struct orc_model orc_model;

typedef struct orc_request {
    const int32_t * phones;
    int32_t         n_phones;
    const float   * bert;     /* [1024][n_phones], NULL = zeros */
    const int32_t * prompt;
    int32_t         n_prompt;
} orc_request;

#define ORC_KV_F16        1u   /* round K/V to fp16 when written to the cache (device storage) */
#define ORC_EOS_MASK_ALL  2u   /* mask EOS at every step */

typedef struct orc_gen_out {
    int32_t * tokens;      /* [B][tok_stride] */
    int32_t   tok_stride;
    int32_t * tok_len;     /* [B] */
    int32_t * lens;        /* [B] finish order */
    int32_t * finish_seq;  /* [B] or NULL */
    int32_t * sampled;     /* [max_steps][B] sampler choice before oracle override, or NULL */
    float   * logits;      /* [max_steps][B][V] logits entering each step, or NULL */
    float   * probs0;      /* [max_steps][V] sequence 0 probabilities, or NULL */
    int32_t   n_steps;
    double    prefill_ms;  /* wall clock of the prefill */
    double    decode_ms;   /* wall clock of the decode loop */
    /* optional: layer kv_layer's K/V cache after the loop, [B][NH][kv_cols][HD], columns
     * [0, kv_cols) (the prefill's S columns, then one column per decode step); NULL = not wanted */
    int32_t   kv_layer;
    int32_t   kv_cols;
    float   * kv_k;
    float   * kv_v;
} orc_gen_out;

orc_model * orc_model_load(const char * gguf_path, char * err, int errlen);
void        orc_model_free(orc_model * m);
/* info[0..9] = D, NH, HD, NL, V, EOS, PHONES, BERT, FFN, head_type */
void        orc_model_info(const orc_model * m, int32_t * info);

int orc_generate(orc_model * m, const orc_request * reqs, int B, int top_k, float top_p,
                 float temperature, float rep, uint64_t seed_base, int early_stop_num,
                 int max_steps, const int32_t * oracle, int n_oracle, const uint64_t * seeds,
                 unsigned flags, int nthreads, orc_gen_out * out);

/* prefill, returning layer `layer`'s K/V cache [B][NH][S][HD] (after the ORC_KV_F16 rounding if
 * set), the last-position logits [B][V] and S */
int orc_prefill_kv(orc_model * m, const orc_request * reqs, int B, unsigned flags, int nthreads,
                   int layer, float * k_out, float * v_out, float * logits, int32_t * S_out);

/* prefill only: last-position logits [B][V] */
int orc_first_logits(orc_model * m, const orc_request * reqs, int B, unsigned flags, int nthreads,
                     float * logits);

#ifdef __cplusplus
}
#endif

#endif

/*
 * gsvk.h — C ABI of the MI355X (gfx950) AR / text-to-semantic decoder.
 *
 * This is the thin layer between the C++ host code (the gsv_ar class, include/gsv_ar.h) and the
 * hand-written HIP kernels. Every entry point takes plain pointers and sizes, returns an int
 * status (GSVK_OK == 0) and never exits the process. gsvk_last_error() gives the message of the
 * last failure on the calling thread.
 *
 * Two groups of entry points:
 *
 *  1. Model runtime (gsvk_model_*, gsvk_generate, gsvk_first_logits, gsvk_kv_*): the work that the
 *     reference does in src/gsv_ar.cpp through ggml graphs. Host buffers stay caller-owned,
 *     device buffers stay model-owned. One model = one HIP device + one HIP stream; a model is
 *     not thread-safe (callers serialise on it, as the reference's callers do).
 *
 *  2. Device ops (gsvk_op_*): one kernel launch each, on caller-owned DEVICE memory and a caller
 *     stream (hipStream_t passed as void*, NULL = default stream). They are the same kernels the
 *     runtime uses, exposed so that each can be checked and timed alone.
 *
 * Conventions: fp16 values are passed as uint16_t bit patterns; Q8_0 "blocks" are the GGUF block
 * layout (34 bytes: fp16 scale d, then 32 int8 quants). On the device Q8_0 rows use the "sliced"
 * layout: quants qs[row][j][blk][t] = q[row][32*blk + 4*j + t] (j < 8, t < 4) and scales
 * d[row][blk] (fp16 for weights, fp32 for activations); slice j of a row is what lane j of
 * ggml-cpu's 8-lane x86 dot accumulates, so the device reproduces its summation order.
 */
#ifndef GSVK_H
#define GSVK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define GSVK_OK          0
#define GSVK_ERR_ARG     1   /* invalid argument or shape */
#define GSVK_ERR_HIP     2   /* a HIP runtime call failed */
#define GSVK_ERR_IO      3   /* file open / read failed */
#define GSVK_ERR_FORMAT  4   /* GGUF content missing or of an unsupported type */
#define GSVK_ERR_NOMEM   5   /* device or host allocation failed */
#define GSVK_ERR_STATE   6   /* call out of order (e.g. decode before prefill) */
#define GSVK_ERR_NODEV   7   /* no usable HIP device */

/* Message of the last failed call on this thread ("" if none). */
const char * gsvk_last_error(void);

/* Number of visible HIP devices (0 when none). */
int gsvk_device_count(int * n);

/* Parse a device string with the reference's syntax (src/gsv_device.h:19-37) extended for HIP:
 * "", "gpu", "hip", "rocm", "vulkan", "cuda" -> device 0; "gpu:N", "hip:N", "N" -> device N.
 * "cpu" is rejected (this build has no CPU path): returns GSVK_ERR_NODEV. */
int gsvk_parse_device(const char * s, int * device);

/* ======================================================================================
 * 1. Model runtime
 * ====================================================================================== */

typedef struct gsvk_model gsvk_model;

typedef struct gsvk_model_info {
    int d_model;        /* ar.hidden_dim (512) */
    int n_head;         /* ar.head (16) */
    int head_dim;       /* d_model / n_head (32) */
    int n_layer;        /* ar.n_layer (24) */
    int vocab;          /* ar.vocab_size (1025) */
    int eos;            /* ar.eos (1024) */
    int phone_vocab;    /* ar.phoneme_vocab_size (732) */
    int bert_dim;       /* 1024 */
    int ffn_dim;        /* rows of ffn1_w (2048) */
    int head_type;      /* GGML type of ar.predict: 0 F32, 1 F16, 8 Q8_0 */
    float text_alpha;   /* ar.text_pe_alpha */
    float audio_alpha;  /* ar.audio_pe_alpha */
    int prompt_len;     /* prompt length seen by the last generate / first_logits (0 = none) */
    int kv_batch;       /* batch of the resident KV cache (0 = none) */
    int kv_lmax;        /* key slots per sequence of the resident KV cache */
} gsvk_model_info;

/* Load a gsv AR GGUF (tools/export_gguf/convert_ar.py contract) onto HIP device `device`.
 * Replaces gsv_ar::load (src/gsv_ar.cpp:490-705). The layer projections may be Q8_0, F16 or F32
 * (the exporter's attn= / ffn= options, tools/export_gguf/export.py:53-54); a model with an F16 or
 * F32 projection decodes on a per-op path (ggml's F16 / F32 dot orders, F16 with fp16-rounded
 * activations) and ignores gsvk_model_set_decode_path's explicit choices (they fail). */
int gsvk_model_load(const char * gguf_path, int device, int verbose, gsvk_model ** out);
void gsvk_model_free(gsvk_model * m);
int gsvk_model_get_info(const gsvk_model * m, gsvk_model_info * info);

/* One request: replaces gsv_ar_request (src/gsv_ar.h:13-17).
 * bert is [bert_dim][n_phones] row-major (bert[k*n_phones + t]); NULL means all zero. */
typedef struct gsvk_request {
    const int32_t * phones;
    int32_t         n_phones;
    const float   * bert;
    const int32_t * prompt;
    int32_t         n_prompt;
} gsvk_request;

/* Sampler settings: same fields and meaning as gsv_sampler_cfg (src/gsv_sampler.h:18-23). */
typedef struct gsvk_sampler_cfg {
    int   top_k;
    float top_p;
    float temperature;
    float repetition_penalty;
} gsvk_sampler_cfg;

/* gsvk_generate flags */
#define GSVK_GEN_EOS_MASK_ALL  1u  /* mask EOS at every step (benchmarks: fixed-length runs) */
#define GSVK_GEN_PROB_DUMP     2u  /* write sequence 0's per-step probabilities to out->probs0 */

/* Output buffers, all caller-owned host memory.
 *  tokens     : [B][tok_stride] int32; row b receives prompt + generated tokens minus the
 *               stopping token (gsv_ar_result.tokens semantics, src/gsv_ar.cpp:782, 790, 813)
 *  tok_len    : [B] number of valid entries of each tokens row
 *  lens       : [B] generated-token counts in FINISH order (gsv_ar_result.lens, :783, 791, 814)
 *  finish_seq : [B] optional (may be NULL): the sequence index of each lens entry
 *  probs0     : optional [max_steps][vocab] (GSVK_GEN_PROB_DUMP), sequence 0's probabilities
 *  n_steps    : number of decode-loop iterations that ran */
typedef struct gsvk_gen_out {
    int32_t * tokens;
    int32_t   tok_stride;
    int32_t * tok_len;
    int32_t * lens;
    int32_t * finish_seq;
    float   * probs0;
    int32_t   n_steps;
    /* optional progress callback, called once per decode step that ran (n_steps calls in all,
     * step = 0, 1, ...), a step or two behind the GPU while it decodes (gsvprog::tick in the
     * reference, src/gsv_ar.cpp:761-763) */
    void   (*progress)(void * user, int step);
    void    * progress_user;
    /* wall-clock split measured by the runtime, stream-synchronised on both sides */
    double    prefill_ms;
    double    decode_ms;
} gsvk_gen_out;

/* Time buckets of the last generate (prefill phases also after first_logits / prefill), the ones
 * GSV_AR_PROFILE prints (src/gsv_ar.cpp:18-42: prof_report). Prefill: host packing of the requests,
 * uploads, the kernels, the logits read-back (device phases timed with HIP events). Decode: the
 * graph capture, the state uploads, the step loop (the GPU's decode, sampling and embedding
 * included: they run on the device), the results read-back. */
typedef struct {
    double pf_build_ms, pf_copy_ms, pf_compute_ms, pf_io_ms;
    double dec_build_ms, dec_copy_ms, dec_compute_ms, dec_other_ms;
    int steps;
} gsvk_profile;
int gsvk_model_get_profile(gsvk_model * m, gsvk_profile * out);

/* The persistent decode's kernel (GSVK_DECODE_PERSIST: all 24 layers of a step) at the model's
 * current step, launched `launches` times back to back on the model's stream between two HIP
 * events: its mean duration per launch. Every launch repeats that step's layers on the same inputs
 * (writing the same K/V column the step writes); the head and the sampler do not run. Needs a
 * decode state (after a prefill or generate) on a path and batch where the persistent decode runs.
 * No counterpart in the reference; for benchmarks (the decode's dominant kernel, timed alone). */
int gsvk_model_time_decode_kernel(gsvk_model * m, int launches, float * ms_per_launch);

/* The persistent decode's phase stamps, in a library built with `build.py --phase-stamps` only
 * (lib/libgsvk_stamps.so; otherwise GSVK_ERR_STATE): for each of the 256 workgroups, 1024 int64
 * values, [layer * 16 + event] = the 100 MHz s_memrealtime counter when thread 0 reached the event
 * in the last persistent launch (0 barrier seen, 1 input row quantised, 2 QKV and K/V append done,
 * 3 attention merged, 4 out-projection partial row stored, 5 flag stored; 8 barrier seen, 9 LN1
 * row quantised, 10 FFN1 blocks quantised, 11 FFN2 partial row stored, 12 flag stored), and at
 * [63 * 16] the launch's start, [63 * 16 + 1] the workgroup's XCD. `n` must be at least 256 * 1024.
 * No counterpart in the reference; for profiling. */
int gsvk_phase_stamps(int64_t * out, size_t n);

/* Full batched generation: replaces gsv_ar::generate (src/gsv_ar.cpp:719-824).
 * oracle (teacher forcing) may be NULL; seeds may be NULL (then seed_base + 0x9E3779B9*b). */
int gsvk_generate(gsvk_model * m, const gsvk_request * reqs, int B, const gsvk_sampler_cfg * cfg,
                  uint64_t seed_base, int early_stop_num, int max_steps,
                  const int32_t * oracle, int n_oracle, const uint64_t * seeds, unsigned flags,
                  gsvk_gen_out * out);

/* Prefill only, last-position logits [B][vocab]: replaces gsv_ar::first_logits (:707-717). */
int gsvk_first_logits(gsvk_model * m, const gsvk_request * reqs, int B, float * logits_out);

/* Which kernels run a decode step (the arithmetic of src/gsv_ar.cpp:380-467 in every case):
 *  GSVK_DECODE_AUTO  the library's choice (default, the fastest at each batch): up to 32
 *                    sequences the persistent decode where it runs (PERSIST), else the two-launch
 *                    layer; from 33 the matrix-core GEMMs;
 *  GSVK_DECODE_GEMV  up to 16 sequences the GEMV chain whose projections and LayerNorms are
 *                    bit-exact with ggml-cpu's x86 order (4 launches per layer);
 *  GSVK_DECODE_FUSED up to 64 sequences two launches per layer (attention + out-projection
 *                    partial rows per head; LN1 + FFN1 + FFN2 partial rows per group of hidden
 *                    units): the same int32 block dots, fp32 sums over heads and groups in a fixed
 *                    order (agrees with the GEMV chain to fp32 rounding);
 *  GSVK_DECODE_MFMA  the matrix-core GEMMs at any batch;
 *  GSVK_DECODE_PERSIST up to 32 sequences, all 24 layers of a step in one launch: the two-launch
 *                    layer's work and arithmetic (the same bits), each XCD running whole
 *                    sequences with its 32 workgroups synchronised through per-workgroup flag
 *                    words in its L2; needs the 256-CU gfx950 device (checked), not in exact mode
 *                    or a continuous batch. A run whose workgroups could not synchronise (a
 *                    bounded wait gave up) is repeated on the two-launch layer, which the model
 *                    then keeps using; GSVK_NO_PERSIST in the environment turns it off.
 * An explicit choice that does not cover the batch (or model: FUSED needs an F16 / F32 head) makes
 * the decode fail with an error naming it; it never falls back to another path. No counterpart
 * in the reference (it has one CPU path); for tests and benchmarks. */
#define GSVK_DECODE_AUTO   0
#define GSVK_DECODE_GEMV   1
#define GSVK_DECODE_FUSED  2
#define GSVK_DECODE_MFMA   3
#define GSVK_DECODE_PERSIST 4
int gsvk_model_set_decode_path(gsvk_model * m, int path);

/* Exact mode (on != 0): every projection, LayerNorm, quantisation and attention row of the
 * prefill and the decode in ggml-cpu's x86 arithmetic order, so that logits and tokens are those
 * of the CPU reference bit for bit: the GEMV chain at every row count (no matrix-core GEMM) and
 * the attention of each (row, head) as flash_attn_ext's sequential online softmax with glibc's
 * expf (gsvk_op_attn_exact). Slower than the default kernels; above 16 sequences the decode runs
 * the chain in groups of 16 rows one after another (a model with F16 / F32 projections: at most
 * 16 sequences). No counterpart in the reference (whose one CPU path is this arithmetic); for callers that need
 * its exact tokens and for tests. */
int gsvk_model_set_exact(gsvk_model * m, int on);

/* Prefill on the fp16 matrix cores (on != 0): the projections of a prefill with enough rows for
 * the matrix-core GEMMs multiply the Q8_0 activations, turned into fp16(d * q), by copies of the
 * Q8_0 weights dequantised once to fp16 (fp16(d * q), made at the first such prefill and kept
 * with the model, 2 bytes per weight) on v_mfma_f32_32x32x16_f16 instead of the int8 products
 * and their per-block fp32 scaling, and the attention's weighted sum is one fp16 product
 * (gsvk_op_attn_prefill path 3). Both operands are rounded to fp16, so the projections are within
 * about 6e-4 of their row's scale of ggml's (the bar for them is 2e-3) instead of fp32 rounding,
 * and so are the K/V rows the prefill writes. No effect on the decode or in exact mode.
 * Off by default; no counterpart in the reference (an option for callers that prefer a faster
 * prefill to agreement within fp32 rounding). */
int gsvk_model_set_prefill_f16(gsvk_model * m, int on);

/* Free the resident KV cache: replaces gsv_ar::release_cache (:826). */
int gsvk_release_cache(gsvk_model * m);

/* ---- step-level entry points (the lockstep loop of gsv_ar::generate, split for callers that
 *      drive it themselves: schedulers, tests, benchmarks) ---- */

/* Allocate (or reuse) the resident KV cache for B sequences of up to lmax positions
 * (src/gsv_ar.cpp:94-118). K and V are fp16 [n_layer][B][n_head][lmax+1][head_dim]. */
int gsvk_kv_alloc(gsvk_model * m, int B, int lmax);

/* Prefill B requests (src/gsv_ar.cpp:186-293): builds inputs on the device, runs all layers,
 * fills the KV cache for positions [0, S) and returns last-position logits [B][vocab] (may be
 * NULL). *S_out receives S = max(n_phones) + n_prompt. Resets the decode position to S. */
int gsvk_prefill(gsvk_model * m, const gsvk_request * reqs, int B, float * logits_out, int * S_out);

/* One decode step (src/gsv_ar.cpp:798-809 + 380-467): embeds last_tok[b] at PE position
 * prompt_len + step, appends K/V at column S + step, and returns logits [B][vocab] (may be NULL).
 * step advances by one per call. */
int gsvk_decode_step(gsvk_model * m, const int32_t * last_tok, float * logits_out);

/* Copy the device KV cache of layer `layer` to host fp16 buffers, each [B][n_head][lmax+1][hd]
 * (for checking the write/gather indexing). */
int gsvk_kv_read(gsvk_model * m, int layer, uint16_t * k_out, uint16_t * v_out);

/* ---- A batch that sequences join and leave while it decodes (continuous batching) ----------
 * The reference batches requests per generate call (tools/svc_core.h:1244-1340: a group of
 * requests with the same prompt, then src/gsv_ar.cpp:719-824 until the last finishes). These
 * calls keep one batch decoding while requests join and leave it, each with the semantics of a
 * generate of its own (same tokens for the same seed: per row the arithmetic does not depend on
 * the other rows). The batch decodes in lockstep over a shared KV column; a request joins with a
 * prefill of its own into a free cache row, left-padded so that it ends at that column. Any
 * other prefill / generate / release call closes the session. */

/* Open a session: `capacity` rows, requests of at most max_prefill = phones + prompt_len rows,
 * the prompt length every request has, at most max_steps decode steps over the whole session
 * (prompt_len + max_steps <= 4096). cfg, early_stop_num and flags (GSVK_GEN_EOS_MASK_ALL) as
 * gsvk_generate, the early-stop rule applied to each request's own tokens. */
int gsvk_cb_open(gsvk_model * m, int capacity, int max_prefill, int max_steps, int prompt_len,
                 const gsvk_sampler_cfg * cfg, int early_stop_num, unsigned flags);

/* Prefill one request into a free row; its first token is sampled at the next step. It decodes
 * at most max_steps steps (the session's remaining steps bound it). seed as gsvk_generate's seeds
 * (0 -> 1). *slot receives the row. */
int gsvk_cb_add(gsvk_model * m, const gsvk_request * req, uint64_t seed, int max_steps, int * slot);

/* Run n_steps decode steps of every row holding a running request; *n_running (may be NULL)
 * receives the number still running after them (-1 when n_steps is 0). */
int gsvk_cb_step(gsvk_model * m, int n_steps, int * n_running);

/* If the request in row `slot` has finished (EOS, early stop or its step limit), copy its tokens
 * (prompt + generated, without the stopping token, as gsvk_generate) to tokens[capacity], set
 * *n_tokens, *len (the finishing step, or the step limit) and *finished = 1, and free the row;
 * else set *finished = 0 and leave it. tokens may be NULL (the request is dropped). */
int gsvk_cb_take(gsvk_model * m, int slot, int32_t * tokens, int capacity, int * n_tokens, int * len,
                 int * finished);

/* Close the session (the cache and buffers stay allocated for the next call). */
int gsvk_cb_close(gsvk_model * m);

/* Sampler choices of the last gsvk_generate before teacher forcing replaced them:
 * [n_steps][B], -1 where a sequence had already finished (greedy-token checks). */
int gsvk_last_sampled(gsvk_model * m, int n_steps, int32_t * out);

/* ======================================================================================
 * 2. Device ops (device pointers, caller stream)
 * ====================================================================================== */

/* GGUF Q8_0 blocks -> fp32 (w = fp32(d) * q). nblocks blocks, out has 32*nblocks floats. */
int gsvk_op_q8_dequant(const void * blocks, int64_t nblocks, float * out, void * stream);

/* GGUF Q8_0 blocks [rows][k/32] -> sliced layout qs [rows][k] int8 + d [rows][k/32] fp16. */
int gsvk_op_q8_repack(const void * blocks, int64_t rows, int64_t k, int8_t * qs, uint16_t * d,
                      void * stream);

/* Activation quantisation of fp32 rows [rows][k] to Q8_0 exactly as ggml-cpu's x86 quantiser:
 * per 32-block amax, d = fp16(amax/127), q = round-half-even(x * (127/amax)).
 * xq receives the quants in the sliced layout, xd fp32(d) per block ([rows][k/32]). */
int gsvk_op_q8_quantize(const float * x, int64_t rows, int64_t k, int8_t * xq, float * xd,
                        void * stream);

/* y[m][n] = W[n] . x[m] on Q8_0 rows in the sliced layout, ggml-cpu's x86 order: per lane j,
 * acc_j = fma(fp32(wd[n][blk]) * xd[m][blk], dot4_i8(group j of blk), acc_j) over the blocks,
 * then ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)); (+ bias[n] if bias) then act (0 none, 1 relu).
 * k % 128 == 0. */
int gsvk_op_q8_gemv(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k,
                    const int8_t * xq, const float * xd, int64_t m, const float * bias, int act,
                    float * y, void * stream);

/* Q8_0 x Q8_0 GEMM on the matrix cores (int8 MFMA, one 32-value block per instruction, fp32
 * per-block scaling): the projections of src/gsv_ar.cpp:244-263 over many rows (prefill). The
 * same product as gsvk_op_q8_gemv, but both operands have their quants in NATURAL order (wq
 * [n][k] = the GGUF blocks' quants without the scales, xq [m][k]) with the scales apart (wd fp16
 * [n][k/32], xd fp32 [m][k/32] holding fp16 values, as every Q8_0 scale does); the fp32
 * accumulation runs block by block instead of in
 * ggml-cpu's 8-lane x86 order, so results agree to fp32 rounding. n must be a multiple of 32
 * (of 128 above 256 rows), k 512 or 2048; bias and y 16-byte aligned. Up to 256 rows the
 * product runs in tiles of 32 columns with the K range split over a workgroup's 4 waves (decode
 * at large batch), above in tiles of 128 x 128. */
int gsvk_op_q8_gemm(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k, const int8_t * xq,
                    const float * xd, int64_t m, const float * bias, int act, float * y, void * stream);

/* gsvk_op_q8_gemm with the other outputs of the projections' epilogue: y may be NULL, and yq/yd
 * (both or neither) receive the Q8_0 quantisation of each 32-column block of the output (quants
 * [m][n], fp32 scales [m][n/32] holding fp16 values), which the next GEMM reads (the FFN1 output
 * of src/gsv_ar.cpp:255-260 as the FFN2 input). tile_rows (small-batch kernel only): row tiles of
 * 32 per workgroup, 1, 2 or 4, 0 = the library's choice. tiled = 1: wq/wd, xq/xd and yq/yd are
 * in the matrix-core operand order instead of natural order: for each 32-row tile and block, 1 KB
 * in which bytes [16L, 16L+16), L = 32h + i, hold the quants [16h, 16h+16) of row i of the tile,
 * and the tile's 32 scales of the block in row order; row counts padded to a multiple of 32 (the
 * small-batch kernel, any m). */
int gsvk_op_q8_gemm_ex(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k,
                       const int8_t * xq, const float * xd, int64_t m, const float * bias, int act,
                       float * y, int8_t * yq, float * yd, int tile_rows, int tiled, void * stream);

/* w16[n][k] = fp16(d * q) (nearest even) of a Q8_0 matrix in natural order (quants wq [n][k],
 * fp16 scales wd [n][k/32]): the weights of the prefill's fp16 mode (gsvk_model_set_prefill_f16).
 * wq and w16 16-byte aligned. */
int gsvk_op_q8_dequant_f16(const int8_t * wq, const uint16_t * wd, int64_t n, int64_t k, uint16_t * w16,
                           void * stream);

/* The projection of the prefill's fp16 mode: y = act(X . W^T + bias) with X the Q8_0 activations
 * (xq [m][k] natural order, fp32 scales xd [m][k/32] holding fp16 values) taken as fp16(d * q) and
 * W the fp16 weights w16 [n][k] of gsvk_op_q8_dequant_f16, on the fp16 matrix cores with fp32
 * accumulation; y and/or yq/yd (the Q8_0 quantisation of each 32-column block of the output) as
 * in gsvk_op_q8_gemm_ex. n a multiple of 128, k 512 or 2048. Replaces the same mul_mat nodes as
 * gsvk_op_q8_gemm (src/gsv_ar.cpp:245-260) within fp16 operand rounding. */
int gsvk_op_q8h_gemm(const uint16_t * w16, int64_t n, int64_t k, const int8_t * xq, const float * xd,
                     int64_t m, const float * bias, int act, float * y, int8_t * yq, float * yd, void * stream);

/* y = W . Q8_0(LayerNorm((res + r) + ln_bias) * wb[0:512] + wb[512:1024]) (+ bias) then act:
 * the decoder's fused kernel with its LayerNorm input stage (rows of 512; n % 32 == 0). The
 * LayerNorm output is also stored to ln_out when given. r, ln_bias, bias may be NULL. */
int gsvk_op_ln_gemv(const int8_t * wq, const uint16_t * wd, int64_t n, const float * res,
                    const float * r, const float * ln_bias, const float * wb, int64_t m,
                    const float * bias, int act, float * y, float * ln_out, void * stream);

/* Fused LayerNorm (PATCH ggml_compute_forward_layernorm_affine):
 * v = x + r + bias; y = (v - mean) / sqrt(var + eps) * wb[0:n] + wb[n:2n], sums in double.
 * r and bias may be NULL. If yq/yd are given, y is also quantised to Q8_0 (n % 32 == 0). */
int gsvk_op_layernorm(const float * x, const float * r, const float * bias, const float * wb,
                      int64_t rows, int64_t n, float eps, float * y, int8_t * yq, float * yd,
                      void * stream);

/* Fused add + activation (PATCH ggml_compute_forward_add_act): y = act(a + b[i % ne0]),
 * act 0 none, 1 relu, 2 gelu(erf), 3 mish. */
int gsvk_op_add_act(const float * a, const float * b, int64_t n, int64_t ne0, int act, float * y,
                    void * stream);

/* Dot products of F16 (wtype 1) or F32 (wtype 0) weight rows W [n][k] with fp32 rows x [m][k]:
 * y[m][n], in ggml-cpu's x86 summation order (mode 0: ggml_vec_dot_f16/_f32, 4x8 lanes;
 * mode 1: tinyBLAS, 8 lanes, k % 8 == 0). F16 weights take fp16-rounded activations. */
int gsvk_op_fdot(const void * w, int wtype, int64_t n, int64_t k, const float * x, int64_t m,
                 float * y, int mode, void * stream);

/* QKV projection + decode attention of one layer in one launch (the decode path's fused kernel:
 * the work of src/gsv_ar.cpp:392 (QKV), :398-399 (K/V append) and :404 (flash_attn_ext) for one
 * new token per sequence). Input row b: LayerNorm((res + r) + ln_bias) with wb = [w; b] (r and
 * ln_bias may be NULL), quantised to Q8_0; wq/wd: sliced Q8_0 QKV weights [3*512][512]; bias
 * [3*512]. The new k, v are appended to the fp16 caches k, v [B][nh][lstride][32] at column *col
 * (device int) and attention runs over keys [kv_begin[b], *col]. out [B][512] fp32; oq/od
 * optional Q8_0 copy; ln_out optional LayerNorm output [B][512]. nh * 32 must be 512.
 * Fails (GSVK_ERR_ARG) for shapes whose rows the standalone attention would split. */
/* 1 when gsvk_op_qkv_attn accepts this shape (the standalone attention would not split rows). */
int gsvk_qkv_attn_supported(int B, int nh, int64_t max_keys);
int gsvk_op_qkv_attn(const int8_t * wq, const uint16_t * wd, const float * bias, const float * res,
                     const float * r, const float * ln_bias, const float * wb, int B, int nh,
                     uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                     const int32_t * col, float scale, float * out, int8_t * oq, float * od,
                     float * ln_out, void * stream);
/* The same launch with the attention in ggml-cpu's order (flash_attn_ext's sequential online
 * softmax, src/gsv_ar.cpp:404, with glibc's expf), bit for bit with the CPU reference: exact mode's
 * decode kernel (gsvk_model_set_exact). Any row length (the keys are taken in chunks of 384). */
int gsvk_op_qkv_attn_exact(const int8_t * wq, const uint16_t * wd, const float * bias, const float * res,
                           const float * r, const float * ln_bias, const float * wb, int B, int nh,
                           uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                           const int32_t * col, float scale, float * out, int8_t * oq, float * od,
                           float * ln_out, void * stream);

/* One call of the device sampler for B rows: gsv_logits_to_probs followed by gsv_sample with the
 * row's gsv_rng (src/gsv_sampler.cpp:8-89). Device memory: logits [B][V] (not modified);
 * hist [B][hist_stride] holding n_hist[b] tokens per row, of which the last <= 4096 are the
 * repetition-penalty window (both NULL = no history); rng [B] xorshift64* states, advanced by
 * V draws; tok_out [B]; probs_out [B][V] or NULL. ws: gsvk_sample_workspace_bytes(V) bytes of
 * device memory. V <= 2048. The call synchronises the stream. */
size_t gsvk_sample_workspace_bytes(int V);
int gsvk_op_sample(const float * logits, int B, int V, const int32_t * hist, int hist_stride,
                   const int32_t * n_hist, const gsvk_sampler_cfg * cfg, uint64_t * rng,
                   int32_t * tok_out, float * probs_out, void * ws, void * stream);

/* Single-query attention over a per-sequence fp16 KV cache (decode; ggml_flash_attn_ext with
 * one query row). q fp32 [B][nh][hd]; K/V fp16 [B][nh][lstride][hd]; valid keys of sequence b
 * are [kv_begin[b], kv_end[b]) (device int32 arrays). out fp32 [B][nh*hd] (head-major).
 * If oq/od are given the output is also quantised to Q8_0 (one block per head, hd == 32).
 * ws: device workspace of gsvk_attn_workspace_bytes() bytes. hd must be 32. */
size_t gsvk_attn_workspace_bytes(int B, int nh, int64_t max_keys);
int gsvk_op_attn_decode(const float * q, const uint16_t * k, const uint16_t * v, int B, int nh,
                        int hd, int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end,
                        int64_t max_keys, float scale, float * out, uint16_t * out_f16,
                        int8_t * oq, float * od, void * ws, void * stream);

/* gsvk_op_attn_decode without the ws argument, for callers that cannot allocate device memory
 * (code under graph capture, serving loops that forbid hipMalloc). No counterpart in the
 * reference. It allocates nothing: the split partials and merge counters live in a device array
 * the library holds on each GPU until the process ends (8 MiB, one per GPU). Shapes whose
 * gsvk_attn_workspace_bytes() exceed 8 MiB are rejected with GSVK_ERR_ARG. stream must belong to
 * the current device. Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams or threads) race and must be serialised by the caller. */
int gsvk_op_attn_decode_noalloc(const float * q, const uint16_t * k, const uint16_t * v, int B,
                                int nh, int hd, int64_t lstride, const int32_t * kv_begin,
                                const int32_t * kv_end, int64_t max_keys, float scale, float * out,
                                uint16_t * out_f16, int8_t * oq, float * od, void * stream);

/* Decode attention in ggml-cpu's order (ggml_compute_forward_flash_attn_ext_f16_one_chunk,
 * ggml/src/ggml-cpu/ops.cpp, as src/gsv_ar.cpp:412 calls it): for each (sequence b, head h) the
 * keys [kv_begin[b], kv_end[b]) of the fp16 caches k, v [B][nh][lstride][32] in order, score
 * dot(k, q) * scale in ggml_vec_dot_f32's lane order, the online softmax with glibc's expf,
 * out [B][nh*32] = acc / S; oq/od (both or neither) get the sliced Q8_0 copy. Same arguments as
 * gsvk_op_attn_decode without its split. */
int gsvk_op_attn_exact(const float * q, const uint16_t * k, const uint16_t * v, int B, int nh,
                       int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end, float scale,
                       float * out, int8_t * oq, float * od, void * stream);

/* y[i] = expf(x[i]) with the results of glibc's x86-64 expf, computed on the device (the
 * exponential of gsvk_op_attn_exact; replaces the libm call inside ggml's softmax). */
int gsvk_op_expf_exact(const float * x, int64_t n, float * y, void * stream);

/* The decode layer of up to 64 sequences in two launches (GSVK_DECODE_FUSED; d_model 512, 16
 * heads of 32, FFN 2048). Launch 1, per (head, sequence): the input row x = LayerNorm((res +
 * parts[0] + ... + parts[15]) + ln_bias) with ln_wb = [w; b] (parts [16][B][512]: the previous
 * layer's FFN2 partial rows), or, when res is NULL, emb[tok[b]] + alpha * pe[*pos + pos_add]
 * (row clamped into pe_rows); x stored to x_out [B][512]; q, k, v of the head with the QKV
 * weights wq/wd (sliced Q8_0 [1536][512]) + bqkv; k, v appended to the fp16 caches k, v
 * [B][16][lstride][32] at column *col; attention over [kv_begin[b], *col]; the head's output
 * quantised to one Q8_0 block times the out projection (woq/wod: Q8_0 [512][512] in the
 * matrix-core operand order of gsvk_op_q8_gemm_ex) gives the partial row p1[head][b][0:512].
 * Replaces the QKV projection, K/V append, flash_attn_ext and out projection of
 * src/gsv_ar.cpp:392-407; sum_h p1[h] is the out projection. */
int gsvk_op_dec_attn(int B, const float * res, const float * parts, const float * ln_bias,
                     const float * ln_wb, const float * emb, const float * pe, const int32_t * tok,
                     const int32_t * pos, int pos_add, float alpha, int vocab, int pe_rows,
                     float * x_out, const int8_t * wq, const uint16_t * wd, const float * bqkv,
                     uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                     const int32_t * col, float scale, const int8_t * woq, const uint16_t * wod,
                     float * p1, void * stream);
/* Launch 2, per (group of 128 hidden units, sequence): n1 = LayerNorm((res + p1[0] + ... +
 * p1[15]) + bo) with ln1_wb, stored to n1_out [B][512]; h = relu(W1 . n1 + b1) for the group's
 * units (w1q/w1d sliced Q8_0 [2048][512]), quantised to Q8_0; p2[group][b][0:512] = the FFN2
 * columns of the group (w2q/w2d: Q8_0 [512][2048] in the matrix-core operand order) times those
 * blocks. Replaces LN1, FFN1 + ReLU and FFN2 of src/gsv_ar.cpp:408-411; sum_g p2[g] is FFN2. */
int gsvk_op_dec_ffn(int B, const float * res, const float * p1, const float * bo, const float * ln1_wb,
                    float * n1_out, const int8_t * w1q, const uint16_t * w1d, const float * b1,
                    const int8_t * w2q, const uint16_t * w2d, float * p2, void * stream);

/* Prefill self-attention (the flash_attn_ext of src/gsv_ar.cpp:257 over all B*S rows, masks of
 * src/gsv_ar.cpp:215-223): qkv fp32 [B][S][3*nh*hd] (Q, K, V of head h at h*hd, D + h*hd,
 * 2*D + h*hd); pad device int32 [B]; query s of sequence b sees keys [pad[b], max_len) when
 * s < max_len, else [pad[b], s]. out fp32 [B][S][nh*hd]; oq/od (both or neither) its Q8_0 copy
 * (fp32 scales; the quants in the layout of the projection that reads them: sliced from the
 * lane-per-query kernel, natural order from the matrix-core kernel). path 0 picks the kernel the
 * prefill uses for B*S rows, 1 the lane-per-query kernel, 2 the matrix-core kernel, 3 the
 * matrix-core kernel with the weighted sum as one product of fp16 probabilities and fp16 values
 * (the prefill's fp16 mode, gsvk_model_set_prefill_f16; about 5e-4 of the output's scale), 4 the
 * matrix-core kernel as the decoder's prefill dispatches it (sequences longest first; a wave whose
 * 32 queries are all left-padding rows computes nothing and those rows are zero; the other rows
 * equal path 2's to the bit; it reads pad to the host and synchronises the stream). hd must be 32;
 * qkv and out 16-byte aligned. */
int gsvk_op_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                         int hd, float scale, int path, float * out, int8_t * oq, float * od,
                         void * stream);

/* ======================================================================================
 * 3. BERT text encoder (src/gsv_bert.{h,cpp}: chinese-roberta-wwm-ext-large, post-LN, the
 *    features the AR prefill takes as a request's `bert` input)
 * ====================================================================================== */

typedef struct gsvk_bert gsvk_bert;

typedef struct {
    int hidden, heads, inter, layers_used, vocab, max_pos;
    float ln_eps;
    int weight_type;   /* GGML type of the projection weights in the file (0 F32, 1 F16, 8 Q8_0) */
} gsvk_bert_info;

/* Load a gsv BERT GGUF (the tensor contract of src/gsv_bert.cpp:398-431, keys bert.* with the
 * reference's defaults) onto HIP device `device`. Projection weights may be F32, F16 or Q8_0;
 * all are held and multiplied in fp32. Only the first layers_used layers are loaded. Replaces
 * gsv_bert::load (src/gsv_bert.cpp:313-457). */
int gsvk_bert_load(const char * path, int device, int verbose, gsvk_bert ** out);
void gsvk_bert_free(gsvk_bert * m);
int gsvk_bert_get_info(const gsvk_bert * m, gsvk_bert_info * info);

/* Encoder over B sequences: sequence b is ids_flat[b*Tmax .. b*Tmax + lens[b]) (token ids with
 * [CLS]/[SEP], 1 <= lens[b] <= Tmax <= max_pos), positions 0..lens[b]-1, token type 0, attending
 * only to its own tokens. Output of layer n_layers (0 = the embedding LayerNorm; < 0 or past
 * layers_used = all used layers) as [hidden][lens[b]] row-major per sequence, the sequences back
 * to back in out (host, hidden * sum(lens) floats). Replaces gsv_bert::impl::run / run_g
 * (src/gsv_bert.cpp:97-233). */
int gsvk_bert_encode(gsvk_bert * m, int B, const int32_t * ids_flat, const int32_t * lens, int Tmax,
                     int n_layers, float * out);

#ifdef __cplusplus
}
#endif

#endif /* GSVK_H */

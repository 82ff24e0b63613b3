/*
 * gsv_oracle.c — CPU restatement of gsv.cpp's AR decoder path (see gsv_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker and the timed CPU baseline. Product code never uses it.
 *
 * Compiled with: gcc -O3 -mavx2 -mfma -mf16c -fopenmp -ffp-contract=off (the reference's
 * release flags, docs/build.md:66, plus explicit FMAs where GCC's GNU-mode contraction puts them).
 */
#include "gsv_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define QB 34

/* ============================================================================ fp16 */

uint16_t orc_f32_to_f16(float f) { return _cvtss_sh(f, 0); }          /* RNE, like F16C */
float    orc_f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

static inline uint16_t rd16(const uint8_t * p) { return (uint16_t) (p[0] | (p[1] << 8)); }

/* ============================================================================ Q8_0 */

/* ggml quantize_row_q8_0_ref: what the GGUF exporter (gguf-py / ggml_quantize_chunk) stores.
 * (gguf-py rounds with np.round-half-away too; the fixtures are generated with this rule.) */
void orc_q8_quantize_ref(const float * x, int64_t n, uint8_t * blocks) {
    const int64_t nb = n / QK;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(x[i * QK + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t * b = blocks + i * QB;
        const uint16_t dh = orc_f32_to_f16(d);
        b[0] = (uint8_t) (dh & 0xff);
        b[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < QK; j++) b[2 + j] = (uint8_t) (int8_t) roundf(x[i * QK + j] * id);
    }
}

/* ggml-cpu x86 quantize_row_q8_0 (AVX2 branch): amax via max of |x|, d = amax / 127 stored as
 * fp16, multiplier id = 127 / amax (0 for an all-zero block), round to nearest even. */
void orc_q8_quantize_x86(const float * x, int64_t n, uint8_t * blocks) {
    const int64_t nb = n / QK;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint8_t * b = blocks + i * QB;
        const uint16_t dh = orc_f32_to_f16(d);
        b[0] = (uint8_t) (dh & 0xff);
        b[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < QK; j++) b[2 + j] = (uint8_t) (int8_t) (int) nearbyintf(xb[j] * id);
    }
}

void orc_q8_dequant(const uint8_t * blocks, int64_t nblocks, float * out) {
    for (int64_t i = 0; i < nblocks; i++) {
        const uint8_t * b = blocks + i * QB;
        const float d = orc_f16_to_f32(rd16(b));
        for (int j = 0; j < QK; j++) out[i * QK + j] = d * (float) (int8_t) b[2 + j];
    }
}

/* hsum_float_8: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
static inline float hsum8(const float * a) {
    const float r0 = a[0] + a[4], r1 = a[1] + a[5], r2 = a[2] + a[6], r3 = a[3] + a[7];
    return (r0 + r2) + (r1 + r3);
}

float orc_q8_dot_scalar(const uint8_t * w, const uint8_t * x, int64_t nblocks) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t i = 0; i < nblocks; i++) {
        const uint8_t * wb = w + i * QB;
        const uint8_t * xb = x + i * QB;
        const float d = orc_f16_to_f32(rd16(wb)) * orc_f16_to_f32(rd16(xb));
        for (int l = 0; l < 8; l++) {
            int s = 0;
            for (int t = 0; t < 4; t++) s += (int) (int8_t) wb[2 + 4 * l + t] * (int) (int8_t) xb[2 + 4 * l + t];
            acc[l] = fmaf(d, (float) s, acc[l]);
        }
    }
    return hsum8(acc);
}

static inline float hsum_m256(__m256 x) {
    __m128 r = _mm_add_ps(_mm256_extractf128_ps(x, 1), _mm256_castps256_ps128(x));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}

float orc_q8_dot(const uint8_t * w, const uint8_t * x, int64_t nblocks) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int64_t i = 0; i < nblocks; i++) {
        const uint8_t * wb = w + i * QB;
        const uint8_t * xb = x + i * QB;
        const __m256 d = _mm256_set1_ps(orc_f16_to_f32(rd16(wb)) * orc_f16_to_f32(rd16(xb)));
        const __m256i qw = _mm256_loadu_si256((const __m256i *) (wb + 2));
        const __m256i qx = _mm256_loadu_si256((const __m256i *) (xb + 2));
        const __m256i aw = _mm256_sign_epi8(qw, qw);
        const __m256i sx = _mm256_sign_epi8(qx, qw);
        const __m256i p16 = _mm256_maddubs_epi16(aw, sx);
        const __m256 q = _mm256_cvtepi32_ps(_mm256_madd_epi16(p16, ones));
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum_m256(acc);
}

void orc_q8_matmul(const uint8_t * W, int64_t N, int64_t K, const float * X, int64_t M, float * Y,
                   int nthreads) {
    const int64_t nb = K / QK;
    const size_t rb = (size_t) nb * QB;
    uint8_t * Xq = (uint8_t *) malloc(rb * (size_t) M);
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t m = 0; m < M; m++) orc_q8_quantize_x86(X + m * K, K, Xq + m * rb);
    const int64_t NT = 16;
    const int64_t ntile = (N + NT - 1) / NT;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1) collapse(2)
    for (int64_t mt = 0; mt < (M + 63) / 64; mt++)
        for (int64_t t = 0; t < ntile; t++)
            for (int64_t m = mt * 64; m < M && m < mt * 64 + 64; m++)
                for (int64_t n = t * NT; n < N && n < t * NT + NT; n++)
                    Y[m * N + n] = orc_q8_dot(W + n * rb, Xq + m * rb, nb);
    free(Xq);
}

/* ============================================================================ F16 / F32 dots */

/* ggml_vec_dot_f16 / _f32, AVX path: sum[4] of 8 lanes over steps of 32, GGML_F32x8_REDUCE,
 * scalar leftovers (fused, as GCC contracts `sumf += x*y`). */
static float vdot_ggml(const float * x, const float * y, int64_t n) {
    float s[4][8];
    memset(s, 0, sizeof(s));
    const int64_t np = n & ~(int64_t) 31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) s[j][l] = fmaf(x[i + 8 * j + l], y[i + 8 * j + l], s[j][l]);
    for (int l = 0; l < 8; l++) {
        s[0][l] = s[0][l] + s[2][l];
        s[1][l] = s[1][l] + s[3][l];
    }
    for (int l = 0; l < 8; l++) s[0][l] = s[0][l] + s[1][l];
    float t0[4];
    for (int i = 0; i < 4; i++) t0[i] = s[0][i] + s[0][i + 4];
    float r = (t0[0] + t0[1]) + (t0[2] + t0[3]);
    for (int64_t i = np; i < n; i++) r = fmaf(x[i], y[i], r);
    return r;
}

/* tinyBLAS: one 8-lane accumulator over k in steps of 8 (k % 8 == 0), hsum */
static float vdot_tinyblas(const float * x, const float * y, int64_t n) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t i = 0; i < n; i += 8)
        for (int l = 0; l < 8; l++) a[l] = fmaf(x[i + l], y[i + l], a[l]);
    return hsum8(a);
}

void orc_f16_matmul(const uint16_t * W, int64_t N, int64_t K, const float * X, int64_t M,
                    float * Y, int mode, int nthreads) {
    float * Xr = (float *) malloc(sizeof(float) * (size_t) (M * K));
    for (int64_t i = 0; i < M * K; i++) Xr[i] = orc_f16_to_f32(orc_f32_to_f16(X[i]));
#pragma omp parallel num_threads(nthreads)
    {
        float * wr = (float *) malloc(sizeof(float) * (size_t) K);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; n++) {
            for (int64_t k = 0; k < K; k++) wr[k] = orc_f16_to_f32(W[n * K + k]);
            for (int64_t m = 0; m < M; m++)
                Y[m * N + n] = mode == 0 ? vdot_ggml(wr, Xr + m * K, K) : vdot_tinyblas(wr, Xr + m * K, K);
        }
        free(wr);
    }
    free(Xr);
}

void orc_f32_matmul(const float * W, int64_t N, int64_t K, const float * X, int64_t M, float * Y,
                    int mode, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t m = 0; m < M; m++)
            Y[m * N + n] = (mode == 0 || (K % 8) != 0) ? vdot_ggml(W + n * K, X + m * K, K)
                                                        : vdot_tinyblas(W + n * K, X + m * K, K);
}

/* ============================================================================ patch ops */

void orc_layernorm(const float * x, const float * r, const float * bias, const float * wb,
                   int64_t rows, int64_t n, float eps, float * y) {
    const float * w = wb;
    const float * b = wb + n;
    for (int64_t row = 0; row < rows; row++) {
        const float * xr = x + row * n;
        const float * rr = r ? r + row * n : NULL;
        float * yr = y + row * n;
        double sum = 0.0, sum2 = 0.0;
        for (int64_t i = 0; i < n; i++) {
            const float v = xr[i] + (rr ? rr[i] : 0.0f) + (bias ? bias[i] : 0.0f);
            sum += v;
            sum2 += (double) v * (double) v;
        }
        const float mean = (float) (sum / (double) n);
        const float var = fmaf(-mean, mean, (float) (sum2 / (double) n));
        const float inv = 1.0f / sqrtf(var + eps);
        for (int64_t i = 0; i < n; i++) {
            const float v = xr[i] + (rr ? rr[i] : 0.0f) + (bias ? bias[i] : 0.0f);
            yr[i] = fmaf((v - mean) * inv, w[i], b[i]);
        }
    }
}

void orc_add_act(const float * a, const float * b, int64_t n, int64_t ne0, int act, float * y) {
    for (int64_t i = 0; i < n; i++) {
        const float v = a[i] + b[i % ne0];
        float o = v;
        if (act == 1) o = v > 0.0f ? v : 0.0f;
        else if (act == 2) o = 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
        else if (act == 3) {
            const float sp = v > 20.0f ? v : log1pf(expf(v));
            o = v * tanhf(sp);
        }
        y[i] = o;
    }
}

/* ============================================================================ attention */

/* ggml_compute_forward_flash_attn_ext_f16_one_chunk with F32 K/V, one query row:
 * online softmax over the unmasked keys in order. kq dot = ggml_vec_dot_f32. */
void orc_attn_row(const float * q, const float * k, const float * v, int64_t kstride, int hd,
                  int64_t L, const uint8_t * mask_skip, float scale, float * out) {
    float S = 0.0f, M = -INFINITY;
    float acc[256];
    for (int d = 0; d < hd; d++) acc[d] = 0.0f;
    for (int64_t j = 0; j < L; j++) {
        if (mask_skip && mask_skip[j]) continue;
        const float * kj = k + j * kstride;
        const float * vj = v + j * kstride;
        float s = vdot_ggml(kj, q, hd);
        s = s * scale;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            for (int d = 0; d < hd; d++) acc[d] = acc[d] * ms;
        } else {
            vs = expf(s - M);
        }
        for (int d = 0; d < hd; d++) acc[d] = fmaf(vj[d], vs, acc[d]);
        S = fmaf(S, ms, vs);
    }
    const float Sinv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int d = 0; d < hd; d++) out[d] = acc[d] * Sinv;
}

void orc_expf_n(const float * x, int64_t n, float * y) {
    for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

void orc_attn_decode_f16(const float * q, const uint16_t * k, const uint16_t * v, int B, int nh,
                         int hd, int64_t lstride, const int32_t * kv_begin,
                         const int32_t * kv_end, float scale, float * out, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1) collapse(2)
    for (int b = 0; b < B; b++)
        for (int h = 0; h < nh; h++) {
            const int64_t bh = (int64_t) b * nh + h;
            const int beg = kv_begin[b] < 0 ? 0 : kv_begin[b];
            const int end = kv_end[b] > lstride ? (int) lstride : kv_end[b];
            const int64_t L = end > beg ? end - beg : 0;
            float * kf = (float *) malloc(sizeof(float) * (size_t) (L * hd + 1));
            float * vf = (float *) malloc(sizeof(float) * (size_t) (L * hd + 1));
            for (int64_t j = 0; j < L; j++)
                for (int d = 0; d < hd; d++) {
                    kf[j * hd + d] = orc_f16_to_f32(k[(bh * lstride + beg + j) * hd + d]);
                    vf[j * hd + d] = orc_f16_to_f32(v[(bh * lstride + beg + j) * hd + d]);
                }
            orc_attn_row(q + bh * hd, kf, vf, hd, hd, L, NULL, scale, out + bh * hd);
            free(kf);
            free(vf);
        }
}

/* ============================================================================ sampler */

typedef struct { float v; int i; } vi_t;

static int cmp_desc_stable(const void * a, const void * b) {
    const vi_t * x = (const vi_t *) a;
    const vi_t * y = (const vi_t *) b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : (x->i > y->i);
}

static int cmp_float_desc(const void * a, const void * b) {
    const float x = *(const float *) a, y = *(const float *) b;
    return x > y ? -1 : (x < y ? 1 : 0);
}

void orc_logits_to_probs(int top_k, float top_p, float temperature, float rep, float * logits,
                         int V, const int32_t * prev, int n_prev, float * probs) {
    /* 1) repetition penalty, once per occurrence */
    if (prev != NULL && n_prev > 0 && rep != 1.0f) {
        for (int i = 0; i < n_prev; i++) {
            const int t = prev[i];
            if (t < 0 || t >= V) continue;
            const float s = logits[t];
            logits[t] = (s < 0.0f) ? s * rep : s / rep;
        }
    }
    /* 2) top-p over a stable descending order (ties keep index order) */
    if (top_p < 1.0f) {
        vi_t * a = (vi_t *) malloc(sizeof(vi_t) * (size_t) V);
        for (int i = 0; i < V; i++) { a[i].v = logits[i]; a[i].i = i; }
        qsort(a, (size_t) V, sizeof(vi_t), cmp_desc_stable);
        const float mx = logits[a[0].i];
        float sum = 0.0f;
        for (int k = 0; k < V; k++) sum += expf(logits[a[k].i] - mx);
        const float inv_sum = 1.0f / sum;
        float cum = 0.0f;
        for (int k = 0; k < V; k++) {
            cum = fmaf(expf(logits[a[k].i] - mx), inv_sum, cum);
            if (k > 0 && cum > top_p) logits[a[k].i] = -INFINITY;
        }
        free(a);
    }
    /* 3) temperature */
    const float t = temperature > 1e-5f ? temperature : 1e-5f;
    for (int i = 0; i < V; i++) logits[i] /= t;
    /* 4) top-k: pivot = k-th largest (with multiplicity), keep >= pivot */
    if (top_k > 0 && top_k < V) {
        float * tmp = (float *) malloc(sizeof(float) * (size_t) V);
        memcpy(tmp, logits, sizeof(float) * (size_t) V);
        qsort(tmp, (size_t) V, sizeof(float), cmp_float_desc);
        const float pivot = tmp[top_k - 1];
        for (int i = 0; i < V; i++)
            if (logits[i] < pivot) logits[i] = -INFINITY;
        free(tmp);
    }
    /* 5) softmax, fp32 accumulation in index order */
    float mx = -INFINITY;
    for (int i = 0; i < V; i++) mx = fmaxf(mx, logits[i]);
    float sum = 0.0f;
    for (int i = 0; i < V; i++) {
        probs[i] = (logits[i] == -INFINITY) ? 0.0f : expf(logits[i] - mx);
        sum += probs[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < V; i++) probs[i] *= inv;
}

uint64_t orc_rng_next(uint64_t * state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    return s * 0x2545F4914F6CDD1Dull;
}

float orc_rng_exponential(uint64_t * state) {
    const float u = (float) ((double) (orc_rng_next(state) >> 40) * (1.0 / 16777216.0));
    return -logf(1.0f - u);
}

/* n draws of orc_rng_exponential in order (test helper: the q values of a run of sampling steps) */
void orc_rng_exponential_n(uint64_t * state, int64_t n, float * out) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_rng_exponential(state);
}

int orc_argmax_probs_over_q(const float * probs, const float * q, int V) {
    int best = 0;
    float bv = -INFINITY;
    for (int i = 0; i < V; i++) {
        const float v = (probs[i] > 0.0f) ? probs[i] / q[i] : 0.0f;
        if (v > bv) { bv = v; best = i; }
    }
    return best;
}

int orc_sample(const float * probs, int V, uint64_t * state) {
    float * q = (float *) malloc(sizeof(float) * (size_t) V);
    for (int i = 0; i < V; i++) q[i] = orc_rng_exponential(state);
    const int r = orc_argmax_probs_over_q(probs, q, V);
    free(q);
    return r;
}

/* ============================================================================ PE */

void orc_pe_table(int D, int npos, float * out) {
    for (int pos = 0; pos < npos; pos++)
        for (int i = 0; i < D; i += 2) {
            const float div = expf((float) i * -(logf(10000.0f) / (float) D));
            out[(size_t) pos * D + i] = sinf((float) pos * div);
            out[(size_t) pos * D + i + 1] = cosf((float) pos * div);
        }
}

/* ============================================================================ GGUF */

enum { GG_U8 = 0, GG_I8, GG_U16, GG_I16, GG_U32, GG_I32, GG_F32, GG_BOOL, GG_STR, GG_ARR, GG_U64,
       GG_I64, GG_F64 };

typedef struct {
    char name[96];
    int nd;
    int64_t ne[4];
    int type;
    uint64_t off;
} gg_tensor;

typedef struct {
    uint8_t * buf;
    size_t size, pos;
    int bad;
} rd_t;

static void rd_bytes(rd_t * r, void * dst, size_t n) {
    if (r->bad || r->pos + n > r->size) { r->bad = 1; memset(dst, 0, n); return; }
    memcpy(dst, r->buf + r->pos, n);
    r->pos += n;
}
static uint64_t rd_u64(rd_t * r) { uint64_t v; rd_bytes(r, &v, 8); return v; }
static uint32_t rd_u32(rd_t * r) { uint32_t v; rd_bytes(r, &v, 4); return v; }

static size_t gg_scalar_size(int t) {
    switch (t) {
        case GG_U8: case GG_I8: case GG_BOOL: return 1;
        case GG_U16: case GG_I16: return 2;
        case GG_U32: case GG_I32: case GG_F32: return 4;
        case GG_U64: case GG_I64: case GG_F64: return 8;
        default: return 0;
    }
}

static void rd_skip_value(rd_t * r, int t) {
    if (t == GG_STR) { const uint64_t n = rd_u64(r); if (r->pos + n > r->size) r->bad = 1; else r->pos += n; return; }
    if (t == GG_ARR) {
        const int et = (int) rd_u32(r);
        const uint64_t n = rd_u64(r);
        for (uint64_t i = 0; i < n && !r->bad; i++) rd_skip_value(r, et);
        return;
    }
    const size_t s = gg_scalar_size(t);
    if (s == 0 || r->pos + s > r->size) { r->bad = 1; return; }
    r->pos += s;
}

static size_t gg_nbytes(const gg_tensor * t) {
    int64_t n = 1;
    for (int i = 0; i < t->nd; i++) n *= t->ne[i];
    if (t->type == 0) return (size_t) n * 4;
    if (t->type == 1) return (size_t) n * 2;
    if (t->type == 8) return (size_t) (n / QK) * QB;
    return 0;
}

typedef struct {
    const void * w;       /* [N][K] rows: Q8_0 blocks, F16 or F32 */
    int type;             /* 8 Q8_0, 1 F16, 0 F32 */
    const float * b;
} lin_t;

typedef struct {
    lin_t qkv, out, f1, f2;
    float * ln1, * ln2;   /* [w;b] */
} layer_t;

struct orc_model {
    int D, NH, HD, NL, V, EOS, PH, BERT, FFN, head_type;
    uint8_t * file;
    size_t fsize;
    const void * head;
    const float * text_emb, * audio_emb;
    float * bert_aug;     /* [D][BERT+1] */
    float text_alpha, audio_alpha;
    layer_t * L;
    float * pe;           /* [4096][D] */
};

#define PE_MAX 4096

static gg_tensor * gg_find(gg_tensor * ts, int n, const char * name) {
    for (int i = 0; i < n; i++)
        if (strcmp(ts[i].name, name) == 0) return &ts[i];
    return NULL;
}

orc_model * orc_model_load(const char * path, char * err, int errlen) {
#define FAIL(...) do { snprintf(err, (size_t) errlen, __VA_ARGS__); goto fail; } while (0)
    orc_model * m = (orc_model *) calloc(1, sizeof(orc_model));
    gg_tensor * ts = NULL;
    FILE * f = fopen(path, "rb");
    if (!f) { snprintf(err, (size_t) errlen, "cannot open %s", path); free(m); return NULL; }
    fseek(f, 0, SEEK_END);
    m->fsize = (size_t) ftell(f);
    fseek(f, 0, SEEK_SET);
    m->file = (uint8_t *) malloc(m->fsize);
    if (fread(m->file, 1, m->fsize, f) != m->fsize) { fclose(f); FAIL("short read"); }
    fclose(f);
    {
        rd_t r = {m->file, m->fsize, 0, 0};
        uint32_t magic = rd_u32(&r);
        if (magic != 0x46554747u) FAIL("not a GGUF file");
        const uint32_t ver = rd_u32(&r);
        if (ver < 2) FAIL("GGUF version %u unsupported", ver);
        const uint64_t nt = rd_u64(&r), nkv = rd_u64(&r);
        uint32_t align = 32;
        m->D = 512; m->NH = 16; m->NL = 24; m->V = 1025; m->PH = 732; m->EOS = 1024;
        for (uint64_t i = 0; i < nkv && !r.bad; i++) {
            const uint64_t kl = rd_u64(&r);
            char key[256] = {0};
            if (kl >= sizeof(key)) { r.bad = 1; break; }
            rd_bytes(&r, key, kl);
            const int t = (int) rd_u32(&r);
            if (t == GG_U32 || t == GG_I32) {
                const uint32_t v = rd_u32(&r);
                if (!strcmp(key, "ar.hidden_dim")) m->D = (int) v;
                else if (!strcmp(key, "ar.head")) m->NH = (int) v;
                else if (!strcmp(key, "ar.n_layer")) m->NL = (int) v;
                else if (!strcmp(key, "ar.vocab_size")) m->V = (int) v;
                else if (!strcmp(key, "ar.phoneme_vocab_size")) m->PH = (int) v;
                else if (!strcmp(key, "ar.eos")) m->EOS = (int) v;
                else if (!strcmp(key, "general.alignment")) align = v;
            } else {
                rd_skip_value(&r, t);
            }
        }
        ts = (gg_tensor *) calloc(nt ? nt : 1, sizeof(gg_tensor));
        for (uint64_t i = 0; i < nt && !r.bad; i++) {
            const uint64_t nl = rd_u64(&r);
            if (nl >= sizeof(ts[i].name)) { r.bad = 1; break; }
            rd_bytes(&r, ts[i].name, nl);
            ts[i].nd = (int) rd_u32(&r);
            if (ts[i].nd < 1 || ts[i].nd > 4) { r.bad = 1; break; }
            for (int d = 0; d < 4; d++) ts[i].ne[d] = 1;
            for (int d = 0; d < ts[i].nd; d++) ts[i].ne[d] = (int64_t) rd_u64(&r);
            ts[i].type = (int) rd_u32(&r);
            ts[i].off = rd_u64(&r);
        }
        if (r.bad) FAIL("truncated GGUF header");
        const size_t data = (r.pos + align - 1) / align * align;
        for (uint64_t i = 0; i < nt; i++) {
            const size_t nb = gg_nbytes(&ts[i]);
            if (nb == 0 || data + ts[i].off + nb > m->fsize) FAIL("tensor %s out of range or unsupported type %d", ts[i].name, ts[i].type);
            ts[i].off += data;
        }
        m->HD = m->D / m->NH;
        m->BERT = 1024;
        const int n = (int) nt;
        char nm[96];
        m->L = (layer_t *) calloc((size_t) m->NL, sizeof(layer_t));
        for (int li = 0; li < m->NL; li++) {
            layer_t * L = &m->L[li];
#define GETW(lin, suffix) do { snprintf(nm, sizeof nm, "transformer.block%d." suffix, li); gg_tensor * t = gg_find(ts, n, nm); \
            if (!t) FAIL("missing tensor %s", nm); if (t->type != 8 && t->type != 1 && t->type != 0) \
            FAIL("%s: projection weights must be Q8_0, F16 or F32", nm); (lin).w = m->file + t->off; (lin).type = t->type; } while (0)
#define GETF(field, suffix) do { snprintf(nm, sizeof nm, "transformer.block%d." suffix, li); gg_tensor * t = gg_find(ts, n, nm); \
            if (!t) FAIL("missing tensor %s", nm); if (t->type != 0) FAIL("%s must be F32", nm); field = (const float *) (m->file + t->off); } while (0)
            const float * n1w, * n1b, * n2w, * n2b;
            GETW(L->qkv, "qkv_w"); GETF(L->qkv.b, "qkv_b");
            GETW(L->out, "out_w"); GETF(L->out.b, "out_b");
            GETW(L->f1, "ffn1_w"); GETF(L->f1.b, "ffn1_b");
            GETW(L->f2, "ffn2_w"); GETF(L->f2.b, "ffn2_b");
            GETF(n1w, "norm1_w"); GETF(n1b, "norm1_b"); GETF(n2w, "norm2_w"); GETF(n2b, "norm2_b");
            if (li == 0) {
                snprintf(nm, sizeof nm, "transformer.block0.ffn1_w");
                m->FFN = (int) gg_find(ts, n, nm)->ne[1];
            }
            L->ln1 = (float *) malloc(sizeof(float) * 2 * (size_t) m->D);
            L->ln2 = (float *) malloc(sizeof(float) * 2 * (size_t) m->D);
            memcpy(L->ln1, n1w, sizeof(float) * (size_t) m->D);
            memcpy(L->ln1 + m->D, n1b, sizeof(float) * (size_t) m->D);
            memcpy(L->ln2, n2w, sizeof(float) * (size_t) m->D);
            memcpy(L->ln2 + m->D, n2b, sizeof(float) * (size_t) m->D);
#undef GETW
#undef GETF
        }
        gg_tensor * t;
        if (!(t = gg_find(ts, n, "ar.predict"))) FAIL("missing ar.predict");
        if (t->type != 0 && t->type != 1 && t->type != 8) FAIL("ar.predict type %d unsupported", t->type);
        m->head_type = t->type;
        m->head = m->file + t->off;
        if (!(t = gg_find(ts, n, "ar.text_emb")) || t->type != 0) FAIL("ar.text_emb missing or not F32");
        m->text_emb = (const float *) (m->file + t->off);
        if (!(t = gg_find(ts, n, "ar.audio_emb")) || t->type != 0) FAIL("ar.audio_emb missing or not F32");
        m->audio_emb = (const float *) (m->file + t->off);
        gg_tensor * bp = gg_find(ts, n, "ar.bert_proj");
        gg_tensor * bb = gg_find(ts, n, "ar.bert_proj_b");
        if (!bp || bp->type != 0 || !bb || bb->type != 0) FAIL("ar.bert_proj(_b) missing or not F32");
        m->bert_aug = (float *) malloc(sizeof(float) * (size_t) m->D * (m->BERT + 1));
        for (int d = 0; d < m->D; d++) {
            memcpy(m->bert_aug + (size_t) d * (m->BERT + 1), (const float *) (m->file + bp->off) + (size_t) d * m->BERT,
                   sizeof(float) * (size_t) m->BERT);
            m->bert_aug[(size_t) d * (m->BERT + 1) + m->BERT] = ((const float *) (m->file + bb->off))[d];
        }
        if (!(t = gg_find(ts, n, "ar.text_pe_alpha"))) FAIL("missing ar.text_pe_alpha");
        m->text_alpha = *(const float *) (m->file + t->off);
        if (!(t = gg_find(ts, n, "ar.audio_pe_alpha"))) FAIL("missing ar.audio_pe_alpha");
        m->audio_alpha = *(const float *) (m->file + t->off);
        m->pe = (float *) malloc(sizeof(float) * (size_t) PE_MAX * m->D);
        orc_pe_table(m->D, PE_MAX, m->pe);
    }
    free(ts);
    return m;
fail:
    free(ts);
    orc_model_free(m);
    return NULL;
#undef FAIL
}

void orc_model_free(orc_model * m) {
    if (!m) return;
    if (m->L) {
        for (int i = 0; i < m->NL; i++) { free(m->L[i].ln1); free(m->L[i].ln2); }
        free(m->L);
    }
    free(m->bert_aug);
    free(m->pe);
    free(m->file);
    free(m);
}

void orc_model_info(const orc_model * m, int32_t * info) {
    info[0] = m->D; info[1] = m->NH; info[2] = m->HD; info[3] = m->NL; info[4] = m->V;
    info[5] = m->EOS; info[6] = m->PH; info[7] = m->BERT; info[8] = m->FFN; info[9] = m->head_type;
}

/* ============================================================================ forward */

typedef struct {
    int B, Lmax;    /* Lmax+1 slots per (b, h) */
    float * k, * v; /* [NL][B][NH][Lmax+1][HD] */
} cache_t;

static inline size_t cidx(const orc_model * m, const cache_t * c, int li, int b, int h, int l) {
    return ((((size_t) li * c->B + b) * m->NH + h) * (size_t) (c->Lmax + 1) + l) * m->HD;
}

static void head_logits(const orc_model * m, const float * x, int M, int mode, float * out, int nt) {
    if (m->head_type == 1) orc_f16_matmul((const uint16_t *) m->head, m->V, m->D, x, M, out, mode, nt);
    else if (m->head_type == 0) orc_f32_matmul((const float *) m->head, m->V, m->D, x, M, out, mode, nt);
    else orc_q8_matmul((const uint8_t *) m->head, m->V, m->D, x, M, out, nt);
}

/* y[M][N] = W[N][K] . x[M][K], ggml_mul_mat of a projection (src/gsv_ar.cpp:244, :260-263, :392,
 * :407-411): Q8_0 weights take the x86-quantised activations and the int8 block dot; F16 and F32
 * weights ggml_vec_dot_f16 / _f32 (mode 0) or llamafile's tinyBLAS (mode 1, the prefill's
 * multi-column products, as for the head), F16 with the activations rounded to fp16 (ggml's
 * vec_dot_type). */
static void proj(const lin_t * l, int64_t N, int64_t K, const float * x, int64_t M, float * y, int mode, int nt) {
    if (l->type == 8) orc_q8_matmul((const uint8_t *) l->w, N, K, x, M, y, nt);
    else if (l->type == 1) orc_f16_matmul((const uint16_t *) l->w, N, K, x, M, y, mode, nt);
    else orc_f32_matmul((const float *) l->w, N, K, x, M, y, mode, nt);
}

/* one transformer layer over R rows after attention has produced attn[R][D] */
static void layer_tail(const orc_model * m, const layer_t * L, float * cur, const float * attn,
                       int64_t R, int mode, int nt, float * o, float * n1, float * h, float * h2) {
    const int D = m->D, F = m->FFN;
    proj(&L->out, D, D, attn, R, o, mode, nt);
    orc_layernorm(cur, o, L->out.b, L->ln1, R, D, 1e-5f, n1);
    proj(&L->f1, F, D, n1, R, h, mode, nt);
    orc_add_act(h, L->f1.b, R * F, F, 1, h);
    proj(&L->f2, D, F, h, R, h2, mode, nt);
    orc_layernorm(n1, h2, L->f2.b, L->ln2, R, D, 1e-5f, cur);
}

static inline float kv_round(float x, unsigned flags) {
    return (flags & ORC_KV_F16) ? orc_f16_to_f32(orc_f32_to_f16(x)) : x;
}

/* prefill (run_first, src/gsv_ar.cpp:228-293). Returns last-position logits [B][V]. */
/* prefill self-attention (src/gsv_ar.cpp:215-223 masks, :257 flash_attn_ext): qkv [B][S][3*D]
 * (Q, K, V of head h at h*hd, D + h*hd, 2*D + h*hd); query qi of sequence b sees keys
 * [pad[b], max_len) when qi < max_len, else [pad[b], qi]. out [B][S][D]. */
void orc_attn_prefill(const float * qkv, int B, int S, int max_len, const int32_t * pad, int nh,
                      int hd, float scale, float * out, int nt) {
    const int D = nh * hd;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) collapse(2)
    for (int b = 0; b < B; b++)
        for (int hh = 0; hh < nh; hh++) {
            uint8_t * skip = (uint8_t *) malloc((size_t) S);
            for (int qi = 0; qi < S; qi++) {
                for (int k = 0; k < S; k++) {
                    int mk;
                    if (k < pad[b]) mk = 1;
                    else if (qi < max_len) mk = (k >= max_len);
                    else mk = (k > qi);
                    skip[k] = (uint8_t) mk;
                }
                const float * base = qkv + (size_t) b * S * 3 * D;
                orc_attn_row(base + (size_t) qi * 3 * D + hh * hd, base + D + hh * hd,
                             base + 2 * D + hh * hd, 3 * D, hd, S, skip, scale,
                             out + ((size_t) b * S + qi) * D + hh * hd);
            }
            free(skip);
        }
}

static void prefill(const orc_model * m, const orc_request * reqs, int B, int S, int max_len,
                    cache_t * c, unsigned flags, int nt, float * logits) {
    const int D = m->D, NH = m->NH, HD = m->HD, F = m->FFN, BD = m->BERT;
    const int P = reqs[0].n_prompt;
    const int64_t R = (int64_t) B * S;
    float * cur = (float *) calloc((size_t) R * D, sizeof(float));
    /* build_inputs (:186-225) + in-graph BERT projection (:241) */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int b = 0; b < B; b++) {
        const int T = reqs[b].n_phones;
        const int pad = max_len - T;
        float * feat = (float *) malloc(sizeof(float) * (size_t) (BD + 1));
        for (int t = 0; t < T; t++) {
            float * dst = cur + ((size_t) b * S + pad + t) * D;
            const float * tok = m->text_emb + (size_t) reqs[b].phones[t] * D;
            for (int d = 0; d < D; d++) dst[d] = fmaf(m->text_alpha, m->pe[(size_t) t * D + d], tok[d]);
            for (int k = 0; k < BD; k++) feat[k] = reqs[b].bert ? reqs[b].bert[(size_t) k * T + t] : 0.0f;
            feat[BD] = 1.0f;
            for (int d = 0; d < D; d++) dst[d] = dst[d] + vdot_ggml(m->bert_aug + (size_t) d * (BD + 1), feat, BD + 1);
        }
        for (int t = 0; t < P; t++) {
            float * dst = cur + ((size_t) b * S + max_len + t) * D;
            const float * e = m->audio_emb + (size_t) reqs[b].prompt[t] * D;
            for (int d = 0; d < D; d++) dst[d] = fmaf(m->audio_alpha, m->pe[(size_t) t * D + d], e[d]);
        }
        free(feat);
    }
    float * qkv = (float *) malloc(sizeof(float) * (size_t) R * 3 * D);
    float * attn = (float *) malloc(sizeof(float) * (size_t) R * D);
    float * o = (float *) malloc(sizeof(float) * (size_t) R * D);
    float * n1 = (float *) malloc(sizeof(float) * (size_t) R * D);
    float * h = (float *) malloc(sizeof(float) * (size_t) R * F);
    float * h2 = (float *) malloc(sizeof(float) * (size_t) R * D);
    const float scale = 1.0f / sqrtf((float) HD);
    for (int li = 0; li < m->NL; li++) {
        const layer_t * L = &m->L[li];
        proj(&L->qkv, 3 * D, D, cur, R, qkv, S >= 2 ? 1 : 0, nt);
        for (int64_t r = 0; r < R; r++)
            for (int i = 0; i < 3 * D; i++) qkv[r * 3 * D + i] = qkv[r * 3 * D + i] + L->qkv.b[i];
        {
            int32_t * pads = (int32_t *) malloc(sizeof(int32_t) * (size_t) B);
            for (int b = 0; b < B; b++) pads[b] = max_len - reqs[b].n_phones;
            orc_attn_prefill(qkv, B, S, max_len, pads, NH, HD, scale, attn, nt);
            free(pads);
        }
        /* KV cache copy of all S positions (:271-275) */
        for (int b = 0; b < B; b++)
            for (int s = 0; s < S; s++)
                for (int hh = 0; hh < NH; hh++)
                    for (int d = 0; d < HD; d++) {
                        const float * row = qkv + ((size_t) b * S + s) * 3 * D;
                        c->k[cidx(m, c, li, b, hh, s) + d] = kv_round(row[D + hh * HD + d], flags);
                        c->v[cidx(m, c, li, b, hh, s) + d] = kv_round(row[2 * D + hh * HD + d], flags);
                    }
        layer_tail(m, L, cur, attn, R, S >= 2 ? 1 : 0, nt, o, n1, h, h2);
    }
    /* logits of the last position (:266-269); tinyBLAS order for >= 2 columns */
    float * last = (float *) malloc(sizeof(float) * (size_t) B * D);
    for (int b = 0; b < B; b++) memcpy(last + (size_t) b * D, cur + ((size_t) b * S + S - 1) * D, sizeof(float) * (size_t) D);
    head_logits(m, last, B, S >= 2 ? 1 : 0, logits, nt);
    free(last); free(cur); free(qkv); free(attn); free(o); free(n1); free(h); free(h2);
}

/* decode step (run_decode, src/gsv_ar.cpp:296-358): x_in [B][D] at cache column len */
static void decode(const orc_model * m, const float * x_in, int B, const int * pad, int len,
                   cache_t * c, unsigned flags, int nt, float * logits) {
    const int D = m->D, NH = m->NH, HD = m->HD, F = m->FFN;
    float * cur = (float *) malloc(sizeof(float) * (size_t) B * D);
    memcpy(cur, x_in, sizeof(float) * (size_t) B * D);
    float * qkv = (float *) malloc(sizeof(float) * (size_t) B * 3 * D);
    float * attn = (float *) malloc(sizeof(float) * (size_t) B * D);
    float * o = (float *) malloc(sizeof(float) * (size_t) B * D);
    float * n1 = (float *) malloc(sizeof(float) * (size_t) B * D);
    float * h = (float *) malloc(sizeof(float) * (size_t) B * F);
    float * h2 = (float *) malloc(sizeof(float) * (size_t) B * D);
    const float scale = 1.0f / sqrtf((float) HD);
    for (int li = 0; li < m->NL; li++) {
        const layer_t * L = &m->L[li];
        proj(&L->qkv, 3 * D, D, cur, B, qkv, 0, nt);
        for (int64_t r = 0; r < B; r++)
            for (int i = 0; i < 3 * D; i++) qkv[r * 3 * D + i] = qkv[r * 3 * D + i] + L->qkv.b[i];
        for (int b = 0; b < B; b++)
            for (int hh = 0; hh < NH; hh++)
                for (int d = 0; d < HD; d++) {
                    c->k[cidx(m, c, li, b, hh, len) + d] = kv_round(qkv[(size_t) b * 3 * D + D + hh * HD + d], flags);
                    c->v[cidx(m, c, li, b, hh, len) + d] = kv_round(qkv[(size_t) b * 3 * D + 2 * D + hh * HD + d], flags);
                }
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) collapse(2)
        for (int b = 0; b < B; b++)
            for (int hh = 0; hh < NH; hh++) {
                const int L0 = pad[b] < len + 1 ? pad[b] : len + 1;
                orc_attn_row(qkv + (size_t) b * 3 * D + hh * HD, c->k + cidx(m, c, li, b, hh, L0),
                             c->v + cidx(m, c, li, b, hh, L0), HD, HD, len + 1 - L0, NULL, scale,
                             attn + (size_t) b * D + hh * HD);
            }
        layer_tail(m, L, cur, attn, B, 0, nt, o, n1, h, h2);
    }
    head_logits(m, cur, B, 0, logits, nt);
    free(cur); free(qkv); free(attn); free(o); free(n1); free(h); free(h2);
}

static int check_reqs(const orc_model * m, const orc_request * reqs, int B, int * S, int * max_len) {
    *max_len = 0;
    for (int b = 0; b < B; b++) {
        if (reqs[b].n_phones < 0 || reqs[b].n_prompt != reqs[0].n_prompt) return -1;
        for (int t = 0; t < reqs[b].n_phones; t++) if (reqs[b].phones[t] < 0 || reqs[b].phones[t] >= m->PH) return -2;
        for (int t = 0; t < reqs[b].n_prompt; t++) if (reqs[b].prompt[t] < 0 || reqs[b].prompt[t] >= m->V) return -2;
        if (reqs[b].n_phones > *max_len) *max_len = reqs[b].n_phones;
    }
    *S = *max_len + reqs[0].n_prompt;
    if (*max_len > PE_MAX || reqs[0].n_prompt > PE_MAX) return -3;
    return 0;
}

int orc_prefill_kv(orc_model * m, const orc_request * reqs, int B, unsigned flags, int nthreads,
                   int layer, float * k_out, float * v_out, float * logits, int32_t * S_out) {
    int S, max_len;
    if (B <= 0 || layer < 0 || layer >= m->NL || check_reqs(m, reqs, B, &S, &max_len) != 0) return -1;
    cache_t c = {B, S + 8, NULL, NULL};
    const size_t n = (size_t) m->NL * B * m->NH * (size_t) (c.Lmax + 1) * m->HD;
    c.k = (float *) calloc(n, sizeof(float));
    c.v = (float *) calloc(n, sizeof(float));
    prefill(m, reqs, B, S, max_len, &c, flags, nthreads, logits);
    for (int b = 0; b < B; b++)
        for (int h = 0; h < m->NH; h++)
            for (int s = 0; s < S; s++)
                for (int d = 0; d < m->HD; d++) {
                    const size_t o = (((size_t) b * m->NH + h) * S + s) * m->HD + d;
                    if (k_out) k_out[o] = c.k[cidx(m, &c, layer, b, h, s) + d];
                    if (v_out) v_out[o] = c.v[cidx(m, &c, layer, b, h, s) + d];
                }
    if (S_out) *S_out = S;
    free(c.k);
    free(c.v);
    return 0;
}

int orc_first_logits(orc_model * m, const orc_request * reqs, int B, unsigned flags, int nthreads,
                     float * logits) {
    int S, max_len;
    if (B <= 0 || check_reqs(m, reqs, B, &S, &max_len) != 0) return -1;
    cache_t c = {B, S + 8, NULL, NULL};
    const size_t n = (size_t) m->NL * B * m->NH * (size_t) (c.Lmax + 1) * m->HD;
    c.k = (float *) calloc(n, sizeof(float));
    c.v = (float *) calloc(n, sizeof(float));
    prefill(m, reqs, B, S, max_len, &c, flags, nthreads, logits);
    free(c.k);
    free(c.v);
    return 0;
}

/* generate (src/gsv_ar.cpp:719-824) */
int orc_generate(orc_model * m, const orc_request * reqs, int B, int top_k, float top_p,
                 float temperature, float rep, uint64_t seed_base, int early_stop_num,
                 int max_steps, const int32_t * oracle, int n_oracle, const uint64_t * seeds,
                 unsigned flags, int nthreads, orc_gen_out * out) {
    int S, max_len;
    if (B <= 0 || check_reqs(m, reqs, B, &S, &max_len) != 0) return -1;
    const int P = reqs[0].n_prompt;
    const int V = m->V, D = m->D;
    if (P + max_steps > PE_MAX) return -3;
    if (out->tok_stride < P + max_steps) return -4;
    int * pad = (int *) malloc(sizeof(int) * (size_t) B);
    for (int b = 0; b < B; b++) pad[b] = max_len - reqs[b].n_phones;
    cache_t c = {B, S + max_steps + 8, NULL, NULL};
    const size_t n = (size_t) m->NL * B * m->NH * (size_t) (c.Lmax + 1) * m->HD;
    c.k = (float *) calloc(n, sizeof(float));
    c.v = (float *) calloc(n, sizeof(float));
    if (!c.k || !c.v) { free(c.k); free(c.v); free(pad); return -5; }
    float * lg = (float *) malloc(sizeof(float) * (size_t) B * V);
    const double t0 = omp_get_wtime();
    prefill(m, reqs, B, S, max_len, &c, flags, nthreads, lg);
    const double t1 = omp_get_wtime();
    out->prefill_ms = (t1 - t0) * 1e3;

    int32_t * y = out->tokens;               /* y[b] lives in its output row */
    int * ny = (int *) malloc(sizeof(int) * (size_t) B);
    int * idx_list = (int *) malloc(sizeof(int) * (size_t) B);
    uint64_t * rng = (uint64_t *) malloc(sizeof(uint64_t) * (size_t) B);
    for (int b = 0; b < B; b++) {
        memcpy(y + (size_t) b * out->tok_stride, reqs[b].prompt, sizeof(int32_t) * (size_t) P);
        ny[b] = P;
        idx_list[b] = -1;
        const uint64_t sd = seeds ? seeds[b] : seed_base + 0x9E3779B9ull * (uint64_t) b;
        rng[b] = sd ? sd : 1;
        out->tok_len[b] = 0;
    }
    int nfin = 0;
    float * row = (float *) malloc(sizeof(float) * (size_t) V);
    float * probs = (float *) malloc(sizeof(float) * (size_t) V);
    float * x_in = (float *) malloc(sizeof(float) * (size_t) B * D);
    int steps = 0;
    for (int idx = 0; idx < max_steps; idx++) {
        steps = idx + 1;
        if (out->logits) memcpy(out->logits + (size_t) idx * B * V, lg, sizeof(float) * (size_t) B * V);
        for (int b = 0; b < B; b++) {
            if (out->sampled) out->sampled[(size_t) idx * B + b] = -1;
            if (idx_list[b] >= 0) continue;
            memcpy(row, lg + (size_t) b * V, sizeof(float) * (size_t) V);
            if (idx < 11 || (flags & ORC_EOS_MASK_ALL)) row[m->EOS] = -INFINITY;
            const int np = ny[b] < 4096 ? ny[b] : 4096;
            const int32_t * prev = y + (size_t) b * out->tok_stride + (ny[b] - np);
            orc_logits_to_probs(top_k, top_p, temperature, rep, row, V, prev, np, probs);
            if (b == 0 && out->probs0) memcpy(out->probs0 + (size_t) idx * V, probs, sizeof(float) * (size_t) V);
            int tok = orc_sample(probs, V, &rng[b]);
            if (out->sampled) out->sampled[(size_t) idx * B + b] = tok;
            if (oracle && idx < n_oracle) tok = oracle[idx];
            y[(size_t) b * out->tok_stride + ny[b]++] = tok;
            if (tok == m->EOS) {
                idx_list[b] = idx;
                out->tok_len[b] = ny[b] - 1;
                if (out->finish_seq) out->finish_seq[nfin] = b;
                out->lens[nfin++] = idx;
            }
        }
        if (early_stop_num != -1 && (ny[0] - P) > early_stop_num) {
            for (int b = 0; b < B; b++)
                if (idx_list[b] < 0) {
                    idx_list[b] = idx;
                    out->tok_len[b] = ny[b] - 1;
                    if (out->finish_seq) out->finish_seq[nfin] = b;
                    out->lens[nfin++] = idx;
                }
        }
        if (nfin == B) break;
        for (int b = 0; b < B; b++) {
            const int tok = y[(size_t) b * out->tok_stride + ny[b] - 1];
            const int pos = P + idx;
            for (int d = 0; d < D; d++)
                x_in[(size_t) b * D + d] = fmaf(m->audio_alpha, m->pe[(size_t) pos * D + d], m->audio_emb[(size_t) tok * D + d]);
        }
        decode(m, x_in, B, pad, S + idx, &c, flags, nthreads, lg);
    }
    for (int b = 0; b < B; b++)
        if (idx_list[b] < 0) {
            out->tok_len[b] = ny[b];
            if (out->finish_seq) out->finish_seq[nfin] = b;
            out->lens[nfin++] = max_steps;
        }
    out->n_steps = steps;
    out->decode_ms = (omp_get_wtime() - t1) * 1e3;
    if ((out->kv_k || out->kv_v) && out->kv_layer >= 0 && out->kv_layer < m->NL && out->kv_cols > 0 &&
        out->kv_cols <= c.Lmax + 1)
        for (int b = 0; b < B; b++)
            for (int h = 0; h < m->NH; h++)
                for (int s = 0; s < out->kv_cols; s++) {
                    const size_t o = (((size_t) b * m->NH + h) * out->kv_cols + s) * m->HD;
                    const size_t src = cidx(m, &c, out->kv_layer, b, h, s);
                    if (out->kv_k) memcpy(out->kv_k + o, c.k + src, sizeof(float) * (size_t) m->HD);
                    if (out->kv_v) memcpy(out->kv_v + o, c.v + src, sizeof(float) * (size_t) m->HD);
                }
    free(row); free(probs); free(x_in); free(lg); free(ny); free(idx_list); free(rng); free(pad);
    free(c.k); free(c.v);
    return 0;
}

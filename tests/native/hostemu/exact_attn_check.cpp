// Host check of exact mode's fused decode kernel (qkv_attn.hip, gsvk_op_qkv_attn_exact) with the
// library's kernels compiled for the CPU (hip/hip_runtime.h, emu.h) under AddressSanitizer: against
// the two launches it replaces, the LayerNorm-input QKV GEMV with the K/V append (layer.hip) and the
// one-wave exact attention (attn_exact.hip, k_attn_exact_decode), on the same inputs. The outputs
// and the appended K/V rows must be equal to the bit, and no access may leave a buffer. Test
// infrastructure only.
//
//   exact_attn_check B lstride col seed
//
// B sequences over fp16 caches [B][16][lstride][32] (N(0, 1) values), the new key at column col,
// the first valid key of sequence b spread over [0, col] (sequence 0: col, only the new key;
// sequence 1: 0).
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "common.h"
#include "layer.h"

namespace gsvk {
static std::string g_err;
void set_error(const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}
const char * get_error() { return g_err.c_str(); }
// the prefill's many-row projection on the matrix cores (fdot_mfma.hip) is linked, never run
int launch_fdot_mfma(const float *, int64_t, int64_t, const float *, int64_t, int64_t, float *, int64_t,
                     hipStream_t) {
    std::fprintf(stderr, "hostemu: matrix-core kernel not emulated\n");
    std::abort();
}
int launch_attn_exact_decode(const float * q, int64_t q_stride, const uint16_t * k, const uint16_t * v, int B,
                             int nh, int64_t lstride, const int32_t * kv_begin, const int32_t * kv_end,
                             float scale, float * out, int8_t * oq, float * od, hipStream_t stream,
                             int oq_layout);
}  // namespace gsvk

extern "C" int gsvk_op_qkv_attn_exact(const int8_t * wq, const uint16_t * wd, const float * bias, const float * res,
                                      const float * r, const float * ln_bias, const float * wb, int B, int nh,
                                      uint16_t * k, uint16_t * v, int64_t lstride, const int32_t * kv_begin,
                                      const int32_t * col, float scale, float * out, int8_t * oq, float * od,
                                      float * ln_out, void * stream);

using namespace gsvk;

template <typename T>
static T * buf(size_t n) {
    T * p = (T *) std::malloc(std::max<size_t>(n, 1) * sizeof(T));
    if (!p) std::exit(2);
    std::memset(p, 0, std::max<size_t>(n, 1) * sizeof(T));
    return p;
}

static uint16_t h16(float f) {
    _Float16 h = (_Float16) f;
    uint16_t u;
    std::memcpy(&u, &h, 2);
    return u;
}

int main(int argc, char ** argv) {
    if (argc < 5) {
        std::fprintf(stderr, "usage: %s B lstride col seed\n", argv[0]);
        return 2;
    }
    const int B = std::atoi(argv[1]), lstride = std::atoi(argv[2]), col = std::atoi(argv[3]);
    std::mt19937_64 rng(std::strtoull(argv[4], nullptr, 0));
    const int D = 512, NH = 16, HD = 32, N3 = 3 * D;
    if (B < 2 || col < 0 || col >= lstride) return 2;
    std::normal_distribution<float> nd(0.0f, 1.0f);
    // QKV weights: sliced quants [1536][512], fp16 scales [1536][16], bias
    int8_t * wq = buf<int8_t>((size_t) N3 * D);
    uint16_t * wd = buf<uint16_t>((size_t) N3 * D / 32);
    float * bias = buf<float>(N3);
    for (size_t i = 0; i < (size_t) N3 * D; i++) wq[i] = (int8_t) ((int) (rng() % 255) - 127);
    for (size_t i = 0; i < (size_t) N3 * D / 32; i++) wd[i] = h16(0.004f * (0.5f + (float) (rng() % 1000) / 1000.0f));
    for (int i = 0; i < N3; i++) bias[i] = 0.1f * nd(rng);
    // LayerNorm input rows and parameters
    float * res = buf<float>((size_t) B * D), * rr = buf<float>((size_t) B * D), * lnb = buf<float>(D);
    float * wb = buf<float>(2 * D);
    for (size_t i = 0; i < (size_t) B * D; i++) { res[i] = nd(rng); rr[i] = 0.5f * nd(rng); }
    for (int i = 0; i < D; i++) { lnb[i] = 0.1f * nd(rng); wb[i] = 1.0f + 0.2f * nd(rng); wb[D + i] = 0.1f * nd(rng); }
    // caches (two copies: each path appends its own K/V)
    const size_t cn = (size_t) B * NH * lstride * HD;
    uint16_t * ka = buf<uint16_t>(cn), * va = buf<uint16_t>(cn), * kb = buf<uint16_t>(cn), * vb = buf<uint16_t>(cn);
    for (size_t i = 0; i < cn; i++) { ka[i] = kb[i] = h16(nd(rng)); va[i] = vb[i] = h16(nd(rng)); }
    int32_t * kv_begin = buf<int32_t>(B), * kv_end = buf<int32_t>(B), * colp = buf<int32_t>(1);
    for (int b = 0; b < B; b++) kv_begin[b] = (int) (rng() % (uint64_t) (col + 1));
    kv_begin[0] = col;
    kv_begin[1] = 0;
    for (int b = 0; b < B; b++) kv_end[b] = col + 1;
    colp[0] = col;
    const float scale = 1.0f / std::sqrt(32.0f);

    // the fused exact kernel
    float * outa = buf<float>((size_t) B * D);
    int8_t * oqa = buf<int8_t>((size_t) B * D);
    float * oda = buf<float>((size_t) B * D / 32);
    float * lna = buf<float>((size_t) B * D);
    if (gsvk_op_qkv_attn_exact(wq, wd, bias, res, rr, lnb, wb, B, NH, ka, va, lstride, kv_begin, colp, scale, outa,
                               oqa, oda, lna, nullptr) != GSVK_OK) {
        std::fprintf(stderr, "qkv_attn_exact failed: %s\n", get_error());
        return 1;
    }
    // the two launches it replaces: QKV GEMV (q stored, K/V appended) + one-wave exact attention
    float * q = buf<float>((size_t) B * D);
    float * lnb_out = buf<float>((size_t) B * D);
    LayerIn in{};
    in.mode = IN_LN;
    in.res = res;
    in.r = rr;
    in.bias = lnb;
    in.wb = wb;
    in.out_x = lnb_out;
    LayerOut qo{};
    qo.y = q;
    qo.y_stride = D;
    qo.n_store = D;
    qo.bias = bias;
    qo.kc = kb;
    qo.vc = vb;
    qo.kv_row0 = D;
    qo.d_model = D;
    qo.n_head = NH;
    qo.lstride = lstride;
    qo.rows_per_seq = 1;
    qo.col_ptr = colp;
    qo.col_add = 0;
    if (launch_layer_gemv(wq, wd, N3, D, B, in, qo, nullptr) != GSVK_OK) {
        std::fprintf(stderr, "layer_gemv failed: %s\n", get_error());
        return 1;
    }
    float * outb = buf<float>((size_t) B * D);
    int8_t * oqb = buf<int8_t>((size_t) B * D);
    float * odb = buf<float>((size_t) B * D / 32);
    if (launch_attn_exact_decode(q, D, kb, vb, B, NH, lstride, kv_begin, kv_end, scale, outb, oqb, odb, nullptr,
                                 Q8_SLICED) != GSVK_OK) {
        std::fprintf(stderr, "attn_exact_decode failed: %s\n", get_error());
        return 1;
    }
    int bad = 0;
    if (std::memcmp(ka, kb, cn * 2) || std::memcmp(va, vb, cn * 2)) {
        std::printf("K/V caches differ\n");
        bad = 1;
    }
    if (std::memcmp(lna, lnb_out, (size_t) B * D * 4)) { std::printf("LayerNorm rows differ\n"); bad = 1; }
    for (size_t i = 0; i < (size_t) B * D; i++)
        if (std::memcmp(&outa[i], &outb[i], 4)) {
            if (bad < 10) std::printf("out[%zu] (b %zu, dim %zu): fused %.9g, two launches %.9g\n", i, i / D, i % D,
                                      outa[i], outb[i]);
            bad++;
        }
    if (std::memcmp(oqa, oqb, (size_t) B * D) || std::memcmp(oda, odb, (size_t) B * D / 32 * 4)) {
        std::printf("Q8_0 copies differ\n");
        bad++;
    }
    std::printf("exact check: B=%d lstride=%d col=%d, keys per row", B, lstride, col);
    for (int b = 0; b < B && b < 8; b++) std::printf(" %d", col + 1 - kv_begin[b]);
    std::printf("%s\n", bad ? " -- MISMATCH" : ": outputs, Q8_0 copies and K/V equal to the bit");
    return bad ? 1 : 0;
}

// ggml-cpu's F32 dot order (MODE 0 of fdot.hip) on the gfx950 fp32 matrix cores, for many
// activation rows (the prefill's BERT projection: ~9k rows x 1025 x 512 at 16 x 1024).
//
// ggml_vec_dot_f32 on x86 keeps 32 fma chains per output: slice p (0..31) sums w[32i+p] *
// x[32i+p] over i in order, then the slices meet in a fixed butterfly (xor 16, 8, 4, 1, 2; see
// fdot.hip), then the k % 32 leftovers are fused in order. v_mfma_f32_16x16x1_4b_f32 adds exactly
// one product to each output of each of its four 16 x 16 blocks, rounded once as an fma does, so a
// slice's chain runs unchanged as a sequence of these instructions (checked bit for bit against
// the oracle).
//
// One wave holds all 32 slices of a 16 x 16 output tile: eight accumulators, acc[q] block b =
// slice q + 8b. Lane l feeds block l / 16 with row l % 16, so for one step of 32 columns it reads
// the 8 contiguous columns 8 (l / 16) .. + 7 of its activation row and of its weight row (two
// 16-byte LDS reads each) and issues the eight products. The butterfly then runs in registers:
// xor 16 and xor 8 pair blocks (VGPRs 4b + v), xor 4, 1 and 2 pair accumulators.
//
// Workgroup: 4 waves, 32 activation rows x 32 weight rows. Both 32-row tiles stream through a
// ring of three LDS buffers of 64 columns by direct global -> LDS loads (one 256-byte row per
// instruction), two chunks ahead of the products; rows are padded to 68 floats, so the 16-byte
// reads of 16 lanes (16 rows) fall in 16 distinct bank quads.
#include "common.h"

namespace gsvk {

namespace {
constexpr int F2_CH = 64;            // columns per chunk (two steps of 32)
constexpr int F2_ROW = F2_CH + 4;    // LDS floats per staged row
constexpr int F2_NB = 3;             // chunk buffers
constexpr int F2_LOADS = 16;         // direct loads per wave and chunk (64 rows / 4 waves)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef float v16f_t __attribute__((ext_vector_type(16)));

#define F2_VMCNT(n) ((((n) & 0xF) | ((((n) >> 4) & 3) << 14)) | (0x7 << 4) | (0xF << 8))

__device__ __forceinline__ void f2_barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef float f4v __attribute__((ext_vector_type(4)));

// A 16-byte LDS read the compiler does not track: its own tracking would wait for every direct
// load in flight before any LDS read (it cannot tell the buffers apart), which would drain the
// chunks issued ahead. The caller waits for the result with f2_wait_lds.
__device__ __forceinline__ f4v f2_lds_read(const float * p) {
    f4v r;
    const uint32_t a = (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) float *) p;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
// every LDS read issued so far has returned; the four values pass through, so no use of them
// is scheduled before the wait
__device__ __forceinline__ void f2_wait_lds(f4v & a, f4v & b, f4v & c, f4v & d) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
}  // namespace

__global__ void __launch_bounds__(256) k_fdot_ggml_mfma16(const float * __restrict__ W, int n, int k,
                                                          const float * __restrict__ X, int64_t xs, int m,
                                                          float * __restrict__ Y, int64_t ys) {
    __shared__ __align__(16) float buf[F2_NB][64][F2_ROW];   // rows 0-31 activations, 32-63 weights
    __shared__ float left[2][32][33];                         // columns np..k-1, same rows
    const int tid = threadIdx.x;
    const int wv = tid >> 6;
    const int l = tid & 63;
    // Workgroup g runs on XCD g % 8 (round-robin dispatch); XCD x takes a contiguous run of
    // tiles, weight tile fastest, so the workgroups that read one activation tile share an L2.
    const int G = gridDim.x, g = blockIdx.x;
    const int per = G >> 3, rem = G & 7, xcd = g & 7;
    const int t = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + (g >> 3);
    const int n0 = (t % (n >> 5)) * 32;
    const int m0 = (t / (n >> 5)) * 32;
    const int np = k & ~31;
    const int nch = np / F2_CH;   // np % F2_CH == 0 (checked at launch)

    // direct loads: wave v copies staged rows 16v .. 16v + 15 (activation rows past m repeat
    // row m - 1; their outputs are not stored), lane l column l of the chunk
    const int wvu = __builtin_amdgcn_readfirstlane(wv);
    const bool xside = wvu < 2;   // (uniform) waves 0-1: activation rows, 2-3: weight rows
    const float * gb = xside ? X : W;
    const int64_t gs = xside ? xs : (int64_t) k;
    const int r0 = xside ? m0 + 16 * wvu : n0 + 16 * (wvu - 2);
    const int rlim = xside ? m - 1 : n - 1;
    auto issue = [&](int c, int b) {
#pragma unroll
        for (int r = 0; r < F2_LOADS; r++) {
            const float * gp = gb + (int64_t) min(r0 + r, rlim) * gs + c * F2_CH;
            __builtin_amdgcn_global_load_lds(gp + l, (lds_void_t *) &buf[b][16 * wvu + r][0], 4, 0, 0);
        }
    };
    issue(0, 0);
    if (nch > 1) issue(1, 1);
    // the leftover columns, once
    for (int e = tid; e < 2 * 32 * 32; e += 256) {
        const int side = e >> 10, row = (e >> 5) & 31, col = e & 31;
        if (np + col < k)
            left[side][row][col] = side ? W[(int64_t) (n0 + row) * k + np + col]
                                        : X[(int64_t) min(m0 + row, m - 1) * xs + np + col];
    }
    __builtin_amdgcn_s_waitcnt(0);   // every load so far (chunks 0 and 1, the leftovers) and LDS store

    // this wave's 16 x 16 output tile within the workgroup's 32 x 32
    const int mw = (wv & 1) * 16, nw = (wv >> 1) * 16;
    const int h = l >> 4;   // the lane's block: slices 8h .. 8h + 7
    const int xo = (mw + (l & 15)) * F2_ROW + 8 * h;
    const int wo = (32 + nw + (l & 15)) * F2_ROW + 8 * h;
    v16f_t acc[8];
#pragma unroll
    for (int q = 0; q < 8; q++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[q][v] = 0.0f;

#pragma unroll 1
    for (int c = 0; c < nch; c++) {
        if (c > 0) {
            // chunk c has landed (chunk c + 1 may still be in flight: loads retire in order)
            if (c + 1 < nch)
                __builtin_amdgcn_s_waitcnt(F2_VMCNT(F2_LOADS));
            else
                __builtin_amdgcn_s_waitcnt(F2_VMCNT(0));
        }
        // every wave's loads of chunk c are visible, and every wave is done with chunk c - 1,
        // whose buffer chunk c + 2 now fills
        f2_barrier();
        if (c + 2 < nch) issue(c + 2, (c + 2) % F2_NB);
        const float * cb = &buf[c % F2_NB][0][0];
#pragma unroll
        for (int st = 0; st < F2_CH / 32; st++) {
            f4v x0 = f2_lds_read(cb + xo + 32 * st);
            f4v x1 = f2_lds_read(cb + xo + 32 * st + 4);
            f4v w0 = f2_lds_read(cb + wo + 32 * st);
            f4v w1 = f2_lds_read(cb + wo + 32 * st + 4);
            f2_wait_lds(x0, x1, w0, w1);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x1f32(x0.x, w0.x, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(x0.y, w0.y, acc[1], 0, 0, 0);
            acc[2] = __builtin_amdgcn_mfma_f32_16x16x1f32(x0.z, w0.z, acc[2], 0, 0, 0);
            acc[3] = __builtin_amdgcn_mfma_f32_16x16x1f32(x0.w, w0.w, acc[3], 0, 0, 0);
            acc[4] = __builtin_amdgcn_mfma_f32_16x16x1f32(x1.x, w1.x, acc[4], 0, 0, 0);
            acc[5] = __builtin_amdgcn_mfma_f32_16x16x1f32(x1.y, w1.y, acc[5], 0, 0, 0);
            acc[6] = __builtin_amdgcn_mfma_f32_16x16x1f32(x1.z, w1.z, acc[6], 0, 0, 0);
            acc[7] = __builtin_amdgcn_mfma_f32_16x16x1f32(x1.w, w1.w, acc[7], 0, 0, 0);
        }
    }

    // the butterfly: slice p = q + 8b meets p ^ 16 (block b ^ 2), p ^ 8 (block b ^ 1), p ^ 4
    // (accumulator q ^ 4), p ^ 1 and p ^ 2; output (i, j) of a block sits in lane j + 16 (i / 4),
    // VGPR 4b + i % 4
    float y[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        float s[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float b0 = acc[q][v] + acc[q][8 + v];       // xor 16: blocks 0 and 2
            const float b1 = acc[q][4 + v] + acc[q][12 + v];  //         blocks 1 and 3
            s[q] = b0 + b1;                                   // xor 8
        }
        const float a0 = s[0] + s[4], a1 = s[1] + s[5], a2 = s[2] + s[6], a3 = s[3] + s[7];   // xor 4
        y[v] = (a0 + a1) + (a2 + a3);                                                      // xor 1, 2
    }
    const int j = nw + (l & 15);
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int i = mw + 4 * h + v;
        float r = y[v];
        for (int kk = 0; kk < k - np; kk++) r = __builtin_fmaf(left[1][j][kk], left[0][i][kk], r);
        if (m0 + i < m) Y[(int64_t) (m0 + i) * ys + n0 + j] = r;
    }
}

// Y[m][n] = W[n][k] . X[m][k] (row strides xs, ys) in ggml_vec_dot_f32's order: n % 32 == 0,
// (k & ~31) % 64 == 0, m > 0.
int launch_fdot_mfma(const float * W, int64_t n, int64_t k, const float * X, int64_t xs, int64_t m, float * Y,
                     int64_t ys, hipStream_t stream) {
    GSVK_REQUIRE(n % 32 == 0 && k >= F2_CH && (k & ~31) % F2_CH == 0 && m > 0 &&
                     (n / 32) * ((m + 31) / 32) < (1LL << 31),
                 "fdot_mfma: bad shape n=%lld k=%lld m=%lld", (long long) n, (long long) k, (long long) m);
    const dim3 grid((unsigned) ((n / 32) * ((m + 31) / 32)));
    hipLaunchKernelGGL(k_fdot_ggml_mfma16, grid, dim3(256), 0, stream, W, (int) n, (int) k, X, xs, (int) m, Y, ys);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

}  // namespace gsvk

// Single-query (decode) attention over a per-sequence fp16 KV cache, for gfx950.
//
// Work decomposition: workgroup (split, head, seq) of NW waves (4 or 8, see attn_waves: a long
// row is spread over up to 8 waves so that its blocks are in flight together instead of one
// after another). The valid keys [begin, end) of a (seq, head) are cut in blocks of 64;
// split s owns a contiguous run of blocks (see attn_plan: one run per row unless batch x heads is
// small and the rows long, or many rows are long enough to be cut in fixed chunks so that the
// launch holds more workgroups than the chip runs at once and rows of unequal length balance).
// Wave w of a workgroup takes blocks w, w+NW, ... of its run.
// Inside a block, lane = (key slot ks = lane/4, quarter qd = lane%4) reads the 16-byte quarter
// [8qd, 8qd+8) of 4 K rows and 4 V rows (all 8 loads issued before any use, and the next block's
// loads issued before this block's arithmetic); one wave-wide load covers 1 KiB of contiguous
// cache. Each wave keeps an online softmax (running max per block, exp2 of log2e-scaled scores);
// the NW waves merge through LDS, and the splits of one (seq, head), if more than one, are merged
// by the last workgroup to finish (device-scope counter, few rows) or by k_attn_merge, a second
// launch (fixed chunks: no device-scope release per workgroup).
//
// Numerics: softmax(q.k * scale) . V over the valid keys with fp32 accumulation; the output is
// divided by the sum (multiplied by its reciprocal), as ggml_flash_attn_ext does.
#include <mutex>

#include "attn_dev.h"

namespace gsvk {

constexpr int ATT_MERGE_WAVES = 16;

// Merge of the nact (<= 64) partials (m, l, o[32]) of one (seq, head) by one wave: lane c reads
// partial c's (m, l), every lane < 32 its o column; output as attn_store_out.
__device__ __forceinline__ void attn_merge_parts(const float * p0, int nact, int lane, int64_t bh,
                                                 int nh, float * __restrict__ out,
                                                 uint16_t * __restrict__ out16,
                                                 int8_t * __restrict__ oq, float * __restrict__ od,
                                                 int oq_layout) {
    const float mc = lane < nact ? ld_coherent(p0 + lane * ATT_PART) : -INFINITY;
    const float lc = lane < nact ? ld_coherent(p0 + lane * ATT_PART + 1) : 0.0f;
    float Mt = mc;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) Mt = fmaxf(Mt, __shfl_xor(Mt, off, 64));
    const float fc = lane < nact ? __builtin_amdgcn_exp2f(mc - Mt) : 0.0f;
    float Lt = lc * fc;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) Lt += __shfl_xor(Lt, off, 64);
    float Ot = 0.0f;
    for (int c = 0; c < nact; c++) {
        const float w = __shfl(fc, c, 64);
        if (lane < ATT_HD) Ot = __builtin_fmaf(ld_coherent(p0 + c * ATT_PART + 2 + lane), w, Ot);
    }
    attn_store_out(Ot * (1.0f / Lt), lane, bh, nh, out, out16, oq, od, oq_layout);
}

template <int NW, bool NT>
__global__ void __launch_bounds__(NW * 64) k_attn_decode(
    const float * __restrict__ q, int64_t q_stride, const uint16_t * __restrict__ kc,
    const uint16_t * __restrict__ vc, int nh, int64_t lstride, const int32_t * __restrict__ kv_begin,
    const int32_t * __restrict__ kv_end, int nsplit, int chunk, float scale_log2,
    float * __restrict__ out, uint16_t * __restrict__ out16, int8_t * __restrict__ oq,
    float * __restrict__ od, int oq_layout, float * __restrict__ part,
    int32_t * __restrict__ counters) {
    const int split = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    // clamp to the buffer so that a bad range can never read outside the cache
    int beg = kv_begin[b];
    int end = kv_end[b];
    beg = beg < 0 ? 0 : beg;
    end = end > (int) lstride ? (int) lstride : end;
    const int nkeys = end > beg ? end - beg : 0;
    const int nblk = (nkeys + ATT_BLK - 1) / ATT_BLK;
    // blocks per split: a row longer than the launch planned for (more than nsplit chunks) gets
    // longer runs, so that no split index reaches nsplit
    const int even = (nblk + nsplit - 1) / nsplit;
    const int bps = chunk > even ? chunk : even;
    const int nact = bps > 0 ? (nblk + bps - 1) / bps : 0;      // splits with work
    if (split >= (nact > 0 ? nact : 1)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ks = lane >> 2;
    const int qd = lane & 3;
    const int64_t bh = (int64_t) b * nh + h;

    __shared__ float s_m[NW];
    __shared__ float s_l[NW];
    __shared__ float s_o[NW][ATT_HD];

    if (nkeys == 0) {   // no valid key: ggml returns 0 (S == 0 -> S_inv = 0)
        if (wave == 0) attn_store_out(0.0f, lane, bh, nh, out, out16, oq, od, oq_layout);
        return;
    }

    float qv[8];
    {
        const float * qp = q + (int64_t) b * q_stride + h * ATT_HD + qd * 8;
        const float4 a = *reinterpret_cast<const float4 *>(qp);
        const float4 c = *reinterpret_cast<const float4 *>(qp + 4);
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w;
        qv[4] = c.x; qv[5] = c.y; qv[6] = c.z; qv[7] = c.w;
    }
    const uint16_t * kb = kc + bh * lstride * ATT_HD + qd * 8;
    const uint16_t * vb = vc + bh * lstride * ATT_HD + qd * 8;
    const int blk0 = split * bps;
    const int blk1 = min(nblk, blk0 + bps);

    float m = -INFINITY, l = 0.0f;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;

    // the first block of this wave is loaded unconditionally (a wave past the last block loads
    // that block again, from L2, and does not use it), then each iteration prefetches the next
    // block before computing the current one: every load count is known to the compiler, so the
    // waits are exact
    const int last_key = end - 1;
    const int nb = blk1 - blk0;
    int blk = blk0 + (wave < nb ? wave : nb - 1);
    KV8 cur;
    load_block<NT>(kb, vb, beg + blk * ATT_BLK, last_key, ks, cur);
    const uint4 z4 = make_uint4(0, 0, 0, 0);
    if (wave < nb) {
        while (blk + NW < blk1) {
            KV8 pre;
            load_block<NT>(kb, vb, beg + (blk + NW) * ATT_BLK, last_key, ks, pre);
            attn_block_step<false>(cur, beg + blk * ATT_BLK, end, ks, qv, scale_log2, -1, z4, z4, m, l, o);
            cur = pre;
            blk += NW;
        }
        attn_block_step<false>(cur, beg + blk * ATT_BLK, end, ks, qv, scale_log2, -1, z4, z4, m, l, o);
    }
    // reduce the 16 key slots of the wave (m is uniform across the wave)
    l = slot_sum(l);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = slot_sum(o[i]);
    if (lane < 4) {
#pragma unroll
        for (int i = 0; i < 8; i++) s_o[wave][lane * 8 + i] = o[i];
        if (lane == 0) {
            s_l[wave] = l;
            s_m[wave] = m;
        }
    }
    __syncthreads();
    if (wave != 0) return;

    // merge the NW waves (a wave without blocks has m = -inf and weight 0)
    float M = s_m[0];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, s_m[w]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        const float f = s_m[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w] - M);
        L = __builtin_fmaf(s_l[w], f, L);
        if (lane < ATT_HD) O = __builtin_fmaf(s_o[w][lane], f, O);
    }

    if (nact == 1) {
        attn_store_out(O * (1.0f / L), lane, bh, nh, out, out16, oq, od, oq_layout);
        return;
    }

    // several splits: publish the partial; k_attn_merge (fixed chunks) or the last workgroup of
    // this (seq, head) merges
    float * pp = part + (bh * nsplit + split) * ATT_PART;
    if (chunk > 0) {
        if (lane < ATT_HD) pp[2 + lane] = O;
        if (lane == 0) {
            pp[0] = M;
            pp[1] = L;
        }
        return;
    }
    if (lane < ATT_HD) st_coherent(pp + 2 + lane, O);
    if (lane == 0) {
        st_coherent(pp + 0, M);
        st_coherent(pp + 1, L);
    }
    __threadfence();
    int lastflag = 0;
    if (lane == 0) {
        const int prev = __hip_atomic_fetch_add(counters + bh, 1, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT);
        lastflag = (prev == nact - 1);
    }
    const int last = __shfl(lastflag, 0, 64);
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    attn_merge_parts(part + bh * nsplit * ATT_PART, nact, lane, bh, nh, out, out16, oq, od, oq_layout);
    if (lane == 0)
        __hip_atomic_store(counters + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge of the fixed-chunk partials of k_attn_decode: workgroup (head group, seq), one wave per
// head of a sequence with more than one chunk (a row of one chunk was stored by its workgroup).
__global__ void __launch_bounds__(ATT_MERGE_WAVES * 64) k_attn_merge(
    const int32_t * __restrict__ kv_begin, const int32_t * __restrict__ kv_end, int nh,
    int64_t lstride, int nsplit, int chunk, const float * __restrict__ part,
    float * __restrict__ out, uint16_t * __restrict__ out16, int8_t * __restrict__ oq,
    float * __restrict__ od, int oq_layout) {
    const int h = blockIdx.x * ATT_MERGE_WAVES + (int) (threadIdx.x >> 6);
    const int b = blockIdx.y;
    if (h >= nh) return;
    int beg = kv_begin[b];
    int end = kv_end[b];
    beg = beg < 0 ? 0 : beg;
    end = end > (int) lstride ? (int) lstride : end;
    const int nkeys = end > beg ? end - beg : 0;
    const int nblk = (nkeys + ATT_BLK - 1) / ATT_BLK;
    const int even = (nblk + nsplit - 1) / nsplit;
    const int bps = chunk > even ? chunk : even;     // as in k_attn_decode
    const int nact = bps > 0 ? (nblk + bps - 1) / bps : 0;
    if (nact <= 1) return;
    const int64_t bh = (int64_t) b * nh + h;
    attn_merge_parts(part + bh * nsplit * ATT_PART, nact, threadIdx.x & 63, bh, nh, out, out16, oq,
                     od, oq_layout);
}

// Waves per workgroup: enough to take every block of the longest row at once (4..8), halved
// while the grid would hold more than 8192 waves (32 per CU, the resident limit of 256 CUs).
int attn_waves(int B, int nh, int64_t max_keys) {
    const int64_t pairs = (int64_t) B * nh;
    const int64_t blocks = (max_keys + ATT_BLK - 1) / ATT_BLK;
    // at most 8: a workgroup of 16 waves starts later and merges more partials than the extra
    // parallelism returns (measured at batch 1-16; equal at 64 and 128)
    int nw = 4;
    while (nw < 8 && nw < blocks) nw *= 2;
    while (nw > 4 && pairs * nw > 8192) nw /= 2;
    return nw;
}

// Splits per (seq, head). Merging splits through the last workgroup needs an agent-scope release
// per workgroup, which on gfx950 writes back the L2 of the workgroup's XCD; that costs more than it
// saves unless the launch would otherwise leave most of the chip idle on long rows. So, with few
// rows: one workgroup per (seq, head) when the rows are short, else enough splits of at least 16
// blocks (1024 keys) to reach ~256 workgroups, at most 64 (the merge reads one split per lane).
// With >= 1024 rows whose longest has >= 48 blocks the workgroups of one (seq, head) per row would
// all be resident at once, each CU holding a random handful of rows of unequal length: the rows
// are cut in chunks of ATT_CHUNK blocks instead (more workgroups than the chip holds, taken up as
// others finish), merged by k_attn_merge. Batch 128 x 16 heads with rows U[1024, 4096]: 129 us
// of attention per layer -> 121 us + 5 us of merge. Rows of at most 2 chunks lose more to the
// extra launch than the balance returns (batch 64 x 16 heads, rows U[256, 2048]: 31 -> 37 us).
constexpr int ATT_CHUNK = 16;
constexpr int64_t ATT_NT_BYTES = (int64_t) 16 << 20;

AttnPlan attn_plan(int B, int nh, int64_t max_keys) {
    const int64_t pairs = (int64_t) B * nh;
    const int64_t blocks = (max_keys + ATT_BLK - 1) / ATT_BLK;
    AttnPlan p{1, 0};
    if (pairs >= 1024) {
        if (blocks >= 3 * ATT_CHUNK) {
            p.chunk = ATT_CHUNK;
            p.nsplit = (int) ((blocks + ATT_CHUNK - 1) / ATT_CHUNK);
        }
        return p;
    }
    if (pairs >= 64 || blocks < 32) return p;
    int64_t ns = (256 + pairs - 1) / pairs;
    if (ns > blocks / 16) ns = blocks / 16;
    if (ns > 64) ns = 64;
    if (ns < 1) ns = 1;
    p.nsplit = (int) ns;
    return p;
}

int attn_nsplit(int B, int nh, int64_t max_keys) { return attn_plan(B, nh, max_keys).nsplit; }

size_t attn_workspace_bytes(int B, int nh, int64_t max_keys) {
    const int ns = attn_nsplit(B, nh, max_keys);
    const size_t part = (size_t) B * nh * ns * ATT_PART * sizeof(float);
    const size_t cnt = (size_t) B * nh * sizeof(int32_t);
    return ((part + 255) / 256) * 256 + cnt;
}

// The counter area (the tail of ws) must be zero before the first call; every call leaves it
// zero again.
int launch_attn_decode(const float * q, int64_t q_stride, const uint16_t * k, const uint16_t * v,
                       int B, int nh, int hd, int64_t lstride, const int32_t * kv_begin,
                       const int32_t * kv_end, int64_t max_keys, float scale, float * out,
                       uint16_t * out16, int8_t * oq, float * od, void * ws, hipStream_t stream,
                       int oq_layout) {
    GSVK_REQUIRE(q && k && v && kv_begin && kv_end && out && ws, "attn_decode: null pointer");
    GSVK_REQUIRE(hd == ATT_HD, "attn_decode: head_dim must be 32 (got %d)", hd);
    GSVK_REQUIRE(q_stride >= (int64_t) nh * hd && q_stride % 4 == 0, "attn_decode: bad q stride");
    GSVK_REQUIRE(B > 0 && B <= 65535 && nh > 0 && nh <= 65535 && lstride > 0 && max_keys >= 0 &&
                     max_keys <= lstride,
                 "attn_decode: bad shape B=%d nh=%d lstride=%lld max_keys=%lld", B, nh,
                 (long long) lstride, (long long) max_keys);
    GSVK_REQUIRE((oq == nullptr) == (od == nullptr), "attn_decode: oq and od go together");
    const AttnPlan plan = attn_plan(B, nh, max_keys);
    const int ns = plan.nsplit;
    GSVK_REQUIRE(ns <= 64, "attn_decode: rows too long for the split merge");
    const size_t part_bytes = (size_t) B * nh * ns * ATT_PART * sizeof(float);
    float * part = (float *) ws;
    int32_t * counters = (int32_t *) ((char *) ws + ((part_bytes + 255) / 256) * 256);
    const dim3 grid((unsigned) ns, (unsigned) nh, (unsigned) B);
    const int nw = attn_waves(B, nh, max_keys);
#define GSVK_ATTN_LAUNCH(W, NT)                                                                  \
    hipLaunchKernelGGL((k_attn_decode<W, NT>), grid, dim3(W * 64), 0, stream, q, q_stride, k, v, nh, \
                       lstride, kv_begin, kv_end, ns, plan.chunk, scale * LOG2E, out, out16, oq, \
                       od, oq_layout, part, counters)
    // streaming loads for a launch of at least ATT_NT_BYTES of K/V rows: a decode of that many
    // per layer reads far more than the MALL holds per step (batch 64 x 16 heads, rows U[256, 2048],
    // 146 MB: 30.4 -> 27.1 us)
    const bool nt = (int64_t) B * nh * max_keys * ATT_HD * 2 * 2 >= ATT_NT_BYTES;
    if (nw == 8) {
        if (nt) GSVK_ATTN_LAUNCH(8, true);
        else GSVK_ATTN_LAUNCH(8, false);
    } else {
        if (nt) GSVK_ATTN_LAUNCH(4, true);
        else GSVK_ATTN_LAUNCH(4, false);
    }
#undef GSVK_ATTN_LAUNCH
    GSVK_LAUNCH_CHECK();
    if (plan.chunk > 0) {
        const int hw = nh < ATT_MERGE_WAVES ? nh : ATT_MERGE_WAVES;
        const dim3 mgrid((unsigned) ((nh + ATT_MERGE_WAVES - 1) / ATT_MERGE_WAVES), (unsigned) B);
        hipLaunchKernelGGL(k_attn_merge, mgrid, dim3(hw * 64), 0, stream, kv_begin, kv_end, nh,
                           lstride, ns, plan.chunk, part, out, out16, oq, od, oq_layout);
        GSVK_LAUNCH_CHECK();
    }
    return GSVK_OK;
}

// ---- the same attention with its workspace in a library-owned device array ------------------
// For callers that cannot allocate (code under graph capture, serving loops that forbid
// hipMalloc): the split partials and merge counters live in `scratch`, one copy per GPU, held
// until the process ends. Every call on a GPU uses that GPU's copy, so calls that overlap on one
// GPU (two streams, two threads) race on it and must be serialised by the caller.
constexpr size_t ATT_SCRATCH_BYTES = (size_t) 8 << 20;
static __device__ __align__(256) unsigned char scratch[ATT_SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;

// Device address of `scratch` on the current device, looked up once per device (the name of the
// array is a host-side stand-in and must never reach a kernel).
int scratch_address(void ** out) {
    static std::mutex mu;
    static void * addr[SCRATCH_MAX_DEVICES] = {};
    int dev = -1;
    GSVK_HIP(hipGetDevice(&dev));
    GSVK_REQUIRE(dev >= 0 && dev < SCRATCH_MAX_DEVICES, "attn_decode_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void) hipGetLastError();
            set_error("attn_decode_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return GSVK_ERR_HIP;
        }
        addr[dev] = p;
    }
    *out = addr[dev];
    return GSVK_OK;
}

__global__ void k_zero_words(int32_t * __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

int launch_attn_decode_noalloc(const float * q, const uint16_t * k, const uint16_t * v, int B, int nh,
                               int hd, int64_t lstride, const int32_t * kv_begin,
                               const int32_t * kv_end, int64_t max_keys, float scale, float * out,
                               uint16_t * out16, int8_t * oq, float * od, hipStream_t stream) {
    GSVK_REQUIRE(B > 0 && B <= 65535 && nh > 0 && nh <= 65535 && max_keys >= 0,
                 "attn_decode_noalloc: bad shape B=%d nh=%d max_keys=%lld", B, nh, (long long) max_keys);
    const size_t need = attn_workspace_bytes(B, nh, max_keys);
    GSVK_REQUIRE(need <= ATT_SCRATCH_BYTES,
                 "attn_decode_noalloc: the shape needs %zu bytes of workspace, more than the %zu of "
                 "the library's scratch array", need, ATT_SCRATCH_BYTES);
    void * ws = nullptr;
    GSVK_TRY(scratch_address(&ws));
    const AttnPlan plan = attn_plan(B, nh, max_keys);
    if (plan.nsplit > 1 && plan.chunk == 0) {
        // the merge counters (the tail of the workspace) must start at zero: a fill kernel, not a
        // memset, so that the call can also be captured into a graph
        const size_t part_bytes = (size_t) B * nh * plan.nsplit * ATT_PART * sizeof(float);
        int32_t * counters = (int32_t *) ((char *) ws + ((part_bytes + 255) / 256) * 256);
        const int n = B * nh;
        hipLaunchKernelGGL(k_zero_words, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream,
                           counters, n);
        GSVK_LAUNCH_CHECK();
    }
    return launch_attn_decode(q, (int64_t) nh * hd, k, v, B, nh, hd, lstride, kv_begin, kv_end,
                              max_keys, scale, out, out16, oq, od, ws, stream);
}

}  // namespace gsvk

extern "C" int gsvk_op_attn_decode_noalloc(const float * q, const uint16_t * k, const uint16_t * v,
                                           int B, int nh, int hd, int64_t lstride,
                                           const int32_t * kv_begin, const int32_t * kv_end,
                                           int64_t max_keys, float scale, float * out,
                                           uint16_t * out_f16, int8_t * oq, float * od,
                                           void * stream) {
    return gsvk::launch_attn_decode_noalloc(q, k, v, B, nh, hd, lstride, kv_begin, kv_end, max_keys,
                                            scale, out, out_f16, oq, od, (hipStream_t) stream);
}

extern "C" size_t gsvk_attn_workspace_bytes(int B, int nh, int64_t max_keys) {
    return gsvk::attn_workspace_bytes(B, nh, max_keys);
}

extern "C" int gsvk_op_attn_decode(const float * q, const uint16_t * k, const uint16_t * v, int B,
                                   int nh, int hd, int64_t lstride, const int32_t * kv_begin,
                                   const int32_t * kv_end, int64_t max_keys, float scale,
                                   float * out, uint16_t * out_f16, int8_t * oq, float * od,
                                   void * ws, void * stream) {
    return gsvk::launch_attn_decode(q, (int64_t) nh * hd, k, v, B, nh, hd, lstride, kv_begin, kv_end,
                                    max_keys, scale, out, out_f16, oq, od, ws, (hipStream_t) stream);
}

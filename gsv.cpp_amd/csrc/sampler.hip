// Device sampler for gfx950: gsv_logits_to_probs + gsv_sample (src/gsv_sampler.cpp:8-89) and
// the per-step bookkeeping of gsv_ar::generate (src/gsv_ar.cpp:762-796), one workgroup per
// sequence, so the decode loop needs no host round trip per step.
//
// Order of operations (not interchangeable, src/gsv_sampler.h:3-10):
//   EOS mask while idx < 11 -> repetition penalty once per occurrence in the last <= 4096
//   tokens -> top-p over a stable descending order -> temperature -> top-k with a pivot (ties
//   kept) -> softmax (fp32, sum in index order) -> argmax(p / q), q_i = -log(1 - U_i),
//   U_i from xorshift64* (the i-th draw of the sequence's stream, first maximum wins).
//
// The sequential parts (the softmax sum, the top-p cumulative sum) run in one lane in index
// order, as in the reference, so the sums round identically. The RNG stream is jumped ahead:
// xorshift64* is linear over GF(2), so the state after n steps is A^n s; lane t of wave 0 starts
// at draw chunk*t from a precomputed matrix and steps sequentially through its chunk.
#include <array>

#include "common.h"
#include "sampler.h"

namespace gsvk {



constexpr int SMP_THREADS = 256;
constexpr int SMP_SORT = 2048;   // >= V
constexpr int SMP_CH = 32;       // >= ceil(V / 64)

__device__ __forceinline__ uint64_t gf2_apply(const uint64_t * __restrict__ cols, uint64_t s) {
    uint64_t r = 0;
#pragma unroll 8
    for (int i = 0; i < 64; i++) r ^= cols[i] & (0ull - ((s >> i) & 1ull));
    return r;
}

__device__ __forceinline__ uint64_t xs_step(uint64_t s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s;
}

// a precedes b in a stable descending sort
__device__ __forceinline__ bool before(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

__device__ void bitonic_sort_desc(float * v, int * idx) {
    for (int size = 2; size <= SMP_SORT; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < SMP_SORT / 2; t += SMP_THREADS) {
                const int i = 2 * t - (t & (stride - 1));
                const int j = i + stride;
                const bool up = (i & size) == 0;     // this run sorts descending when up
                const bool sw = up ? before(v[j], idx[j], v[i], idx[i]) : before(v[i], idx[i], v[j], idx[j]);
                if (sw) {
                    const float tv = v[i]; v[i] = v[j]; v[j] = tv;
                    const int ti = idx[i]; idx[i] = idx[j]; idx[j] = ti;
                }
            }
        }
    }
    __syncthreads();
}

__global__ void __launch_bounds__(SMP_THREADS) k_sample(SampleArgs a) {
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int V = a.V;
    const int idx = *a.step;

    __shared__ float lg[SMP_SORT];
    __shared__ int cnt[SMP_SORT];
    __shared__ float sv[SMP_SORT];
    __shared__ int si[SMP_SORT];
    __shared__ float s_scalar[2];
    __shared__ float s_bestv[1];
    __shared__ int s_besti[1];

    const bool running = a.fin_step[b] < 0 && idx < a.max_steps;
    if (running) {
        for (int v = tid; v < V; v += SMP_THREADS) {
            lg[v] = a.logits[(int64_t) b * V + v];
            cnt[v] = 0;
        }
        __syncthreads();
        if (tid == 0 && (idx < 11 || (a.flags & 1u))) lg[a.eos] = -INFINITY;
        // 1) repetition penalty, once per occurrence in the window
        if (a.rep != 1.0f) {
            const int n = a.ny[b];
            const int np = n < 4096 ? n : 4096;
            const int32_t * h = a.hist + (int64_t) b * a.hist_stride + (n - np);
            for (int i = tid; i < np; i += SMP_THREADS) {
                const int t = h[i];
                if (t >= 0 && t < V) atomicAdd(&cnt[t], 1);
            }
            __syncthreads();
            for (int v = tid; v < V; v += SMP_THREADS) {
                float s = lg[v];
                for (int c = cnt[v]; c > 0; c--) s = (s < 0.0f) ? s * a.rep : s / a.rep;
                lg[v] = s;
            }
        }
        __syncthreads();
        // 2) top-p over the stable descending order
        if (a.top_p < 1.0f) {
            for (int v = tid; v < SMP_SORT; v += SMP_THREADS) {
                sv[v] = v < V ? lg[v] : -INFINITY;
                si[v] = v;
            }
            bitonic_sort_desc(sv, si);
            if (tid == 0) {
                const float mx = lg[si[0]];
                float sum = 0.0f;
                for (int k = 0; k < V; k++) sum = sum + (float) exp((double) (lg[si[k]] - mx));
                const float inv_sum = 1.0f / sum;
                float cum = 0.0f;
                for (int k = 0; k < V; k++) {
                    const int i = si[k];
                    cum = __builtin_fmaf((float) exp((double) (lg[i] - mx)), inv_sum, cum);
                    if (k > 0 && cum > a.top_p) lg[i] = -INFINITY;
                }
            }
            __syncthreads();
        }
        // 3) temperature
        const float temp = a.temperature > 1e-5f ? a.temperature : 1e-5f;
        for (int v = tid; v < V; v += SMP_THREADS) lg[v] = lg[v] / temp;
        __syncthreads();
        // 4-6) wave 0 holds the row in registers: lane t owns indices [t*chunk, t*chunk + chunk)
        // (the same ownership as the RNG chunks of step 6).
        const bool use_k = a.top_k > 0 && a.top_k < V;
        if (use_k && a.top_k > 64) {   // large k: pivot from a full stable sort (all threads)
            for (int v = tid; v < SMP_SORT; v += SMP_THREADS) {
                sv[v] = v < V ? lg[v] : -INFINITY;
                si[v] = v;
            }
            bitonic_sort_desc(sv, si);
            if (tid == 0) s_scalar[1] = sv[a.top_k - 1];
        }
        __syncthreads();
        const int chunk = a.chunk;
        const int base = (tid & 63) * chunk;
        float pv[SMP_CH];
        int total = 0;
        if (tid < 64) {
#pragma unroll
            for (int c = 0; c < SMP_CH; c++) pv[c] = (c < chunk && base + c < V) ? lg[base + c] : -INFINITY;
            // 4) top-k: pivot = k-th largest value counted with multiplicity; values below it are
            // masked (ties with the pivot stay)
            if (use_k) {
                float pivot;
                if (a.top_k <= 64) {
                    float w[SMP_CH];
#pragma unroll
                    for (int c = 0; c < SMP_CH; c++) w[c] = pv[c];
                    pivot = -INFINITY;
                    for (int r = 0; r < a.top_k; r++) {
                        float bv = -INFINITY;
                        int bc = SMP_CH;
#pragma unroll
                        for (int c = 0; c < SMP_CH; c++)
                            if (c < chunk && (w[c] > bv || bc == SMP_CH)) { bv = w[c]; bc = c; }
                        const int mine = bc < SMP_CH ? base + bc : 0x7fffffff;
                        float gv = bv;
                        int gi = mine;
#pragma unroll
                        for (int o = 32; o > 0; o >>= 1) {
                            const float ov = __shfl_xor(gv, o, 64);
                            const int oi = __shfl_xor(gi, o, 64);
                            if (ov > gv || (ov == gv && oi < gi)) { gv = ov; gi = oi; }
                        }
                        pivot = gv;
#pragma unroll
                        for (int c = 0; c < SMP_CH; c++)
                            if (base + c == gi) w[c] = -INFINITY;   // remove one instance
                    }
                } else {
                    pivot = s_scalar[1];
                }
#pragma unroll
                for (int c = 0; c < SMP_CH; c++)
                    if (pv[c] < pivot) pv[c] = -INFINITY;
            }
            // 5) softmax: max, exp; the sum runs in index order over the non-zero terms only
            // (adding +0 leaves an fp32 sum unchanged), compacted into LDS in index order
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < SMP_CH; c++) mx = fmaxf(mx, pv[c]);
            mx = warp_max(mx);
            int cnt = 0;
#pragma unroll
            for (int c = 0; c < SMP_CH; c++) {
                pv[c] = (pv[c] == -INFINITY) ? 0.0f : (float) exp((double) (pv[c] - mx));
                cnt += pv[c] > 0.0f;
            }
            int incl = cnt;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if ((tid & 63) >= o) incl += t;
            }
            total = __shfl(incl, 63, 64);
            int wpos = incl - cnt;
#pragma unroll
            for (int c = 0; c < SMP_CH; c++)
                if (pv[c] > 0.0f) sv[wpos++] = pv[c];
        }
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            for (int i = 0; i < total; i++) sum = sum + sv[i];
            s_scalar[0] = 1.0f / sum;
        }
        __syncthreads();
        // 6) sample: argmax over p > 0 of p / q, q_i = -log(1 - U_i)
        if (tid < 64) {
            const float inv = s_scalar[0];
#pragma unroll
            for (int c = 0; c < SMP_CH; c++) pv[c] = pv[c] * inv;
            if (b == 0 && a.probs_dump) {
#pragma unroll
                for (int c = 0; c < SMP_CH; c++)
                    if (c < chunk && base + c < V) a.probs_dump[(int64_t) idx * V + base + c] = pv[c];
            }
            const uint64_t s0 = a.rng[b];
            uint64_t st = gf2_apply(a.jump + (int64_t) tid * 64, s0);
            float best = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int c = 0; c < SMP_CH; c++) {
                if (c < chunk && base + c < V) {
                    const float p = pv[c];
                    float val = 0.0f;
                    if (p > 0.0f) {
                        const uint64_t x = st * 0x2545F4914F6CDD1Dull;
                        const float u = (float) ((double) (x >> 40) * (1.0 / 16777216.0));
                        const float q = -(float) log((double) (1.0f - u));
                        val = p / q;
                    }
                    if (val > best) { best = val; bi = base + c; }
                    st = xs_step(st);
                }
            }
            // first maximum wins: larger value, then smaller index
            for (int o = 32; o > 0; o >>= 1) {
                const float ob = __shfl_xor(best, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
            }
            if (tid == 0) {
                s_besti[0] = bi;
                s_bestv[0] = best;
                a.rng[b] = gf2_apply(a.adv, s0);
            }
        }
        __syncthreads();
        if (tid == 0) {
            int tok = s_besti[0];
            if (tok < 0 || tok >= V) tok = 0;   // all values were 0: the first index wins
            if (a.sampled_dump) a.sampled_dump[(int64_t) idx * a.B + b] = tok;
            if (a.oracle && idx < a.n_oracle) tok = a.oracle[idx];
            const int n = a.ny[b];
            a.hist[(int64_t) b * a.hist_stride + n] = tok;
            a.ny[b] = n + 1;
            a.last_tok[b] = tok;
            if (tok == a.eos) {
                a.fin_step[b] = idx;
                a.fin_kind[b] = 0;
            }
        }
    }
    // the last workgroup applies the early-stop rule and advances the loop index
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const int prev = __hip_atomic_fetch_add(a.done_counter, 1, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT);
        if (prev == a.B - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (idx < a.max_steps) {
                if (a.early_stop != -1) {
                    const int n0 = __hip_atomic_load(a.ny, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (n0 - a.P > a.early_stop) {
                        for (int bb = 0; bb < a.B; bb++) {
                            if (__hip_atomic_load(a.fin_step + bb, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) < 0) {
                                a.fin_step[bb] = idx;
                                a.fin_kind[bb] = 1;
                            }
                        }
                    }
                }
                int unfinished = 0;
                for (int bb = 0; bb < a.B; bb++)
                    unfinished += __hip_atomic_load(a.fin_step + bb, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT) < 0;
                *a.n_unfinished = unfinished;
                *a.step = idx + 1;
            }
            __hip_atomic_store(a.done_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

int launch_sample(const SampleArgs & a, hipStream_t stream) {
    GSVK_REQUIRE(a.V > 0 && a.V <= SMP_SORT && a.B > 0 && a.chunk * 64 >= a.V && a.chunk <= SMP_CH,
                 "sample: vocabulary %d exceeds %d", a.V, SMP_SORT);
    GSVK_REQUIRE(a.top_k < 0 || a.top_k <= SMP_SORT, "sample: bad top_k");
    hipLaunchKernelGGL(k_sample, dim3((unsigned) a.B), dim3(SMP_THREADS), 0, stream, a);
    GSVK_LAUNCH_CHECK();
    return GSVK_OK;
}

// ---- host: GF(2) matrices of the xorshift64* state transition ----

namespace {
using Mat = std::array<uint64_t, 64>;   // column i = image of basis vector e_i

uint64_t host_step(uint64_t s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s;
}
uint64_t apply(const Mat & m, uint64_t s) {
    uint64_t r = 0;
    for (int i = 0; i < 64; i++)
        if ((s >> i) & 1) r ^= m[i];
    return r;
}
Mat mul(const Mat & a, const Mat & b) {   // a * b
    Mat r;
    for (int i = 0; i < 64; i++) r[i] = apply(a, b[i]);
    return r;
}
Mat power(const Mat & a, uint64_t n) {
    Mat r;
    for (int i = 0; i < 64; i++) r[i] = 1ull << i;
    Mat p = a;
    while (n) {
        if (n & 1) r = mul(p, r);
        p = mul(p, p);
        n >>= 1;
    }
    return r;
}
}  // namespace

// jump: [64][64] = A^(chunk*t + 1) for t < 64; adv: [64] = A^V
void rng_tables(int V, int chunk, uint64_t * jump, uint64_t * adv) {
    Mat A;
    for (int i = 0; i < 64; i++) A[i] = host_step(1ull << i);
    for (int t = 0; t < 64; t++) {
        const Mat m = power(A, (uint64_t) chunk * t + 1);
        for (int i = 0; i < 64; i++) jump[t * 64 + i] = m[i];
    }
    const Mat m = power(A, (uint64_t) V);
    for (int i = 0; i < 64; i++) adv[i] = m[i];
}

}  // namespace gsvk

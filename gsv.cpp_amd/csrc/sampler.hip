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
// xorshift64* is linear over GF(2), so the state after n steps is A^n s. Lane t of wave 0 starts
// at draw chunk*t: M s for the precomputed M = A^(chunk*t + 1) is the XOR over the 8 bytes of s
// of a table entry (M applied to that byte), 8 loads; it then steps sequentially through its
// chunk. The next step's state A^V s comes from the same kind of table.
#include <array>
#include <vector>

#include "common.h"
#include "sampler.h"

namespace gsvk {



constexpr int SMP_THREADS = 256;
constexpr int SMP_SORT = 2048;   // >= V
constexpr int SMP_CH = 32;       // >= ceil(V / 64): the generic instantiation
constexpr int SMP_CH17 = 17;     // ceil(V / 64) for vocabularies of up to 1088 (1025 here)

// Largest of a uint32 over the 64 lanes (DPP rotations within rows, then the row results).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x128, 0xf, 0xf, false));
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x124, 0xf, 0xf, false));
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x122, 0xf, 0xf, false));
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x121, 0xf, 0xf, false));
    const uint32_t a = max((uint32_t) __builtin_amdgcn_readlane((int) v, 0), (uint32_t) __builtin_amdgcn_readlane((int) v, 16));
    const uint32_t b = max((uint32_t) __builtin_amdgcn_readlane((int) v, 32), (uint32_t) __builtin_amdgcn_readlane((int) v, 48));
    return max(a, b);
}

// The k-th largest (1 <= k <= 64, counted with multiplicity) of one uint32 per lane: the largest
// T with #{lanes : v >= T} >= k, built bit by bit from the top (the count only falls as T grows,
// and the largest such T is a lane's value). One compare and one ballot per bit.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t v, int k) {
    uint32_t prefix = 0u;
#pragma unroll
    for (int bit = 31; bit >= 0; bit--) {
        const uint32_t trial = prefix | (1u << bit);
        if ((int) __popcll(__ballot(v >= trial)) >= k) prefix = trial;
    }
    return prefix;
}

// Sum of an int over the 64 lanes, returned to every lane: rotations within each row of 16
// lanes (DPP row_ror 8, 4, 2, 1), then the four row totals read as scalars.
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
           __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

__device__ __forceinline__ uint64_t xs_step(uint64_t s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s;
}

// order-preserving map of a float to uint32 (larger float -> larger key) and back
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
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

template <int CH>
__global__ void __launch_bounds__(SMP_THREADS) k_sample(SampleArgs a) {
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int V = a.V;

    __shared__ float lg[SMP_SORT];
    __shared__ int cnt[SMP_SORT];
    // (64 spare slots past SMP_SORT: a lane's branch-free stores of non-survivors)
    __shared__ __align__(16) float sv[SMP_SORT + 64];
    __shared__ int si[SMP_SORT + 64];
    __shared__ float su[SMP_SORT + 64];
    __shared__ float s_scalar[2];
    __shared__ float s_bestv[1];
    __shared__ int s_besti[1];

    // Every load is issued here, before the first use, those whose addresses depend on no loaded
    // value first: the logits and the first 4096 history entries (the penalty window whenever the
    // row holds at most 4096 tokens). The scheduling barrier keeps them ahead of the scalar loads
    // of the row's state, whose values the compiler would otherwise wait for right away.
    constexpr int LV = SMP_SORT / SMP_THREADS;
    float lv[LV];
#pragma unroll
    for (int r = 0; r < LV; r++) {
        const int v = tid + r * SMP_THREADS;
        lv[r] = v < V ? a.logits[(int64_t) b * V + v] : 0.0f;
    }
    constexpr int HW = 4096 / SMP_THREADS;   // the window: the last <= 4096 tokens, 16 per thread
    const int hspec_n = (a.rep != 1.0f && a.ny) ? (a.hist_stride < 4096 ? a.hist_stride : 4096) : 0;
    int htok[HW];
    {
        const int32_t * h = a.hist + (int64_t) b * a.hist_stride;
#pragma unroll
        for (int r = 0; r < HW; r++) {
            const int i = tid + r * SMP_THREADS;
            htok[r] = i < hspec_n ? h[i] : -1;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the loop index, this row's state, the jump matrices and the advance columns
    const int gidx = a.step ? *a.step : 11;   // no loop state: past the EOS-mask window
    const int idx = gidx - (a.row_start ? a.row_start[b] : 0);   // this row's own step
    const int rmax = a.row_max ? a.row_max[b] : a.max_steps;
    const int fin = a.fin_step ? a.fin_step[b] : -1;
    const int n_hist = a.ny ? a.ny[b] : 0;
    const uint64_t s0 = a.rng[b];
    uint64_t st0 = 0, s_next = 0;   // wave 0: this lane's first draw state; A^V s0
    if (tid < 64) {
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const int byte = (int) ((s0 >> (8 * p)) & 255u);
            st0 ^= a.jump[((int64_t) (p * 256 + byte)) * 64 + tid];
            s_next ^= a.adv[p * 256 + byte];
        }
    }
    const int np = a.rep != 1.0f ? (n_hist < 4096 ? n_hist : 4096) : 0;
    if (n_hist > 4096 && np > 0) {   // a longer row: its window starts at n_hist - 4096 (uniform)
        const int32_t * h = a.hist + (int64_t) b * a.hist_stride + (n_hist - np);
#pragma unroll
        for (int r = 0; r < HW; r++) htok[r] = h[tid + r * SMP_THREADS];
    } else {
#pragma unroll
        for (int r = 0; r < HW; r++)
            if (tid + r * SMP_THREADS >= np) htok[r] = -1;
    }
#pragma unroll
    for (int r = 0; r < LV; r++) {
        const int v = tid + r * SMP_THREADS;
        if (v < V) {
            lg[v] = lv[r];
            cnt[v] = 0;
        }
    }
    asm volatile("" ::"v"(st0), "v"(s_next));   // the table loads complete here, not at first use
    __syncthreads();

    const bool running = fin < 0 && idx >= 0 && idx < rmax;
    if (running) {
        if (tid == 0 && a.step && (idx < 11 || (a.flags & 1u))) lg[a.eos] = -INFINITY;
        // 1) repetition penalty, once per occurrence in the window
        if (np > 0) {
#pragma unroll
            for (int r = 0; r < HW; r++) {
                const int t = htok[r];
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
        // 4-6) wave 0: lane t owns indices [t*chunk, t*chunk + chunk), the same ownership as the
        // RNG chunks, so index order is (lane, slot) order
        if (tid < 64) {
            const int chunk = a.chunk;
            const int lane = tid;
            const int base = lane * chunk;
            float pv[CH];
            uint32_t key[CH];
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const bool ok = c < chunk && base + c < V;
                pv[c] = ok ? lg[base + c] : -INFINITY;
                key[c] = ok ? order_key(pv[c]) : 0u;   // below every value, -inf included
            }
            // 4) top-k: pivot = the top_k-th largest value counted with multiplicity (what
            // nth_element leaves at position k-1), found exactly by a radix select over the
            // order-preserving key, most significant bit first; values below it are masked,
            // ties with it stay
            if (a.top_k > 0 && a.top_k < V) {
                const int k = a.top_k;
                bool found = false;
                uint32_t prefix = 0u;
                if (k <= 64) {
                    // T = k-th largest of the 64 lane maxima: at least k values are >= T, so the
                    // pivot is >= T and the k largest values all lie in {key >= T}. When that set
                    // fits in one wave, its k-th largest (one sort) is the pivot.
                    uint32_t lmax = 0u;
#pragma unroll
                    for (int c = 0; c < CH; c++) lmax = key[c] > lmax ? key[c] : lmax;
                    const uint32_t T = wave_kth_largest(lmax, k);
                    int cmine = 0, cbelow = 0, ctotal = 0;
                    int cpos[CH];
#pragma unroll
                    for (int c = 0; c < CH; c++) {
                        const bool in = key[c] >= T && key[c] != 0u;
                        const uint64_t m = __ballot(in);
                        cbelow += __popcll(m & ((1ull << lane) - 1ull));
                        ctotal += __popcll(m);
                        cpos[c] = in ? cmine : -1;
                        cmine += in;
                    }
                    if (ctotal <= 64) {
                        uint32_t * cand = reinterpret_cast<uint32_t *>(si);
                        cand[lane] = 0u;
                        __builtin_amdgcn_wave_barrier();
#pragma unroll
                        for (int c = 0; c < CH; c++)
                            if (cpos[c] >= 0) cand[cbelow + cpos[c]] = key[c];
                        __builtin_amdgcn_wave_barrier();
                        prefix = wave_kth_largest(cand[lane], k);
                        found = true;
                    }
                }
                int rem = k;
                for (int bit = 31; bit >= 0 && !found; bit--) {
                    const uint32_t sel = (bit == 31 ? 0u : (0xffffffffu << (bit + 1))) | (1u << bit);
                    const uint32_t want = prefix | (1u << bit);
                    int c1 = 0;
#pragma unroll
                    for (int c = 0; c < CH; c++) c1 += (key[c] & sel) == want;
                    c1 = wave_sum_i32(c1);
                    if (c1 >= rem) prefix = want;
                    else rem -= c1;
                }
                const float pivot = key_value(prefix);
#pragma unroll
                for (int c = 0; c < CH; c++)
                    if (pv[c] < pivot) pv[c] = -INFINITY;
            }
            // 5) softmax over the survivors. They are compacted into LDS in index order (position
            // = survivors in lower lanes + survivors in lower slots of this lane), so exp runs
            // once per survivor and the sum runs in index order over the non-zero terms only
            // (adding +0 leaves an fp32 sum unchanged).
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < CH; c++) mx = fmaxf(mx, pv[c]);
            mx = warp_max(mx);
            const uint64_t lt_mask = (1ull << lane) - 1ull;
            int below = 0, total = 0, mine = 0;
            int pos[CH];
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const bool sv_c = pv[c] != -INFINITY;
                const uint64_t m = __ballot(sv_c);
                below += __popcll(m & lt_mask);
                total += __popcll(m);
                pos[c] = sv_c ? mine : -1;
                mine += sv_c;
            }
            // every slot is stored, a non-survivor to a spare slot of its own lane (past the
            // SMP_SORT >= V possible survivors), so that the stores need no branch
            const int spare = SMP_SORT + lane;
#pragma unroll
            for (int c = 0; c < CH; c++) {
                if (pos[c] >= 0) pos[c] += below;
                const int slot = pos[c] >= 0 ? pos[c] : spare;
                sv[slot] = pv[c];
                si[slot] = base + c;
            }
            __builtin_amdgcn_wave_barrier();
            for (int jx = lane; jx < total; jx += 64) sv[jx] = (float) exp((double) (sv[jx] - mx));
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) {   // sequential, in index order; four terms per LDS read
                float sum = 0.0f;
                int jx = 0;
                for (; jx + 4 <= total; jx += 4) {
                    const float4 t4 = *reinterpret_cast<const float4 *>(&sv[jx]);
                    sum = sum + t4.x;
                    sum = sum + t4.y;
                    sum = sum + t4.z;
                    sum = sum + t4.w;
                }
                for (; jx < total; jx++) sum = sum + sv[jx];
                s_scalar[0] = 1.0f / sum;
            }
            __builtin_amdgcn_wave_barrier();
            const float inv = s_scalar[0];
            for (int jx = lane; jx < total; jx += 64) sv[jx] = sv[jx] * inv;
            // 6) sample: argmax over p > 0 of p / q, q_i = -log(1 - U_i), U_i the draw of index i.
            // Each lane walks its chunk of the stream and keeps the draws of its survivors.
            // U = (x >> 40) / 2^24 of x = state * 0x2545F4914F6CDD1D: a 24-bit integer times a
            // power of two, exact in fp32. Computed for every slot (no branch), stored for the
            // survivors, the others to the lane's spare slot.
            uint64_t st = st0;
#pragma unroll
            for (int c = 0; c < CH; c++) {
                if (c < chunk && base + c < V) {
                    const uint64_t x = st * 0x2545F4914F6CDD1Dull;
                    su[pos[c] >= 0 ? pos[c] : spare] = (float) (uint32_t) (x >> 40) * 0x1p-24f;
                    st = xs_step(st);
                }
            }
            __builtin_amdgcn_wave_barrier();
            float* dump = nullptr;
            if (a.probs_dump) dump = a.probs_per_row ? a.probs_dump + (int64_t) b * V
                                                     : (b == 0 ? a.probs_dump + (int64_t) idx * V : nullptr);
            if (dump) {
#pragma unroll
                for (int c = 0; c < CH; c++)
                    if (c < chunk && base + c < V) dump[base + c] = pos[c] >= 0 ? sv[pos[c]] : 0.0f;
            }
            float best = -INFINITY;
            int bi = 0x7fffffff;
            for (int jx = lane; jx < total; jx += 64) {   // increasing index within the lane
                const float p = sv[jx];
                const float val = p > 0.0f ? p / -(float) log((double) (1.0f - su[jx])) : 0.0f;
                if (val > best) { best = val; bi = si[jx]; }
            }
            // first maximum wins: larger value, then smaller index
            for (int o = 32; o > 0; o >>= 1) {
                const float ob = __shfl_xor(best, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
            }
            if (lane == 0) {
                s_besti[0] = bi;
                s_bestv[0] = best;
                a.rng[b] = s_next;
            }
        }
        __syncthreads();
        if (tid == 0) {
            int tok = s_besti[0];
            if (tok < 0 || tok >= V) tok = 0;   // no value > 0: the first index wins
            if (a.tok_out) a.tok_out[b] = tok;
            if (a.step) {
                if (a.sampled_dump) a.sampled_dump[(int64_t) gidx * a.B + b] = tok;
                if (a.oracle && idx < a.n_oracle) tok = a.oracle[idx];
                const int n = n_hist;
                a.hist[(int64_t) b * a.hist_stride + n] = tok;
                a.ny[b] = n + 1;
                a.last_tok[b] = tok;
                if (tok == a.eos) {
                    a.fin_step[b] = idx;
                    a.fin_kind[b] = 0;
                } else if ((a.flags & 2u) && a.early_stop != -1 && n + 1 - a.P > a.early_stop) {
                    a.fin_step[b] = idx;   // the early-stop rule on this row's own tokens
                    a.fin_kind[b] = 1;
                }
            }
        }
    }
    if (!a.step) return;   // single sampling call: no loop state
    // the last workgroup to finish applies the batch-wide early-stop rule, counts the rows that
    // take part in the next step and advances the loop index; its threads take the rows in turn
    __shared__ int s_last, s_unfinished;
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const int prev = __hip_atomic_fetch_add(a.done_counter, 1, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == a.B - 1;
        s_unfinished = 0;
    }
    __syncthreads();
    if (!s_last) return;   // uniform over the workgroup
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (gidx < a.max_steps) {
        const bool stop_all = a.early_stop != -1 && !(a.flags & 2u) &&
                              __hip_atomic_load(a.ny, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - a.P >
                                  a.early_stop;
        int unfinished = 0;
        for (int bb = tid; bb < a.B; bb += SMP_THREADS) {
            bool open = __hip_atomic_load(a.fin_step + bb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < 0;
            const int rs = a.row_start ? a.row_start[bb] : 0;
            if (open && stop_all) {   // every row still open stops at this step
                a.fin_step[bb] = gidx - rs;
                a.fin_kind[bb] = 1;
                open = false;
            }
            // with per-row limits, only the rows that take part in the next step
            unfinished += a.row_max ? (open && gidx + 1 - rs < a.row_max[bb]) : open;
        }
        if (unfinished) atomicAdd(&s_unfinished, unfinished);
        __syncthreads();
        if (tid == 0) {
            if (a.active) *a.active = *a.n_unfinished > 0 ? 1 : 0;   // (the count before this step)
            *a.n_unfinished = s_unfinished;
            if (a.n_unfinished_host)
                __hip_atomic_store(a.n_unfinished_host, s_unfinished, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            *a.step = gidx + 1;
        }
    }
    if (tid == 0) __hip_atomic_store(a.done_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int launch_sample(const SampleArgs & a, hipStream_t stream) {
    GSVK_REQUIRE(a.V > 0 && a.V <= SMP_SORT && a.B > 0 && a.chunk * 64 >= a.V && a.chunk <= SMP_CH,
                 "sample: vocabulary %d exceeds %d", a.V, SMP_SORT);
    GSVK_REQUIRE(a.top_k < 0 || a.top_k <= SMP_SORT, "sample: bad top_k");
    // the per-lane loops run over CH slots: 17 covers the vocabulary of the t2s model exactly
    if (a.chunk <= SMP_CH17)
        hipLaunchKernelGGL(k_sample<SMP_CH17>, dim3((unsigned) a.B), dim3(SMP_THREADS), 0, stream, a);
    else
        hipLaunchKernelGGL(k_sample<SMP_CH>, dim3((unsigned) a.B), dim3(SMP_THREADS), 0, stream, a);
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

// out[p][v] (stride `stride` between v entries) = M applied to byte value v at byte position p
void byte_table(const Mat & m, uint64_t * out, int64_t stride) {
    for (int p = 0; p < 8; p++) {
        uint64_t * row = out + (int64_t) p * 256 * stride;
        row[0] = 0;
        for (int v = 1; v < 256; v++) {
            const int low = __builtin_ctz(v);
            row[(int64_t) v * stride] = row[(int64_t) (v & (v - 1)) * stride] ^ m[8 * p + low];
        }
    }
}
}  // namespace

// jump: [8][256][64], entry (p, v, t) = A^(chunk*t + 1) applied to byte v at byte position p;
// adv: [8][256], the same for A^V
void rng_tables(int V, int chunk, uint64_t * jump, uint64_t * adv) {
    Mat A;
    for (int i = 0; i < 64; i++) A[i] = host_step(1ull << i);
    for (int t = 0; t < 64; t++) byte_table(power(A, (uint64_t) chunk * t + 1), jump + t, 64);
    byte_table(power(A, (uint64_t) V), adv, 1);
}

size_t sample_workspace_bytes() { return (size_t) (RNG_JUMP_WORDS + RNG_ADV_WORDS) * sizeof(uint64_t); }

}  // namespace gsvk

extern "C" size_t gsvk_sample_workspace_bytes(int V) {
    (void) V;
    return gsvk::sample_workspace_bytes();
}

extern "C" int gsvk_op_sample(const float * logits, int B, int V, const int32_t * hist, int hist_stride,
                              const int32_t * n_hist, const gsvk_sampler_cfg * cfg, uint64_t * rng,
                              int32_t * tok_out, float * probs_out, void * ws, void * stream) {
    using namespace gsvk;
    GSVK_REQUIRE(logits && cfg && rng && tok_out && ws, "sample: null pointer");
    GSVK_REQUIRE(B > 0 && V > 0 && V <= SMP_SORT, "sample: bad shape B=%d V=%d (V <= %d)", B, V, SMP_SORT);
    GSVK_REQUIRE((hist == nullptr) == (n_hist == nullptr) && (!hist || hist_stride > 0),
                 "sample: hist and n_hist go together");
    GSVK_REQUIRE(((uintptr_t) ws & 7) == 0, "sample: workspace must be 8-byte aligned");
    const hipStream_t st = (hipStream_t) stream;
    const int chunk = (V + 63) / 64;
    std::vector<uint64_t> tab(RNG_JUMP_WORDS + RNG_ADV_WORDS);
    rng_tables(V, chunk, tab.data(), tab.data() + RNG_JUMP_WORDS);
    uint64_t * jump = (uint64_t *) ws;
    GSVK_HIP(hipMemcpyAsync(jump, tab.data(), tab.size() * 8, hipMemcpyHostToDevice, st));
    SampleArgs a{};
    a.logits = logits;
    a.V = V;
    a.eos = -1;
    a.B = B;
    a.hist = const_cast<int32_t *>(hist);
    a.hist_stride = hist_stride;
    a.ny = const_cast<int32_t *>(n_hist);
    a.rng = rng;
    a.jump = jump;
    a.adv = jump + RNG_JUMP_WORDS;
    a.chunk = chunk;
    a.top_k = cfg->top_k;
    a.top_p = cfg->top_p;
    a.temperature = cfg->temperature;
    a.rep = cfg->repetition_penalty;
    a.max_steps = 1 << 30;
    a.probs_dump = probs_out;
    a.probs_per_row = 1;
    a.tok_out = tok_out;
    GSVK_TRY(launch_sample(a, st));
    GSVK_HIP(hipStreamSynchronize(st));   // the table upload reads host memory
    return GSVK_OK;
}

// Host stand-in for <hip/hip_runtime.h>, for running the library's gfx950 kernels on the CPU under
// AddressSanitizer: every thread of a workgroup is a fiber (emu.h); barriers and the wave-wide
// exchanges the kernels use (shuffles, DPP, ds_swizzle, readlane, ballot) are resolved once every
// live lane of the wave (or thread of the workgroup) has reached them. Test infrastructure only:
// it checks index arithmetic and buffer bounds, not speed, and nothing in the library uses it.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#define __global__
#define __device__
#define __host__
#define __constant__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))
#define __shared__ static

struct dim3 {
    unsigned x = 1, y = 1, z = 1;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

typedef int hipError_t;
constexpr hipError_t hipSuccess = 0;
typedef struct emu_stream * hipStream_t;
enum hipMemcpyKind { hipMemcpyHostToHost, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice };
inline const char * hipGetErrorString(hipError_t) { return "host emulation"; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipGetDevice(int * d) { *d = 0; return hipSuccess; }
inline hipError_t hipMalloc(void ** p, size_t n) { *p = std::malloc(n); return *p ? hipSuccess : 1; }
inline hipError_t hipFree(void * p) { std::free(p); return hipSuccess; }
inline hipError_t hipMemcpyAsync(void * d, const void * s, size_t n, hipMemcpyKind, hipStream_t = nullptr) {
    std::memcpy(d, s, n);
    return hipSuccess;
}
inline hipError_t hipMemcpy(void * d, const void * s, size_t n, hipMemcpyKind) { std::memcpy(d, s, n); return hipSuccess; }
inline hipError_t hipMemsetAsync(void * d, int v, size_t n, hipStream_t = nullptr) { std::memset(d, v, n); return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
#define HIP_SYMBOL(s) (&(s))
template <typename T>
inline hipError_t hipGetSymbolAddress(void ** p, T * sym) { *p = (void *) sym; return hipSuccess; }

// ---- vector types ----
#define EMU_VEC2(N, T) struct N { T x, y; }; inline N make_##N(T a, T b) { return N{a, b}; }
#define EMU_VEC4(N, T) struct N { T x, y, z, w; }; inline N make_##N(T a, T b, T c, T d) { return N{a, b, c, d}; }
EMU_VEC2(int2, int)
EMU_VEC2(uint2, unsigned)
EMU_VEC2(float2, float)
EMU_VEC4(int4, int)
EMU_VEC4(uint4, unsigned)
EMU_VEC4(float4, float)
EMU_VEC4(char4, signed char)

#include "../emu.h"

#define threadIdx (::emu::cur().tid)
#define blockIdx (::emu::cur().bid)
#define blockDim (::emu::cur().bdim)
#define gridDim (::emu::cur().gdim)

using std::max;
using std::min;
inline int max(int a, int b) { return a > b ? a : b; }
inline int min(int a, int b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long max(long a, long b) { return a > b ? a : b; }
inline long min(long a, long b) { return a < b ? a : b; }

inline int __float_as_int(float f) { int i; std::memcpy(&i, &f, 4); return i; }
inline float __int_as_float(int i) { float f; std::memcpy(&f, &i, 4); return f; }
inline unsigned __float_as_uint(float f) { unsigned i; std::memcpy(&i, &f, 4); return i; }
inline float __uint_as_float(unsigned i) { float f; std::memcpy(&f, &i, 4); return f; }
inline int __double2hiint(double d) { uint64_t u; std::memcpy(&u, &d, 8); return (int) (u >> 32); }
inline int __double2loint(double d) { uint64_t u; std::memcpy(&u, &d, 8); return (int) (uint32_t) u; }
inline double __hiloint2double(int hi, int lo) {
    const uint64_t u = ((uint64_t) (uint32_t) hi << 32) | (uint32_t) lo;
    double d; std::memcpy(&d, &u, 8); return d;
}
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __popc(unsigned v) { return __builtin_popcount(v); }

// ---- synchronisation and wave-wide operations (emu.h) ----
inline void __syncthreads() { ::emu::barrier(); }
inline void __threadfence() {}
inline void __threadfence_block() {}
#define __builtin_amdgcn_fence(...) ((void) 0)
#define __builtin_amdgcn_sched_barrier(x) ((void) 0)
#define __builtin_amdgcn_s_waitcnt(x) ((void) 0)
#define __builtin_amdgcn_s_barrier() ::emu::barrier()
inline void __builtin_amdgcn_wave_barrier() { ::emu::wave_sync(); }

template <typename T>
inline T __shfl_xor(T v, int mask, int width = 64) { return ::emu::shfl_xor(v, mask, width); }
template <typename T>
inline T __shfl(T v, int src, int width = 64) { return ::emu::shfl(v, src, width); }
template <typename T>
inline T __shfl_up(T v, unsigned delta, int width = 64) {   // 1-D workgroups: lane = threadIdx.x % 64
    const int lane = (int) (threadIdx.x & 63), base = lane & ~(width - 1), src = lane - (int) delta;
    return ::emu::shfl(v, src >= base ? src : lane, 64);
}
inline unsigned long long __ballot(int pred) { return ::emu::ballot(pred != 0); }
inline int __any(int pred) { return ::emu::ballot(pred != 0) != 0; }
inline int __all(int pred) { return ::emu::ballot(pred != 0) == ::emu::live_mask(); }
inline int __builtin_amdgcn_readlane(int v, int l) { return ::emu::readlane(v, l); }
inline int __builtin_amdgcn_readfirstlane(int v) { return ::emu::readfirstlane(v); }
inline int __builtin_amdgcn_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    return ::emu::update_dpp(old, src, ctrl, row_mask, bank_mask, bound_ctrl);
}
inline int __builtin_amdgcn_mov_dpp(int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    return ::emu::update_dpp(0, src, ctrl, row_mask, bank_mask, bound_ctrl);
}
inline int __builtin_amdgcn_ds_swizzle(int v, int pattern) { return ::emu::ds_swizzle(v, pattern); }

// ---- arithmetic builtins ----
inline float __builtin_amdgcn_exp2f(float x) { return std::exp2(x); }
inline int __builtin_amdgcn_sdot4(int a, int b, int c, bool) {
    int s = c;
    for (int i = 0; i < 4; i++) s += (int) (int8_t) (a >> (8 * i)) * (int) (int8_t) (b >> (8 * i));
    return s;
}

// ---- atomics (one fiber runs at a time) ----
// (__hip_atomic_load / store / fetch_add are clang builtins on the host too; the scopes are not
// predefined there)
#ifndef __HIP_MEMORY_SCOPE_SINGLETHREAD
#define __HIP_MEMORY_SCOPE_SINGLETHREAD 1
#define __HIP_MEMORY_SCOPE_WAVEFRONT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __HIP_MEMORY_SCOPE_SYSTEM 5
#endif
template <typename T, typename U> inline T atomicAdd(T * p, U v) { T o = *p; *p = (T) (o + v); return o; }

// ---- launch ----
#define hipLaunchKernelGGL(K, grid, block, shmem, stream, ...) ::emu::launch(K, dim3(grid), dim3(block), ##__VA_ARGS__)

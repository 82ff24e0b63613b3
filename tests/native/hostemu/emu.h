// Workgroup emulation for the host stand-in of the HIP runtime (hip/hip_runtime.h): the threads
// of one workgroup run as fibers (ucontext) on one OS thread; a barrier or a wave-wide exchange
// suspends the fiber until every live thread of the workgroup (barrier) or lane of the wave
// (exchange) has reached it, then resolves it with wave64 semantics. Workgroups run one after
// another. A fiber starts with swapcontext and switches with _setjmp / _longjmp afterwards (no
// signal-mask system call per switch). AddressSanitizer is told about every stack switch.
#pragma once

#include <setjmp.h>
#include <ucontext.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#include <sanitizer/common_interface_defs.h>
#define EMU_ASAN 1
#endif
#endif

namespace emu {

struct Idx {
    unsigned x = 0, y = 0, z = 0;
};

enum { RUN = 0, AT_BARRIER = 1, AT_WAVE = 2, DONE = 3 };
enum { OP_SHFL_XOR = 1, OP_SHFL, OP_READLANE, OP_READFIRST, OP_BALLOT, OP_DPP, OP_SWIZZLE, OP_SYNC };

struct Thread {
    Idx tid, bid, bdim, gdim;
    ucontext_t ctx;
    jmp_buf jb;
    char * stack = nullptr;
    int state = DONE;
    int lane = 0, wave = 0;
    int op = 0;
    uint64_t a = 0, old = 0;
    int p0 = 0, p1 = 0, p2 = 0, p3 = 0, p4 = 0;
    uint64_t result = 0;
    void * fake = nullptr;
};

constexpr size_t STACK = 512 * 1024;

struct Sched {
    ucontext_t main;
    jmp_buf main_jb;
    std::vector<Thread> th;
    int cur = 0;
    std::function<void()> fn;
    const void * main_bottom = nullptr;
    size_t main_size = 0;
    long long switches = 0;
};

inline Sched & S() {
    static Sched s;
    return s;
}
inline Thread & cur() { return S().th[S().cur]; }

inline void to_main(bool exiting) {
    Thread & t = cur();
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(exiting ? nullptr : &t.fake, S().main_bottom, S().main_size);
#endif
    if (exiting || !_setjmp(t.jb)) _longjmp(S().main_jb, 1);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(cur().fake, &S().main_bottom, &S().main_size);
#endif
}

inline void trampoline() {
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(nullptr, &S().main_bottom, &S().main_size);
#endif
    S().fn();
    cur().state = DONE;
    to_main(true);
}

inline void barrier() {
    cur().state = AT_BARRIER;
    to_main(false);
}

inline uint64_t wave_op(int op, uint64_t a, int p0 = 0, int p1 = 0, int p2 = 0, int p3 = 0, int p4 = 0,
                        uint64_t old = 0) {
    Thread & t = cur();
    t.op = op;
    t.a = a;
    t.old = old;
    t.p0 = p0; t.p1 = p1; t.p2 = p2; t.p3 = p3; t.p4 = p4;
    t.state = AT_WAVE;
    to_main(false);
    return cur().result;
}

template <typename T>
inline uint64_t bits(T v) {
    static_assert(sizeof(T) <= 8, "64-bit payloads at most");
    uint64_t u = 0;
    std::memcpy(&u, &v, sizeof(T));
    return u;
}
template <typename T>
inline T unbits(uint64_t u) {
    T v;
    std::memcpy(&v, &u, sizeof(T));
    return v;
}

template <typename T>
inline T shfl_xor(T v, int mask, int width) { return unbits<T>(wave_op(OP_SHFL_XOR, bits(v), mask, width)); }
template <typename T>
inline T shfl(T v, int src, int width) { return unbits<T>(wave_op(OP_SHFL, bits(v), src, width)); }
inline int readlane(int v, int l) { return unbits<int>(wave_op(OP_READLANE, bits(v), l)); }
inline int readfirstlane(int v) { return unbits<int>(wave_op(OP_READFIRST, bits(v))); }
inline uint64_t ballot(bool p) { return wave_op(OP_BALLOT, p ? 1 : 0); }
inline int update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    return unbits<int>(wave_op(OP_DPP, bits(src), ctrl, row_mask, bank_mask, bound_ctrl ? 1 : 0, 0, bits(old)));
}
inline int ds_swizzle(int v, int pattern) { return unbits<int>(wave_op(OP_SWIZZLE, bits(v), pattern)); }
inline void wave_sync() { (void) wave_op(OP_SYNC, 0); }
inline uint64_t live_mask();

// source lane of a DPP control for lane l (-1: no source)
inline int dpp_src(int ctrl, int l) {
    const int r = l & 15, base = l & ~15;
    if (ctrl >= 0 && ctrl <= 0xff) return (l & ~3) | ((ctrl >> (2 * (l & 3))) & 3);
    if (ctrl >= 0x101 && ctrl <= 0x10f) { const int n = ctrl - 0x100; return r + n <= 15 ? l + n : -1; }
    if (ctrl >= 0x111 && ctrl <= 0x11f) { const int n = ctrl - 0x110; return r - n >= 0 ? l - n : -1; }
    if (ctrl >= 0x121 && ctrl <= 0x12f) { const int n = ctrl - 0x120; return base | ((r - n + 16) & 15); }
    if (ctrl == 0x138) return l >= 1 ? l - 1 : -1;                  // wave_shr:1
    if (ctrl == 0x140) return base | (15 - r);
    if (ctrl == 0x141) return (l & ~7) | (7 - (l & 7));
    if (ctrl == 0x142) return base >= 16 ? base - 1 : -1;           // row_bcast:15
    if (ctrl == 0x143) return base >= 32 ? 31 : -1;                 // row_bcast:31
    std::fprintf(stderr, "emu: DPP control 0x%x not emulated\n", ctrl);
    std::abort();
}

// Resolve the wave ops of wave w when all its live lanes have reached one.
inline bool resolve_wave(int first, int n) {
    auto & th = S().th;
    int op = 0;
    bool any = false;
    for (int i = first; i < first + n; i++) {
        if (th[i].state == DONE) continue;
        if (th[i].state != AT_WAVE) return false;
        if (op && th[i].op != op) {
            std::fprintf(stderr, "emu: lanes of one wave at different exchanges (%d, %d)\n", op, th[i].op);
            std::abort();
        }
        op = th[i].op;
        any = true;
    }
    if (!any) return false;
    uint64_t val[64] = {};
    bool live[64] = {};
    for (int l = 0; l < n; l++) {
        live[l] = th[first + l].state == AT_WAVE;
        val[l] = th[first + l].a;
    }
    uint64_t ballot = 0;
    int firstl = -1;
    for (int l = 0; l < n; l++) {
        if (live[l] && (val[l] & 1)) ballot |= 1ull << l;
        if (live[l] && firstl < 0) firstl = l;
    }
    for (int l = 0; l < n; l++) {
        Thread & t = th[first + l];
        if (!live[l]) continue;
        int src = l;
        switch (op) {
        case OP_SHFL_XOR: {
            const int w = t.p1, idx = l ^ t.p0;
            src = idx >= ((l + w) & ~(w - 1)) ? l : idx;
            t.result = src < n ? val[src] : val[l];
            break;
        }
        case OP_SHFL: {
            const int w = t.p1;
            src = (t.p0 & (w - 1)) + (l & ~(w - 1));
            t.result = src < n ? val[src] : val[l];
            break;
        }
        case OP_READLANE: t.result = (t.p0 >= 0 && t.p0 < n) ? val[t.p0] : 0; break;
        case OP_READFIRST: t.result = val[firstl]; break;
        case OP_BALLOT: t.result = ballot; break;
        case OP_DPP: {
            const int row = l >> 4, bank = (l >> 2) & 3;
            if (!((t.p1 >> row) & 1) || !((t.p2 >> bank) & 1)) { t.result = t.old; break; }
            src = dpp_src(t.p0, l);
            t.result = src < 0 || src >= n ? (t.p3 ? 0 : t.old) : val[src];
            break;
        }
        case OP_SWIZZLE: {
            const int p = t.p0;
            if (p & 0x8000) src = (l & ~3) | ((p >> (2 * (l & 3))) & 3);
            else src = (l & ~31) | ((((l & 31) & (p & 31)) | ((p >> 5) & 31)) ^ ((p >> 10) & 31));
            t.result = src < n ? val[src] : 0;
            break;
        }
        case OP_SYNC: t.result = 0; break;
        default: std::abort();
        }
        t.state = RUN;
    }
    return true;
}

template <typename F>
void launch_fn(dim3 grid, dim3 block, F && fn) {
    Sched & s = S();
    const int nt = (int) (block.x * block.y * block.z);
    if ((int) s.th.size() < nt) s.th.resize(nt);
    for (int i = 0; i < nt; i++)
        if (!s.th[i].stack) s.th[i].stack = (char *) std::malloc(STACK);
    s.fn = fn;
    for (unsigned bz = 0; bz < grid.z; bz++)
        for (unsigned by = 0; by < grid.y; by++)
            for (unsigned bx = 0; bx < grid.x; bx++) {
                for (int i = 0; i < nt; i++) {
                    Thread & t = s.th[i];
                    t.tid = Idx{(unsigned) (i % block.x), (unsigned) ((i / block.x) % block.y),
                                (unsigned) (i / (block.x * block.y))};
                    t.bid = Idx{bx, by, bz};
                    t.bdim = Idx{block.x, block.y, block.z};
                    t.gdim = Idx{grid.x, grid.y, grid.z};
                    t.lane = i & 63;
                    t.wave = i >> 6;
                    t.state = RUN;
                    getcontext(&t.ctx);
                    t.ctx.uc_stack.ss_sp = t.stack;
                    t.ctx.uc_stack.ss_size = STACK;
                    t.ctx.uc_link = nullptr;
                    makecontext(&t.ctx, (void (*)()) trampoline, 0);
                }
                std::vector<char> started(nt, 0);
                for (;;) {
                    bool ran = false;
                    for (int i = 0; i < nt; i++) {
                        if (s.th[i].state != RUN) continue;
                        s.cur = i;
                        void * fake = nullptr;
#ifdef EMU_ASAN
                        __sanitizer_start_switch_fiber(&fake, s.th[i].stack, STACK);
#endif
                        if (!_setjmp(s.main_jb)) {
                            if (started[i]) _longjmp(s.th[i].jb, 1);
                            started[i] = 1;
                            swapcontext(&s.main, &s.th[i].ctx);
                        }
#ifdef EMU_ASAN
                        __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
                        s.switches++;
                        ran = true;
                    }
                    bool resolved = false;
                    for (int w = 0; w * 64 < nt; w++) resolved |= resolve_wave(w * 64, std::min(64, nt - w * 64));
                    int alive = 0, at_bar = 0;
                    for (int i = 0; i < nt; i++) {
                        alive += s.th[i].state != DONE;
                        at_bar += s.th[i].state == AT_BARRIER;
                    }
                    if (alive == 0) break;
                    if (at_bar == alive) {
                        for (int i = 0; i < nt; i++)
                            if (s.th[i].state == AT_BARRIER) s.th[i].state = RUN;
                        resolved = true;
                    }
                    if (!ran && !resolved) {
                        std::fprintf(stderr, "emu: workgroup (%u, %u, %u) deadlocked (%d live, %d at a barrier)\n", bx,
                                     by, bz, alive, at_bar);
                        std::abort();
                    }
                }
            }
}

template <typename... KA, typename... A>
void launch(void (*k)(KA...), dim3 grid, dim3 block, A... args) {
    launch_fn(grid, block, [=]() { k(args...); });
}

inline uint64_t live_mask() {
    // the live lanes of the current wave (those not finished)
    Sched & s = S();
    const int w0 = cur().wave * 64;
    uint64_t m = 0;
    for (int l = 0; l < 64 && w0 + l < (int) s.th.size(); l++)
        if (s.th[w0 + l].state != DONE) m |= 1ull << l;
    return m;
}

}  // namespace emu

// Host check of gsv.cpp_amd/csrc/expf_exact.h: expf_glibc equals this host's expf (the libm the
// oracle and the reference's ggml-cpu call) on every non-NaN float (argument: a step, default 1,
// to check every step-th bit pattern only). Prints the count of floats checked and of those that
// differ; exits 1 if any differs.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "expf_exact.h"

int main(int argc, char ** argv) {
    static const uint64_t tab[32] = GSVK_EXP2_TAB32;
    const uint64_t step = argc > 1 ? std::max(1ull, std::strtoull(argv[1], nullptr, 10)) : 1;
    const unsigned nt = std::max(1u, std::thread::hardware_concurrency());
    std::vector<long long> bad(nt, 0), n(nt, 0);
    std::vector<uint32_t> first(nt, 0);
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++)
        th.emplace_back([&, t] {
            const uint64_t lo = (1ull << 32) / nt * t, hi = t + 1 == nt ? (1ull << 32) : (1ull << 32) / nt * (t + 1);
            for (uint64_t u = (lo + step - 1) / step * step; u < hi; u += step) {
                const uint32_t uu = (uint32_t) u;
                float x;
                std::memcpy(&x, &uu, 4);
                if (std::isnan(x)) continue;
                const float a = expf(x), b = gsvk::expf_glibc(x, tab);
                n[t]++;
                if (std::memcmp(&a, &b, 4) != 0) {
                    if (!bad[t]) first[t] = uu;
                    bad[t]++;
                }
            }
        });
    for (auto & x : th) x.join();
    long long B = 0, N = 0;
    uint32_t f = 0;
    for (unsigned t = 0; t < nt; t++) {
        if (bad[t] && !B) f = first[t];
        B += bad[t];
        N += n[t];
    }
    std::printf("checked %lld floats, %lld differ%s", N, B, B ? "" : "\n");
    if (B) std::printf(" (first 0x%08x)\n", f);
    return B != 0;
}

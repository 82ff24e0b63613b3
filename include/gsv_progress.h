#pragma once
// The engine's coarse synthesis progress (the reference's src/gsv_progress.h, read by its HTTP
// server's /progress): three process-wide counters that the AR stage sets while it decodes.
//
// The names, types and the inline-variable form are the interface: C++17 inline variables with
// default visibility are one object per process, so the counters this library updates are the
// ones the engine's server reads when the engine links libgsvk.so. Only what the AR stage uses is
// declared here: begin (stage 2 = AR, with the step budget) and one tick per decode step.
#include <atomic>

namespace gsvprog {

inline std::atomic<int> stage{0};   // 2 while the AR decoder runs
inline std::atomic<int> cur{0};     // steps done
inline std::atomic<int> total{0};   // step budget

inline void begin(int st, int t = 0) {
    cur.store(0);
    total.store(t);
    stage.store(st);
}

inline void tick() { cur.fetch_add(1); }

}  // namespace gsvprog

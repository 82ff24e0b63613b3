// Device sampler interface (sampler.hip).
#pragma once

#include "common.h"

namespace gsvk {

struct SampleArgs {
    const float * logits;      // [B][V]
    int V, eos, B, P;
    int32_t * hist;            // [B][hist_stride] prompt + generated tokens
    int hist_stride;
    int32_t * ny;              // [B] tokens in hist (null = no history)
    int32_t * fin_step;        // [B] -1 while running (null with step == null)
    int32_t * fin_kind;        // [B] 0 EOS, 1 early stop
    uint64_t * rng;            // [B] xorshift64* state
    const uint64_t * jump;     // [8][256][64] byte tables of A^(chunk*t + 1), see rng_tables
    const uint64_t * adv;      // [8][256] byte tables of A^V
    int chunk;                 // draws per lane of wave 0
    int top_k;
    float top_p, temperature, rep;
    const int32_t * oracle;    // teacher forcing tokens or null
    int n_oracle;
    int32_t * step;            // device loop index; null = one sampling call without loop
                               // state (no EOS mask, no history append, no bookkeeping)
    unsigned flags;            // bit0: mask EOS at every step
    int32_t * last_tok;        // [B]
    float * probs_dump;        // [max_steps][V] for sequence 0 (probs_per_row: [B][V]), or null
    int probs_per_row;
    int32_t * tok_out;         // [B] sampled token (before any oracle override), or null
    int32_t * sampled_dump;    // [max_steps][B] sampler choice before the oracle, or null
    int max_steps;
    int32_t * done_counter;    // zero between calls
    int32_t * n_unfinished;    // written by the last workgroup
    int32_t * n_unfinished_host;   // the same count in mapped pinned host memory (or null): the
                                   // host reads it once the step's event has completed
    int32_t * active;          // or null: set by the last workgroup to whether any row took part
                               // in this step (the count before it, *n_unfinished, was nonzero);
                               // a decode kernel after the sampler may skip a step that is not
    int early_stop;            // -1 = off
    // a batch that sequences join while it decodes: row b takes part from loop index
    // row_start[b] on, for at most row_max[b] steps, its EOS-mask window, oracle, dumps and
    // finish step counted from there; with bit 1 of flags the early-stop rule is applied per row
    // (its own token count) instead of on sequence 0 for the whole batch. Null: every row starts
    // at 0 with max_steps.
    const int32_t * row_start;
    const int32_t * row_max;
};

int launch_sample(const SampleArgs & a, hipStream_t stream);

// A is the GF(2) matrix of one xorshift64* state update. jump (RNG_JUMP_WORDS): entry
// [p][v][t] = A^(chunk*t + 1) applied to the state whose only non-zero byte is v at byte p, so
// that A^(chunk*t + 1) s = XOR over p of jump[p][byte p of s][t]; adv (RNG_ADV_WORDS): [p][v],
// the same for A^V.
constexpr int RNG_JUMP_WORDS = 8 * 256 * 64;
constexpr int RNG_ADV_WORDS = 8 * 256;
void rng_tables(int V, int chunk, uint64_t * jump, uint64_t * adv);

}  // namespace gsvk

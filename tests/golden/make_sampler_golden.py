"""Write tests/golden/sampler_golden.npz: input/output vectors of the reference sampler.

The reference's src/gsv_sampler.cpp has no ggml dependency; oracle/Makefile compiles it from the
reference tree into oracle/_ref/libgsv_sampler_ref.so (in the build container only). This
script calls that library on seeded inputs and stores inputs and outputs as plain arrays:

* logits_to_probs: (cfg, logits, prev) -> (logits after the call, probs), covering repeated
  tokens in the history (penalty once per occurrence), top-k ties, top-p < 1, -inf entries
  (the EOS mask), temperature extremes, top-k >= V, top-k = 1 and disabled filters;
* rng: xorshift64* streams (next()) and exponential draws for several seeds, including 0;
* sample: (probs, seed) -> token and the final RNG state.

Run: python tests/golden/make_sampler_golden.py   (needs oracle/_ref built: make -C oracle)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import ctypes as C  # noqa: E402

import oracle  # noqa: E402

V = 1025
EOS = 1024


def cases(rng):
    out = []
    base = lambda: (rng.standard_normal(V) * 0.5).astype(np.float32)   # noqa: E731
    # defaults of the reference (15 / 1.0 / 1.0 / 1.35) with a prompt-like history
    for i in range(4):
        lg = base()
        if i % 2 == 0:
            lg[EOS] = -np.inf
        prev = rng.integers(0, V, size=rng.integers(1, 400)).astype(np.int32)
        out.append(((15, 1.0, 1.0, 1.35), lg, prev))
    # repeated tokens: one token 7 times, another 3 times, negative and positive logits
    lg = base()
    lg[5], lg[9] = -0.8, 0.9
    out.append(((15, 1.0, 1.0, 1.35), lg, np.array([5] * 7 + [9] * 3 + [1, 2], np.int32)))
    # ties at the top-k pivot (values equal to the k-th largest are kept)
    lg = np.round(base() * 4) / 4
    out.append(((15, 1.0, 1.0, 1.35), lg.astype(np.float32), np.array([], np.int32)))
    out.append(((3, 1.0, 1.0, 1.0), np.full(V, 0.25, np.float32), None))
    # top-p < 1 (stable descending order; rank 0 always kept), with and without top-k
    for tp in (0.9, 0.5, 0.05):
        out.append(((0, tp, 1.0, 1.35), base(), rng.integers(0, V, 50).astype(np.int32)))
    out.append(((15, 0.7, 0.8, 1.35), base(), rng.integers(0, V, 50).astype(np.int32)))
    lg = np.round(base() * 2) / 2
    out.append(((0, 0.6, 1.0, 1.0), lg.astype(np.float32), None))
    # temperature extremes (0 -> 1e-5), top-k >= V, top-k 1 (greedy), all filters off
    out.append(((15, 1.0, 0.0, 1.35), base(), None))
    out.append(((15, 1.0, 5.0, 1.35), base(), None))
    out.append(((V, 1.0, 1.0, 1.35), base(), rng.integers(0, V, 30).astype(np.int32)))
    out.append(((1, 1.0, 1.0, 1.35), base(), rng.integers(0, V, 30).astype(np.int32)))
    out.append(((0, 1.0, 1.0, 1.0), base(), None))
    # history longer than the 4096 window of the caller is the caller's job; long history here
    out.append(((15, 1.0, 1.0, 1.35), base(), rng.integers(0, V, 4096).astype(np.int32)))
    # out-of-range history entries are skipped
    out.append(((15, 1.0, 1.0, 1.35), base(), np.array([-1, V, V + 5, 3], np.int32)))
    return out


def main():
    oracle.build()
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libgsv_sampler_ref.so is missing (needs the reference tree)")
    rng = np.random.default_rng(20261201)
    cs = cases(rng)
    n = len(cs)
    cfg = np.zeros((n, 4), np.float32)
    lg_in = np.zeros((n, V), np.float32)
    lg_out = np.zeros((n, V), np.float32)
    probs = np.zeros((n, V), np.float32)
    prev = np.full((n, 4096), -2, np.int32)      # -2 = padding marker, n_prev holds the length
    n_prev = np.zeros(n, np.int32)
    has_prev = np.zeros(n, np.int32)
    for i, ((k, p, t, r), lg, pv) in enumerate(cs):
        cfg[i] = (k, p, t, r)
        lg_in[i] = lg
        work = lg.copy()
        pr = np.zeros(V, np.float32)
        if pv is not None:
            prev[i, :len(pv)] = pv
            n_prev[i] = len(pv)
            has_prev[i] = 1
            pp = np.ascontiguousarray(pv, np.int32)
            ref.ref_logits_to_probs(k, p, t, r, work, V, pp.ctypes.data_as(C.c_void_p), len(pv), pr)
        else:
            ref.ref_logits_to_probs(k, p, t, r, work, V, None, 0, pr)
        lg_out[i] = work
        probs[i] = pr
    seeds = np.array([0, 1, 12345, 0x9E3779B97F4A7C15, 7 + 0x9E3779B9 * 3, 2 ** 63 + 11], np.uint64)
    streams = np.zeros((len(seeds), 2100), np.uint64)
    exps = np.zeros((len(seeds), 2100), np.float32)
    final_state = np.zeros(len(seeds), np.uint64)
    for i, sd in enumerate(seeds):
        final_state[i] = ref.ref_rng_stream(int(sd), 2100, streams[i])
        ref.ref_rng_exponential(int(sd), 2100, exps[i])
    sample_tok = np.zeros((n, len(seeds)), np.int32)
    sample_state = np.zeros((n, len(seeds)), np.uint64)
    for i in range(n):
        for j, sd in enumerate(seeds):
            st = C.c_uint64(0)
            sample_tok[i, j] = ref.ref_sample(probs[i], V, int(sd), C.byref(st))
            sample_state[i, j] = st.value
    np.savez_compressed(os.path.join(HERE, "sampler_golden.npz"), cfg=cfg, logits_in=lg_in, logits_out=lg_out,
                        probs=probs, prev=prev, n_prev=n_prev, has_prev=has_prev, seeds=seeds,
                        rng_stream=streams, rng_exp=exps, rng_final=final_state, sample_tok=sample_tok,
                        sample_state=sample_state)
    print("wrote", os.path.join(HERE, "sampler_golden.npz"), n, "cases")


if __name__ == "__main__":
    main()

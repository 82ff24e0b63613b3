"""Parity at the workload shapes of the benchmark, with the 24-layer model, through properties
that hold at any size and an oracle check on the sequence the oracle finishes in seconds.

* Prefill of 16 sequences x 1024 rows (valid lengths U[512, 1024], 256 prompt codes; projections
  on the int8 matrix cores, attention on the fp16 matrix cores): each sequence prefilled alone
  gives bit-identical logits (left padding and the rest of the batch change nothing); for the
  shortest one the layer-0 K/V cache is within one fp16 ulp of the oracle's and the greedy token
  of the first logits is the oracle's. Over 24 layers the logits themselves drift from the
  oracle's by about 1e-2 relative: every layer re-quantises its activations to Q8_0, so a single
  rounding-level difference (the device and host expf differ in the last bit now and then) flips
  one int8 value, which moves its whole row by ~1e-3 and spreads through attention. The same drift
  appears with the bit-exact GEMV and the lane-per-query attention, so the bound below (2e-2) is
  that of the model's re-quantisation, not of the matrix-core kernels, whose own outputs are
  checked to 2e-3 (in practice ~1e-6) op by op.
* Decode at batch 128 with KV lengths U[1024, 4096] (27 GB fp16 KV cache): 32 teacher-forced
  greedy steps; the three shortest sequences' choices equal the oracle's run of each sequence
  alone, except at fragile steps (tests/fragile.py).
"""
import numpy as np
import pytest

import fragile as FR
import oracle as O
import synth_model as sm

pytestmark = pytest.mark.gpu


def _lengths(seed, B, lo, hi):
    rng = np.random.Generator(np.random.PCG64(seed))
    L = rng.integers(lo, hi + 1, B)
    L[0] = hi
    return L


def test_prefill_16x1024(gpu, model24_path):
    P = 256
    L = _lengths(0x6A5E0004, 16, 512, 1024)
    reqs = sm.synth_requests(0x6A5E0004, 16, P, L - P)
    g = gpu.Model(model24_path)
    try:
        batch = g.first_logits(reqs)
        assert np.all(np.isfinite(batch))
        short = int(np.argmin(L))
        for b in (0, short, 7):
            print(f"prefill alone: sequence {b}, {L[b]} rows", flush=True)
            alone = g.first_logits([reqs[b]])
            assert np.array_equal(batch[b], alone[0]), b
    finally:
        g.close()
    g = gpu.Model(model24_path)
    try:
        _, S = g.prefill([reqs[short]])
        k_dev, v_dev = g.kv_read(0)
    finally:
        g.close()
    o = O.Model(model24_path)
    try:
        ref = o.first_logits([reqs[short]])
        k_ref, v_ref, _ = o.prefill_kv([reqs[short]], 0, flags=O.ORC_KV_F16)
    finally:
        o.close()
    for dev, r in ((k_dev, k_ref), (v_dev, v_ref)):
        d = dev[:, :, :S, :].view(np.float16).astype(np.float32)
        ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(d - r) <= np.maximum(ulp, 1e-6 * np.abs(r).max()))
        assert np.mean(d != r) <= 0.01
    assert int(batch[short].argmax()) == int(ref[0].argmax())
    rel = np.abs(batch[short] - ref[0]).max() / np.abs(ref[0]).max()
    assert rel <= 2e-2, rel


def test_prefill_16x1024_fp16_mode(gpu, model24_path):
    """The prefill's fp16 mode (gsvk_model_set_prefill_f16: the projections on fp16 operands) at
    the same shape: a sequence prefilled alone gives the logits it has in the batch, bit for bit;
    its layer-0 K/V rows are within 2e-3 of each row's largest magnitude of the oracle's (the
    projections' bar: fp16 operands plus the fp16 cache); its first logits agree with the oracle
    as the default mode's do (2e-2 of their scale after 24 layers of Q8_0 requantisation), with the
    same greedy token; switching the mode off gives the default mode's logits back."""
    P = 256
    L = _lengths(0x6A5E0004, 16, 512, 1024)
    reqs = sm.synth_requests(0x6A5E0004, 16, P, L - P)
    short = int(np.argmin(L))
    g = gpu.Model(model24_path)
    try:
        default = g.first_logits([reqs[short]])
        g.set_prefill_f16(True)
        batch = g.first_logits(reqs)
        assert np.all(np.isfinite(batch))
        print(f"fp16 mode, prefill alone: sequence {short}, {L[short]} rows", flush=True)
        alone = g.first_logits([reqs[short]])
        assert np.array_equal(batch[short], alone[0])
        _, S = g.prefill([reqs[short]])
        k_dev, v_dev = g.kv_read(0)
        g.set_prefill_f16(False)
        back = g.first_logits([reqs[short]])
    finally:
        g.close()
    assert np.array_equal(back, default)
    o = O.Model(model24_path)
    try:
        ref = o.first_logits([reqs[short]])
        k_ref, v_ref, _ = o.prefill_kv([reqs[short]], 0, flags=O.ORC_KV_F16)
    finally:
        o.close()
    for dev, r in ((k_dev, k_ref), (v_dev, v_ref)):
        d = dev[:, :, :S, :].view(np.float16).astype(np.float32)
        # rows (sequence, column) over all heads and dims
        dr = np.moveaxis(d, 2, 1).reshape(d.shape[0], S, -1)
        rr = np.moveaxis(r, 2, 1).reshape(r.shape[0], S, -1)
        row_scale = np.maximum(np.abs(rr).max(axis=2), 1e-6)
        rel = (np.abs(dr - rr).max(axis=2) / row_scale).max()
        print(f"fp16 mode: layer-0 K/V within {rel:.2e} of the row scale", flush=True)
        assert rel <= 2e-3, rel
    assert int(alone[0].argmax()) == int(ref[0].argmax())
    rel = np.abs(alone[0] - ref[0]).max() / np.abs(ref[0]).max()
    assert rel <= 2e-2, rel


def test_decode_batch128_long_kv(gpu, model24_path):
    """Batch 128, KV lengths U[1024, 4096], 32 teacher-forced greedy steps (repetition penalty
    1.35): the generate graph's choices equal those of the per-step path's logits, and for the
    three shortest sequences (each run alone by the oracle) every choice is the oracle's except at
    a fragile step (one whose measured logit drift could change it)."""
    P, steps = 64, 32
    L = _lengths(0x6A5E0005, 128, 1024, 4096)
    reqs = sm.synth_requests(0x6A5E0005, 128, P, L - P, bert=False)
    forced = np.random.default_rng(12).integers(0, 1024, steps).astype(np.int32)
    greedy = (1, 1.0, 1.0, 1.35)
    seeds = list(range(1, 129))
    g = gpu.Model(model24_path)
    try:
        print("decode: batch 128, KV lengths U[1024, 4096], generate", flush=True)
        res = g.generate(reqs, sampler=greedy, max_steps=steps, oracle=forced, seeds=seeds, flags=1,
                         want_sampled=True)
        print("decode: batch 128, per-step logits", flush=True)
        dev = FR.device_step_logits(g, reqs, forced, steps)
        g.release_cache()
    finally:
        g.close()
    assert res["n_steps"] == steps
    o = O.Model(model24_path)
    try:
        for s in np.argsort(L, kind="stable")[:3]:
            print(f"oracle: sequence {s} alone, {L[s]} rows, {steps} steps", flush=True)
            ref = o.generate([reqs[s]], sampler=greedy, max_steps=steps, oracle=forced, seeds=[seeds[s]],
                             flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, want_logits=True)
            assert np.array_equal(res["tokens"][s], ref["tokens"][0])
            n_mis, n_fr, worst = FR.check_choices([reqs[s]], greedy, forced, [seeds[s]], ref,
                                                  {"sampled": res["sampled"][:, [s]]}, dev[:, [s]], steps)
            print(f"sequence {s}: {n_mis} of {steps} choices differ, {n_fr} fragile, drift {worst:.2e}",
                  flush=True)
            assert worst <= 3e-2, worst
    finally:
        o.close()

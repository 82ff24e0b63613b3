"""Models whose projections are stored F16 or F32 (the reference exporter's attn= / ffn= options,
tools/export_gguf/export.py:53-54; the engine's fallback F16 model, src/gsv_engine.cpp:216): the
reference multiplies them through ggml_mul_mat as they are (src/gsv_ar.cpp:244, :392), F16 with
the activations rounded to fp16, F32 on the fp32 activations; no Q8_0 quantisation.

* Exact mode: the prefill's last-row logits and those entering every teacher-forced decode step
  equal the oracle's to the bit, and a sampled free run gives the oracle's tokens.
* Default mode (the default decode and prefill attention kernels): logits within 2e-3 of the
  oracle's scale, every teacher-forced choice the oracle's except at a fragile step.
* A model mixing F16 attention projections with Q8_0 FFN projections, the same.
"""
import numpy as np
import pytest

import fragile as FR
import oracle as O
import synth_model as sm

pytestmark = pytest.mark.gpu

TYPES = [("f16", "f16"), ("f32", "f32"), ("f16", "q8_0")]


@pytest.fixture(scope="module", params=TYPES, ids=[f"attn_{a}-ffn_{f}" for a, f in TYPES])
def float_model(request, tmp_path_factory):
    a, f = request.param
    d = tmp_path_factory.mktemp("fw")
    return sm.write_model(str(d / f"ar3_{a}_{f}.gguf"), seed=0x6A5E0100, n_layer=3, attn_type=a, ffn_type=f)


def _oracle(path, reqs, cfg, steps, seeds, forced=None, want_logits=False):
    o = O.Model(path)
    try:
        return o.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, oracle=forced,
                          flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, want_logits=want_logits)
    finally:
        o.close()


def test_exact_mode_bitexact(gpu, float_model):
    reqs = sm.synth_requests(0x100, 3, 16, [12, 30, 5])          # 3 x 46 prefill rows
    cfg = (15, 1.0, 1.0, 1.35)
    seeds = [5, 6, 7]
    steps = 10
    free = _oracle(float_model, reqs, cfg, steps, seeds)
    forced = free["sampled"][:, 0].astype(np.int32)
    ref = _oracle(float_model, reqs, cfg, steps, seeds, forced, want_logits=True)
    g = gpu.Model(float_model)
    try:
        g.set_exact(True)
        print(f"{float_model}: exact mode, teacher forced", flush=True)
        dev = FR.device_step_logits(g, reqs, forced, steps)
        res = g.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, flags=1)
    finally:
        g.close()
    assert np.array_equal(dev.view(np.uint32), ref["logits"][:steps].view(np.uint32)), \
        np.abs(dev - ref["logits"][:steps]).max()
    for b in range(3):
        assert np.array_equal(res["tokens"][b], free["tokens"][b]), b


def test_default_mode_within_bounds(gpu, float_model):
    reqs = sm.synth_requests(0x101, 4, 16, [20, 60, 9, 33])      # 4 x 76 rows: the matrix-core attention
    cfg = (1, 1.0, 1.0, 1.35)
    seeds = [1, 2, 3, 4]
    steps = 12
    forced = np.random.default_rng(0x102).integers(0, 1024, steps).astype(np.int32)
    ref = _oracle(float_model, reqs, cfg, steps, seeds, forced, want_logits=True)
    g = gpu.Model(float_model)
    try:
        print(f"{float_model}: default mode, teacher forced", flush=True)
        res = g.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, oracle=forced, flags=1, want_sampled=True)
        dev = FR.device_step_logits(g, reqs, forced, steps)
        with pytest.raises(gpu.GsvkError, match="F16 / F32 projections"):
            g.set_decode_path(gpu.GSVK_DECODE_FUSED)
            g.generate(reqs, sampler=cfg, max_steps=2, seeds=seeds, flags=1)
    finally:
        g.close()
    scale = np.abs(ref["logits"][:steps]).max()
    assert np.abs(dev - ref["logits"][:steps]).max() <= 2e-3 * scale
    for b in range(4):
        assert np.array_equal(res["tokens"][b], ref["tokens"][b])
    n_mis, n_fr, worst = FR.check_choices(reqs, cfg, forced, seeds, ref, res, dev, steps)
    print(f"{n_mis} of {4 * steps} choices differ, {n_fr} fragile, drift {worst:.2e}", flush=True)

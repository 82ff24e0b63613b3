"""A model loaded from the pre-swizzled GGUF (gsv.cpp_amd/gguf_tiled.py: layer projections in
the matrix-core operand order, the sliced and natural copies derived on the device) computes the
same bits as the one loaded from the Q8_0 block form: prefill and step logits and the K/V cache,
on the two-launch layer, the GEMV chain and the matrix-core path (batch 20), and in exact mode;
in exact mode the tiled file also gives the oracle's logits to the bit."""
import numpy as np
import pytest

import gguf_tiled as GT
import synth_model as sm

pytestmark = pytest.mark.gpu

GREEDY = (1, 1.0, 1.0, 1.35)


@pytest.fixture(scope="module")
def tiled4(model4_path, tmp_path_factory):
    p = str(tmp_path_factory.mktemp("tiled4") / "ar4.tiled.gguf")
    GT.main([model4_path, p])
    return p


def _run(gpu, path, reqs, forced, steps, path_id=None, exact=False):
    import gsvk
    g = gpu.Model(path)
    try:
        if path_id is not None:
            g.set_decode_path(path_id)
        g.set_exact(exact)
        B = len(reqs)
        S = max(len(r["phones"]) for r in reqs) + len(reqs[0]["prompt"])
        gsvk.check(gsvk.lib().gsvk_kv_alloc(g.h, B, S + steps + 8), "kv_alloc")
        lg, _ = g.prefill(reqs)
        out = [lg]
        for i in range(steps - 1):
            out.append(g.decode_step(np.full(B, forced[i], np.int32)))
        k1, v1 = g.kv_read(1)
        return np.array(out), k1, v1
    finally:
        g.close()


@pytest.mark.parametrize("B,path,exact", [(3, None, False), (3, "GEMV", False), (20, "MFMA", False),
                                          (3, None, True)])
def test_tiled_file_gives_the_same_bits(gpu, model4_path, tiled4, B, path, exact):
    rng = np.random.default_rng(900 + B)
    reqs = sm.synth_requests(901 + B, B, 16, rng.integers(3, 40, B))
    steps = 6
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    pid = None if path is None else getattr(gpu, f"GSVK_DECODE_{path}")
    print(f"canonical vs tiled file, batch {B}, path {path}, exact {exact}", flush=True)
    a = _run(gpu, model4_path, reqs, forced, steps, pid, exact)
    b = _run(gpu, tiled4, reqs, forced, steps, pid, exact)
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    assert np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2])


def test_tiled_file_exact_mode_equals_the_oracle(gpu, model4_path, tiled4):
    """The pre-swizzled file, loaded in exact mode, gives the oracle's logits (the oracle reading
    the reference exporter's Q8_0 block form, tools/export_gguf/convert_ar.py:76-130) to the bit:
    the prefill's last-row logits and those entering every teacher-forced decode step."""
    import oracle as O
    rng = np.random.default_rng(950)
    B = 3
    reqs = sm.synth_requests(951, B, 16, rng.integers(3, 40, B))
    steps = 8
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    o = O.Model(model4_path)
    try:
        ref = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                         flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, want_logits=True)
    finally:
        o.close()
    print("tiled file, exact mode, batch 3 against the oracle", flush=True)
    got, _, _ = _run(gpu, tiled4, reqs, forced, steps, None, True)
    assert np.array_equal(got.view(np.uint32), ref["logits"][:steps].view(np.uint32)), \
        np.abs(got - ref["logits"][:steps]).max()

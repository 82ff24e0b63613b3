"""End-to-end parity of the HIP AR decoder with the oracle (through the C ABI).

* prefill logits within 2e-3 relative of the oracle; left padding changes nothing (bit-exact);
* layer-0 KV cache bit-exact with the oracle's fp16-rounded cache (write indexing of prefill),
  and the decode append at column S bit-exact with a prefill that has the token in its prompt;
* teacher-forced greedy and sampled choices equal to the oracle's except at fragile steps (the
  step's measured logit drift could change the choice), and all equal in exact mode;
* the generate-loop rules (EOS after 11 steps, early stop, lens in finish order, oracle tokens).
"""
import numpy as np
import pytest

import fragile as FR
import oracle as O
import synth_model as sm

pytestmark = pytest.mark.gpu


def _reqs(seed, lens, P=16, bert=True):
    return sm.synth_requests(seed, len(lens), P, lens, bert=bert)


@pytest.fixture(scope="module")
def models(gpu, small_model_path):
    g = gpu.Model(small_model_path)
    o = O.Model(small_model_path)
    yield g, o
    g.close()
    o.close()


def test_first_logits_parity(models):
    g, o = models
    reqs = _reqs(1, [5, 20, 12])
    got = g.first_logits(reqs)
    ref = o.first_logits(reqs)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel <= 2e-3, rel


def test_left_padding_invariance(models):
    """(GEMV path: fewer than 64 prefill rows in the batch and alone.)"""
    g, _ = models
    reqs = _reqs(2, [3, 17, 9], P=4)            # S = 21, 63 rows
    batch = g.first_logits(reqs)
    for b in range(3):
        alone = g.first_logits([reqs[b]])
        assert np.array_equal(batch[b], alone[0]), b


def test_kv_write_layer0_bitexact(models):
    g, o = models
    reqs = _reqs(3, [7, 11])
    _, S = g.prefill(reqs)
    k_dev, v_dev = g.kv_read(0)
    k_ref, v_ref, _ = o.prefill_kv(reqs, 0, flags=O.ORC_KV_F16)
    kd = k_dev[:, :, :S, :].view(np.float16).astype(np.float32)
    vd = v_dev[:, :, :S, :].view(np.float16).astype(np.float32)
    assert np.array_equal(kd, k_ref)
    assert np.array_equal(vd, v_ref)


def test_kv_write_layer0_bitexact_without_bert(models):
    """A request without BERT features gets the projection bias on its text rows instead of the
    projection of a zero feature row: the layer-0 cache stays bit-exact with the oracle, which
    projects the zero row, also in a batch that mixes requests with and without features."""
    g, o = models
    reqs = _reqs(23, [9, 6, 12], P=8)          # 3 x 20 rows: below the matrix-core path
    reqs[1]["bert"] = None
    reqs[2]["bert"] = None
    for batch in (reqs, reqs[1:]):
        _, S = g.prefill(batch)
        k_dev, v_dev = g.kv_read(0)
        k_ref, v_ref, _ = o.prefill_kv(batch, 0, flags=O.ORC_KV_F16)
        assert np.array_equal(k_dev[:, :, :S, :].view(np.float16).astype(np.float32), k_ref)
        assert np.array_equal(v_dev[:, :, :S, :].view(np.float16).astype(np.float32), v_ref)


@pytest.mark.parametrize("lens,what", [
    ([260, 300, 245], "128 x 128 tiles: S = 316, 948 rows; alone: 261 rows and more"),
    ([70, 100], "32-column tiles, K split over 4 waves: S = 116, 232 rows; alone: 86 and 116 rows"),
])
def test_prefill_on_matrix_cores(models, lens, what):
    """Prefills of 64 rows and more run the projections on the MFMA GEMM (fp32 accumulation per
    block, not in ggml-cpu's 8-lane order): logits within 2e-3 of the oracle, the layer-0 K/V
    within one fp16 ulp of the oracle's (the fp32 values differ by rounding, which can move a
    value across an fp16 rounding boundary), and left padding changes nothing as long as the
    batch and the request alone fall in the same row range of the GEMM (up to 256 rows: the
    32-column kernel sums 4 K quarters, above: the 128 x 128 kernel accumulates through K)."""
    g, o = models
    reqs = _reqs(11, lens)
    got = g.first_logits(reqs)
    ref = o.first_logits(reqs)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 2e-3
    _, S = g.prefill(reqs)
    k_dev, v_dev = g.kv_read(0)
    k_ref, v_ref, _ = o.prefill_kv(reqs, 0, flags=O.ORC_KV_F16)
    for dev, ref16 in ((k_dev, k_ref), (v_dev, v_ref)):
        d = dev[:, :, :S, :].view(np.float16).astype(np.float32)
        r = ref16
        # one fp16 ulp of the value, or (near zero) an fp32 rounding of the largest value
        ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float32)
        tol = np.maximum(ulp, 1e-6 * np.abs(r).max())
        assert np.all(np.abs(d - r) <= tol), np.abs(d - r).max()
        assert np.mean(d != r) <= 0.01
    for b in range(len(lens)):
        alone = g.first_logits([reqs[b]])
        assert np.array_equal(got[b], alone[0]), (what, b)


def test_kv_append_matches_prefill(models):
    """decode_step appends K/V at column S: equal to a prefill whose prompt ends with the token."""
    g, _ = models
    reqs = _reqs(4, [6, 10])
    _, S = g.prefill(reqs)
    tok = np.array([77, 901], np.int32)
    g.decode_step(tok)
    k1, v1 = g.kv_read(0)
    col_dec_k = k1[:, :, S, :].copy()
    col_dec_v = v1[:, :, S, :].copy()
    # untouched columns keep the prefill values
    reqs2 = []
    for b, r in enumerate(reqs):
        r2 = dict(r)
        r2["prompt"] = np.concatenate([r["prompt"], [tok[b]]]).astype(np.int32)
        reqs2.append(r2)
    # the shared-prompt rule needs equal prompts per batch: run each sequence alone
    for b in range(2):
        _, S2 = g.prefill([reqs2[b]])
        k2, v2 = g.kv_read(0)
        pad = max(6, 10) - len(reqs[b]["phones"])
        # alone, sequence b has no left padding: its column S - pad holds the appended token
        assert np.array_equal(k2[0, :, S2 - 1, :], col_dec_k[b]), b
        assert np.array_equal(v2[0, :, S2 - 1, :], col_dec_v[b]), b
        assert S2 - 1 == S - pad


def _forced_parity(gpu, path, reqs, cfg, steps, forced, seeds, exact_too=True):
    """Teacher-forced choices of the default path (fragile steps only may differ) and, below 17
    sequences, of exact mode (every choice and every step's logits the oracle's)."""
    o = O.Model(path)
    try:
        ref = o.generate(reqs, sampler=cfg, max_steps=steps, oracle=forced, seeds=seeds,
                         flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, want_logits=True)
    finally:
        o.close()
    g = gpu.Model(path)
    try:
        res = g.generate(reqs, sampler=cfg, max_steps=steps, oracle=forced, seeds=seeds, flags=1, want_sampled=True)
        dev = FR.device_step_logits(g, reqs, forced, steps)
        if exact_too:
            g.set_exact(True)
            res_x = g.generate(reqs, sampler=cfg, max_steps=steps, oracle=forced, seeds=seeds, flags=1,
                               want_sampled=True)
            dev_x = FR.device_step_logits(g, reqs, forced, steps)
    finally:
        g.close()
    assert res["n_steps"] == ref["n_steps"] == steps
    for b in range(len(reqs)):
        assert np.array_equal(res["tokens"][b], ref["tokens"][b])   # the teacher-forced history
    n_mis, n_fragile, worst = FR.check_choices(reqs, cfg, forced, seeds, ref, res, dev, steps)
    print(f"{len(reqs)} x {steps} choices: {n_mis} differ, {n_fragile} fragile, drift {worst:.2e}", flush=True)
    assert worst <= 3e-2, worst
    if exact_too:
        assert np.array_equal(res_x["sampled"], ref["sampled"])
        assert np.array_equal(dev_x.view(np.uint32), ref["logits"][:steps].view(np.uint32))


def test_teacher_forced_greedy_tokens(gpu, model4_path):
    """Greedy (top-k 1, repetition penalty 1.35), 2 sequences x 40 steps, forced random tokens."""
    reqs = _reqs(5, [40, 25], P=24)
    steps = 40
    forced = np.random.default_rng(6).integers(0, 1024, steps).astype(np.int32)   # no EOS
    _forced_parity(gpu, model4_path, reqs, (1, 1.0, 1.0, 1.35), steps, forced, [1, 2])


@pytest.mark.parametrize("B", [20, 64])
def test_decode_batch64_on_matrix_cores(gpu, model4_path, B):
    """From batch 17 the decode step runs its projections as MFMA GEMMs (LayerNorms and the
    embedding as launches of their own, Q8_0 operands in the matrix-core order, a partial last
    tile of 32 rows at batch 20): fp32 accumulation per block instead of the x86 8-lane order, so
    a choice may differ from the oracle's only at a fragile step (teacher forcing keeps the
    histories equal)."""
    rng = np.random.default_rng(24)
    lens = rng.integers(3, 21, B)
    reqs = _reqs(25, lens, P=8)
    steps = 8
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    _forced_parity(gpu, model4_path, reqs, (1, 1.0, 1.0, 1.35), steps, forced, list(range(1, B + 1)),
                   exact_too=False)


def test_generate_rules_match_oracle(models):
    """EOS via teacher forcing at step 14 (after the 11-step EOS mask), early stop, lens order."""
    g, o = models
    reqs = _reqs(7, [9, 4, 13], P=12)
    forced = np.random.default_rng(8).integers(0, 1024, 30).astype(np.int32)
    forced[14] = 1024
    for kw in ({"max_steps": 30, "oracle": forced},
               {"max_steps": 30, "oracle": forced, "early_stop": 6},
               {"max_steps": 9, "oracle": forced}):
        res = g.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), seeds=[11, 12, 13], **kw)
        ref = o.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), seeds=[11, 12, 13], flags=O.ORC_KV_F16, **kw)
        assert res["n_steps"] == ref["n_steps"], kw
        assert list(res["lens"]) == list(ref["lens"]), kw
        assert list(res["finish_seq"]) == list(ref["finish_seq"]), kw
        for b in range(3):
            assert np.array_equal(res["tokens"][b], ref["tokens"][b]), (kw, b)


def test_sampling_matches_oracle(gpu, small_model_path):
    """top-k 15 sampling with per-sequence seeds, 24 steps: teacher forced with the oracle's own
    sequence-0 tokens, every choice the oracle's except at fragile steps (default path) and every
    one in exact mode; and exact mode's free run gives the oracle's free-run tokens."""
    reqs = _reqs(9, [10, 6], P=16)
    cfg = (15, 1.0, 1.0, 1.35)
    seeds = [101, 202]
    o = O.Model(small_model_path)
    try:
        free = o.generate(reqs, sampler=cfg, max_steps=24, seeds=seeds, flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL)
    finally:
        o.close()
    forced = free["sampled"][:, 0].astype(np.int32)
    _forced_parity(gpu, small_model_path, reqs, cfg, 24, forced, seeds)
    g = gpu.Model(small_model_path)
    try:
        g.set_exact(True)
        res = g.generate(reqs, sampler=cfg, max_steps=24, seeds=seeds, flags=1)
    finally:
        g.close()
    for b in range(2):
        assert np.array_equal(res["tokens"][b], free["tokens"][b]), b


def test_top_p_and_temperature(models):
    g, o = models
    reqs = _reqs(10, [8], P=8)
    for cfg in [(0, 0.8, 0.7, 1.0), (5, 0.5, 1.3, 1.35), (1025, 1.0, 1.0, 1.0)]:
        res = g.generate(reqs, sampler=cfg, max_steps=8, seeds=[5], flags=1)
        ref = o.generate(reqs, sampler=cfg, max_steps=8, seeds=[5], flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL)
        assert np.array_equal(res["tokens"][0][:8 + 4], ref["tokens"][0][:8 + 4]), cfg


def test_prefill_workspace_reuse(models):
    """The prefill workspace is kept by the model and grown to the largest prefill seen: a large
    prefill, then a smaller one (reusing the start of the pool), then the large one again give the
    same logits as on first use, bit for bit, on both paths (GEMM from 64 rows, GEMV below)."""
    g, _ = models
    big = _reqs(21, [90, 40, 120])        # 3 x (120 + 16) rows: matrix-core path
    small = _reqs(22, [5, 9])             # 2 x (9 + 16) rows: GEMV path
    first = g.first_logits(big)
    s1 = g.first_logits(small)
    again = g.first_logits(big)
    s2 = g.first_logits(small)
    assert np.array_equal(first, again)
    assert np.array_equal(s1, s2)
    g.release_cache()                     # frees the pool too; the next prefill allocates anew
    assert np.array_equal(g.first_logits(big), first)


def _cb_scenario(g, reqs, seeds, steps, P, cfg, flags, early_stop):
    """Five requests through a continuous batch of 3 rows: two start, one joins 5 steps in, one
    takes the row a finished request left, one joins late. Returns each request's tokens."""
    g.cb_open(capacity=3, max_prefill=64, max_steps=80, prompt_len=P, sampler=cfg, early_stop=early_stop,
              flags=flags)
    got = {}
    slots = {}

    def add(i):
        slots[i] = g.cb_add(reqs[i], seeds[i], steps[i])

    def take_done():
        for i, sl in list(slots.items()):
            fin, toks, _ = g.cb_take(sl)
            if fin:
                got[i] = toks
                del slots[i]

    add(0)
    add(1)
    g.cb_step(5)
    take_done()
    add(2)                      # joins 5 steps in
    g.cb_step(7)
    take_done()                 # request 1 has run its 12 steps
    add(3)                      # into the row request 1 left
    g.cb_step(12)
    take_done()
    add(4)
    g.cb_step(10)
    take_done()
    assert sorted(got) == [0, 1, 2, 3, 4] and not slots
    g.cb_close()
    return got


@pytest.mark.parametrize("flags,early_stop", [(1, -1), (0, 6)])
def test_continuous_batch_matches_generate(gpu, model4_path, flags, early_stop):
    """Requests that join a decoding batch (a prefill of their own into a free row, left-padded to
    the batch's KV column) and leave it when done produce the tokens of a generate of their own,
    bit for bit: per row the arithmetic does not depend on the other rows. Rows are reused after
    a request leaves; with early stop the rule counts each request's own tokens."""
    P = 8
    cfg = (15, 1.0, 1.0, 1.35)
    reqs = _reqs(41, [20, 9, 30, 14, 25], P=P)
    seeds = [101, 202, 303, 404, 505]
    steps = [24, 12, 16, 20, 10]
    g = gpu.Model(model4_path)
    try:
        refs = []
        for r, sd, st in zip(reqs, seeds, steps):
            res = g.generate([r], sampler=cfg, max_steps=st, seeds=[sd], flags=flags, early_stop=early_stop)
            refs.append(res["tokens"][0])
        got = _cb_scenario(g, reqs, seeds, steps, P, cfg, flags, early_stop)
        for i in range(5):
            assert np.array_equal(got[i], refs[i]), (i, got[i], refs[i])
        # the model runs a plain generate again after the session
        res = g.generate([reqs[0]], sampler=cfg, max_steps=steps[0], seeds=[seeds[0]], flags=flags,
                         early_stop=early_stop)
        assert np.array_equal(res["tokens"][0], refs[0])
    finally:
        g.close()


@pytest.mark.parametrize("flags,early_stop", [(1, -1), (0, 6)])
def test_continuous_batch_exact_matches_oracle(gpu, model4_path, flags, early_stop):
    """The same continuous batch in exact mode (ggml-cpu's arithmetic order) gives, for every
    request, the tokens of the oracle's generate of that request alone
    (src/gsv_ar.cpp:719-824 with one request): joining a running batch, left-padded to its KV
    column, with PE positions counted from the request's own start, changes nothing a request
    computes (tools/svc_core.h:1244-1340 is the reference batcher this replaces)."""
    P = 8
    cfg = (15, 1.0, 1.0, 1.35)
    reqs = _reqs(41, [20, 9, 30, 14, 25], P=P)
    seeds = [101, 202, 303, 404, 505]
    steps = [24, 12, 16, 20, 10]
    o = O.Model(model4_path)
    try:
        refs = [o.generate([r], sampler=cfg, max_steps=st, seeds=[sd], early_stop=early_stop,
                           flags=O.ORC_KV_F16 | (O.ORC_EOS_MASK_ALL if flags & 1 else 0))["tokens"][0]
                for r, sd, st in zip(reqs, seeds, steps)]
    finally:
        o.close()
    g = gpu.Model(model4_path)
    try:
        g.set_exact(True)
        got = _cb_scenario(g, reqs, seeds, steps, P, cfg, flags, early_stop)
    finally:
        g.close()
    for i in range(5):
        assert np.array_equal(got[i], refs[i]), (i, got[i], refs[i])
    if flags == 0:
        assert any(len(refs[i]) < P + steps[i] for i in range(5))   # some request stopped early

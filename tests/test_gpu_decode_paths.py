"""The decode step's kernel paths against each other, the oracle and the known-answer closed forms.

* GSVK_DECODE_GEMV: four launches per layer, projections and LayerNorms bit-exact with the
  oracle (ggml-cpu's x86 order).
* GSVK_DECODE_FUSED (the persistent decode's fallback up to 32 sequences): two launches per layer; the out projection
  and FFN2 are summed over heads / hidden groups as partial rows, so they agree with the GEMV
  chain to fp32 rounding; everything before the first of those sums (the layer-0 input, QKV, the
  K/V append of layer 0) is unchanged and stays bit-exact.
* GSVK_DECODE_PERSIST (the default up to 32 sequences where the device allows): the two-launch
  layer's work in one launch per step, each XCD running whole sequences; the same bits as FUSED.
"""
import numpy as np
import pytest

import known_models as KM
import oracle as O
import synth_model as sm

pytestmark = pytest.mark.gpu

GREEDY = (1, 1.0, 1.0, 1.35)


def _reqs(seed, lens, P):
    return sm.synth_requests(seed, len(lens), P, lens)


def _step_logits(g, reqs, forced, steps, path):
    """Prefill then `steps` decode steps fed the forced tokens; logits entering each step."""
    g.set_decode_path(path)
    B = len(reqs)
    S = max(len(r["phones"]) for r in reqs) + len(reqs[0]["prompt"])
    import gsvk
    gsvk.check(gsvk.lib().gsvk_kv_alloc(g.h, B, S + steps + 8), "kv_alloc")
    lg, _ = g.prefill(reqs)
    out = [lg]
    for i in range(steps - 1):
        out.append(g.decode_step(np.full(B, forced[i], np.int32)))
    return np.array(out)


@pytest.mark.parametrize("B", [1, 3, 8, 9, 16])
def test_fused_layer_matches_gemv_chain(gpu, model4_path, B):
    """(Batches 1-8 run the FFN launch as 32 hidden groups, 9 and above as 16.)
    Logits of every decode step of the two paths, same forced tokens: equal to fp32 rounding
    at the median step; a step where some layer's Q8_0 re-quantisation of an activation lands on
    the other side of a rounding boundary moves by that one int8 step (amax / 127 of a block),
    which the later layers spread: within 1e-2 of the row's scale (the same bound as the drift
    of the oracle's own re-quantisation, test_gpu_configs.py). Layer-0 K/V equal to the bit."""
    rng = np.random.default_rng(60 + B)
    reqs = _reqs(61 + B, rng.integers(3, 40, B), 16)
    steps = 12
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    g = gpu.Model(model4_path)
    try:
        print(f"fused vs GEMV chain, batch {B}", flush=True)
        a = _step_logits(g, reqs, forced, steps, gpu.GSVK_DECODE_GEMV)
        ka, va = g.kv_read(0)
        b = _step_logits(g, reqs, forced, steps, gpu.GSVK_DECODE_FUSED)
        kb, vb = g.kv_read(0)
    finally:
        g.close()
    assert np.array_equal(a[0], b[0])                       # the prefill is the same kernels
    rel = np.abs(a - b).max(axis=2) / np.abs(a).max(axis=2)
    assert np.median(rel[1:]) <= 1e-5, np.median(rel[1:])
    assert rel.max() <= 1e-2, rel.max()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)


@pytest.mark.parametrize("B", [17, 32, 64])
def test_fused_layer_matches_mfma_path(gpu, model4_path, B):
    """Above 16 sequences (where the GEMV chain does not run) the two-launch layer against the
    matrix-core path: logits of every step equal to fp32 rounding at the median, within 1e-2 of
    the row's scale at the worst step (re-quantisation flips, as against the GEMV chain); the
    prefill is the same kernels."""
    rng = np.random.default_rng(80 + B)
    reqs = _reqs(81 + B, rng.integers(3, 40, B), 16)
    steps = 10
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    g = gpu.Model(model4_path)
    try:
        print(f"fused vs matrix-core path, batch {B}", flush=True)
        a = _step_logits(g, reqs, forced, steps, gpu.GSVK_DECODE_MFMA)
        b = _step_logits(g, reqs, forced, steps, gpu.GSVK_DECODE_FUSED)
    finally:
        g.close()
    assert np.array_equal(a[0], b[0])
    rel = np.abs(a - b).max(axis=2) / np.abs(a).max(axis=2)
    assert np.median(rel[1:]) <= 1e-5, np.median(rel[1:])
    assert rel.max() <= 1e-2, rel.max()


@pytest.mark.parametrize("B", [32, 64])
def test_fused_decode_kv_matches_oracle_large_batch(gpu, model4_path, B):
    """The two-launch layer at 32 and 64 sequences: the layer-0 K/V rows of every decode step are
    the oracle's cache bit for bit (the embedding at PE position P + idx and its QKV in the x86
    order), as at batch 16."""
    rng = np.random.default_rng(90 + B)
    reqs = _reqs(91 + B, rng.integers(3, 24, B), 16)
    steps = 6
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    g = gpu.Model(model4_path)
    o = O.Model(model4_path)
    try:
        print(f"fused decode K/V, batch {B}", flush=True)
        g.set_decode_path(gpu.GSVK_DECODE_FUSED)
        g.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced, flags=1)
        k0, v0 = g.kv_read(0)
        ref = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                         flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, kv_layer=0)
    finally:
        g.close()
        o.close()
    rk, rv = ref["kv"]
    S = max(len(r["phones"]) for r in reqs) + 16
    sl = slice(S, S + steps)
    for b in range(B):
        assert np.array_equal(k0[b, :, sl].view(np.float16).astype(np.float32), rk[b, :, sl]), b
        assert np.array_equal(v0[b, :, sl].view(np.float16).astype(np.float32), rv[b, :, sl]), b


@pytest.mark.parametrize("path", ["GEMV", "FUSED"])
def test_decode_kv_cache_matches_oracle(gpu, model4_path, path):
    """The K/V rows every decode step appends (layer 0: the embedding at PE position P + idx, its
    QKV at column S + idx) are the oracle's cache after the same teacher-forced steps, bit for
    bit, on both paths; the later layers' rows within fp16 rounding of the attention's last-bit
    differences."""
    rng = np.random.default_rng(70)
    reqs = _reqs(71, [12, 30, 5, 21], 16)
    steps = 10
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    g = gpu.Model(model4_path)
    o = O.Model(model4_path)
    try:
        g.set_decode_path(getattr(gpu, f"GSVK_DECODE_{path}"))
        g.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced, flags=1)
        k0, v0 = g.kv_read(0)
        k3, _ = g.kv_read(3)
        ref = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                         flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, kv_layer=0)
        ref3 = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                          flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, kv_layer=3)
    finally:
        g.close()
        o.close()
    rk, rv = ref["kv"]
    S = max(len(r["phones"]) for r in reqs) + 16
    assert rk.shape[2] == S + steps
    for b, r in enumerate(reqs):
        pad = S - 16 - len(r["phones"])
        # decode columns: bit for bit
        sl = slice(S, S + steps)
        assert np.array_equal(k0[b, :, sl].view(np.float16).astype(np.float32), rk[b, :, sl]), b
        assert np.array_equal(v0[b, :, sl].view(np.float16).astype(np.float32), rv[b, :, sl]), b
        # prefill columns (4 x 46 rows: the matrix-core GEMM, fp32 sums per block): within one
        # fp16 ulp
        for dev, ref_ in ((k0, rk), (v0, rv)):
            d = dev[b, :, pad:S].view(np.float16).astype(np.float32)
            rr = ref_[b, :, pad:S]
            assert np.all(np.abs(d - rr) <= np.spacing(np.abs(rr).astype(np.float16)).astype(np.float32)), b
        d3 = k3[b, :, S:S + steps].view(np.float16).astype(np.float32)
        r3 = ref3["kv"][0][b, :, S:S + steps]
        assert np.abs(d3 - r3).max() <= 2e-2 * np.abs(r3).max()


@pytest.fixture(scope="module")
def zero2_gpu(tmp_path_factory):
    d = tmp_path_factory.mktemp("kmg")
    return KM.write(str(d / "zero2.gguf"), 11, [{}, {}])


@pytest.fixture(scope="module")
def idqkv_gpu(tmp_path_factory):
    d = tmp_path_factory.mktemp("kmg")
    return KM.write(str(d / "idqkv.gguf"), 12, [{"qkv": "id"}])


@pytest.mark.parametrize("path", ["GEMV", "FUSED"])
def test_decode_logits_known_answer(gpu, zero2_gpu, path):
    """Zero projections: the logits entering step idx + 1 are the closed form of the token of step
    idx embedded at PE position P + idx (tests/known_models.py), on the device as in the oracle."""
    mpath, p, perm, scale = zero2_gpu
    pe = KM.pe(64)
    P = 6
    reqs = _reqs(22, [4, 7, 11], P)
    forced = np.array([17, 900, 3, 1000, 250, 64], np.int32)
    g = gpu.Model(mpath)
    try:
        lg = _step_logits(g, reqs, forced, len(forced), getattr(gpu, f"GSVK_DECODE_{path}"))
    finally:
        g.close()
    x = KM.decode_input64(p, reqs[0]["prompt"][P - 1], P - 1, pe)
    for idx in range(len(forced)):
        if idx > 0:
            x = KM.decode_input64(p, forced[idx - 1], P + idx - 1, pe)
        ref = KM.head64(KM.zero_layers64(p, x, 2), perm, scale)
        bound = 2.0 ** -10 * np.abs(ref) + 1e-6
        for b in range(3):
            assert np.all(np.abs(lg[idx, b] - ref) <= bound), (idx, b)


@pytest.mark.parametrize("path", ["GEMV", "FUSED"])
def test_decode_kv_known_answer(gpu, idqkv_gpu, path):
    """Identity QKV: the K row appended at column S + idx is the quantised input row + b_k, the
    input being the token of step idx at PE position P + idx (bound from the activation
    quantisation), and equals the oracle's to the bit."""
    mpath, p, perm, scale = idqkv_gpu
    pe = KM.pe(64)
    P = 5
    reqs = _reqs(24, [3, 8], P)
    forced = np.array([40, 41, 1020, 7, 300, 12, 999], np.int32)
    n = len(forced)
    g = gpu.Model(mpath)
    o = O.Model(mpath)
    try:
        g.set_decode_path(getattr(gpu, f"GSVK_DECODE_{path}"))
        g.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=n, oracle=forced, seeds=[3, 4], flags=1)
        k0, _ = g.kv_read(0)
        ref = o.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=n, oracle=forced, seeds=[3, 4],
                         flags=O.ORC_EOS_MASK_ALL | O.ORC_KV_F16, kv_layer=0)
    finally:
        g.close()
        o.close()
    S = 8 + P
    bk = p["transformer.block0.qkv_b"][KM.D:2 * KM.D].astype(np.float64)
    for idx in range(n):
        x = KM.decode_input64(p, forced[idx], P + idx, pe)
        bound = KM.block_amax(x) * KM.Q8_ERR * 1.001 + 2.0 ** -10 * np.abs(x + bk) + 1e-6
        for b in range(2):
            dev = k0[b, :, S + idx].view(np.float16).astype(np.float64).reshape(-1)
            assert np.all(np.abs(dev - (x + bk)) <= bound), (idx, b)
            assert np.array_equal(k0[b, :, S + idx].view(np.float16).astype(np.float32), ref["kv"][0][b, :, S + idx])


# ---------------------------------------------------------------------------- the two kernels alone

def _q8_weights(gpu, torch, rng, n, k, tiled=False):
    """Random Q8_0 weights [n][k]: (sliced quants, fp16 scales) as the GEMV reads them, and with
    tiled=True also the matrix-core operand order the two-launch layer reads."""
    from test_gpu_ops import _dev, blocks_to_split, to_tiled
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    blk = sm.q8_quantize_ref(W).ravel()
    qs = torch.zeros(n * k, dtype=torch.int8, device="cuda")
    d = torch.zeros(n * k // 32, dtype=torch.int16, device="cuda")
    gpu.op_q8_repack(_dev(blk, torch), n, k, qs, d)
    if not tiled:
        return qs, d
    qn, dn = blocks_to_split(blk, n, k)
    qt, dt = to_tiled(qn, dn.view(np.int16))
    return qs, d, _dev(qt, torch), _dev(dt, torch)


def _seq_sum(parts):
    """parts[0] + parts[1] + ... in that order, in fp32 (the kernels' order)."""
    r = parts[0].copy()
    for p in parts[1:]:
        r = (r + p).astype(np.float32)
    return r


@pytest.mark.parametrize("B", [1, 5, 16])
def test_dec_attn_op_matches_separate_kernels(gpu, B):
    """Launch 1 against the GEMV chain's kernels on the same inputs: the LayerNorm row and the
    K/V append bit for bit; the sum of the 16 per-head partial rows is the out projection of the
    same Q8_0 attention output, to fp32 summation order (2e-6 of its scale)."""
    import torch
    from test_gpu_ops import _dev
    rng = np.random.default_rng(8000 + B)
    D, nh, lstride = 512, 16, 700
    wq, wd = _q8_weights(gpu, torch, rng, 3 * D, D)
    wos, wod_s, woq, wod = _q8_weights(gpu, torch, rng, D, D, tiled=True)
    bqkv = rng.standard_normal(3 * D).astype(np.float32) * 0.02
    res = rng.standard_normal((B, D)).astype(np.float32)
    parts = (rng.standard_normal((16, B, D)) * 0.1).astype(np.float32)
    lb = (rng.standard_normal(D) * 0.02).astype(np.float32)
    wb = np.concatenate([1 + 0.05 * rng.standard_normal(D), 0.05 * rng.standard_normal(D)]).astype(np.float32)
    kc = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16)
    vc = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16)
    col = lstride - 5
    begins = rng.integers(0, 200, B).astype(np.int32)
    begins[0] = 0
    scale = float(1.0 / np.sqrt(32.0))
    d = lambda a: _dev(a, torch)
    kb, colt = d(begins), torch.tensor([col], dtype=torch.int32, device="cuda")
    # the two-launch layer's first kernel
    k1, v1 = d(kc).view(torch.int16), d(vc).view(torch.int16)
    x1 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    p1 = torch.zeros((16, B, D), dtype=torch.float32, device="cuda")
    gpu.op_dec_attn(B, wq, wd, d(bqkv), k1, v1, kb, colt, scale, woq, wod, p1, x_out=x1, res=d(res),
                    parts=d(parts), ln_bias=d(lb), ln_wb=d(wb))
    # the GEMV chain's kernels
    k2, v2 = d(kc), d(vc)
    qkv = torch.zeros((B, 3 * D), dtype=torch.float32, device="cuda")
    x2 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    gpu.op_ln_gemv(wq, wd, 3 * D, d(res), d(_seq_sum(parts)), d(lb), d(wb), d(bqkv), 0, qkv, ln_out=x2)
    k2[:, :, col, :] = qkv[:, D:2 * D].reshape(B, nh, 32).half()
    v2[:, :, col, :] = qkv[:, 2 * D:].reshape(B, nh, 32).half()
    att = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    oq = torch.zeros(B * D, dtype=torch.int8, device="cuda")
    od = torch.zeros(B * nh, dtype=torch.float32, device="cuda")
    ws = torch.zeros(gpu.attn_workspace_bytes(B, nh, lstride), dtype=torch.uint8, device="cuda")
    ke = torch.full((B,), col + 1, dtype=torch.int32, device="cuda")
    gpu.op_attn_decode(qkv[:, :D].reshape(B, nh, 32).contiguous(), k2.view(torch.int16), v2.view(torch.int16), kb,
                       ke, lstride, scale, att, oq=oq, od=od, ws=ws)
    y = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    gpu.op_q8_gemv(wos, wod_s, D, D, oq, od, B, None, 0, y)
    torch.cuda.synchronize()
    assert torch.equal(x1, x2)
    assert torch.equal(k1, k2.view(torch.int16)) and torch.equal(v1, v2.view(torch.int16))
    yref = y.cpu().numpy().astype(np.float64)
    ysum = p1.cpu().numpy().astype(np.float64).sum(axis=0)
    assert np.abs(ysum - yref).max() <= 2e-6 * np.abs(yref).max()


@pytest.mark.parametrize("B", [1, 5, 16])
def test_dec_ffn_op_matches_separate_kernels(gpu, B):
    """Launch 2 against the GEMV chain's kernels on the same inputs: LN1 bit for bit; the sum of
    the 16 per-group partial rows is FFN2 of the same Q8_0 hidden row, to fp32 summation order."""
    import torch
    from test_gpu_ops import _dev
    rng = np.random.default_rng(8100 + B)
    D, F = 512, 2048
    w1q, w1d = _q8_weights(gpu, torch, rng, F, D)
    w2s, w2d_s, w2q, w2d = _q8_weights(gpu, torch, rng, D, F, tiled=True)
    b1 = (rng.standard_normal(F) * 0.02).astype(np.float32)
    res = rng.standard_normal((B, D)).astype(np.float32)
    p1 = (rng.standard_normal((16, B, D)) * 0.1).astype(np.float32)
    bo = (rng.standard_normal(D) * 0.02).astype(np.float32)
    wb = np.concatenate([1 + 0.05 * rng.standard_normal(D), 0.05 * rng.standard_normal(D)]).astype(np.float32)
    d = lambda a: _dev(a, torch)
    n1 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    p2 = torch.zeros((16, B, D), dtype=torch.float32, device="cuda")
    gpu.op_dec_ffn(B, d(res), d(p1), d(bo), d(wb), n1, w1q, w1d, d(b1), w2q, w2d, p2)
    h = torch.zeros((B, F), dtype=torch.float32, device="cuda")
    n1r = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    gpu.op_ln_gemv(w1q, w1d, F, d(res), d(_seq_sum(p1)), d(bo), d(wb), d(b1), 1, h, ln_out=n1r)
    hq = torch.zeros(B * F, dtype=torch.int8, device="cuda")
    hd = torch.zeros(B * F // 32, dtype=torch.float32, device="cuda")
    gpu.op_q8_quantize(h, hq, hd)
    y = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    gpu.op_q8_gemv(w2s, w2d_s, D, F, hq, hd, B, None, 0, y)
    torch.cuda.synchronize()
    assert torch.equal(n1, n1r)
    yref = y.cpu().numpy().astype(np.float64)
    ysum = p2.cpu().numpy().astype(np.float64).sum(axis=0)
    assert np.abs(ysum - yref).max() <= 2e-6 * np.abs(yref).max()


@pytest.mark.parametrize("B", [1, 3, 8, 9, 16, 17, 32])
def test_persistent_decode_equals_two_launch_layer(gpu, model4_path, B):
    """The persistent decode (all layers of a step in one launch, per-XCD barriers) against the
    two launches per layer: the logits entering every teacher-forced step, the K/V of every layer
    and the sampled tokens of a generate, all to the bit. Batches 1-8: one sequence per XCD, 32
    FFN groups; 9-16: up to two; 17-32: up to four (two items per workgroup and phase)."""
    rng = np.random.default_rng(500 + B)
    reqs = _reqs(501 + B, rng.integers(3, 60, B), 16)
    steps = 10
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    cfg = (15, 1.0, 1.0, 1.35)
    seeds = list(range(1, B + 1))
    g = gpu.Model(model4_path)
    try:
        print(f"persistent vs two-launch, batch {B}", flush=True)
        a = _step_logits(g, reqs, forced, steps, gpu.GSVK_DECODE_FUSED)
        kva = [g.kv_read(li) for li in (0, 3)]
        ra = g.generate(reqs, sampler=cfg, max_steps=24, seeds=seeds, flags=1)
        b = _step_logits(g, reqs, forced, steps, gpu.GSVK_DECODE_PERSIST)
        kvb = [g.kv_read(li) for li in (0, 3)]
        rb = g.generate(reqs, sampler=cfg, max_steps=24, seeds=seeds, flags=1)
        g.set_decode_path(gpu.GSVK_DECODE_AUTO)
        rc = g.generate(reqs, sampler=cfg, max_steps=24, seeds=seeds, flags=1)
    finally:
        g.close()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.abs(a - b).max()
    ncol = max(len(r["phones"]) for r in reqs) + 16 + steps - 1    # the columns the steps wrote
    for (ka, va), (kb, vb) in zip(kva, kvb):
        assert np.array_equal(ka[:, :, :ncol], kb[:, :, :ncol]) and np.array_equal(va[:, :, :ncol], vb[:, :, :ncol])
    for r in (rb, rc):
        assert r["n_steps"] == ra["n_steps"]
        for i in range(B):
            assert np.array_equal(r["tokens"][i], ra["tokens"][i]), i


@pytest.mark.parametrize("B, early_stop, max_steps, flags", [(5, 9, 23, 0), (3, -1, 23, 1), (9, 13, 30, 1)])
def test_persistent_generate_steps_per_launch(gpu, model4_path, B, early_stop, max_steps, flags):
    """generate on the persistent decode launches 4 steps per graph (the last max_steps % 4 one by
    one) and its kernel returns at once in steps after the last row finished: the tokens, lengths,
    finish order and step count equal the two-launch layer's (one step per launch), with a
    batch-wide early stop in the middle of a launch and without one."""
    rng = np.random.default_rng(900 + B)
    reqs = _reqs(901 + B, rng.integers(3, 60, B), 16)
    cfg = (15, 1.0, 1.0, 1.35)
    seeds = list(range(1, B + 1))
    g = gpu.Model(model4_path)
    try:
        print(f"generate: batch {B}, early stop {early_stop}, {max_steps} steps", flush=True)
        res = {}
        for path in ("FUSED", "PERSIST", "FUSED"):
            g.set_decode_path(getattr(gpu, "GSVK_DECODE_" + path))
            r = g.generate(reqs, sampler=cfg, early_stop=early_stop, max_steps=max_steps, seeds=seeds, flags=flags)
            res.setdefault(path, r)
    finally:
        g.close()
    a, b = res["FUSED"], res["PERSIST"]
    if early_stop >= 0:
        assert a["n_steps"] < max_steps
    assert b["n_steps"] == a["n_steps"]
    assert np.array_equal(b["lens"], a["lens"]) and np.array_equal(b["finish_seq"], a["finish_seq"])
    for i in range(B):
        assert np.array_equal(b["tokens"][i], a["tokens"][i]), i


def test_decode_kernel_timing_leaves_the_state(gpu, model4_path):
    """gsvk_model_time_decode_kernel (the bench's timing of the persistent kernel alone) repeats the
    current step's kernel: a positive duration, and a generate afterwards gives the tokens it gave
    before. Where the persistent decode does not run (batch 33 on the default path) it is an error."""
    rng = np.random.default_rng(777)
    reqs = _reqs(778, rng.integers(3, 60, 4), 16)
    cfg = (15, 1.0, 1.0, 1.35)
    g = gpu.Model(model4_path)
    try:
        r0 = g.generate(reqs, sampler=cfg, max_steps=12, seeds=[1, 2, 3, 4], flags=1)
        ms = g.time_decode_kernel(5)
        r1 = g.generate(reqs, sampler=cfg, max_steps=12, seeds=[1, 2, 3, 4], flags=1)
        big = _reqs(779, rng.integers(3, 30, 33), 16)
        g.generate(big, sampler=cfg, max_steps=4, seeds=list(range(1, 34)), flags=1)
        with pytest.raises(gpu.GsvkError):
            g.time_decode_kernel(2)
    finally:
        g.close()
    assert 0.0 < ms < 50.0
    for i in range(4):
        assert np.array_equal(r0["tokens"][i], r1["tokens"][i]), i

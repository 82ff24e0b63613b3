"""Exact mode (gsvk_model_set_exact) and its kernels, bit for bit against the oracle.

* gsvk_op_expf_exact: glibc's expf restated on the device (gsv.cpp_amd/csrc/expf_exact.h) against
  this host's libm expf (the oracle's) on a strided sweep of all float bit patterns.
* gsvk_op_attn_exact: flash_attn_ext's sequential online softmax against orc_attn_decode_f16 on
  ragged rows (empty, one key, chunk edges, the whole cache), scores that set a new maximum at
  every key, ties, and scores spread over +-80.
* gsvk_op_qkv_attn_exact (exact mode's fused decode kernel) against the GEMV's q and the oracle's
  attention over the appended cache, bit for bit.
* A model in exact mode: the prefill's K/V (every column, at a row count where the default path
  runs the matrix-core GEMM), the logits entering every teacher-forced decode step and the decode
  K/V columns of layers 0 and 3 equal the oracle's to the bit; a decode of 17 sequences is refused.
"""
import numpy as np
import pytest

import oracle as O
import synth_model as sm

pytestmark = pytest.mark.gpu

GREEDY = (1, 1.0, 1.0, 1.35)


def _dev(a, torch):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_device_expf_matches_libm(gpu):
    import torch
    u = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    dense = np.linspace(-104.0, 0.0, 1 << 20, dtype=np.float32)        # the softmax's arguments
    specials = np.array([0.0, -0.0, np.inf, -np.inf, float.fromhex('0x1.62e42ep6'), float.fromhex('0x1.62e430p6'),
                         float.fromhex('-0x1.9fe368p6'), float.fromhex('-0x1.9fe36ap6'), 1e-30, -1e-30,
                         1.401298464324817e-45], np.float32)
    x = np.concatenate([u.view(np.float32), dense, specials])
    x = x[~np.isnan(x)]
    print(f"expf over {x.size} floats", flush=True)
    xt = _dev(x, torch)
    yt = torch.empty_like(xt)
    gpu.op_expf_exact(xt, yt)
    torch.cuda.synchronize()
    y = yt.cpu().numpy()
    ref = O.expf(x)
    bad = np.flatnonzero(y.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, (bad.size, x[bad[:4]], y[bad[:4]], ref[bad[:4]])


def _attn_inputs(rng, B, nh, lstride):
    q = rng.standard_normal((B, nh, 32)).astype(np.float32)
    k = rng.standard_normal((B, nh, lstride, 32)).astype(np.float32)
    v = rng.standard_normal((B, nh, lstride, 32)).astype(np.float32)
    # sequence 1: every key's score above the last (a new maximum, so a rescale, at every key)
    ramp = np.linspace(0.0, 6.0, lstride, dtype=np.float32)
    k[1] = q[1][:, None, :] * ramp[None, :, None] / np.maximum((q[1] ** 2).sum(-1), 1e-3)[:, None, None]
    # sequence 2: repeated keys (equal scores: the else branch with expf(0) = 1)
    k[2, :, 1::2] = k[2, :, 0::2][:, : lstride // 2]
    # sequence 3: scores spread over about +-80
    q[3] *= 12.0
    return q, k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("B,lstride", [(6, 700), (16, 1100)])
def test_attn_exact_op_matches_oracle(gpu, B, lstride):
    import torch
    rng = np.random.default_rng(400 + B)
    nh = 16
    q, k, v = _attn_inputs(rng, B, nh, lstride)
    begins = rng.integers(0, 60, B).astype(np.int32)
    ends = np.minimum(lstride, begins + rng.integers(1, lstride, B)).astype(np.int32)
    begins[0], ends[0] = 7, 7                       # empty: output 0
    begins[1], ends[1] = 0, lstride                 # the whole cache, rising scores
    begins[2], ends[2] = 2, 2 + 256                 # exactly one chunk of 256
    begins[3], ends[3] = 1, 1 + 257                 # one key into the second chunk
    begins[4], ends[4] = 30, 31                     # one key: that V row
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32.0)))
    out = torch.zeros((B, nh * 32), dtype=torch.float32, device="cuda")
    oq = torch.zeros(B * nh * 32, dtype=torch.int8, device="cuda")
    od = torch.zeros(B * nh, dtype=torch.float32, device="cuda")
    print(f"attn_exact B={B} lstride={lstride}", flush=True)
    gpu.op_attn_exact(_dev(q, torch), _dev(k, torch).view(torch.int16), _dev(v, torch).view(torch.int16),
                      _dev(begins, torch), _dev(ends, torch), scale, out, oq, od)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.attn_decode_f16(q, k, v, begins, ends, scale)
    bad = np.argwhere(got.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, (len(bad), bad[:4], np.abs(got - ref).max())
    assert np.all(got[0] == 0.0)
    assert np.array_equal(got[4], v[4, :, 30, :].view(np.float16).astype(np.float32).reshape(-1))
    # the sliced Q8_0 copy is the x86 quantisation of the output (one block per head)
    blocks = O.q8_quantize_x86(got).reshape(B, nh, 34)
    q_ref = blocks[:, :, 2:].view(np.int8).reshape(B, nh * 32)
    qs = oq.cpu().numpy().reshape(B, 8, nh, 4).transpose(0, 2, 1, 3).reshape(B, nh * 32)
    assert np.array_equal(qs, q_ref)


@pytest.mark.parametrize("B,lstride", [(4, 300), (16, 1100)])
def test_qkv_attn_exact_op_matches_oracle(gpu, B, lstride):
    """Exact mode's fused decode kernel (gsvk_op_qkv_attn_exact: LN input, QKV, K/V append and the
    attention in ggml-cpu's order in chunks of 256 keys) against the LN-input GEMV (bit-exact with
    ggml's dot) and the oracle's attention over the appended cache: output bit for bit, the same K/V
    rows; a row of the new key only, one that reaches column 0, and one whose every key sets a new
    maximum."""
    import torch
    from test_gpu_ops import _dev as dev
    rng = np.random.default_rng(420 + B)
    D, nh, n = 512, 16, 1536
    W = rng.standard_normal((n, D)).astype(np.float32) * 0.02
    wq = torch.zeros(n * D, dtype=torch.int8, device="cuda")
    wd = torch.zeros(n * D // 32, dtype=torch.int16, device="cuda")
    gpu.op_q8_repack(dev(sm.q8_quantize_ref(W).ravel(), torch), n, D, wq, wd)
    bias = dev(rng.standard_normal(n).astype(np.float32) * 0.02, torch)
    res = dev(rng.standard_normal((B, D)).astype(np.float32), torch)
    r = dev(rng.standard_normal((B, D)).astype(np.float32) * 0.5, torch)
    lb = dev(rng.standard_normal(D).astype(np.float32) * 0.02, torch)
    wb = dev(np.concatenate([1 + 0.05 * rng.standard_normal(D), 0.05 * rng.standard_normal(D)]).astype(np.float32),
             torch)
    qkv = torch.zeros((B, n), dtype=torch.float32, device="cuda")
    gpu.op_ln_gemv(wq, wd, n, res, r, lb, wb, bias, 0, qkv)
    torch.cuda.synchronize()
    q = qkv[:, :D].cpu().numpy().reshape(B, nh, 32)
    k = rng.standard_normal((B, nh, lstride, 32)).astype(np.float32)
    v = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16)
    ramp = np.linspace(0.0, 6.0, lstride, dtype=np.float32)     # sequence 2: rising scores
    k[2] = q[2][:, None, :] * ramp[None, :, None] / np.maximum((q[2] ** 2).sum(-1), 1e-3)[:, None, None]
    k = k.astype(np.float16)
    col = lstride - 3
    begins = rng.integers(0, col + 1, B).astype(np.int32)
    begins[0], begins[1], begins[2] = col, 0, 0
    kc, vc = dev(k, torch), dev(v, torch)
    col_d = torch.tensor([col], dtype=torch.int32, device="cuda")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32.0)))
    out = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    print(f"qkv_attn_exact B={B} lstride={lstride}", flush=True)
    gpu.op_qkv_attn(wq, wd, bias, res, r, lb, wb, kc, vc, dev(begins, torch), col_d, scale, out, exact=True)
    torch.cuda.synchronize()
    k2, v2 = k.copy(), v.copy()
    k2[:, :, col, :] = qkv[:, D:2 * D].cpu().numpy().reshape(B, nh, 32).astype(np.float16)
    v2[:, :, col, :] = qkv[:, 2 * D:].cpu().numpy().reshape(B, nh, 32).astype(np.float16)
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), k2.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), v2.view(np.uint16))
    ends = np.full(B, col + 1, np.int32)
    ref = O.attn_decode_f16(q, k2.view(np.uint16), v2.view(np.uint16), begins, ends, scale)
    got = out.cpu().numpy()
    bad = np.argwhere(got.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, (len(bad), bad[:4], np.abs(got - ref).max())
    assert np.array_equal(got[0], v2[0, :, col, :].astype(np.float32).reshape(-1))   # one key: its V row


def _forced_logits(g, reqs, forced, steps):
    import gsvk
    B = len(reqs)
    S = max(len(r["phones"]) for r in reqs) + len(reqs[0]["prompt"])
    gsvk.check(gsvk.lib().gsvk_kv_alloc(g.h, B, S + steps + 8), "kv_alloc")
    lg, _ = g.prefill(reqs)
    out = [lg]
    for i in range(steps - 1):
        out.append(g.decode_step(np.full(B, forced[i], np.int32)))
    return np.array(out)


def test_exact_mode_prefill_and_decode_bitexact(gpu, model4_path):
    rng = np.random.default_rng(410)
    reqs = sm.synth_requests(411, 4, 16, [12, 30, 5, 21])     # 4 x 46 prefill rows
    steps = 10
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    g = gpu.Model(model4_path)
    o = O.Model(model4_path)
    try:
        g.set_exact(True)
        print("exact mode: generate, 4 layers, batch 4", flush=True)
        g.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced, flags=1)
        k0, v0 = g.kv_read(0)
        k3, v3 = g.kv_read(3)
        print("exact mode: step logits", flush=True)
        dev = _forced_logits(g, reqs, forced, steps)
        ref = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                         flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, kv_layer=0, want_logits=True)
        ref3 = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                          flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, kv_layer=3)
    finally:
        g.close()
        o.close()
    assert np.array_equal(dev.view(np.uint32), ref["logits"][:steps].view(np.uint32)), \
        np.abs(dev - ref["logits"][:steps]).max()
    S = max(len(r["phones"]) for r in reqs) + 16
    for (dk, dv), (rk, rv) in (((k0, v0), ref["kv"]), ((k3, v3), ref3["kv"])):
        assert rk.shape[2] == S + steps
        for b, r in enumerate(reqs):
            pad = S - 16 - len(r["phones"])
            sl = slice(pad, S + steps)
            assert np.array_equal(dk[b, :, sl].view(np.float16).astype(np.float32), rk[b, :, sl]), b
            assert np.array_equal(dv[b, :, sl].view(np.float16).astype(np.float32), rv[b, :, sl]), b


def test_exact_mode_decodes_past_16_sequences_in_row_groups(gpu, model4_path):
    """Exact mode at 20 sequences: the GEMV chain in row groups of 16 and 4, one after another;
    logits and the K/V of rows in both groups equal the oracle's to the bit."""
    rng = np.random.default_rng(412)
    B = 20
    reqs = sm.synth_requests(412, B, 8, list(rng.integers(3, 25, B)))
    steps = 6
    forced = rng.integers(0, 1024, steps).astype(np.int32)
    g = gpu.Model(model4_path)
    o = O.Model(model4_path)
    try:
        g.set_exact(True)
        print("exact mode: generate, 4 layers, batch 20", flush=True)
        res = g.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced, flags=1)
        assert res["n_steps"] == steps
        k3, v3 = g.kv_read(3)
        print("exact mode: step logits, batch 20", flush=True)
        dev = _forced_logits(g, reqs, forced, steps)
        ref = o.generate(reqs, sampler=GREEDY, max_steps=steps, oracle=forced,
                         flags=O.ORC_KV_F16 | O.ORC_EOS_MASK_ALL, kv_layer=3, want_logits=True)
    finally:
        g.close()
        o.close()
    assert np.array_equal(dev.view(np.uint32), ref["logits"][:steps].view(np.uint32)), \
        np.abs(dev - ref["logits"][:steps]).max()
    rk, rv = ref["kv"]
    S = max(len(r["phones"]) for r in reqs) + 8
    for b in (0, 15, 16, 19):   # rows of both groups
        pad = S - 8 - len(reqs[b]["phones"])
        sl = slice(pad, S + steps)
        assert np.array_equal(k3[b, :, sl].view(np.float16).astype(np.float32), rk[b, :, sl]), b
        assert np.array_equal(v3[b, :, sl].view(np.float16).astype(np.float32), rv[b, :, sl]), b

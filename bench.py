#!/usr/bin/env python3
"""AR decode throughput of the MI355X (gfx950) text-to-semantic decoder on one GPU.

Workload (the batched-decode configuration the metric is quoted on): the GPT-SoVITS t2s-shaped
decoder (24 layers, d_model 512, 16 heads x 32, FFN 2048, Q8_0 projections, F16 head, synthetic
weights from a fixed seed), batch 16, prompt lengths uniform in [100, 400] (phones = length - 64,
64 shared semantic prompt codes), fp16 KV cache, top-k 15 / top-p 1.0 / temperature 1.0 sampling
with per-sequence xorshift64* seeds, EOS masked so that every sequence decodes all steps.

A "step" is one decode iteration of the whole batch (sampler + 24 layers + head, one HIP graph
launch). The timed region covers exactly --steps steps with the inputs and the prompt's KV cache
resident on the device (the prefill runs before it and is reported separately).

    python bench.py [--gpus 1] [--steps 500] [--warmup 16] [--no-cpu]
    python bench.py --exact-only [--steps 20]      (exact mode alone, for a kernel trace)

Prints one JSON line. The roofline object times the dominant decode kernel (the persistent decode
kernel, all 24 layers of a step in one launch, at batch <= 32) alone with HIP events on the
model's stream (gsvk_model_time_decode_kernel), at the mid-run state of the line's own steps; its
traffic is the HBM-counter ratio of profiles/decode_persist_b16_hbm.md at that shape times those
algorithmic bytes. cpu_baseline times the oracle (the CPU restatement of the reference path) on this host's
cores on the same requests and the same steps, repeated to at least 10 s of decode; with the
oracle as the checker it also counts, under teacher forcing, the steps whose device choice differs
from the oracle's (default path and exact mode, batch 16 and batch 1). extra.exact_mode times
exact mode (ggml-cpu's arithmetic order, the oracle's logits to the bit) on the same workloads.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "gsv.cpp_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
SEED = 0x6A5E0002
N_LAYER, D, NH, HD, FFN, V = 24, 512, 16, 32, 2048, 1025


def workload_requests(B=16, seed=SEED):
    import synth_model as sm
    rng = np.random.Generator(np.random.PCG64(seed))
    P_b = rng.integers(100, 401, B)
    reqs = sm.synth_requests(seed, B, 64, P_b - 64)
    return reqs


def decode_bytes_per_step(reqs, step_kv):
    """Algorithmic HBM bytes of one decode step: Q8_0 weights + biases/LN + F16 head + the valid
    fp16 K/V rows read by attention + the new K/V rows written."""
    w = N_LAYER * (3 * D * D + D * D + 2 * FFN * D) // 32 * 34
    small = N_LAYER * (3 * D + D + FFN + D + 4 * D) * 4
    head = V * D * 2
    T = np.array([len(r["phones"]) for r in reqs])
    P = len(reqs[0]["prompt"])
    valid = T + P + step_kv + 1                       # keys [pad_b, S + step] per sequence
    kv_read = int(valid.sum()) * N_LAYER * 2 * D * 2
    kv_write = len(reqs) * N_LAYER * 2 * D * 2
    return w + small + head + kv_read + kv_write


def prefill_requests(B=16, S=1024, P=256, lo=512, seed=0x6A5E0004, bert=True):
    """Prefill workload: B sequences of valid length U[lo, S] from the seed (one of them exactly S),
    each P shared prompt codes after L_b - P phones, so that the padded batch is B x S rows."""
    import synth_model as sm
    rng = np.random.Generator(np.random.PCG64(seed))
    L = rng.integers(lo, S + 1, B)
    L[0] = S
    return sm.synth_requests(seed, B, P, L - P, bert=bert)


def prefill_flops(reqs):
    """Algorithmic FLOPs of the prefill over the valid rows: the Q8_0 projections (2 per weight per
    row) and attention (QK^T and PV, 4 * head_dim per query-key pair over the reference's masks:
    text rows see the T_b text keys, the semantic row j (0-based) sees T_b + j + 1 keys)."""
    P = len(reqs[0]["prompt"])
    proj = 2 * (3 * D * D + D * D + 2 * FFN * D)
    f = 0
    for r in reqs:
        T = len(r["phones"])
        pairs = T * T + sum(T + j + 1 for j in range(P))
        f += (T + P) * proj + pairs * NH * 4 * HD
    return f * N_LAYER


def time_events(fn, iters, torch):
    """Average duration of fn(i) for i < iters: the launches are captured in one graph (so host
    launch cost is not measured) and the replay is timed with HIP events on its stream."""
    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def kernel_shape(reqs, steps):
    """The mid-run shape of a decode run of `steps` steps: loop index steps // 2, every sequence's
    valid keys [pad_b, S + idx]."""
    T = np.array([len(r["phones"]) for r in reqs])
    P = len(reqs[0]["prompt"])
    max_len = int(T.max())
    S = max_len + P
    mid = steps // 2
    return {"S": S, "mid": mid, "pad": (max_len - T).astype(np.int32), "nkeys": int((S + mid + 1 - (max_len - T)).sum()),
            "lstride": S + steps + 8 + 1}


def kernel_roofline(gsvk, torch, reqs, steps):
    """Time the decode-step kernels alone at the mid-run shape of the line's own run (`steps`
    steps), each in a captured graph of many launches timed with HIP events on its stream,
    rotating through weight copies and K/V caches larger than the 256 MB MALL."""
    B = len(reqs)
    sh = kernel_shape(reqs, steps)
    S, mid, lstride = sh["S"], sh["mid"], sh["lstride"]
    kv_begin = torch.tensor(sh["pad"], dtype=torch.int32, device="cuda")
    kv_end = torch.full((B,), S + mid + 1, dtype=torch.int32, device="cuda")
    col = torch.tensor([S + mid], dtype=torch.int32, device="cuda")
    nkeys = sh["nkeys"]
    kv_bytes = nkeys * NH * 2 * HD * 2
    res = {}
    rot = N_LAYER
    scale = 1.0 / np.sqrt(32.0)
    small = B <= 32   # the two-launch layer's range (the persistent decode's fallback there)
    kc = torch.randn((rot, B, NH, lstride, HD), dtype=torch.float16, device="cuda").view(torch.int16)
    vc = torch.randn((rot, B, NH, lstride, HD), dtype=torch.float16, device="cuda").view(torch.int16)
    qkv_w = 3 * D * D // 32 * 34
    out_w = D * D // 32 * 34
    ffn_w = FFN * D // 32 * 34
    rnd_q = lambda n: torch.randint(-127, 128, (rot, n), dtype=torch.int8, device="cuda")
    rnd_d = lambda n: (torch.rand((rot, n), device="cuda") * 0.001).half().view(torch.int16)
    if small:
        # the two-launch layer of the decode (the default up to batch 32)
        wq, wd = rnd_q(3 * D * D), rnd_d(3 * D * D // 32)
        woq, wod = rnd_q(D * D), rnd_d(D * D // 32)
        w1q, w1d = rnd_q(FFN * D), rnd_d(FFN * D // 32)
        w2q, w2d = rnd_q(FFN * D), rnd_d(FFN * D // 32)
        bq = torch.randn(3 * D, device="cuda") * 0.02
        b1 = torch.randn(FFN, device="cuda") * 0.02
        bo = torch.randn(D, device="cuda") * 0.02
        xres = torch.randn((B, D), device="cuda")
        parts = torch.randn((16, B, D), device="cuda") * 0.1
        wb = torch.cat([torch.ones(D), torch.zeros(D)]).cuda()
        x_out = torch.zeros((B, D), device="cuda")
        n1 = torch.zeros((B, D), device="cuda")
        p1 = torch.zeros((16, B, D), device="cuda")
        p2 = torch.zeros((16, B, D), device="cuda")

        def dec_attn(i):
            r = i % rot
            gsvk.op_dec_attn(B, wq[r], wd[r], bq, kc[r], vc[r], kv_begin, col, scale, woq[r], wod[r], p1,
                             x_out=x_out, res=xres, parts=parts, ln_bias=bo, ln_wb=wb)

        def dec_ffn(i):
            r = i % rot
            gsvk.op_dec_ffn(B, xres, parts, bo, wb, n1, w1q[r], w1d[r], b1, w2q[r], w2d[r], p2)
        ms = time_events(dec_attn, 240, torch)
        ab = kv_bytes + qkv_w + out_w
        res["dec_attn"] = {"ms": ms, "bytes": ab, "gbs": ab / ms / 1e6, "launches_per_step": N_LAYER,
                           "in_decode": False}
        ms = time_events(dec_ffn, 240, torch)
        fb = 2 * ffn_w
        res["dec_ffn"] = {"ms": ms, "bytes": fb, "gbs": fb / ms / 1e6, "launches_per_step": N_LAYER,
                          "in_decode": False}
        del wq, wd, woq, wod, w1q, w1d, w2q, w2d
    # the standalone decode attention (the matrix-core path's, from batch 33)
    q = torch.randn((B, NH, HD), dtype=torch.float32, device="cuda")
    out = torch.zeros((B, NH * HD), dtype=torch.float32, device="cuda")
    oq = torch.zeros(B * D, dtype=torch.int8, device="cuda")
    od = torch.zeros(B * NH, dtype=torch.float32, device="cuda")
    ws = torch.zeros(gsvk.attn_workspace_bytes(B, NH, lstride), dtype=torch.uint8, device="cuda")

    def attn(i):
        gsvk.op_attn_decode(q, kc[i % rot], vc[i % rot], kv_begin, kv_end, lstride, scale, out, oq=oq,
                            od=od, ws=ws)
    ms = time_events(attn, 240, torch)
    res["attn_decode"] = {"ms": ms, "bytes": kv_bytes, "gbs": kv_bytes / ms / 1e6, "launches_per_step": N_LAYER,
                          "in_decode": not small}
    del kc, vc
    return res, sh


def persist_kernel(g, reqs, steps, launches=100):
    """The persistent decode's kernel (the 24 layers of a step in one launch, the decode's dominant
    kernel up to batch 32) alone, at the mid-run state of a run of `steps` steps: a generate of
    steps // 2 + 1 steps leaves the state of loop index steps // 2, whose kernel is then launched
    `launches` times back to back and timed with HIP events on the model's stream
    (gsvk_model_time_decode_kernel). Algorithmic bytes per launch: the 24 layers' Q8_0 weights,
    biases and LayerNorm vectors, the valid K/V rows read and the new K/V rows written (the step's
    head is another kernel)."""
    mid = steps // 2
    B = len(reqs)
    g.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=mid + 1, seeds=list(range(1, B + 1)), flags=1)
    ms = g.time_decode_kernel(launches)
    b = decode_bytes_per_step(reqs, mid) - V * D * 2
    sh = kernel_shape(reqs, steps)
    return {"ms": ms, "bytes": b, "gbs": b / ms / 1e6, "launches_per_step": 1, "in_decode": True,
            "mid": mid, "nkeys": sh["nkeys"]}


def attn_microkernel(gsvk, torch, seed=0x6A5E0003, B=64, sets=8):
    """Decode attention alone: batch 64 x 16 heads x 32, one query per sequence, KV lengths uniform
    in [256, 2048] from the seed, fp16 K/V ~ N(0,1), fp16 output. Rotates over `sets` K/V buffer
    sets (8 x 268 MB, > MALL) so that every launch reads HBM."""
    rng = np.random.Generator(np.random.PCG64(seed))
    L = rng.integers(256, 2049, B)
    lstride = 2048
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    kc = torch.randn((sets, B, NH, lstride, HD), dtype=torch.float16, device="cuda", generator=g)
    vc = torch.randn((sets, B, NH, lstride, HD), dtype=torch.float16, device="cuda", generator=g)
    q = torch.randn((B, NH, HD), dtype=torch.float32, device="cuda", generator=g)
    kv_begin = torch.zeros(B, dtype=torch.int32, device="cuda")
    kv_end = torch.tensor(L, dtype=torch.int32, device="cuda")
    out = torch.zeros((B, NH * HD), dtype=torch.float32, device="cuda")
    out16 = torch.zeros((B, NH * HD), dtype=torch.float16, device="cuda")
    ws = torch.zeros(gsvk.attn_workspace_bytes(B, NH, lstride), dtype=torch.uint8, device="cuda")
    scale = 1.0 / np.sqrt(32.0)

    def attn(i):
        gsvk.op_attn_decode(q, kc[i % sets], vc[i % sets], kv_begin, kv_end, lstride, scale, out, out16=out16,
                            ws=ws)
    ms = time_events(attn, 160, torch)
    b = int(L.sum()) * NH * 2 * HD * 2
    del kc, vc
    return {"us": round(ms * 1e3, 2), "bytes": b, "GBs": round(b / ms / 1e6, 1),
            "frac": round(b / ms / 1e6 / HBM_PEAK_GBS, 4), "batch": B, "kv_len": "U[256,2048]"}


def copy_probe(torch, nbytes=256 << 20):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE counters give the factor
    that turns those counters into bytes for the decode kernels."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    return nbytes


PROFILES_HBM = (os.path.join("profiles", "decode_persist_b16_hbm.md"),
                os.path.join("profiles", "decode_layer_b16_hbm.md"))


def traffic_ratio(kernel, shape=None):
    """(HBM traffic / algorithmic bytes per launch, the shape it was measured at, the summary) of
    `kernel` from the committed counter summaries: two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE) over `bench.py --kernels-only` at that shape, each scaled by what the counter reads
    for a 256 MiB copy; the line measured at `shape` when there is one, else the first. None when
    no summary holds the kernel."""
    found = []
    for rel in PROFILES_HBM:
        path = os.path.join(ROOT, rel)
        if not os.path.exists(path):
            continue
        for line in open(path):
            f = line.split()
            if len(f) >= 5 and f[0] == "traffic_ratio" and f[1] == kernel:
                found.append((float(f[2]), " ".join(f[4:]), rel))
    for t in found:
        if t[1] == shape:
            return t
    return found[0] if found else None


def physical_cores():
    """Physical cores of this host (unique (core, socket) pairs of lscpu -p), or None."""
    import subprocess
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, check=True).stdout
    except Exception:
        return None
    pairs = {tuple(l.split(",")) for l in out.splitlines() if l and not l.startswith("#")}
    return len(pairs) or None


def cpu_baseline(reqs, steps, min_s=10.0):
    """The oracle (the CPU restatement of the reference's ggml path) on this host: the same
    requests and the same `steps` decode steps as the GPU line (each run preceded by its own,
    untimed prefill), repeated until at least min_s seconds of CPU work have run; the rate is the
    tokens of the timed decode loops over their total time."""
    import oracle
    import synth_model as sm
    nthreads = oracle.nthreads_default()
    path = sm.cached_model(os.path.join(ROOT, "_fixtures"), n_layer=N_LAYER)
    m = oracle.Model(path)
    runs, dec_ms, pf_ms = 0, 0.0, 0.0
    try:
        while runs == 0 or dec_ms + pf_ms < min_s * 1e3:
            r = m.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=steps, seeds=list(range(1, len(reqs) + 1)),
                           flags=oracle.ORC_EOS_MASK_ALL, nthreads=nthreads)
            runs += 1
            dec_ms += r["decode_ms"]
            pf_ms += r["prefill_ms"]
    finally:
        m.close()
    tok_s = len(reqs) * steps * runs / (dec_ms / 1e3)
    return {"value": round(tok_s, 2), "unit": "tokens/s", "cores": nthreads, "physical_cores": physical_cores(),
            "kind": "port",
            "sample": f"batch {len(reqs)}, the same requests and the same {steps} decode steps as the GPU line, "
                      f"{runs} run(s): {dec_ms / 1e3:.2f} s of decode timed (their prefills, {pf_ms / 1e3:.1f} s, "
                      f"untimed); F32 KV cache, OpenMP over {nthreads} threads"}


def token_parity(g, reqs, cfg, steps, seeds):
    """Token identity against the oracle (the checker, fp16 KV as on the device) on the same
    requests, sampler, seeds and steps. The oracle runs freely; its sequence-0 tokens are then
    forced on both sides (the reference's oracle_tokens), so that every step of every sequence
    sees the same history, and the device's choice before the override is compared with the
    oracle's at every step. Reported for the default path and for exact mode, plus whether exact
    mode's free run gives the oracle's free-run tokens."""
    import gsvk
    import oracle
    import synth_model as sm
    path = sm.cached_model(os.path.join(ROOT, "_fixtures"), n_layer=N_LAYER)
    o = oracle.Model(path)
    fl = oracle.ORC_KV_F16 | oracle.ORC_EOS_MASK_ALL
    try:
        free = o.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, flags=fl)
        forced = free["sampled"][:, 0].astype(np.int32)
        ref = o.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, oracle=forced, flags=fl)
    finally:
        o.close()
    flags = gsvk.GSVK_GEN_EOS_MASK_ALL
    out = {"choices": len(reqs) * steps}
    for mode in ("default", "exact"):
        g.set_exact(mode == "exact")
        try:
            r = g.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, oracle=forced, flags=flags,
                           want_sampled=True)
            d = {"teacher_forced_differ": int((r["sampled"] != ref["sampled"][:steps]).sum())}
            if mode == "exact":
                rf = g.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, flags=flags)
                d["free_run_tokens_equal"] = all(np.array_equal(rf["tokens"][b], free["tokens"][b])
                                                 for b in range(len(reqs)))
        finally:
            g.set_exact(False)
        out[mode] = d
    return out


def prefill_line(g, torch):
    """Prefill of batch 16 x 1024 rows (valid lengths U[512, 1024], 256 prompt codes), 24 layers:
    median wall time of 3 calls after one warm-up, and TFLOP/s over prefill_flops; the same in the
    fp16 mode (projections on fp16 operands, gsvk_model_set_prefill_f16; its weight copies are made
    in the warm-up call)."""
    pr = prefill_requests()
    fl = prefill_flops(pr)

    def timed():
        g.first_logits(pr)
        torch.cuda.synchronize()
        t = []
        for _ in range(3):
            t0 = time.perf_counter()
            g.first_logits(pr)
            t.append(time.perf_counter() - t0)
        return float(np.median(t))

    pf_s = timed()
    g.set_prefill_f16(True)
    try:
        f16_s = timed()
    finally:
        g.set_prefill_f16(False)
    return {"ms": round(pf_s * 1e3, 2), "tflops": round(fl / pf_s / 1e12, 1),
            "frac_fp16_peak": round(fl / pf_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "algorithmic_tflop": round(fl / 1e12, 3),
            "fp16_mode_ms": round(f16_s * 1e3, 2), "fp16_mode_tflops": round(fl / f16_s / 1e12, 1),
            "workload": "16 x 1024 rows, valid U[512,1024], 256 prompt codes, wall time of the whole "
                        "prefill call incl. head logits"}


def b128_line(g, flags):
    """High-batch long context: batch 128, KV lengths U[1024, 4096] (64 prompt codes), 256 greedy
    steps (the projections run as matrix-core GEMMs at this batch)."""
    hb = prefill_requests(B=128, S=4096, P=64, lo=1024, seed=0x6A5E0005, bert=False)
    seeds = list(range(1, 129))
    g.generate(hb, sampler=(1, 1.0, 1.0, 1.0), max_steps=4, seeds=seeds, flags=flags)
    rb = g.generate(hb, sampler=(1, 1.0, 1.0, 1.0), max_steps=256, seeds=seeds, flags=flags)
    ms5 = rb["decode_ms"] / 256
    b5 = np.mean([decode_bytes_per_step(hb, s) for s in range(0, 256, 16)])
    return {"tok_s": round(128 * 256 / (rb["decode_ms"] / 1e3), 1), "ms_per_step": round(ms5, 4),
            "step_bytes_mb": round(b5 / 1e6, 1),
            "step_hbm_frac": round(b5 / (ms5 / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "prefill_ms": round(rb["prefill_ms"], 1),
            "workload": "128 sequences, KV lengths U[1024,4096] (phones + 64 prompt codes, "
                        "no BERT features), 256 greedy steps"}


def bert_line(torch):
    """The BERT text encoder at the shape of chinese-roberta-wwm-ext-large (hidden 1024, 16 heads,
    FFN 4096, 22 of 24 layers, vocab 21128; synthetic F16 weights, the file type the engine loads:
    fp16 products with fp32 sums): median wall time of 5 encode calls after one warm-up, for one
    64-token sentence and for 8 sentences of 64 tokens in one call, with TFLOP/s over the
    algorithmic flops (2 per weight per token, 4 x hidden per visible query-key pair) against the
    fp16 matrix-core peak."""
    import gsvk
    import synth_model as sm
    d = os.path.join(ROOT, "_fixtures")
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, "gsv_bert_large_f16.gguf")
    if not os.path.exists(path):
        sm.write_bert_model(path, n_layer=22, layers_used=22, vocab=21128, wtype="f16")
    m = gsvk.Bert(path)
    rng = np.random.default_rng(0x6A5E0006)
    res = {}
    L, D, F = m.info["layers_used"], m.info["hidden"], m.info["inter"]
    for name, B, T in (("t64", 1, 64), ("b8_t64", 8, 64)):
        seqs = [rng.integers(0, 21128, size=T).astype(np.int32) for _ in range(B)]
        m.encode(seqs)
        t = []
        for _ in range(5):
            t0 = time.perf_counter()
            m.encode(seqs)
            t.append(time.perf_counter() - t0)
        s = float(np.median(t))
        fl = B * T * L * (2.0 * (4 * D * D + 2 * D * F) + 4.0 * T * D)
        res[name] = {"ms": round(s * 1e3, 3), "tflops": round(fl / s / 1e12, 2),
                     "frac_fp16_peak": round(fl / s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    m.close()
    res["workload"] = ("BERT encoder, hidden 1024, 16 heads, FFN 4096, 22 layers, F16 weights (fp16 "
                       "products, fp32 sums, fp32 attention and LayerNorm); wall time of encode (ids "
                       "upload to features on the host)")
    return res


def exact_line(g, B, steps, warmup, cfg, flags):
    """Exact mode (gsvk_model_set_exact) on the batch-B workload over `steps` steps and on the batch-1
    workload (128 phones + 64 prompt codes, 300 greedy steps, repetition penalty 1.35)."""
    import synth_model as sm
    reqs = workload_requests(B)
    r1 = sm.synth_requests(0x6A5E0001, 1, 64, [128])
    cfg1 = (1, 1.0, 1.0, 1.35)
    g.set_exact(True)
    try:
        g.generate(r1, sampler=cfg1, max_steps=8, seeds=[1], flags=flags)
        rx1 = g.generate(r1, sampler=cfg1, max_steps=300, seeds=[1], flags=flags)
        g.generate(reqs, sampler=cfg, max_steps=max(warmup, 1), seeds=list(range(1, B + 1)), flags=flags)
        rx = g.generate(reqs, sampler=cfg, max_steps=steps, seeds=list(range(1, B + 1)), flags=flags)
    finally:
        g.set_exact(False)
    return {"tok_s": round(B * steps / (rx["decode_ms"] / 1e3), 1),
            "ms_per_step": round(rx["decode_ms"] / steps, 4),
            "tok_s_b1": round(300 / (rx1["decode_ms"] / 1e3), 1),
            "ms_per_step_b1": round(rx1["decode_ms"] / 300, 4),
            "what": "gsvk_model_set_exact: the same workloads with ggml-cpu's arithmetic "
                    "order throughout (logits equal to the oracle's to the bit)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-b128", action="store_true", help="skip the batch-128 long-context decode line")
    ap.add_argument("--prefill-only", action="store_true", help="time only the batch-16 x 1024 prefill")
    ap.add_argument("--b128-only", action="store_true", help="time only the batch-128 long-context decode")
    ap.add_argument("--bert-only", action="store_true", help="time only the BERT text encoder")
    ap.add_argument("--no-bert", action="store_true", help="skip the BERT text encoder line")
    ap.add_argument("--exact-only", action="store_true",
                    help="time only exact mode (the batch's workload and batch 1) and print it")
    ap.add_argument("--kernels-only", action="store_true",
                    help="time only the per-kernel roofline launches (for counter runs) and print them")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this decoder runs each batch on a single MI355X and has no "
              f"multi-GPU path (--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)

    import torch

    import gsvk
    import synth_model as sm

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    if args.kernels_only:
        kreqs = workload_requests(args.batch)
        kr, sh = kernel_roofline(gsvk, torch, kreqs, args.steps)
        if args.batch <= 32:
            gk = gsvk.Model(sm.cached_model(os.path.join(ROOT, "_fixtures"), n_layer=N_LAYER), device=0)
            try:
                kr["dec_persist"] = persist_kernel(gk, kreqs, args.steps)
            finally:
                gk.close()
        res = {k: {"us": round(v["ms"] * 1e3, 3), "bytes": v["bytes"], "GBs": round(v["gbs"], 1),
                   "in_decode": v["in_decode"]} for k, v in kr.items()}
        res["shape"] = {"batch": args.batch, "steps": args.steps, "mid_step": sh["mid"], "valid_keys": sh["nkeys"]}
        res["attn_microkernel_b64"] = attn_microkernel(gsvk, torch)
        res["copy_probe_bytes"] = copy_probe(torch)
        print(json.dumps({"kernels_only": res}))
        return
    if args.bert_only:
        print(json.dumps({"bert_encode": bert_line(torch)}))
        return
    path = sm.cached_model(os.path.join(ROOT, "_fixtures"), n_layer=N_LAYER)
    g = gsvk.Model(path, device=0)
    if args.prefill_only:
        print(json.dumps({"prefill_b16_s1024": prefill_line(g, torch)}))
        g.close()
        return
    if args.b128_only:
        print(json.dumps({"b128_long": b128_line(g, gsvk.GSVK_GEN_EOS_MASK_ALL)}))
        g.close()
        return
    cfg = (15, 1.0, 1.0, 1.35)
    flags = gsvk.GSVK_GEN_EOS_MASK_ALL
    if args.exact_only:
        print(json.dumps({"exact_mode": exact_line(g, args.batch, args.steps, args.warmup, cfg, flags)}))
        g.close()
        return

    def run(B, steps, warmup):
        reqs = workload_requests(B)
        seeds = list(range(1, B + 1))
        if warmup:
            g.generate(reqs, sampler=cfg, max_steps=warmup, seeds=seeds, flags=flags)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        r = g.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, flags=flags)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        assert r["n_steps"] == steps and all(len(t) == len(reqs[0]["prompt"]) + steps for t in r["tokens"])
        return reqs, r, wall

    reqs, r, wall = run(args.batch, args.steps, args.warmup)
    B = args.batch
    dec_s = r["decode_ms"] / 1e3
    tok_s = B * args.steps / dec_s
    ms_step = r["decode_ms"] / args.steps
    step_bytes = np.mean([decode_bytes_per_step(reqs, s) for s in range(0, args.steps, max(1, args.steps // 16))])
    Tn = np.array([len(r["phones"]) for r in reqs])
    step_kv_lo = Tn.min() + len(reqs[0]["prompt"]) + 1
    step_kv_hi = Tn.max() + len(reqs[0]["prompt"]) + args.steps
    extra = {"prefill_ms": round(r["prefill_ms"], 2), "wall_s_incl_prefill": round(wall, 3),
             "step_bytes_mb": round(step_bytes / 1e6, 1),
             "step_hbm_frac": round(step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}
    # batch 1 as the reference's single-sequence case: 128 phones + 64 prompt codes (prefill 192),
    # 300 greedy steps (repetition penalty 1.35) with EOS masked
    r1 = sm.synth_requests(0x6A5E0001, 1, 64, [128])
    cfg1 = (1, 1.0, 1.0, 1.35)
    g.generate(r1, sampler=cfg1, max_steps=8, seeds=[1], flags=flags)
    rb = g.generate(r1, sampler=cfg1, max_steps=300, seeds=[1], flags=flags)
    extra["tok_s_b1"] = round(300 / (rb["decode_ms"] / 1e3), 1)
    extra["ms_per_step_b1"] = round(rb["decode_ms"] / 300, 4)
    extra["b1_workload"] = "1 sequence, 128 phones + 64 prompt codes, 300 greedy steps, repetition penalty 1.35"
    # exact mode (ggml-cpu's arithmetic order throughout: the oracle's logits to the bit) on the same
    # two workloads
    extra["exact_mode"] = exact_line(g, B, args.steps, args.warmup, cfg, flags)
    # the decode's dominant kernel alone at the timed run's mid-run state (batch <= 16)
    pk = persist_kernel(g, reqs, args.steps) if (not args.no_kernels and B <= 32) else None
    # batch 64: the batch-16 workload's request shape at 64 sequences, 200 steps
    _, rb, _ = run(64, 200, 8)
    extra["tok_s_b64"] = round(64 * 200 / (rb["decode_ms"] / 1e3), 1)
    extra["ms_per_step_b64"] = round(rb["decode_ms"] / 200, 4)
    extra["prefill_b16_s1024"] = prefill_line(g, torch)
    if not args.no_b128:
        extra["b128_long"] = b128_line(g, flags)
        g.release_cache()
    g.close()
    if not args.no_bert:
        extra["bert_encode"] = bert_line(torch)

    roof = None
    if not args.no_kernels:
        kr, sh = kernel_roofline(gsvk, torch, reqs, args.steps)
        if pk is not None:
            kr["dec_persist"] = pk
        extra["kernels"] = {k: {"us": round(v["ms"] * 1e3, 2), "GBs": round(v["gbs"], 1),
                                "frac": round(v["gbs"] / HBM_PEAK_GBS, 4), "in_decode": v["in_decode"]}
                            for k, v in kr.items()}
        extra["attn_microkernel_b64"] = attn_microkernel(gsvk, torch)
        dom = max((k for k in kr if kr[k]["in_decode"]), key=lambda k: kr[k]["ms"] * kr[k]["launches_per_step"])
        d = kr[dom]
        shape = (f"batch {B}, mid-run of {args.steps} steps (loop index {sh['mid']}), "
                 f"{sh['nkeys']} valid keys per head")
        tr = traffic_ratio(dom, shape)
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(d["gbs"], 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
                "traffic": None if tr is None else int(round(tr[0] * d["bytes"])),
                "bytes_per_launch": int(d["bytes"]), "us_per_launch": round(d["ms"] * 1e3, 3),
                "shape": shape,
                "timing": "HIP events around back-to-back launches on the launching stream"
                          + (" (gsvk_model_time_decode_kernel)" if dom == "dec_persist" else
                             " (one captured graph of 240 launches)"),
                "traffic_basis": None if tr is None else
                {"ratio": tr[0], "measured_at": tr[1], "profile": tr[2]}}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(reqs, args.steps)
        g = gsvk.Model(path, device=0)
        try:
            cpu["token_parity"] = {
                "batch16": token_parity(g, reqs, cfg, args.steps, list(range(1, B + 1))),
                "batch1": token_parity(g, r1, cfg1, 300, [1]),
                "what": "the oracle (fp16 KV) as the checker: its tokens forced on both sides, the "
                        "device's choice before the override compared at every step; default path "
                        "and exact mode"}
        finally:
            g.close()

    line = {
        "metric": "AR decode tokens/sec at batch 1/16/64; attn+Q8_0 GEMV % of HBM roofline",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q8_0 int8 dot, fp32 accumulate, fp16 KV",
        "data": "synthetic (random-init weights from a fixed seed, seeded requests)",
        "config": {"workload": f"batched AR decode, 24-layer t2s decoder (d512, 16x32 heads, FFN 2048, Q8_0, "
                               f"F16 head), batch {B}, prompt lengths U[100,400] (64 prompt codes), fp16 KV, "
                               f"top-k 15 sampling, the first {args.steps} decode steps of the configuration's 500 "
                               f"(KV {int(step_kv_lo)}-{int(step_kv_hi)} keys per sequence over the timed steps)",
                   "batch": B, "decode_steps": args.steps, "prompt_codes": 64,
                   "kv": "fp16", "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()

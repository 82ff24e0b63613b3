"""Per-phase timeline of the persistent decode (k_dec_persist) from its phase stamps.

    python gsv.cpp_amd/build.py --phase-stamps          # lib/libgsvk_stamps.so
    python gsv.cpp_amd/phase_stamps.py [--batch 16] [--steps 20]

Runs a generate of the decode benchmark's request shape (prompt lengths U[100, 400] from the
benchmark's seed, 64 shared prompt codes; batch 1: 128 phones + 64 codes) on the 24-layer
synthetic model with the stamps library, then reads the stamps of the last persistent launch
(gsvk_phase_stamps: thread 0 of every workgroup records the 100 MHz s_memrealtime counter at each
event of each layer's two phases). A phase starts when the barrier before it completes, i.e. when
the last of the XCD's 32 workgroups stored its flag for the phase before; the table gives, per
event, the time from that completion (medians and maxima over the workgroups of every XCD that
holds a sequence and over layers 1-23). The stamps' own stores add a few tens of nanoseconds per
event to the kernel.
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)

WGS, SLOTS = 256, 64 * 16
TICK_US = 0.01   # s_memrealtime: 100 MHz
ATTN = [(0, "barrier seen"), (1, "input row (LN2 / embedding) quantised"), (2, "QKV + K/V append"),
        (3, "attention merged"), (4, "out-projection partial row stored"), (5, "flag stored")]
FFN = [(8, "barrier seen"), (9, "LN1 row quantised"), (10, "FFN1 blocks quantised"),
       (11, "FFN2 partial row stored"), (12, "flag stored")]


def workload(B: int):
    import synth_model as sm
    if B == 1:
        return sm.synth_requests(0x6A5E0001, 1, 64, [128])
    rng = np.random.Generator(np.random.PCG64(0x6A5E0002))
    P_b = rng.integers(100, 401, B)
    return sm.synth_requests(0x6A5E0002, B, 64, P_b - 64)


def run(B: int, steps: int) -> np.ndarray:
    import gsvk
    import synth_model as sm
    gsvk.LIB_PATH = os.path.join(HERE, "lib", "libgsvk_stamps.so")
    model = gsvk.Model(sm.cached_model(os.path.join(ROOT, "_fixtures"), n_layer=24), device=0)
    try:
        reqs = workload(B)
        cfg = (1 if B == 1 else 15, 1.0, 1.0, 1.35)
        seeds = list(range(1, B + 1))
        model.generate(reqs, sampler=cfg, max_steps=16, seeds=seeds, flags=gsvk.GSVK_GEN_EOS_MASK_ALL)
        r = model.generate(reqs, sampler=cfg, max_steps=steps, seeds=seeds, flags=gsvk.GSVK_GEN_EOS_MASK_ALL)
        print(f"batch {B}, {steps} steps: {r['decode_ms'] / steps:.4f} ms per step", flush=True)
        buf = np.zeros(WGS * SLOTS, np.int64)
        gsvk.check(gsvk.lib().gsvk_phase_stamps(buf.ctypes.data_as(C.c_void_p), C.c_size_t(buf.size)),
                   "phase_stamps")
    finally:
        model.close()
    return buf.reshape(WGS, SLOTS)


def analyse(st: np.ndarray, B: int, n_layer: int = 24) -> list[str]:
    xcd = st[:, 63 * 16 + 1]
    start = st[:, 63 * 16]
    rows = {(phase, ev): [] for phase, evs in (("attention", ATTN), ("FFN", FFN)) for ev, _ in evs}
    per_layer = []
    for x in range(min(B, 8)):   # the XCDs that hold a sequence (x, x + 8, ...)
        wg = np.where(xcd == x)[0]
        if wg.size != 32:
            continue
        s = st[wg].reshape(32, 64, 16)
        per_layer.append((s[:, n_layer - 1, 12].max() - start[wg].min()) * TICK_US / n_layer)
        for li in range(1, n_layer):
            bar_a = s[:, li - 1, 12].max()   # the last FFN flag of layer li - 1
            bar_f = s[:, li, 5].max()        # the last attention flag of layer li
            t0 = start[wg].min()   # (a workgroup without an item in a phase has no stamps of this launch)
            for ev, _ in ATTN:
                v = s[:, li, ev]
                rows[("attention", ev)].extend(((v[v >= t0] - bar_a) * TICK_US).tolist())
            for ev, _ in FFN:
                v = s[:, li, ev]
                rows[("FFN", ev)].extend(((v[v >= t0] - bar_f) * TICK_US).tolist())
    out = [f"kernel time per layer (launch start to the last flag of layer {n_layer - 1}, / {n_layer}), per XCD: "
           + ", ".join(f"{v:.2f}" for v in per_layer) + " us", "",
           "| phase | event (from the barrier's completion) | median us | max us |", "|---|---|---:|---:|"]
    for phase, evs in (("attention", ATTN), ("FFN", FFN)):
        for ev, name in evs:
            v = np.array(rows[(phase, ev)])
            out.append(f"| {phase} | {name} | {np.median(v):.2f} | {v.max():.2f} |")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--steps", type=int, default=20)
    a = ap.parse_args()
    st = run(a.batch, a.steps)
    print("\n".join(analyse(st, a.batch)))


if __name__ == "__main__":
    main()

"""Helpers shared by the token-parity tests: which teacher-forced choices may differ from the
oracle's.

The default decode path's logits differ from the oracle's by the drift of Q8_0 re-quantisation
(a rounding-level difference that lands on a rounding boundary flips one int8 value of an
activation block). With e = max |device - oracle| over the penalised logits of a step, the step
is fragile when some other token could win under a perturbation of every logit by at most e:
tok = argmax over the top-k set of z_i - log q_i (q the step's exponential draws), so either tok
can leave that set or another token that can be in it scores within 2e of tok (greedy: the top two
penalised logits within 2e). A choice may differ from the oracle's only at a fragile step.
"""
import numpy as np

import oracle as O

V, EOS = 1025, 1024


def penalised(cfg, z, hist, mask_eos=True):
    """The sampler's row after EOS masking, the repetition penalty and the temperature (top_k = V
    and top_p = 1 leave it whole): the oracle's own pinned function."""
    row = np.array(z, np.float32)
    if mask_eos:
        row[EOS] = -np.inf
    out, _ = O.logits_to_probs((V, 1.0, cfg[2], cfg[3]), row, hist)
    return out


def decision(cfg, z, hist, q, mask_eos=True):
    """The sampler's choice for the logits z entering a step, with the step's exponential draws q:
    the oracle's pinned gsv_logits_to_probs and argmax p / q."""
    row = np.array(z, np.float32)
    if mask_eos:
        row[EOS] = -np.inf
    _, probs = O.logits_to_probs(cfg, row, hist)
    return int(O.lib().orc_argmax_probs_over_q(probs, np.ascontiguousarray(q, np.float32), V))


def fragile(cfg, zrow, q, e, tok):
    """Could a perturbation of every logit by at most e change the choice tok?"""
    k = cfg[0]
    fin = np.isfinite(zrow)
    zs = np.sort(zrow[fin])[::-1]
    kk = min(k, int(fin.sum()))
    zk = zs[kk - 1]
    zk1 = zs[kk] if kk < len(zs) else -np.inf
    cand = fin & (zrow >= zk - 2 * e)
    cand[tok] = False
    if not cand.any():
        return False
    if zrow[tok] <= zk1 + 2 * e:
        return True
    score = zrow.astype(np.float64) - np.log(q.astype(np.float64))
    return bool(np.any(score[cand] >= score[tok] - 2 * e - 1e-6))


def device_step_logits(g, reqs, forced, steps):
    """Prefill + steps - 1 decode steps fed the forced tokens: the logits entering each step."""
    import gsvk
    B = len(reqs)
    S = max(len(r["phones"]) for r in reqs) + len(reqs[0]["prompt"])
    gsvk.check(gsvk.lib().gsvk_kv_alloc(g.h, B, S + steps + 8), "kv_alloc")
    lg, _ = g.prefill(reqs)
    out = np.zeros((steps, B, V), np.float32)
    out[0] = lg
    for i in range(steps - 1):
        out[i + 1] = g.decode_step(np.full(B, forced[i], np.int32))
    return out


def check_choices(reqs, cfg, forced, seeds, ref, res, dev, steps):
    """Every teacher-forced choice of the device (res["sampled"], from the generate graph) equals
    its own decision over its step logits dev, the oracle's equals its decision over ref["logits"],
    and the two differ only at fragile steps. Returns (mismatches, fragile steps, worst drift as a
    fraction of the row scale)."""
    B = len(reqs)
    P = len(reqs[0]["prompt"])
    draws = [O.rng_exponential_n(s, steps * V).reshape(steps, V) for s in seeds]
    n_mis = n_fragile = 0
    worst = 0.0
    for b in range(B):
        hist = np.concatenate([reqs[b]["prompt"], forced]).astype(np.int32)
        for i in range(steps):
            h = hist[:P + i]
            zo = penalised(cfg, ref["logits"][i, b], h)
            zd = penalised(cfg, dev[i, b], h)
            fin = np.isfinite(zo)
            e = float(np.abs(zd[fin] - zo[fin]).max())
            worst = max(worst, e / float(np.abs(zo[fin]).max()))
            q = draws[b][i]
            tok_o = decision(cfg, ref["logits"][i, b], h, q)
            tok_d = decision(cfg, dev[i, b], h, q)
            assert tok_o == ref["sampled"][i, b], (b, i)            # the oracle's own choice
            assert tok_d == res["sampled"][i, b], (b, i)            # the device's own choice
            fr = fragile(cfg, zo, q, e, tok_o)
            n_fragile += fr
            if tok_d != tok_o:
                n_mis += 1
                assert fr, (b, i, tok_d, tok_o, e)
    return n_mis, n_fragile, worst

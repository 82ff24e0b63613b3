"""The device sampler against the reference's own sampler: tests/golden/sampler_golden.npz holds
inputs and outputs of src/gsv_sampler.cpp (gsv_logits_to_probs, gsv_rng, gsv_sample) compiled from
the reference's source. Every case runs through gsvk_op_sample (one launch of the kernel the
decode loop uses) with each golden seed.

Tolerance: the masks (which entries are zero) and the sampled tokens and RNG states must be
identical. Probabilities may differ by a few ulp: the reference uses glibc expf, the device
(float)exp(double), i.e. the correctly rounded value, which glibc's expf is not always."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def _run(gpu, z, seed):
    import torch
    n, V = z["logits_in"].shape
    logits = torch.tensor(z["logits_in"], device="cuda")
    hist = torch.tensor(z["prev"], device="cuda")
    n_hist = torch.tensor(np.where(z["has_prev"] > 0, z["n_prev"], 0).astype(np.int32), device="cuda")
    toks = np.zeros(n, np.int32)
    states = np.zeros(n, np.uint64)
    probs = np.zeros((n, V), np.float32)
    # one call per configuration (the sampler settings are per call)
    for i in range(n):
        k, p, t, r = z["cfg"][i]
        st = np.array([seed if seed != 0 else 1], np.uint64)          # gsv_rng: seed 0 -> 1
        rng = torch.tensor(st.view(np.int64), device="cuda")
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        pr = torch.zeros((1, V), dtype=torch.float32, device="cuda")
        gpu.op_sample(logits[i:i + 1], (int(k), float(p), float(t), float(r)), rng, tok, hist=hist[i:i + 1],
                      n_hist=n_hist[i:i + 1], probs_out=pr)
        toks[i] = int(tok.cpu()[0])
        states[i] = rng.cpu().numpy().view(np.uint64)[0]
        probs[i] = pr.cpu().numpy()[0]
    return toks, states, probs


def test_probs_match_reference(gpu, golden):
    _, _, probs = _run(gpu, golden, int(golden["seeds"][1]))
    ref = golden["probs"]
    for i in range(ref.shape[0]):
        assert np.array_equal(probs[i] == 0, ref[i] == 0), f"case {i}: different mask"
        nz = ref[i] > 0
        rel = np.abs(probs[i][nz] - ref[i][nz]) / ref[i][nz]
        assert rel.max() <= 4 * 2.0 ** -23, (i, rel.max())


@pytest.mark.parametrize("j", range(6))
def test_tokens_and_rng_match_reference(gpu, golden, j):
    seed = int(golden["seeds"][j])
    toks, states, _ = _run(gpu, golden, seed)
    assert np.array_equal(toks, golden["sample_tok"][:, j]), (toks, golden["sample_tok"][:, j])
    assert np.array_equal(states, golden["sample_state"][:, j])


def test_batch_rows_are_independent(gpu, golden):
    """All 19 default-config-like rows in one launch give the same tokens as one row per launch."""
    import torch
    z = golden
    sel = [i for i in range(z["cfg"].shape[0]) if tuple(z["cfg"][i]) == (15.0, 1.0, 1.0, np.float32(1.35))]
    assert len(sel) >= 4
    seed = int(z["seeds"][2])
    toks1, st1, _ = _run(gpu, z, seed)
    logits = torch.tensor(z["logits_in"][sel], device="cuda")
    hist = torch.tensor(z["prev"][sel], device="cuda")
    n_hist = torch.tensor(np.where(z["has_prev"][sel] > 0, z["n_prev"][sel], 0).astype(np.int32), device="cuda")
    rng = torch.tensor(np.full(len(sel), seed, np.uint64).view(np.int64), device="cuda")
    tok = torch.zeros(len(sel), dtype=torch.int32, device="cuda")
    gpu.op_sample(logits, (15, 1.0, 1.0, 1.35), rng, tok, hist=hist, n_hist=n_hist)
    assert np.array_equal(tok.cpu().numpy(), toks1[sel])
    assert np.array_equal(rng.cpu().numpy().view(np.uint64), st1[sel])


@pytest.mark.parametrize("top_k", [1, 2, 15, 40, 61, 62, 64, 65, 100, 500, 1024])
@pytest.mark.parametrize("kind", ["normal", "ties", "coarse", "neg_inf"])
def test_top_k_pivot_against_oracle(gpu, top_k, kind):
    """top-k pivot (k-th largest with multiplicity, ties kept) over rows that reach every path of
    the device selection: k <= 64 with a small candidate set, k <= 64 with many ties (the
    candidate set overflows one wave), k just above the 61 lanes that hold values, and k > 64."""
    import torch
    import oracle as O
    rng = np.random.default_rng(1000 + top_k)
    V, B = 1025, 4
    if kind == "normal":
        lg = rng.standard_normal((B, V)).astype(np.float32)
    elif kind == "ties":
        lg = (np.round(rng.standard_normal((B, V)) * 3) / 3).astype(np.float32)
    elif kind == "coarse":
        lg = rng.integers(0, 3, (B, V)).astype(np.float32)
    else:
        lg = rng.standard_normal((B, V)).astype(np.float32)
        lg[:, rng.integers(0, V, 900)] = -np.inf
    seeds = [11, 12, 13, 14]
    cfg = (top_k, 1.0, 1.0, 1.0)
    probs = torch.zeros((B, V), dtype=torch.float32, device="cuda")
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.tensor(np.array(seeds, np.uint64).view(np.int64), device="cuda")
    gpu.op_sample(torch.tensor(lg, device="cuda"), cfg, st, tok, probs_out=probs)
    got = probs.cpu().numpy()
    for b in range(B):
        _, ref = O.logits_to_probs(cfg, lg[b], None)
        assert np.array_equal(got[b] == 0, ref == 0), (kind, top_k, b, int((got[b] > 0).sum()), int((ref > 0).sum()))
        nz = ref > 0
        assert np.abs(got[b][nz] - ref[nz]).max() <= 4 * 2.0 ** -23 * ref[nz].max()
        t_ref, s_ref = O.sample(ref, seeds[b])
        assert int(tok.cpu()[b]) == t_ref
        assert int(st.cpu().numpy().view(np.uint64)[b]) == s_ref

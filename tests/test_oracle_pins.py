"""CPU tests that pin the oracle (the CPU restatement of the reference path) before it is trusted.

Every function of the oracle is checked against something other than itself:
  * the sampler against golden vectors written by the reference's own gsv_sampler.cpp
    (tests/golden/sampler_golden.npz) and against an independent Python restatement of xorshift64*;
  * Q8_0 against closed forms and known-answer blocks, the int8 dot against fp64 and against a
    lane-by-lane scalar restatement (bit-exact);
  * LayerNorm against closed forms (constant row, 1..512) and fp64;
  * add + activation against the reference's own fixture (tests/test_add_act.cpp:66-101);
  * the PE table against fp64 sin/cos;
  * attention against an fp64 softmax and its invariants, the prefill masks by perturbation;
  * masks and the generate loop against properties of src/gsv_ar.cpp (left padding changes
    nothing, text queries never see semantic keys, causality) and hand-derived traces of the loop.
"""
import math
import os

import numpy as np
import pytest

import oracle as O
import synth_model as sm

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.fixture(scope="module")
def tiny_path(tmp_path_factory):
    d = tmp_path_factory.mktemp("m")
    return sm.write_model(str(d / "tiny.gguf"), seed=5, n_layer=2, d_model=64, n_head=2, ffn=128,
                          vocab=129, phone_vocab=40, eos=128)


# ------------------------------------------------------------------------------- sampler

def test_sampler_matches_reference_golden(golden):
    for i in range(golden["cfg"].shape[0]):
        k, p, t, r = golden["cfg"][i]
        prev = golden["prev"][i, :golden["n_prev"][i]] if golden["has_prev"][i] else None
        lg, probs = O.logits_to_probs((int(k), float(p), float(t), float(r)), golden["logits_in"][i], prev)
        assert np.array_equal(lg, golden["logits_out"][i]), i
        assert np.array_equal(probs.view(np.uint32), golden["probs"][i].view(np.uint32)), i


def test_rng_matches_reference_golden(golden):
    for i, sd in enumerate(golden["seeds"]):
        s, final = O.rng_stream(int(sd), 2100)
        assert np.array_equal(s, golden["rng_stream"][i])
        assert final == int(golden["rng_final"][i])
        e, _ = O.rng_exponential(int(sd), 2100)
        assert np.array_equal(e.view(np.uint32), golden["rng_exp"][i].view(np.uint32))


def test_sample_matches_reference_golden(golden):
    for i in range(golden["probs"].shape[0]):
        for j, sd in enumerate(golden["seeds"]):
            tok, st = O.sample(golden["probs"][i], int(sd))
            assert tok == golden["sample_tok"][i, j] and st == int(golden["sample_state"][i, j])


def test_rng_independent_restatement():
    """xorshift64*: s ^= s>>12; s ^= s<<25; s ^= s>>27; out = s * 0x2545F4914F6CDD1D (mod 2^64);
    seed 0 -> 1 (src/gsv_sampler.h:33-42), restated with Python integers."""
    M = (1 << 64) - 1
    for seed in (0, 1, 99, 0xDEADBEEFCAFEF00D):
        s = seed if seed else 1
        ref = []
        for _ in range(50):
            s ^= s >> 12
            s ^= (s << 25) & M
            s ^= s >> 27
            ref.append((s * 0x2545F4914F6CDD1D) & M)
        got, _ = O.rng_stream(seed, 50)
        assert [int(x) for x in got] == ref
        u = np.float32(float(ref[0] >> 40) / 16777216.0)
        e, _ = O.rng_exponential(seed, 1)
        assert abs(float(e[0]) - (-math.log(1.0 - float(u)))) <= 2e-7 * max(1.0, abs(float(e[0])))


def test_sampler_special_cases():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal(1025).astype(np.float32)
    # top_k = 1 -> one-hot at the argmax; top_k >= V and top_p = 1 -> plain softmax
    _, p1 = O.logits_to_probs((1, 1.0, 1.0, 1.0), lg, None)
    assert p1[np.argmax(lg)] == 1.0 and p1.sum() == 1.0
    _, pall = O.logits_to_probs((1025, 1.0, 1.0, 1.0), lg, None)
    e = np.exp(lg.astype(np.float64) - lg.max())
    assert np.allclose(pall, e / e.sum(), rtol=1e-5, atol=1e-9)
    # the penalty applies once per occurrence: a token seen 3 times is divided by 1.35^3
    l2, _ = O.logits_to_probs((0, 1.0, 1.0, 1.35), np.array([2.0, -2.0, 1.0] + [0.0] * 29, np.float32),
                              np.array([0, 0, 0, 1], np.int32))
    assert abs(l2[0] - 2.0 / 1.35 ** 3) < 1e-6 and abs(l2[1] - (-2.0 * 1.35)) < 1e-6 and l2[2] == 1.0


# ------------------------------------------------------------------------------- Q8_0

def test_q8_known_answer_blocks():
    blocks = np.zeros((4, 34), np.uint8)
    blocks[0, 0:2] = np.array([0], np.float16).view(np.uint8)               # d = 0 -> zeros
    blocks[0, 2:] = np.arange(32).astype(np.int8).view(np.uint8)
    blocks[1, 0:2] = np.array([0.5], np.float16).view(np.uint8)             # +-127 extremes
    blocks[1, 2:] = np.array([127, -127] * 16, np.int8).view(np.uint8)
    blocks[2, 0:2] = np.array([-0.0], np.float16).view(np.uint8)            # negative zero scale
    blocks[2, 2:] = np.full(32, 3, np.int8).view(np.uint8)
    blocks[3, 0:2] = np.array([6.1035e-05], np.float16).view(np.uint8)      # smallest normal fp16
    blocks[3, 2:] = np.arange(-16, 16).astype(np.int8).view(np.uint8)
    out = O.q8_dequant(blocks).reshape(4, 32)
    assert np.all(out[0] == 0)
    assert np.array_equal(out[1], np.array([63.5, -63.5] * 16, np.float32))
    assert np.all(out[2] == 0) and np.all(np.signbit(out[2]))
    d = np.float32(np.float16(6.1035e-05))
    assert np.array_equal(out[3], d * np.arange(-16, 16).astype(np.float32))


def test_q8_activation_quantiser_known_answers():
    x = np.zeros(96, np.float32)
    x[:32] = np.arange(-16, 16, dtype=np.float32)          # amax 16: id = 127/16
    x[32:64] = 0.0                                          # zero block: d = 0, q = 0
    x[64:96] = np.float32(2.5) * np.sign(np.arange(32) - 15.5).astype(np.float32)   # +-amax -> +-127
    b = O.q8_quantize_x86(x).reshape(3, 34)
    q = b[:, 2:].view(np.int8)
    d = b[:, 0:2].copy().view(np.float16)[:, 0]
    assert d[0] == np.float16(16 / 127) and d[1] == 0 and d[2] == np.float16(2.5 / 127)
    id0 = np.float32(127) / np.float32(16)
    assert np.array_equal(q[0], np.rint(np.arange(-16, 16, dtype=np.float32) * id0).astype(np.int8))
    assert np.all(q[1] == 0) and np.array_equal(np.abs(q[2]), np.full(32, 127, np.int8))
    # round half to even: 0.5*(2k+1) ties at id = 1
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:6] = [0.5, 1.5, 2.5, -0.5, -2.5]
    q = O.q8_quantize_x86(t)[2:].view(np.int8)
    assert list(q[1:6]) == [0, 2, 2, 0, -2]
    # the weight quantiser rounds half away from zero (roundf)
    q = O.q8_quantize_ref(t)[2:].view(np.int8)
    assert list(q[1:6]) == [1, 2, 3, -1, -3]


def test_q8_dot_exact_and_fp64():
    rng = np.random.default_rng(2)
    for k in (512, 2048):
        W = rng.standard_normal((20, k)).astype(np.float32) * 0.02
        X = rng.standard_normal((3, k)).astype(np.float32)
        wb = O.q8_quantize_ref(W).reshape(20, -1)
        xb = O.q8_quantize_x86(X).reshape(3, -1)
        wf = O.q8_dequant(wb).reshape(20, k).astype(np.float64)
        xf = O.q8_dequant(xb).reshape(3, k).astype(np.float64)
        for n in range(20):
            for m in range(3):
                a = O.lib().orc_q8_dot(wb[n].copy(), xb[m].copy(), k // 32)
                s = O.lib().orc_q8_dot_scalar(wb[n].copy(), xb[m].copy(), k // 32)
                assert np.float32(a).view(np.uint32) == np.float32(s).view(np.uint32)
                exact = float(wf[n] @ xf[m])
                assert abs(a - exact) <= 1e-5 * np.abs(wf[n] * xf[m]).sum()
        Y = O.q8_matmul(wb.ravel(), 20, k, X)
        assert np.allclose(Y, xf @ wf.T, rtol=0, atol=1e-4)


def test_fp_dots_against_fp64():
    rng = np.random.default_rng(3)
    W = rng.standard_normal((40, 1025)).astype(np.float32)
    X = rng.standard_normal((2, 1025)).astype(np.float32)
    ref = X.astype(np.float64) @ W.astype(np.float64).T
    for mode in (0, 1):
        Y = O.f32_matmul(W, X, mode)
        assert np.allclose(Y, ref, rtol=0, atol=1e-3)
    W16 = W[:, :512].astype(np.float16)
    X16 = X[:, :512].astype(np.float16).astype(np.float64)
    ref16 = X16 @ W16.astype(np.float64).T
    for mode in (0, 1):
        assert np.allclose(O.f16_matmul(W16.view(np.uint16), X[:, :512], mode), ref16, rtol=0, atol=1e-3)


# ------------------------------------------------------------------------------- LayerNorm / act

def test_layernorm_closed_forms():
    n = 512
    wb = np.concatenate([np.full(n, 1.7), np.linspace(-1, 1, n)]).astype(np.float32)
    y = O.layernorm(np.full((1, n), 3.25, np.float32), None, None, wb)
    assert np.array_equal(y[0], wb[n:])                    # constant row -> b exactly
    x = np.arange(1, n + 1, dtype=np.float32)[None, :]
    y = O.layernorm(x, None, None, np.concatenate([np.ones(n), np.zeros(n)]).astype(np.float32))
    mean, var = (n + 1) / 2, (n * n - 1) / 12
    assert np.allclose(y[0], (np.arange(1, n + 1) - mean) / np.sqrt(var + 1e-5), rtol=0, atol=2e-6)
    rng = np.random.default_rng(4)
    x, r = rng.standard_normal((5, n)).astype(np.float32), rng.standard_normal((5, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    wb = np.concatenate([rng.standard_normal(n), rng.standard_normal(n)]).astype(np.float32)
    v = x.astype(np.float64) + r + bias
    ref = (v - v.mean(1, keepdims=True)) / np.sqrt(v.var(1, keepdims=True) + 1e-5) * wb[:n] + wb[n:]
    assert np.allclose(O.layernorm(x, r, bias, wb), ref, rtol=0, atol=1e-5)


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_add_act_reference_fixture(act):
    """tests/test_add_act.cpp:66-101 (NE0 = 64, NR = 7, tolerance 2e-3, 5e-3 for GELU)."""
    NE0, NR = 64, 7
    i = np.arange(NE0 * NR)
    a = (0.02 * ((i * 37 % 101) - 50) + 0.5).astype(np.float32)
    b = (0.01 * ((np.arange(NE0) * 13) % 29 - 14)).astype(np.float32)
    v = (a.reshape(NR, NE0) + b).ravel().astype(np.float64)
    ref = {0: v, 1: np.maximum(v, 0), 2: 0.5 * v * (1 + np.vectorize(math.erf)(v / math.sqrt(2))),
           3: v * np.tanh(np.log1p(np.exp(v)))}[act]
    assert np.abs(O.add_act(a, b, act) - ref).max() <= (5e-3 if act == 2 else 2e-3)


def test_pe_table_closed_form():
    D, npos = 512, 4096
    pe = O.pe_table(D, npos)
    i = np.arange(0, D, 2).astype(np.float64)
    div = np.exp(-i * math.log(10000.0) / D)                  # fp64 closed form
    for pos in (0, 1, 17, 1000, 4095):
        arg = pos * div
        # the reference rounds div and pos*div to float: |d arg| <= 3 ulp(arg)
        tol = 3.0 * arg * 2.0 ** -23 + 3e-7
        assert np.all(np.abs(pe[pos, 0::2] - np.sin(arg)) <= tol)
        assert np.all(np.abs(pe[pos, 1::2] - np.cos(arg)) <= tol)
    assert np.array_equal(pe[0, 0::2], np.zeros(D // 2, np.float32))
    assert np.array_equal(pe[0, 1::2], np.ones(D // 2, np.float32))


# ------------------------------------------------------------------------------- attention

def _attn64(q, k, v, skip, scale):
    s = (k.astype(np.float64) @ q.astype(np.float64)) * scale
    s[skip] = -np.inf
    if np.all(skip):
        return np.zeros(q.shape[0])
    p = np.exp(s - s.max())
    return (p[:, None] * v).sum(0) / p.sum()


def test_attention_row_bruteforce_and_invariants():
    rng = np.random.default_rng(5)
    scale = np.float32(1.0) / np.sqrt(np.float32(32))
    lib = O.lib()
    for L in (1, 2, 7, 64, 300):
        q = rng.standard_normal(32).astype(np.float32)
        k = rng.standard_normal((L, 32)).astype(np.float32)
        v = rng.standard_normal((L, 32)).astype(np.float32)
        skip = (rng.random(L) < 0.3).astype(np.uint8)
        skip[0] = 0
        out = np.zeros(32, np.float32)
        lib.orc_attn_row(q, k, v, 32, 32, L, skip.ctypes.data, scale, out)
        assert np.allclose(out, _attn64(q, k, v, skip.astype(bool), float(scale)), rtol=0, atol=1e-5)
        # masked keys do not matter; a single valid key returns its V row; constant V returns V
        k2, v2 = k.copy(), v.copy()
        k2[skip.astype(bool)] = 1e3
        v2[skip.astype(bool)] = -7.0
        out2 = np.zeros(32, np.float32)
        lib.orc_attn_row(q, k2, v2, 32, 32, L, skip.ctypes.data, scale, out2)
        assert np.array_equal(out, out2)
    one = np.ones(3, np.uint8)
    one[1] = 0
    out = np.zeros(32, np.float32)
    lib.orc_attn_row(q, k[:3].copy(), v[:3].copy(), 32, 32, 3, one.ctypes.data, scale, out)
    assert np.array_equal(out, v[1])


def test_attention_prefill_masks_by_perturbation():
    """Prefill attention: every output row is the fp64 softmax over some key set; which set is
    fixed by perturbing K/V rows and seeing which outputs move (a text query never sees a
    semantic key or a left-pad key; a semantic query sees itself and nothing after it)."""
    rng = np.random.default_rng(9)
    B, S, max_len, nh, hd = 2, 40, 15, 2, 32
    D = nh * hd
    pad = np.array([0, 6], np.int32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    qkv = rng.standard_normal((B, S, 3 * D)).astype(np.float32)
    out = O.attn_prefill(qkv, max_len, pad, nh, scale, nthreads=2)
    # each row equals the fp64 softmax over the key set the perturbations below establish
    for b in range(B):
        for s in range(S):
            keys = np.arange(pad[b], max_len if s < max_len else s + 1)
            for h in range(nh):
                q = qkv[b, s, h * hd:(h + 1) * hd]
                k = qkv[b, keys, D + h * hd:D + (h + 1) * hd]
                v = qkv[b, keys, 2 * D + h * hd:2 * D + (h + 1) * hd]
                ref = _attn64(q, k, v, np.zeros(len(keys), bool), scale)
                assert np.allclose(out[b, s, h * hd:(h + 1) * hd], ref, rtol=0, atol=2e-6)
    for b in range(B):
        for j in range(S):
            p = qkv.copy()
            p[b, j, D:] = rng.standard_normal(2 * D) * 5
            o2 = O.attn_prefill(p, max_len, pad, nh, scale, nthreads=2)
            moved = np.any(o2[b] != out[b], axis=1)
            assert np.array_equal(o2[1 - b], out[1 - b])
            if j < pad[b]:
                expect = np.zeros(S, bool)                           # left pad: seen by nobody
            elif j < max_len:
                expect = np.ones(S, bool)                            # text key: seen by all
            else:
                expect = np.arange(S) >= j                           # semantic key: itself and later
            assert np.array_equal(moved, expect), (b, j)


# ------------------------------------------------------------------------------- model semantics

def test_gguf_contract_read(tiny_path):
    m = O.Model(tiny_path)
    assert (m.D, m.NH, m.HD, m.NL, m.V, m.EOS, m.PH, m.FFN, m.head_type) == (64, 2, 32, 2, 129, 128, 40, 128, 1)


def test_left_padding_changes_nothing(tiny_path):
    m = O.Model(tiny_path)
    reqs = sm.synth_requests(1, 3, 6, [2, 9, 5], phone_vocab=40, code_vocab=129)
    batch = m.first_logits(reqs, nthreads=2)
    for b in range(3):
        assert np.array_equal(batch[b], m.first_logits([reqs[b]], nthreads=2)[0])


def test_text_queries_do_not_see_semantic_keys(tiny_path):
    """Layer-1 K at text positions depends only on text (x queries are masked off the y keys);
    at a prompt position it depends only on earlier positions (y queries are causal)."""
    m = O.Model(tiny_path)
    reqs = sm.synth_requests(2, 1, 8, [6], phone_vocab=40, code_vocab=129)
    k1, _, _ = m.prefill_kv(reqs, 1, nthreads=2)
    r2 = [dict(reqs[0])]
    r2[0]["prompt"] = reqs[0]["prompt"].copy()
    r2[0]["prompt"][5] = (r2[0]["prompt"][5] + 1) % 129
    k2, _, _ = m.prefill_kv(r2, 1, nthreads=2)
    T = 6
    assert np.array_equal(k1[:, :, :T + 5], k2[:, :, :T + 5])      # text + prompt before the change
    assert not np.array_equal(k1[:, :, T + 5:], k2[:, :, T + 5:])   # the change and after


def test_generate_loop_rules(tiny_path):
    """Hand-derived traces of src/gsv_ar.cpp:762-815 under teacher forcing."""
    m = O.Model(tiny_path)
    reqs = sm.synth_requests(3, 3, 4, [3, 5, 2], phone_vocab=40, code_vocab=129)
    P = 4
    forced = np.array([7, 8, 9, 10, 11, 128, 12, 13, 14, 15, 16, 17, 18, 128, 19], np.int32)
    # EOS forced at step 5 (the EOS mask before step 11 applies to sampling, not to oracle tokens)
    r = m.generate(reqs, max_steps=15, oracle=forced, seeds=[1, 2, 3], nthreads=2)
    assert r["n_steps"] == 6 and list(r["lens"]) == [5, 5, 5] and list(r["finish_seq"]) == [0, 1, 2]
    for b in range(3):
        assert list(r["tokens"][b]) == list(reqs[b]["prompt"]) + [7, 8, 9, 10, 11]
    # early stop: more than 2 generated tokens in sequence 0 stops everyone at step 2
    r = m.generate(reqs, max_steps=15, oracle=forced, early_stop=2, nthreads=2)
    assert r["n_steps"] == 3 and list(r["lens"]) == [2, 2, 2]
    assert all(list(t) == list(reqs[b]["prompt"]) + [7, 8] for b, t in enumerate(r["tokens"]))
    # max_steps without EOS: full histories, lens = max_steps
    r = m.generate(reqs, max_steps=4, oracle=forced, nthreads=2)
    assert r["n_steps"] == 4 and list(r["lens"]) == [4, 4, 4]
    assert all(len(t) == P + 4 for t in r["tokens"])
    # sampled EOS is impossible before step 11 without the oracle
    r = m.generate(reqs, max_steps=11, sampler=(0, 1.0, 1.0, 1.0), seeds=[5, 6, 7], nthreads=2)
    assert all(128 not in list(t[P:]) for t in r["tokens"])


def test_rng_exponential_n_is_the_same_stream():
    """The bulk draw helper the workload tests use equals the golden-pinned one-draw function."""
    for seed in (0, 1, 7, 2 ** 63 + 5):
        a, _ = O.rng_exponential(seed, 2100)
        assert np.array_equal(O.rng_exponential_n(seed, 2100).view(np.uint32), a.view(np.uint32))

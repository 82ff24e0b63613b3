"""CPU known-answer tests of the oracle's layer composition (src/gsv_ar.cpp:186-293, :296-358,
:719-824; src/gsv_bert.cpp:141-155).

The component pins (tests/test_oracle_pins.py) fix each op; these fix how the ops are chained:
which terms enter each LayerNorm, where the BERT projection and its bias apply, the PE position
and alpha of every row (prefill and decode), the attention masks, the cache column of each decode
step and the head over the last row. Each test runs the oracle on a model whose projections are
zero or exact identities (tests/known_models.py) and compares with a float64 closed form under a
bound derived from the Q8_0 activation quantisation; each also checks that the plausible wrong
compositions (a dropped bias, a PE position off by one, a swapped alpha, a wrong mask) miss that
bound by a wide margin, so the test has the power to catch them.
"""
import numpy as np
import pytest

import bert_oracle as BO
import known_models as KM
import oracle as O
import synth_model as sm

N_THREADS = 4


@pytest.fixture(scope="module")
def zero2(tmp_path_factory):
    """2 layers, every projection zero."""
    d = tmp_path_factory.mktemp("km")
    return KM.write(str(d / "zero2.gguf"), 11, [{}, {}])


@pytest.fixture(scope="module")
def idqkv(tmp_path_factory):
    """1 layer: Wqkv = [I; I; I] (q = k = v = the quantised input + bias), the rest zero."""
    d = tmp_path_factory.mktemp("km")
    return KM.write(str(d / "idqkv.gguf"), 12, [{"qkv": "id"}])


@pytest.fixture(scope="module")
def attnout(tmp_path_factory):
    """2 layers: layer 0 Wq = Wk = 0, Wv = I, Wo = I (attention = mean of the visible V rows);
    layer 1 Wqkv = [I; I; I] (its K cache shows layer 0's output of every row)."""
    d = tmp_path_factory.mktemp("km")
    vcols = np.concatenate([np.full(2 * KM.D, -1), np.arange(KM.D)])
    return KM.write(str(d / "attnout.gguf"), 13, [{"qkv": vcols, "out": "id"}, {"qkv": "id"}])


def _reqs(seed, lens, P, bert=(True,)):
    reqs = sm.synth_requests(seed, len(lens), P, lens)
    for i, r in enumerate(reqs):
        if not bert[i % len(bert)]:
            r["bert"] = None
    return reqs


def _excess(got, ref, bound):
    """max of |got - ref| / bound (<= 1 means within the bound)."""
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref) / bound))


# ---------------------------------------------------------------------------- prefill logits

def test_first_logits_zero_projections(zero2):
    """n1 = LN1(x + b_o), x' = LN2(n1 + b_2) per layer, then the head over the LAST row, whose
    input is the last prompt code at PE position P-1 with audio_alpha."""
    path, p, perm, scale = zero2
    m = O.Model(path)
    pe = KM.pe(64)
    reqs = _reqs(21, [5, 9, 1], 7)
    got = m.first_logits(reqs, nthreads=N_THREADS)
    P = 7
    x = KM.decode_input64(p, reqs[0]["prompt"][P - 1], P - 1, pe)
    ref = KM.head64(KM.zero_layers64(p, x, 2), perm, scale)
    bound = 2.0 ** -10 * np.abs(ref) + 1e-6
    for b in range(3):
        assert _excess(got[b], ref, bound) <= 1.0
    # the wrong compositions miss the bound by far
    wrong = {
        "b_o not in LN1": lambda p2: p2.__setitem__("transformer.block0.out_b", 0 * p["transformer.block0.out_b"]),
        "b_2 not in LN2": lambda p2: p2.__setitem__("transformer.block1.ffn2_b", 0 * p["transformer.block1.ffn2_b"]),
        "LN1 and LN2 swapped": lambda p2: (p2.__setitem__("transformer.block0.norm1_w", p["transformer.block0.norm2_w"]),
                                           p2.__setitem__("transformer.block0.norm2_w", p["transformer.block0.norm1_w"])),
    }
    for what, edit in wrong.items():
        p2 = dict(p)
        edit(p2)
        alt = KM.head64(KM.zero_layers64(p2, x, 2), perm, scale)
        assert _excess(got[0], alt, bound) > 100, what
    for what, alt_x in {"PE position P": KM.decode_input64(p, reqs[0]["prompt"][P - 1], P, pe),
                        "text alpha": p["ar.audio_emb"][reqs[0]["prompt"][P - 1]] + KM.TEXT_ALPHA * pe[P - 1],
                        "first prompt row": KM.decode_input64(p, reqs[0]["prompt"][0], 0, pe)}.items():
        alt = KM.head64(KM.zero_layers64(p, alt_x, 2), perm, scale)
        assert _excess(got[0], alt, bound) > 100, what
    # one layer only (the second layer's LN pair dropped)
    alt = KM.head64(KM.zero_layers64(p, x, 1), perm, scale)
    assert _excess(got[0], alt, bound) > 100


# ---------------------------------------------------------------------------- decode logits

def test_decode_logits_zero_projections(zero2):
    """The logits entering loop step idx + 1 come from the token of step idx embedded at PE
    position prompt_len + idx with audio_alpha (src/gsv_ar.cpp:798-807)."""
    path, p, perm, scale = zero2
    m = O.Model(path)
    pe = KM.pe(64)
    P = 6
    reqs = _reqs(22, [4, 7], P)
    forced = np.array([17, 900, 3, 1000, 250, 64], np.int32)
    r = m.generate(reqs, sampler=(1, 1.0, 1.0, 1.0), max_steps=len(forced), oracle=forced, seeds=[1, 2],
                   flags=O.ORC_EOS_MASK_ALL, nthreads=N_THREADS, want_logits=True)
    lg = r["logits"]
    assert lg.shape[0] == len(forced)
    for idx in range(len(forced) - 1):
        x = KM.decode_input64(p, forced[idx], P + idx, pe)
        ref = KM.head64(KM.zero_layers64(p, x, 2), perm, scale)
        bound = 2.0 ** -10 * np.abs(ref) + 1e-6
        for b in range(2):
            assert _excess(lg[idx + 1, b], ref, bound) <= 1.0, idx
        for what, alt_x in {"PE position + 1": KM.decode_input64(p, forced[idx], P + idx + 1, pe),
                            "PE position - 1": KM.decode_input64(p, forced[idx], P + idx - 1, pe),
                            "PE position idx": KM.decode_input64(p, forced[idx], idx, pe),
                            "text alpha": p["ar.audio_emb"][forced[idx]] + KM.TEXT_ALPHA * pe[P + idx]}.items():
            alt = KM.head64(KM.zero_layers64(p, alt_x, 2), perm, scale)
            assert _excess(lg[idx + 1, 0], alt, bound) > 100, (what, idx)


# ---------------------------------------------------------------------------- the layer input

def _kv_bound(x, bias):
    """|K - (x + bias)| for K = dequant(quant_x86(x)) + bias in fp32."""
    return KM.block_amax(x) * KM.Q8_ERR * 1.001 + 2e-7 * (np.abs(x) + np.abs(bias)) + 1e-7


def _heads(a):
    """[B][NH][S][HD] -> [B][S][D] (head h holds dims 32h .. 32h + 31)."""
    B, nh, S, hd = a.shape
    return a.transpose(0, 2, 1, 3).reshape(B, S, nh * hd)


def test_prefill_inputs_and_kv_cache(idqkv):
    """The layer-0 K and V of every prefill row equal the row's input x plus the bias: text rows
    with the BERT projection and its bias (or the bias alone without features), prompt rows
    without either, left-pad rows zero; text PE positions start at 0 after the pad, prompt PE
    positions at 0 after max_len."""
    path, p, perm, scale = idqkv
    m = O.Model(path)
    pe = KM.pe(64)
    reqs = _reqs(23, [6, 13, 1, 9], 5, bert=(True, True, False, True))
    k, v, _ = m.prefill_kv(reqs, 0, nthreads=N_THREADS)
    x, S, max_len = KM.inputs64(p, reqs, pe)
    bk = p["transformer.block0.qkv_b"][KM.D:2 * KM.D].astype(np.float64)
    bv = p["transformer.block0.qkv_b"][2 * KM.D:].astype(np.float64)
    K, Vv = _heads(k), _heads(v)
    assert _excess(K, x + bk, _kv_bound(x, bk)) <= 1.0
    assert _excess(Vv, x + bv, _kv_bound(x, bv)) <= 1.0
    # the wrong inputs miss the bound
    Wb, bb = p["ar.bert_proj"].astype(np.float64), p["ar.bert_proj_b"].astype(np.float64)
    b = 0                                      # 6 phones after 7 pad rows
    T = len(reqs[b]["phones"])
    pad = max_len - T
    assert pad > 0
    t = 3
    row = K[b, pad + t]
    good = x[b, pad + t] + bk
    bnd = _kv_bound(x[b, pad + t], bk)
    te = p["ar.text_emb"][reqs[b]["phones"][t]]
    alts = {
        "no BERT projection": good - Wb @ reqs[b]["bert"][:, t],
        "no BERT bias": good - bb,
        "PE position pad + t": te + KM.TEXT_ALPHA * pe[pad + t] + Wb @ reqs[b]["bert"][:, t] + bb + bk,
        "audio alpha on text": te + KM.AUDIO_ALPHA * pe[t] + Wb @ reqs[b]["bert"][:, t] + bb + bk,
    }
    for what, alt in alts.items():
        assert _excess(row, alt, bnd) > 50, what
    prow = K[b, max_len + 2]
    pgood = x[b, max_len + 2] + bk
    pb = _kv_bound(x[b, max_len + 2], bk)
    for what, alt in {"BERT bias on a prompt row": pgood + bb,
                      "prompt PE after the text": pgood + KM.AUDIO_ALPHA * (pe[max_len + 2] - pe[2]),
                      "text alpha on prompt": pgood + (KM.TEXT_ALPHA - KM.AUDIO_ALPHA) * pe[2]}.items():
        assert _excess(prow, alt, pb) > 50, what
    # pad rows: the bias alone (x = 0)
    assert np.all(K[2, :max_len - 1] == bk.astype(np.float32))


def test_decode_kv_append_column_and_position(idqkv):
    """Decode step idx writes K/V of its token, embedded at PE position P + idx, at cache column
    S + idx of every sequence; the prefill columns are left as they were."""
    path, p, perm, scale = idqkv
    m = O.Model(path)
    pe = KM.pe(64)
    P = 5
    reqs = _reqs(24, [3, 8], P)
    forced = np.array([40, 41, 1020, 7, 300, 12, 999], np.int32)
    n = len(forced)
    r = m.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=n, oracle=forced, seeds=[3, 4],
                   flags=O.ORC_EOS_MASK_ALL, nthreads=N_THREADS, kv_layer=0)
    k, v = r["kv"]
    kp, vp, _ = m.prefill_kv(reqs, 0, nthreads=N_THREADS)
    S = kp.shape[2]
    assert k.shape[2] == S + n
    assert np.array_equal(k[:, :, :S], kp) and np.array_equal(v[:, :, :S], vp)
    bk = p["transformer.block0.qkv_b"][KM.D:2 * KM.D].astype(np.float64)
    K = _heads(k)
    for idx in range(n):
        x = KM.decode_input64(p, forced[idx], P + idx, pe)
        for b in range(2):
            assert _excess(K[b, S + idx], x + bk, _kv_bound(x, bk)) <= 1.0, idx
        alt = KM.decode_input64(p, forced[idx], P + idx + 1, pe) + bk
        assert _excess(K[0, S + idx], alt, _kv_bound(x, bk)) > 50
    # the ORC_KV_F16 cache is the same values rounded to fp16 (the device's storage)
    r16 = m.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=n, oracle=forced, seeds=[3, 4],
                     flags=O.ORC_EOS_MASK_ALL | O.ORC_KV_F16, nthreads=N_THREADS, kv_layer=0)
    assert np.array_equal(r16["kv"][0], k.astype(np.float16).astype(np.float32))


# ---------------------------------------------------------------------------- attention + out

def _q8(x):
    """x after the x86 activation quantisation and dequantisation (the pinned oracle functions),
    row by row: what an identity Q8_0 projection passes on."""
    x32 = np.asarray(x, np.float32)
    return O.q8_dequant(O.q8_quantize_x86(x32)).reshape(x32.shape).astype(np.float64)


def _attn_layer64(p, x, S, max_len, pads, mask_kind="reference"):
    """Layer 0 of the attnout model: q and k are the constant biases, so attention is the plain
    mean of the visible V rows (v = quant(x) + b_v); o = quant(attention); then the two
    LayerNorms. float64, with the three activation quantisations of the path modelled by the
    pinned quantiser (x -> v, attention -> o, and the caller's layer-1 input)."""
    B = x.shape[0]
    b0 = "transformer.block0"
    bv = p[f"{b0}.qkv_b"][2 * KM.D:].astype(np.float64)
    v = _q8(x) + bv
    out = np.zeros_like(x)
    for b in range(B):
        for s in range(S):
            if mask_kind == "reference":
                keys = range(pads[b], max_len) if s < max_len else range(pads[b], s + 1)
            elif mask_kind == "text causal":
                keys = range(pads[b], s + 1) if s >= pads[b] else range(pads[b], max_len)
            elif mask_kind == "semantic sees all":
                keys = range(pads[b], max_len) if s < max_len else range(pads[b], S)
            elif mask_kind == "pads visible":
                keys = range(0, max_len) if s < max_len else range(0, s + 1)
            keys = list(keys)
            out[b, s] = v[b, keys].mean(axis=0) if keys else 0.0
    n1 = KM.ln64(x + _q8(out) + p[f"{b0}.out_b"], p[f"{b0}.norm1_w"], p[f"{b0}.norm1_b"])
    return KM.ln64(n1 + p[f"{b0}.ffn2_b"], p[f"{b0}.norm2_w"], p[f"{b0}.norm2_b"])


def test_prefill_attention_masks_and_out_projection(attnout):
    """Layer 0 output of every row (seen through layer 1's K cache): LN2(LN1(x + mean of the
    visible V rows + b_o) + b_2), text queries seeing [pad, max_len), semantic queries [pad, q].
    The closed form models the quantisations exactly, so it agrees with the oracle to fp32
    rounding except where that rounding moves a value across a quantisation boundary (one step,
    amax/127, of that element; a few elements in a thousand)."""
    path, p, perm, scale = attnout
    m = O.Model(path)
    pe = KM.pe(64)
    reqs = _reqs(25, [7, 12, 3], 6)
    k1, _, _ = m.prefill_kv(reqs, 1, nthreads=N_THREADS)
    x, S, max_len = KM.inputs64(p, reqs, pe)
    pads = [max_len - len(r["phones"]) for r in reqs]
    bk1 = p["transformer.block1.qkv_b"][KM.D:2 * KM.D].astype(np.float64)
    K1 = _heads(k1).astype(np.float64)

    def check(cur):
        ref = _q8(cur) + bk1
        d = np.abs(K1 - ref)
        close = d <= 1e-4 * (1.0 + np.abs(ref))
        step = KM.block_amax(cur) / 127.0 * 1.01 + 1e-4
        return float(close.mean()), bool(np.all(d <= step + 0.05 * np.abs(ref)))

    frac, bounded = check(_attn_layer64(p, x, S, max_len, pads))
    assert frac >= 0.99 and bounded, frac
    for kind in ("text causal", "semantic sees all", "pads visible"):
        frac_alt, _ = check(_attn_layer64(p, x, S, max_len, pads, kind))
        assert frac_alt < 0.9, (kind, frac_alt)
    p2 = dict(p)
    p2["transformer.block0.out_b"] = 0 * p["transformer.block0.out_b"]
    frac_alt, _ = check(_attn_layer64(p2, x, S, max_len, pads))
    assert frac_alt < 0.1, frac_alt


# ---------------------------------------------------------------------------- BERT encoder

def _bert_params(seed, n_layer, D=64, F=256, vocab=40, max_pos=16, ident=False):
    rng = np.random.default_rng(seed)
    W = {"bert.word_emb": rng.standard_normal((vocab, D)), "bert.pos_emb": rng.standard_normal((max_pos, D)),
         "bert.type_emb": rng.standard_normal((2, D)), "bert.emb_ln_w": rng.uniform(0.5, 1.5, D),
         "bert.emb_ln_b": rng.standard_normal(D) * 0.3}
    for li in range(n_layer):
        q = f"bert.l{li}."
        W[q + "qkv_w"] = np.zeros((3 * D, D))
        W[q + "attn_out_w"] = np.zeros((D, D))
        W[q + "ff1_w"] = np.zeros((F, D))
        W[q + "ff2_w"] = np.zeros((D, F))
        if ident:
            W[q + "qkv_w"][2 * D:, :] = np.eye(D)                 # v = x; q = k = 0
            W[q + "attn_out_w"] = np.eye(D)
            W[q + "ff1_w"][:D, :] = np.eye(D)
            W[q + "ff2_w"][:, :D] = np.eye(D)
        W[q + "qkv_b"] = rng.standard_normal(3 * D) * 0.5
        W[q + "attn_out_b"] = rng.standard_normal(D) * 0.5
        W[q + "ff1_b"] = rng.standard_normal(F) * 0.5
        W[q + "ff2_b"] = rng.standard_normal(D) * 0.5
        for n in ("attn_ln", "out_ln"):
            W[q + n + "_w"] = rng.uniform(0.5, 1.5, D)
            W[q + n + "_b"] = rng.standard_normal(D) * 0.3
    return W


def _bert_closed(W, ids, n_layers, ident, drop=None):
    import math
    ids = np.asarray(ids)
    T = len(ids)
    x = (W["bert.word_emb"][ids] + W["bert.pos_emb"][:T]) + W["bert.type_emb"][0]
    x = KM.ln64(x, W["bert.emb_ln_w"], W["bert.emb_ln_b"], 1e-12)
    gelu = np.vectorize(lambda t: 0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))))
    for li in range(n_layers):
        q = f"bert.l{li}."
        D = x.shape[1]
        bv = W[q + "qkv_b"][2 * D:]
        a = (x + bv).mean(axis=0, keepdims=True) if ident else bv[None, :]   # uniform attention
        o = a if ident else 0.0
        x = KM.ln64(x + o + (0 if drop == "b_o" else W[q + "attn_out_b"]), W[q + "attn_ln_w"], W[q + "attn_ln_b"], 1e-12)
        h = gelu((np.pad(x, ((0, 0), (0, W[q + "ff1_b"].size - D))) if ident else 0.0) + W[q + "ff1_b"])
        f = h[:, :D] if ident else 0.0
        x = KM.ln64(x + f + (0 if drop == "b_2" else W[q + "ff2_b"]), W[q + "out_ln_w"], W[q + "out_ln_b"], 1e-12)
    return x.T


@pytest.mark.parametrize("ident", [False, True])
@pytest.mark.parametrize("n_layers", [1, 2])
def test_bert_encoder_composition(ident, n_layers):
    """src/gsv_bert.cpp:147-155 with zero / identity projections: x = LN1(x + Wo.a + b_o),
    x = LN2(x + W2.gelu(W1.x + b1) + b2), a = softmax attention over the sequence's own tokens
    (uniform here: q = k = 0)."""
    W = _bert_params(31 + n_layers, n_layers, ident=ident)
    ids = [3, 17, 5, 39, 0, 11]
    got = BO.encode(W, ids, n_layers, 64, 4, 1e-12)
    ref = _bert_closed(W, ids, n_layers, ident)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-9)
    for drop in ("b_o", "b_2"):
        assert np.max(np.abs(got - _bert_closed(W, ids, n_layers, ident, drop))) > 1e-2


# ---------------------------------------------------------------------------- decode attention

def _dec_attn_model(tmp_path_factory, name, seed, k_ident):
    """1 layer: Wq = 0 (q = b_q), Wk = I (k = the quantised input + b_k) or 0 (k = b_k), Wv = I,
    Wo = I; FFN zero. The head reads LN2(LN1(x + quant(attention) + b_o) + b_2)."""
    d = tmp_path_factory.mktemp("km")
    kcols = np.arange(KM.D) if k_ident else np.full(KM.D, -1)
    cols = np.concatenate([np.full(KM.D, -1), kcols, np.arange(KM.D)])
    return KM.write(str(d / name), seed, [{"qkv": cols, "out": "id"}])


@pytest.fixture(scope="module")
def dec_mean(tmp_path_factory):
    """q and k constant: decode attention is the plain mean of the visible V rows."""
    return _dec_attn_model(tmp_path_factory, "dec_mean.gguf", 14, False)


@pytest.fixture(scope="module")
def dec_soft(tmp_path_factory):
    """k varies per key: the softmax weights exp(scale * b_q . k_j) depend on the scale."""
    return _dec_attn_model(tmp_path_factory, "dec_soft.gguf", 15, True)


def _dec_attn_logits64(p, perm, scale, x, K0, V0, b, keys, sc):
    """Logits of a decode row of sequence b whose layer input is x: per head h, softmax over the
    cache columns `keys` of sc * (b_q[h] . K0[b, h, j]), times V0[b, h, j]; o = quant(attention);
    x' = LN2(LN1(x + o + b_o) + b_2) (zero FFN); then the head. float64 from the layer-0 cache
    (whose values the K/V tests above pin)."""
    b0 = "transformer.block0"
    bq = p[f"{b0}.qkv_b"][:KM.D].astype(np.float32).astype(np.float64)
    keys = np.asarray(list(keys))
    a = np.zeros(KM.D)
    for h in range(KM.NH):
        sl = slice(h * KM.HD, (h + 1) * KM.HD)
        Kh = K0[b, h, keys].astype(np.float64)
        Vh = V0[b, h, keys].astype(np.float64)
        s = sc * (Kh @ bq[sl])
        w = np.exp(s - s.max())
        a[sl] = (w / w.sum()) @ Vh
    n1 = KM.ln64(x + _q8(a) + p[f"{b0}.out_b"], p[f"{b0}.norm1_w"], p[f"{b0}.norm1_b"])
    return KM.head64(KM.ln64(n1 + p[f"{b0}.ffn2_b"], p[f"{b0}.norm2_w"], p[f"{b0}.norm2_b"]), perm, scale)


def _close_frac(got, ref):
    """Fraction of logits within the fp16-head bound of the closed form. The closed form models the
    attention output's quantisation with the pinned quantiser; fp32 rounding moves a value across
    a quantisation boundary for a few elements in a thousand, so the bar is a fraction."""
    got = np.asarray(got, np.float64)
    return float(np.mean(np.abs(got - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-5))


@pytest.mark.parametrize("model", ["dec_mean", "dec_soft"])
def test_decode_attention_keys_scale_and_new_key(model, request):
    """Decode step idx of sequence b attends over cache columns [pad_b, S + idx]: the left-pad
    columns (whose V is the bias alone, x = 0) are hidden, the first valid column is seen, and the
    key just appended at column S + idx is included; scores are scaled by 1/sqrt(32)
    (src/gsv_ar.cpp:404-405 flash_attn_ext scale, :445-452 the decode mask)."""
    path, p, perm, scale = request.getfixturevalue(model)
    m = O.Model(path)
    pe = KM.pe(64)
    P = 5
    reqs = _reqs(26, [3, 8, 6], P, bert=(True, False, True))
    forced = np.array([40, 1001, 7, 300, 12, 999], np.int32)
    n = len(forced)
    flags = O.ORC_EOS_MASK_ALL | (O.ORC_KV_F16 if model == "dec_soft" else 0)
    r = m.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=n, oracle=forced, seeds=[3, 4, 5],
                   flags=flags, nthreads=N_THREADS, want_logits=True, kv_layer=0)
    lg = r["logits"]
    K0, V0 = r["kv"]
    max_len = max(len(q["phones"]) for q in reqs)
    S = max_len + P
    assert K0.shape[2] == S + n
    pads = [max_len - len(q["phones"]) for q in reqs]
    assert pads[0] > 0 and pads[1] == 0
    sc = 1.0 / np.sqrt(32.0)
    miss = {}
    for idx in range(n - 1):
        x = KM.decode_input64(p, forced[idx], P + idx, pe)
        col = S + idx
        for b in range(len(reqs)):
            got = lg[idx + 1, b]
            ref = _dec_attn_logits64(p, perm, scale, x, K0, V0, b, range(pads[b], col + 1), sc)
            assert _close_frac(got, ref) >= 0.99, (model, idx, b)
            alts = {"pad columns visible": (range(0, col + 1), sc),
                    "first valid column dropped": (range(pads[b] + 1, col + 1), sc),
                    "new key excluded": (range(pads[b], col), sc),
                    "keys up to the prefill only": (range(pads[b], S), sc)}
            if model == "dec_soft":
                alts["scale 1"] = (range(pads[b], col + 1), 1.0)
                alts["scale 1/32"] = (range(pads[b], col + 1), 1.0 / 32.0)
            for what, (keys, s2) in alts.items():
                if list(keys) == list(range(pads[b], col + 1)) and s2 == sc:
                    continue                     # identical to the reference for this row (pad 0)
                alt = _dec_attn_logits64(p, perm, scale, x, K0, V0, b, keys, s2)
                miss.setdefault(what, []).append(_close_frac(got, alt))
    expect = {"pad columns visible", "first valid column dropped", "new key excluded",
              "keys up to the prefill only"} | ({"scale 1", "scale 1/32"} if model == "dec_soft" else set())
    assert set(miss) == expect
    for what, fr in miss.items():
        assert max(fr) < 0.5, (model, what, max(fr))


# ---------------------------------------------------------------------------- FFN activation

def _ffn_exact_edit(seed):
    """Layer 0 with LN1 weight 0, so n1 = LN1(.) = norm1_b exactly, and norm1_b, b_1 multiples of
    1/16 whose every 32-block (of n1, and of the hidden row h = relu(n1[r % 512] + b_1[r])) has
    amax exactly 127/16: the x86 quantiser then maps each of those rows to itself (127/amax = 16,
    d = 2^-4), the identity FFN1 and FFN2 are exact, and the pre-activations take both signs."""
    def edit(p):
        rng = np.random.default_rng(seed)
        b = "transformer.block0"
        n1 = rng.integers(-40, 41, KM.D).astype(np.float64)
        pos = rng.integers(0, 32, KM.D // 32)
        n1[np.arange(KM.D // 32) * 32 + pos] = 127.0
        m = rng.integers(-20, 21, KM.FFN).astype(np.float64)
        r = np.arange(KM.FFN)
        m[(r % 32) == pos[(r % KM.D) // 32]] = 0.0
        p[f"{b}.norm1_w"] = np.zeros(KM.D, np.float32)
        p[f"{b}.norm1_b"] = (n1 / 16.0).astype(np.float32)
        p[f"{b}.ffn1_b"] = (m / 16.0).astype(np.float32)
    return edit


@pytest.fixture(scope="module")
def ffn_exact(tmp_path_factory):
    """1 layer: attention and out projection zero, FFN1 = FFN2 = identity (exact, see the edit)."""
    d = tmp_path_factory.mktemp("km")
    return KM.write(str(d / "ffn_exact.gguf"), 16, [{"ffn1": "id", "ffn2": "id"}], edit=_ffn_exact_edit(17))


def _ffn_logits64(p, perm, scale, act="relu", drop=None):
    import math
    b = "transformer.block0"
    n1 = p[f"{b}.norm1_b"].astype(np.float64)
    pre = n1 + (0.0 if drop == "b_1" else p[f"{b}.ffn1_b"][:KM.D].astype(np.float64))
    if act == "relu":
        f = np.maximum(pre, 0.0)
    elif act == "gelu":
        f = np.array([0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))) for t in pre])
    else:
        f = pre
    res = 0.0 if drop == "n1 residual" else n1
    x = KM.ln64(res + f + p[f"{b}.ffn2_b"], p[f"{b}.norm2_w"], p[f"{b}.norm2_b"])
    return KM.head64(x, perm, scale)


def test_ffn_relu_between_the_projections(ffn_exact):
    """x' = LN2(n1 + W2 . relu(W1 . n1 + b_1) + b_2): the FFN activation is ReLU (ggml ADD_ACT,
    PATCH:1586-1620; src/gsv_ar.cpp:262, :408), with b_1 inside it and n1 as the residual. Checked
    on the prefill's last row and on every decode row (the layer output does not depend on the row
    here, since n1 = norm1_b)."""
    path, p, perm, scale = ffn_exact
    m = O.Model(path)
    reqs = _reqs(27, [4, 9], 6)
    ref = _ffn_logits64(p, perm, scale)
    bound = 2.0 ** -10 * np.abs(ref) + 1e-6
    got = m.first_logits(reqs, nthreads=N_THREADS)
    forced = np.array([5, 600, 1000], np.int32)
    r = m.generate(reqs, sampler=(1, 1.0, 1.0, 1.0), max_steps=len(forced), oracle=forced, seeds=[1, 2],
                   flags=O.ORC_EOS_MASK_ALL | O.ORC_KV_F16, nthreads=N_THREADS, want_logits=True)
    rows = [got[0], got[1]] + [r["logits"][i, b] for i in range(1, len(forced)) for b in range(2)]
    for row in rows:
        assert _excess(row, ref, bound) <= 1.0
    pre = p["transformer.block0.norm1_b"].astype(np.float64) + p["transformer.block0.ffn1_b"][:KM.D]
    assert (pre < -0.5).sum() > 100 and (pre > 0.5).sum() > 100     # both signs, away from 0
    for what, alt in {"GELU": _ffn_logits64(p, perm, scale, "gelu"),
                      "no activation": _ffn_logits64(p, perm, scale, "none"),
                      "b_1 dropped": _ffn_logits64(p, perm, scale, drop="b_1"),
                      "n1 residual dropped": _ffn_logits64(p, perm, scale, drop="n1 residual")}.items():
        assert _excess(rows[0], alt, bound) > 10, what


# ---------------------------------------------------------------------------- F16 / F32 projections

@pytest.fixture(scope="module", params=["f32", "f16"])
def ffn_float(request, tmp_path_factory):
    """1 layer of F16 or F32 projections (the exporter's attn= / ffn= options): attention and out
    projection zero, FFN1 = FFN2 = identity (1.0 and 0.0, exact in both types); F32 head."""
    d = tmp_path_factory.mktemp("kmf")
    t = request.param
    return t, KM.write(str(d / f"ffn_{t}.gguf"), 18, [{"ffn1": "id", "ffn2": "id"}], attn_type=t, ffn_type=t,
                       head_type="f32")


def _ffn_float_logits64(p, perm, scale, x, wtype, round16=True, act="relu"):
    """x' = LN2(n1 + W2 . relu(W1 . n1 + b_1) + b_2) with n1 = LN1(x + b_o) and identity W1, W2:
    F16 weights take their activations rounded to fp16 (n1 into FFN1, h into FFN2)."""
    b = "transformer.block0"
    n1 = KM.ln64(x + p[f"{b}.out_b"], p[f"{b}.norm1_w"], p[f"{b}.norm1_b"])
    r16 = (lambda a: np.asarray(a).astype(np.float32).astype(np.float16).astype(np.float64)) \
        if (wtype == "f16" and round16) else (lambda a: np.asarray(a).astype(np.float32).astype(np.float64))
    pre = r16(n1) + p[f"{b}.ffn1_b"][:KM.D].astype(np.float64)
    h = np.maximum(pre.astype(np.float32).astype(np.float64), 0.0) if act == "relu" else pre
    xo = KM.ln64(n1 + r16(h) + p[f"{b}.ffn2_b"], p[f"{b}.norm2_w"], p[f"{b}.norm2_b"])
    return KM.head64_f32(xo, perm, scale)


def test_f16_f32_projections(ffn_float):
    """Projections stored F16 or F32 (src/gsv_ar.cpp:244, :392 multiply them through ggml_mul_mat;
    the engine's fallback F16 model, src/gsv_engine.cpp:216): F32 weights take the fp32
    activations, F16 weights the activations rounded to fp16 (ggml's vec_dot_type), with no Q8_0
    quantisation; checked through identity FFN matrices on the prefill's last row (tinyBLAS order)
    and the decode rows (vec_dot order), where both orders are exact."""
    wtype, (path, p, perm, scale) = ffn_float
    m = O.Model(path)
    pe = KM.pe(64)
    P = 6
    reqs = _reqs(28, [4, 9], P)
    forced = np.array([5, 600, 1000, 77], np.int32)
    got0 = m.first_logits(reqs, nthreads=N_THREADS)
    r = m.generate(reqs, sampler=(1, 1.0, 1.0, 1.0), max_steps=len(forced), oracle=forced, seeds=[1, 2],
                   flags=O.ORC_EOS_MASK_ALL, nthreads=N_THREADS, want_logits=True)
    rows = [(got0[b], KM.decode_input64(p, reqs[b]["prompt"][P - 1], P - 1, pe)) for b in range(2)]
    rows += [(r["logits"][i + 1, b], KM.decode_input64(p, forced[i], P + i, pe))
             for i in range(len(forced) - 1) for b in range(2)]
    for got, x in rows:
        ref = _ffn_float_logits64(p, perm, scale, x, wtype)
        close = np.abs(np.asarray(got, np.float64) - ref) <= 2e-6 * np.abs(ref) + 1e-6
        assert close.mean() >= 0.99, (wtype, close.mean())
        # the wrong compositions: Q8_0-style or no rounding of the activations, no activation
        for what, alt in {"no fp16 rounding": _ffn_float_logits64(p, perm, scale, x, wtype, round16=False),
                          "no activation": _ffn_float_logits64(p, perm, scale, x, wtype, act="none"),
                          "Q8_0 activations": KM.head64_f32(KM.ln64(
                              KM.ln64(x + p["transformer.block0.out_b"], p["transformer.block0.norm1_w"],
                                      p["transformer.block0.norm1_b"]) * 0 + 0, np.ones(KM.D), np.zeros(KM.D)),
                              perm, scale)}.items():
            if what == "no fp16 rounding" and wtype == "f32":
                continue
            if what == "Q8_0 activations":
                b0 = "transformer.block0"
                n1 = KM.ln64(x + p[f"{b0}.out_b"], p[f"{b0}.norm1_w"], p[f"{b0}.norm1_b"])
                h = np.maximum(_q8(n1) + p[f"{b0}.ffn1_b"][:KM.D], 0.0)
                alt = KM.head64_f32(KM.ln64(n1 + _q8(h) + p[f"{b0}.ffn2_b"], p[f"{b0}.norm2_w"],
                                            p[f"{b0}.norm2_b"]), perm, scale)
            frac = np.mean(np.abs(np.asarray(got, np.float64) - alt) <= 2e-6 * np.abs(alt) + 1e-6)
            assert frac < 0.9, (wtype, what, frac)   # the bar above is 0.99

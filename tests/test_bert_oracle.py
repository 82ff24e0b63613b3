"""CPU pins of the BERT oracle (oracle/bert_oracle.py) and host checks of the BERT C ABI.

The oracle restates src/gsv_bert.cpp:128-155; each function is checked here against what the
mathematics fixes, so that a dropped term, a wrong sign or a transposed operand fails."""
import math

import numpy as np
import pytest

import bert_oracle as BO
import gsvk
import synth_model as sm


def test_layernorm_closed_forms():
    # constant row -> b exactly; [1..n] -> analytic mean and variance
    n = 1024
    w = np.linspace(0.5, 1.5, n)
    b = np.linspace(-0.1, 0.1, n)
    np.testing.assert_array_equal(BO.layernorm(np.full((1, n), 3.25), w, b, 1e-12), b[None, :])
    v = np.arange(1, n + 1, dtype=np.float64)[None, :]
    mean, var = (n + 1) / 2.0, (n * n - 1) / 12.0
    np.testing.assert_allclose(BO.layernorm(v, w, b, 1e-12), (v - mean) / math.sqrt(var) * w + b, rtol=1e-12)


def test_gelu_erf_known_values():
    assert BO.gelu_erf(np.array([0.0]))[0] == 0.0
    x = np.array([-3.0, -1.0, -0.5, 0.5, 1.0, 2.0, 6.0])
    ref = [0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))) for t in x]
    np.testing.assert_allclose(BO.gelu_erf(x), ref, rtol=1e-14)
    # gelu(x) - gelu(-x) = x; gelu(1) = Phi(1)
    np.testing.assert_allclose(BO.gelu_erf(x) - BO.gelu_erf(-x), x, rtol=1e-13)
    assert abs(BO.gelu_erf(np.array([1.0]))[0] - 0.8413447460685429) < 1e-15


def test_attention_bruteforce_and_invariants():
    rng = np.random.default_rng(3)
    T, hd = 7, 64
    q, k, v = rng.standard_normal((3, T, hd))
    s = 0.125
    out = BO.attention(q, k, v, s)
    for i in range(T):
        e = np.array([math.exp(s * float(q[i] @ k[j])) for j in range(T)])
        np.testing.assert_allclose(out[i], (e / e.sum()) @ v, rtol=1e-12)
    # one key: the output is that value row; constant V: V
    np.testing.assert_allclose(BO.attention(q[:1], k[:1], v[:1], s), v[:1], rtol=1e-15)
    cv = np.tile(v[:1], (T, 1))
    np.testing.assert_allclose(BO.attention(q, k, cv, s), cv, rtol=1e-13)


def test_encode_embedding_only(tmp_path):
    path, W = sm.write_bert_model(str(tmp_path / "b.gguf"), n_layer=1, layers_used=1, vocab=50, max_pos=16)
    ids = [1, 7, 3, 49]
    x = (W["bert.word_emb"][ids].astype(np.float64) + W["bert.pos_emb"][:4]) + W["bert.type_emb"][0]
    ref = BO.layernorm(x, W["bert.emb_ln_w"], W["bert.emb_ln_b"], 1e-12).T
    np.testing.assert_allclose(BO.encode(W, ids, 0, 1024, 16, 1e-12), ref, rtol=1e-13)


def test_synthetic_writer_dequantises_like_the_loader(tmp_path):
    _, W16 = sm.write_bert_model(str(tmp_path / "h.gguf"), n_layer=1, layers_used=1, vocab=40, max_pos=8,
                                 wtype="f16")
    _, W8 = sm.write_bert_model(str(tmp_path / "q.gguf"), n_layer=1, layers_used=1, vocab=40, max_pos=8,
                                wtype="q8_0")
    _, W32 = sm.write_bert_model(str(tmp_path / "f.gguf"), n_layer=1, layers_used=1, vocab=40, max_pos=8)
    a = W32["bert.l0.ff1_w"]
    np.testing.assert_array_equal(W16["bert.l0.ff1_w"], a.astype(np.float16).astype(np.float32))
    assert np.max(np.abs(W8["bert.l0.ff1_w"] - a)) <= np.max(np.abs(a)) / 127.0
    np.testing.assert_array_equal(W8["bert.l0.ff1_b"], W32["bert.l0.ff1_b"])   # biases stay F32


def test_bert_load_rejects_bad_files(tmp_path):
    p = tmp_path / "not.gguf"
    p.write_bytes(b"GGUF\x03\x00\x00\x00")
    with pytest.raises(gsvk.GsvkError):
        gsvk.Bert(str(p))
    with pytest.raises(gsvk.GsvkError):
        gsvk.Bert(str(tmp_path / "missing.gguf"))


def test_encode_f16_activations_round_each_projection_input(tmp_path):
    """act_f16 rounds the inputs of the four projections to fp16 and nothing else: with weights
    and activations exactly representable in fp16 the two modes agree, and in general they differ
    by about fp16 rounding."""
    path, W = sm.write_bert_model(str(tmp_path / "b.gguf"), n_layer=1, layers_used=1, vocab=30, max_pos=8,
                                  wtype="f16")
    ids = [3, 1, 4, 1, 5]
    a = BO.encode(W, ids, 1, 1024, 16, 1e-12)
    b = BO.encode(W, ids, 1, 1024, 16, 1e-12, act_f16=True)
    d = np.max(np.abs(a - b)) / np.max(np.abs(a))
    assert 1e-6 < d < 1e-2
    np.testing.assert_array_equal(BO.encode(W, ids, 0, 1024, 16, 1e-12, act_f16=True),
                                  BO.encode(W, ids, 0, 1024, 16, 1e-12))


def test_q8_quantiser_is_the_pinned_x86_one():
    """bert_oracle.q8_quantize_x86 (numpy) against the C oracle's orc_q8_quantize_x86, itself pinned
    by known-answer blocks (tests/test_oracle_pins.py): same quants and fp16 scales, ties
    included."""
    import oracle as O
    rng = np.random.default_rng(21)
    x = rng.standard_normal((7, 256)).astype(np.float32)
    x[0, :32] = 0.0                                     # all-zero block
    x[1, :32] = np.linspace(-1, 1, 32)                  # +-amax
    x[2, :32] = np.arange(32, dtype=np.float32) - 15.5  # halves: exact ties after the scale
    q, d = BO.q8_quantize_x86(x)
    blocks = O.q8_quantize_x86(x).reshape(7, 8, 34)
    np.testing.assert_array_equal(q, blocks[:, :, 2:].view(np.int8))
    np.testing.assert_array_equal(d, blocks[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float64))


def test_q8_matmul_is_exact_block_products():
    """q8_matmul against an independent evaluation: dequantised operands (d q, exact in float64)
    multiplied in float64 give the same sums of exact block products to within fp64 rounding,
    and against the plain float product to within the quantisation error."""
    rng = np.random.default_rng(22)
    n, k = 64, 128
    w = (rng.standard_normal((n, k)) * 0.03).astype(np.float32)
    blocks = sm.q8_quantize_ref(w)
    x = rng.standard_normal((5, k))
    y = BO.q8_matmul(x, blocks, n, k)
    qx, dx = BO.q8_quantize_x86(x.astype(np.float32))
    xd = (qx.astype(np.float64) * dx[..., None]).reshape(5, k)
    wd = sm.q8_dequant(blocks, k).reshape(n, k).astype(np.float64)
    np.testing.assert_allclose(y, xd @ wd.T, rtol=0, atol=1e-12 * np.abs(xd @ wd.T).max())
    assert np.abs(y - x @ w.T.astype(np.float64)).max() <= 0.02 * np.abs(x @ w.T).max()

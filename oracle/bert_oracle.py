"""CPU restatement of the reference's BERT text encoder (src/gsv_bert.cpp), in numpy float64.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP encoder, never as the
product path.

The reference builds this graph with ggml (src/gsv_bert.cpp:128-155); its arithmetic lives in
ggml-cpu (mul_mat, flash_attn_ext, the patch's layernorm_affine / add_act), which is not part of
/root/reference, so this restatement follows the graph and the published formulas, in float64:

  x   = LN_emb((word[id] + pos[t]) + type[0])                         (:141-145)
  per layer li < n_layers (post-LN, HF BertLayer):                    (:147-155)
    qkv = Wqkv . x + bqkv; q, k, v = rows [0, D), [D, 2D), [2D, 3D); head h = 64h .. 64h+63
    a   = softmax(q_h k_h^T / sqrt(64)) v_h, over the tokens of the same sequence (:257 mask)
    x   = LN1(x + Wo . a + bo)                                        (ln_affine, :150)
    x   = LN2(x + W2 . gelu_erf(W1 . x + b1) + b2)                    (:151-154)
  LN(v) = (v - mean) / sqrt(var + eps) * w + b over the hidden dim (PATCH:1533-1584)
  gelu_erf(v) = 0.5 v (1 + erf(v / sqrt 2))                            (PATCH GGML_ACT_GELU_ERF)
Output [hidden][T] (:220-228).

Pins (tests/test_oracle_pins.py): LayerNorm and GELU against closed forms and math.erf;
attention against a brute-force softmax and its one-key / constant-V invariants; the whole
forward at n_layers = 0 against the embedding formula. The ggml-cpu summation orders are not
restated (parity of the HIP encoder is within a tolerance).
"""
from __future__ import annotations

import math

import numpy as np

_erf = np.vectorize(math.erf, otypes=[np.float64])


def layernorm(v: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    """Row-wise LayerNorm of the fused layernorm_affine (PATCH:1533-1584)."""
    v = np.asarray(v, np.float64)
    mean = v.mean(axis=-1, keepdims=True)
    var = ((v - mean) ** 2).mean(axis=-1, keepdims=True)
    return (v - mean) / np.sqrt(var + eps) * np.asarray(w, np.float64) + np.asarray(b, np.float64)


def gelu_erf(v: np.ndarray) -> np.ndarray:
    """GGML_ACT_GELU_ERF of the patch's add_act: 0.5 v (1 + erf(v / sqrt 2))."""
    v = np.asarray(v, np.float64)
    return 0.5 * v * (1.0 + _erf(v / math.sqrt(2.0)))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """softmax(q k^T * scale) v for one head: q [T][hd], k, v [T][hd] (no mask: one sequence)."""
    s = (np.asarray(q, np.float64) @ np.asarray(k, np.float64).T) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ np.asarray(v, np.float64)


def q8_quantize_x86(x32: np.ndarray):
    """ggml-cpu's x86 Q8_0 quantisation of float32 rows [R][K] (K % 32 == 0): per block of 32,
    d = fp16(amax / 127), q = round-half-even(x * (127 / amax)) in float32 (0 for an all-zero block).
    Returns (q int8 [R][K/32][32], d float64 [R][K/32])."""
    x32 = np.asarray(x32, np.float32)
    R, K = x32.shape
    xb = x32.reshape(R, K // 32, 32)
    amax = np.abs(xb).max(axis=-1)
    d = (amax / np.float32(127.0)).astype(np.float16).astype(np.float64)
    with np.errstate(divide="ignore"):
        idv = np.where(amax != 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    q = np.rint(xb * idv[..., None]).astype(np.int8)
    return q, d


def q8_matmul(x: np.ndarray, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """ggml mul_mat of Q8_0 weights (GGUF blocks of an [n][k] matrix) with float activations:
    the activations are quantised (q8_quantize_x86 of their float32 values, ggml-cpu's vec_dot type
    for Q8_0), then y[m][n] = sum over blocks of d_x d_w (exact integer block dot), in float64."""
    qx, dx = q8_quantize_x86(np.asarray(x, np.float64).astype(np.float32))
    b = np.asarray(blocks, np.uint8).reshape(n, k // 32, 34)
    dw = b[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    qw = b[:, :, 2:].view(np.int8).astype(np.int32)
    s = np.einsum("mbk,nbk->mnb", qx.astype(np.int32), qw)
    return np.einsum("mnb,mb,nb->mn", s.astype(np.float64), dx, dw)


def encode(W: dict, ids, n_layers: int, hidden: int, heads: int, eps: float, act_f16: bool = False,
           act_q8: bool = False) -> np.ndarray:
    """One sequence of token ids -> [hidden][T] after n_layers layers (0: the embedding LN).
    act_f16: the projections' inputs are rounded to fp16 first, as ggml-cpu does for F16 weights
    (their vec_dot type is F16: ggml_cpu_fp32_to_fp16 of the activations, then F16 x F16 dots).
    act_q8: Q8_0 weights (W holds their blocks under name + "#q8"), multiplied as ggml-cpu does:
    activations quantised to Q8_0 (x86), exact integer block dots (q8_matmul)."""
    ids = np.asarray(ids, np.int64)
    T = len(ids)
    D, hd = hidden, hidden // heads
    g = lambda n: np.asarray(W[n], np.float64)
    x = (g("bert.word_emb")[ids] + g("bert.pos_emb")[:T]) + g("bert.type_emb")[0]
    x = layernorm(x, g("bert.emb_ln_w"), g("bert.emb_ln_b"), eps)
    scale = 1.0 / math.sqrt(hd)
    r = (lambda a: a.astype(np.float32).astype(np.float16).astype(np.float64)) if act_f16 else (lambda a: a)

    def mm(a, name):   # a . W^T of the projection `name`
        if act_q8:
            n_, k_ = W[name].shape
            return q8_matmul(a, W[name + "#q8"], n_, k_)
        return r(a) @ g(name).T

    for li in range(n_layers):
        p = f"bert.l{li}."
        qkv = mm(x, p + "qkv_w") + g(p + "qkv_b")
        a = np.empty((T, D))
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            a[:, sl] = attention(qkv[:, sl], qkv[:, D:2 * D][:, sl], qkv[:, 2 * D:][:, sl], scale)
        x = layernorm(x + mm(a, p + "attn_out_w") + g(p + "attn_out_b"), g(p + "attn_ln_w"),
                      g(p + "attn_ln_b"), eps)
        hh = gelu_erf(mm(x, p + "ff1_w") + g(p + "ff1_b"))
        x = layernorm(x + mm(hh, p + "ff2_w") + g(p + "ff2_b"), g(p + "out_ln_w"), g(p + "out_ln_b"), eps)
    return x.T.copy()

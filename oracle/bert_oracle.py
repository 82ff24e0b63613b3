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


def encode(W: dict, ids, n_layers: int, hidden: int, heads: int, eps: float, act_f16: bool = False) -> np.ndarray:
    """One sequence of token ids -> [hidden][T] after n_layers layers (0: the embedding LN).
    act_f16: the projections' inputs are rounded to fp16 first, as ggml-cpu does for F16 weights
    (their vec_dot type is F16: ggml_cpu_fp32_to_fp16 of the activations, then F16 x F16 dots)."""
    ids = np.asarray(ids, np.int64)
    T = len(ids)
    D, hd = hidden, hidden // heads
    g = lambda n: np.asarray(W[n], np.float64)
    x = (g("bert.word_emb")[ids] + g("bert.pos_emb")[:T]) + g("bert.type_emb")[0]
    x = layernorm(x, g("bert.emb_ln_w"), g("bert.emb_ln_b"), eps)
    scale = 1.0 / math.sqrt(hd)
    r = (lambda a: a.astype(np.float32).astype(np.float16).astype(np.float64)) if act_f16 else (lambda a: a)
    for li in range(n_layers):
        p = f"bert.l{li}."
        qkv = r(x) @ g(p + "qkv_w").T + g(p + "qkv_b")
        a = np.empty((T, D))
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            a[:, sl] = attention(qkv[:, sl], qkv[:, D:2 * D][:, sl], qkv[:, 2 * D:][:, sl], scale)
        x = layernorm(x + r(a) @ g(p + "attn_out_w").T + g(p + "attn_out_b"), g(p + "attn_ln_w"),
                      g(p + "attn_ln_b"), eps)
        hh = gelu_erf(r(x) @ g(p + "ff1_w").T + g(p + "ff1_b"))
        x = layernorm(x + r(hh) @ g(p + "ff2_w").T + g(p + "ff2_b"), g(p + "out_ln_w"), g(p + "out_ln_b"), eps)
    return x.T.copy()

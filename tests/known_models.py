"""Known-answer decoder models for pinning the layer composition of src/gsv_ar.cpp.

Each model keeps the GGUF contract of the real export (full width: d_model 512, 16 heads,
FFN 2048) but chooses its projection weights so that the output of the whole forward pass has a
closed form that this file evaluates in float64 from the model's own tensors:

* a zero Q8_0 matrix contributes nothing (every block has d = 0, q = 0);
* an "identity" Q8_0 matrix (synth_model.q8_blocks: one 1.0 per row, stored d = 2**-6, q = 64, so
  fp32(d_w * d_x) * 64 * q_x is exactly the dequantised activation) passes its input through the
  activation quantisation only, whose error per element is at most
  amax(block) * (1/254 + 2**-11) (x86 quantiser: q = round(x * 127/amax), d = fp16(amax/127)).

What the closed forms restate is the composition the reference graph builds
(src/gsv_ar.cpp:186-225 inputs, :228-269 prefill, :296-358 / :380-467 decode, :798-807 the decode
embedding):
    x_text[t]   = text_emb[phone[t]] + text_alpha * PE[t] + bert_proj . bert[:, t] + bert_proj_b
    x_prompt[t] = audio_emb[prompt[t]] + audio_alpha * PE[t]
    x_pad       = 0
    per layer:  qkv = Wqkv . x + b_qkv
                a   = softmax(q k^T / sqrt(32)) v   (text queries see [pad, max_len), semantic
                                                    queries [pad, q]; decode sees [pad, len])
                n1  = LN1(x + Wo . a + b_o)
                x   = LN2(n1 + W2 . relu(W1 . n1 + b1) + b2)
    logits of the last row = predict . x
    decode step idx embeds its token at PE position prompt_len + idx, K/V at column S + idx.
"""
from __future__ import annotations

import numpy as np

import synth_model as sm

D, NH, HD, FFN, V, PH, BERT = 512, 16, 32, 2048, 1025, 732, 1024
TEXT_ALPHA, AUDIO_ALPHA = 0.75, 1.25
Q8_ERR = 1.0 / 254.0 + 2.0 ** -11        # |dequant(quant(x)) - x| <= amax(block) * Q8_ERR


def zero_q8(n, k):
    return np.zeros(n * k // 32 * 34, np.uint8)


def params(seed: int, n_layer: int):
    """Random non-projection tensors with large, distinct values (so that a dropped or swapped
    term moves the result far outside the quantisation bounds) and a head of signed unit rows."""
    rng = np.random.default_rng(seed)
    f16 = lambda a: a.astype(np.float16).astype(np.float32)
    p = {
        "ar.text_emb": f16(rng.standard_normal((PH, D)) * 0.5),
        "ar.audio_emb": f16(rng.standard_normal((V, D)) * 0.5),
        "ar.bert_proj": (rng.standard_normal((D, BERT)) * 0.05).astype(np.float32),
        "ar.bert_proj_b": (rng.standard_normal(D) * 0.5).astype(np.float32),
    }
    # head row i = s_i * e_{perm[i % 512]}, s_i in {+-1, +-1/2, +-1/4}: exact in fp16 and exact
    # products, so logits[i] = s_i * fp16(x[perm[i % 512]])
    perm = rng.permutation(D)
    scale = (1.0 / (1 << (np.arange(V) // D))) * np.where(rng.random(V) < 0.5, -1.0, 1.0)
    head = np.zeros((V, D), np.float32)
    head[np.arange(V), perm[np.arange(V) % D]] = scale
    p["ar.predict"] = head
    for li in range(n_layer):
        b = f"transformer.block{li}"
        p[f"{b}.qkv_b"] = (rng.standard_normal(3 * D) * 0.5).astype(np.float32)
        p[f"{b}.out_b"] = (rng.standard_normal(D) * 0.5).astype(np.float32)
        p[f"{b}.ffn1_b"] = (rng.standard_normal(FFN) * 0.5).astype(np.float32)
        p[f"{b}.ffn2_b"] = (rng.standard_normal(D) * 0.5).astype(np.float32)
        for n in ("norm1", "norm2"):
            p[f"{b}.{n}_w"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
            p[f"{b}.{n}_b"] = (rng.standard_normal(D) * 0.3).astype(np.float32)
    return p, perm, scale


def write(path, seed, layers, edit=None, **kw):
    """layers: per layer a dict of {"qkv", "out", "ffn1", "ffn2"} -> "zero" | "id" | cols array
    (see synth_model.q8_blocks); missing entries are zero. edit(p), if given, changes the random
    non-projection tensors in place before the file is written. Returns (path, tensors, perm,
    scale)."""
    n_layer = len(layers)
    p, perm, scale = params(seed, n_layer)
    if edit is not None:
        edit(p)
    shapes = {"qkv": (3 * D, D), "out": (D, D), "ffn1": (FFN, D), "ffn2": (D, FFN)}
    fkind = {"qkv": kw.get("attn_type", "q8_0"), "out": kw.get("attn_type", "q8_0"),
             "ffn1": kw.get("ffn_type", "q8_0"), "ffn2": kw.get("ffn_type", "q8_0")}
    for li, spec in enumerate(layers):
        for name, (n, k) in shapes.items():
            kind = spec.get(name, "zero")
            if fkind[name] != "q8_0":      # F16 / F32 weights: the matrix itself (exact 1.0 and 0.0)
                cols = None if isinstance(kind, str) else np.asarray(kind)
                Wm = np.zeros((n, k), np.float32)
                if not (isinstance(kind, str) and kind == "zero"):
                    c = np.arange(n) % k if cols is None else cols
                    Wm[np.arange(n)[c >= 0], c[c >= 0]] = 1.0
                p[f"transformer.block{li}.{name}_w"] = Wm
                continue
            if isinstance(kind, str) and kind == "zero":
                blk = zero_q8(n, k)
            elif isinstance(kind, str) and kind == "id":
                blk = sm.q8_blocks(n, k)
            else:
                blk = sm.q8_blocks(n, k, cols=kind)
            p[f"transformer.block{li}.{name}_w"] = blk
    sm.write_model(path, seed=seed, n_layer=n_layer, override=p, text_alpha=TEXT_ALPHA,
                   audio_alpha=AUDIO_ALPHA, **kw)
    return path, p, perm, scale


# ---- float64 closed forms --------------------------------------------------------------------

def ln64(v, w, b, eps=1e-5):
    v = np.asarray(v, np.float64)
    mean = v.mean(axis=-1, keepdims=True)
    var = ((v - mean) ** 2).mean(axis=-1, keepdims=True)
    return (v - mean) / np.sqrt(var + eps) * np.asarray(w, np.float64) + np.asarray(b, np.float64)


def ln_err(v, w, dv, eps=1e-5):
    """Bound on |LN(v + e) - LN(v)| per element when |e| <= dv (first order, x1.25 margin):
    |w_i| / sigma * dv * (2 + |z_i|), z = the normalised row."""
    v = np.asarray(v, np.float64)
    mean = v.mean(axis=-1, keepdims=True)
    sig = np.sqrt(((v - mean) ** 2).mean(axis=-1, keepdims=True) + eps)
    z = np.abs((v - mean) / sig)
    return 1.25 * np.abs(np.asarray(w, np.float64)) / sig * np.asarray(dv, np.float64)[..., None] * (2.0 + z)


def block_amax(x):
    """amax of each element's 32-block (same shape as x)."""
    x = np.asarray(x, np.float64)
    a = np.abs(x.reshape(x.shape[:-1] + (-1, 32))).max(axis=-1)
    return np.repeat(a, 32, axis=-1)


def pe(npos):
    import oracle as O
    return O.pe_table(D, npos).astype(np.float64)


def inputs64(p, reqs, pe_tab):
    """x [B][S][D] of the prefill (src/gsv_ar.cpp:186-225, :241), float64. Returns (x, S, max_len)."""
    B = len(reqs)
    P = len(reqs[0]["prompt"])
    max_len = max(len(r["phones"]) for r in reqs)
    S = max_len + P
    x = np.zeros((B, S, D))
    te, ae = p["ar.text_emb"].astype(np.float64), p["ar.audio_emb"].astype(np.float64)
    Wb, bb = p["ar.bert_proj"].astype(np.float64), p["ar.bert_proj_b"].astype(np.float64)
    for b, r in enumerate(reqs):
        T = len(r["phones"])
        pad = max_len - T
        for t in range(T):
            feat = np.zeros(BERT) if r.get("bert") is None else r["bert"][:, t].astype(np.float64)
            x[b, pad + t] = te[r["phones"][t]] + TEXT_ALPHA * pe_tab[t] + Wb @ feat + bb
        for t in range(P):
            x[b, max_len + t] = ae[r["prompt"][t]] + AUDIO_ALPHA * pe_tab[t]
    return x, S, max_len


def decode_input64(p, tok, pos, pe_tab):
    """Embedding of a decode step (src/gsv_ar.cpp:798-807): audio_emb[tok] + audio_alpha * PE[pos]."""
    return p["ar.audio_emb"][tok].astype(np.float64) + AUDIO_ALPHA * pe_tab[pos]


def zero_layers64(p, x, n_layer):
    """The decoder over rows x with every projection zero: n1 = LN1(x + b_o), x = LN2(n1 + b_2)."""
    for li in range(n_layer):
        b = f"transformer.block{li}"
        n1 = ln64(x + p[f"{b}.out_b"], p[f"{b}.norm1_w"], p[f"{b}.norm1_b"])
        x = ln64(n1 + p[f"{b}.ffn2_b"], p[f"{b}.norm2_w"], p[f"{b}.norm2_b"])
    return x


def head64_f32(x, perm, scale):
    """F32 head of signed unit rows: exact products of the fp32 activations."""
    xs = np.asarray(x, np.float64).astype(np.float32).astype(np.float64)
    return xs[..., perm[np.arange(V) % D]] * scale


def head64(x, perm, scale):
    """F16 head of signed unit rows: activations rounded to fp16 (ggml's F16 vec_dot type)."""
    xh = np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)
    return xh[..., perm[np.arange(V) % D]] * scale

"""Synthetic gsv AR model writer (GGUF v3), for tests and benchmarks.

Writes a t2s-shaped decoder with the exact tensor names, shapes, types and ``ar.*`` keys of the
reference exporter (tools/export_gguf/convert_ar.py:91-130, ``--q8`` = attn/ffn Q8_0 per
tools/export_gguf/export.py:51-52; norms, biases, alphas and bert_proj F32 per convert_ar.py:76-89)
and random weights from a fixed seed:

* projection weights (qkv/out/ffn1/ffn2) N(0, 0.02), quantised to Q8_0 with ggml's reference
  quantiser (d = amax/127 stored fp16, q = roundf(x / d), half away from zero);
* biases N(0, 0.02); LayerNorm weights 1 + N(0, 0.05) and biases N(0, 0.05) (not the identity, so
  that a swapped or dropped affine term is visible);
* embeddings N(0, 0.02) rounded to fp16 and stored F32 (the loader requires F32,
  src/gsv_ar.cpp:632-637); ``ar.predict`` N(0, 0.02) in F16 (or F32 / Q8_0 on request);
* ``bert_proj`` N(0, 0.02) F32, PE alphas 1.0.

numpy's PCG64 generator makes the file identical for a given seed on every machine with this
numpy, so the GPU box regenerates the same model instead of shipping 80 MB.
"""
from __future__ import annotations

import os
import struct

import numpy as np

GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
_GG_U32, _GG_F32, _GG_STR = 4, 6, 8
ALIGN = 32


def q8_quantize_ref(x: np.ndarray) -> np.ndarray:
    """ggml quantize_row_q8_0_ref over the last axis -> uint8 [..., nblk*34] GGUF blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    shp = x.shape
    assert shp[-1] % 32 == 0
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = (xb * idv[:, None]).astype(np.float32).astype(np.float64)
    q = np.trunc(v + np.copysign(0.5, v)).astype(np.int8)        # roundf: half away from zero
    out = np.empty((xb.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(shp[:-1] + (shp[-1] // 32 * 34,))


def q8_dequant(blocks: np.ndarray, k: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks).reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1, k)


class _Writer:
    def __init__(self):
        self.kv: list[bytes] = []
        self.tensors: list[tuple[str, tuple, int, bytes]] = []

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def add_u32(self, key, v):
        self.kv.append(self._str(key) + struct.pack("<II", _GG_U32, v))

    def add_f32(self, key, v):
        self.kv.append(self._str(key) + struct.pack("<If", _GG_F32, v))

    def add_str(self, key, v):
        self.kv.append(self._str(key) + struct.pack("<I", _GG_STR) + self._str(v))

    def add_tensor(self, name, torch_shape, ggml_type, data: bytes):
        ne = tuple(reversed(torch_shape))      # ggml order: ne0 = last torch dim
        self.tensors.append((name, ne, ggml_type, data))

    def write(self, path):
        head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.kv)))
        for kv in self.kv:
            head += kv
        off = 0
        offsets = []
        for name, ne, t, data in self.tensors:
            offsets.append(off)
            off += (len(data) + ALIGN - 1) // ALIGN * ALIGN
        for (name, ne, t, data), o in zip(self.tensors, offsets):
            head += self._str(name) + struct.pack("<I", len(ne))
            for n in ne:
                head += struct.pack("<Q", n)
            head += struct.pack("<IQ", t, o)
        pad = (-len(head)) % ALIGN
        head += b"\0" * pad
        tmp = path + ".tmp%d" % os.getpid()
        with open(tmp, "wb") as f:
            f.write(head)
            for name, ne, t, data in self.tensors:
                f.write(data)
                f.write(b"\0" * ((-len(data)) % ALIGN))
        os.replace(tmp, path)


def write_model(path: str, seed: int = 0x6A5E0000, n_layer: int = 24, d_model: int = 512,
                n_head: int = 16, ffn: int = 2048, vocab: int = 1025, phone_vocab: int = 732,
                eos: int = 1024, head_type: str = "f16", bert_dim: int = 1024,
                override: dict | None = None, text_alpha: float = 1.0, audio_alpha: float = 1.0,
                attn_type: str = "q8_0", ffn_type: str = "q8_0") -> str:
    """Write the synthetic model to ``path`` (returns path).

    override maps tensor names to the values to store instead of the random ones (the random
    stream is drawn as usual, so the other tensors do not change): fp32 arrays of the tensor's
    shape, stored in the tensor's type (Q8_0 through q8_quantize_ref, F16 rounded), or, for a
    Q8_0 tensor, a uint8 array of ready GGUF blocks (exact scales, see q8_blocks).

    attn_type (qkv_w, out_w) and ffn_type (ffn1_w, ffn2_w): "q8_0", "f16" or "f32", the projection
    types of the reference exporter's attn= / ffn= options (tools/export_gguf/export.py:53-54)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    D = d_model
    override = override or {}

    def normal(shape, std):
        return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    w = _Writer()
    w.add_str("general.architecture", "gsv.ar")
    w.add_str("general.name", "gsv-ar-synthetic")
    w.add_u32("ar.hidden_dim", D)
    w.add_u32("ar.head", n_head)
    w.add_u32("ar.n_layer", n_layer)
    w.add_u32("ar.vocab_size", vocab)
    w.add_u32("ar.phoneme_vocab_size", phone_vocab)
    w.add_u32("ar.eos", eos)
    w.add_f32("ar.bert_dim", float(bert_dim))
    w.add_u32("general.alignment", ALIGN)

    f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32).tobytes()
    emb16 = lambda a: a.astype(np.float16).astype(np.float32)

    def put(name, shape, ggml_type, values):
        v = override.get(name, values)
        if ggml_type == GGML_Q8_0:
            if v.dtype == np.uint8:
                assert v.size == int(np.prod(shape)) // 32 * 34, name
                data = np.ascontiguousarray(v).tobytes()
            else:
                data = q8_quantize_ref(np.asarray(v, np.float32).reshape(shape)).tobytes()
        elif ggml_type == GGML_F16:
            data = np.asarray(v, np.float32).reshape(shape).astype(np.float16).tobytes()
        else:
            data = f32(np.asarray(v, np.float32).reshape(shape))
        w.add_tensor(name, shape, ggml_type, data)

    put("ar.text_emb", (phone_vocab, D), GGML_F32, emb16(normal((phone_vocab, D), 0.02)))
    put("ar.audio_emb", (vocab, D), GGML_F32, emb16(normal((vocab, D), 0.02)))
    put("ar.bert_proj", (D, bert_dim), GGML_F32, normal((D, bert_dim), 0.02))
    put("ar.bert_proj_b", (D,), GGML_F32, normal((D,), 0.02))
    put("ar.text_pe_alpha", (1,), GGML_F32, np.full(1, text_alpha, np.float32))
    put("ar.audio_pe_alpha", (1,), GGML_F32, np.full(1, audio_alpha, np.float32))
    pred = normal((vocab, D), 0.02)
    if head_type == "f16":
        put("ar.predict", (vocab, D), GGML_F16, pred)
    elif head_type == "f32":
        put("ar.predict", (vocab, D), GGML_F32, pred)
    elif head_type == "q8_0":
        put("ar.predict", (vocab, D), GGML_Q8_0, pred)
    else:
        raise ValueError("head_type must be f16, f32 or q8_0")
    types = {"q8_0": GGML_Q8_0, "f16": GGML_F16, "f32": GGML_F32}
    ta, tf = types[attn_type], types[ffn_type]
    for li in range(n_layer):
        p = f"transformer.block{li}"
        put(f"{p}.qkv_w", (3 * D, D), ta, normal((3 * D, D), 0.02))
        put(f"{p}.qkv_b", (3 * D,), GGML_F32, normal((3 * D,), 0.02))
        put(f"{p}.out_w", (D, D), ta, normal((D, D), 0.02))
        put(f"{p}.out_b", (D,), GGML_F32, normal((D,), 0.02))
        put(f"{p}.norm1_w", (D,), GGML_F32, 1.0 + normal((D,), 0.05))
        put(f"{p}.norm1_b", (D,), GGML_F32, normal((D,), 0.05))
        put(f"{p}.ffn1_w", (ffn, D), tf, normal((ffn, D), 0.02))
        put(f"{p}.ffn1_b", (ffn,), GGML_F32, normal((ffn,), 0.02))
        put(f"{p}.ffn2_w", (D, ffn), tf, normal((D, ffn), 0.02))
        put(f"{p}.ffn2_b", (D,), GGML_F32, normal((D,), 0.02))
        put(f"{p}.norm2_w", (D,), GGML_F32, 1.0 + normal((D,), 0.05))
        put(f"{p}.norm2_b", (D,), GGML_F32, normal((D,), 0.05))
    w.write(path)
    return path


def q8_blocks(n: int, k: int, cols=None, scale_log2: int = -6) -> np.ndarray:
    """GGUF Q8_0 blocks of an n x k matrix whose row r holds one non-zero, exactly 1.0, at column
    cols[r] (default r % k), stored as d = 2**scale_log2 (exact in fp16) and q = 2**-scale_log2;
    cols[r] < 0 leaves row r zero. All other blocks have d = 0, q = 0."""
    cols = np.arange(n) % k if cols is None else np.asarray(cols)
    q = 2 ** (-scale_log2)
    assert 1 <= q <= 127
    blk = np.zeros((n, k // 32, 34), np.uint8)
    d16 = np.array([2.0 ** scale_log2], np.float16).view(np.uint8)
    for r in range(n):
        c = int(cols[r])
        if c < 0:
            continue
        blk[r, c // 32, 0:2] = d16
        blk[r, c // 32, 2 + c % 32] = np.uint8(q)
    return blk.reshape(-1)


def cached_model(cache_dir: str, **kw) -> str:
    """Path of the synthetic model for these arguments, written on first use."""
    os.makedirs(cache_dir, exist_ok=True)
    key = "_".join(f"{k}{v}" for k, v in sorted(kw.items())) or "default"
    path = os.path.join(cache_dir, f"gsv_ar_{key}.gguf")
    if not os.path.exists(path):
        write_model(path, **kw)
    return path


def synth_requests(seed: int, B: int, prompt_len: int, phone_lens, bert: bool = True,
                   phone_vocab: int = 732, code_vocab: int = 1025, bert_dim: int = 1024):
    """Seeded requests: phones U{0..phone_vocab-1}, one shared prompt U{0..code_vocab-1},
    bert U(-1, 1) ([bert_dim][T] row-major) as in tests/bench_ar_width.cpp:44-55."""
    rng = np.random.Generator(np.random.PCG64(seed))
    prompt = rng.integers(0, code_vocab, size=prompt_len, dtype=np.int32)
    reqs = []
    for b in range(B):
        T = int(phone_lens[b])
        ph = rng.integers(0, phone_vocab, size=T, dtype=np.int32)
        be = rng.uniform(-1.0, 1.0, size=(bert_dim, T)).astype(np.float32) if bert else None
        reqs.append({"phones": ph, "bert": be, "prompt": prompt.copy()})
    return reqs


def write_bert_model(path: str, seed: int = 0x6A5E0010, n_layer: int = 4, layers_used: int = 2,
                     hidden: int = 1024, heads: int = 16, inter: int = 4096, vocab: int = 1000,
                     max_pos: int = 512, wtype: str = "f32", ln_eps: float = 1e-12):
    """A synthetic BERT GGUF with the tensor contract of src/gsv_bert.cpp:398-431 (keys bert.*,
    tensors bert.word_emb .. bert.l{i}.out_ln_b; projection weights in `wtype`, the rest F32, as
    tools/export_gguf/convert_bert.py writes them). Returns (path, weights): the fp32 values the
    loader holds (F16 rounded, Q8_0 dequantised; for Q8_0 also the blocks, under name + "#q8"),
    for the oracle."""
    rng = np.random.Generator(np.random.PCG64(seed))
    D, F = hidden, inter

    def normal(shape, std):
        return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32).tobytes()
    w = _Writer()
    w.add_str("general.architecture", "gsv.bert")
    w.add_str("general.name", "gsv-bert-synthetic")
    w.add_u32("bert.n_layer", n_layer)
    w.add_u32("bert.hidden", D)
    w.add_u32("bert.head", heads)
    w.add_u32("bert.inter", F)
    w.add_f32("bert.ln_eps", ln_eps)
    w.add_u32("bert.vocab", vocab)
    w.add_u32("bert.max_pos", max_pos)
    w.add_u32("bert.layers_used", layers_used)
    w.add_u32("general.alignment", ALIGN)
    W = {}

    def add(name, a, proj=False):
        if proj and wtype == "f16":
            h = a.astype(np.float16)
            w.add_tensor(name, a.shape, GGML_F16, h.tobytes())
            W[name] = h.astype(np.float32)
        elif proj and wtype == "q8_0":
            blocks = q8_quantize_ref(a)
            w.add_tensor(name, a.shape, GGML_Q8_0, blocks.tobytes())
            W[name] = q8_dequant(blocks, a.shape[-1]).reshape(a.shape)
            W[name + "#q8"] = blocks          # the blocks themselves (an oracle that quantises activations)
        else:
            w.add_tensor(name, a.shape, GGML_F32, f32(a))
            W[name] = a.astype(np.float32)

    add("bert.word_emb", normal((vocab, D), 0.05))
    add("bert.pos_emb", normal((max_pos, D), 0.05))
    add("bert.type_emb", normal((2, D), 0.05))
    add("bert.emb_ln_w", 1.0 + normal((D,), 0.05))
    add("bert.emb_ln_b", normal((D,), 0.05))
    for li in range(n_layer):
        p = f"bert.l{li}."
        add(p + "qkv_w", normal((3 * D, D), 0.03), proj=True)
        add(p + "qkv_b", normal((3 * D,), 0.02))
        add(p + "attn_out_w", normal((D, D), 0.03), proj=True)
        add(p + "attn_out_b", normal((D,), 0.02))
        add(p + "attn_ln_w", 1.0 + normal((D,), 0.05))
        add(p + "attn_ln_b", normal((D,), 0.05))
        add(p + "ff1_w", normal((F, D), 0.03), proj=True)
        add(p + "ff1_b", normal((F,), 0.02))
        add(p + "ff2_w", normal((D, F), 0.03), proj=True)
        add(p + "ff2_b", normal((D,), 0.02))
        add(p + "out_ln_w", 1.0 + normal((D,), 0.05))
        add(p + "out_ln_b", normal((D,), 0.05))
    w.write(path)
    return path, W

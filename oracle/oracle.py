"""ctypes binding of the CPU oracle (liboracle.so) and of the reference sampler (_ref/).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by bench.py's
CPU-baseline leg, always as the checker or the timed CPU baseline, never as the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libgsv_sampler_ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")

ORC_KV_F16 = 1
ORC_EOS_MASK_ALL = 2


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class _Req(C.Structure):
    _fields_ = [("phones", C.c_void_p), ("n_phones", C.c_int32), ("bert", C.c_void_p),
                ("prompt", C.c_void_p), ("n_prompt", C.c_int32)]


class _GenOut(C.Structure):
    _fields_ = [("tokens", C.c_void_p), ("tok_stride", C.c_int32), ("tok_len", C.c_void_p),
                ("lens", C.c_void_p), ("finish_seq", C.c_void_p), ("sampled", C.c_void_p),
                ("logits", C.c_void_p), ("probs0", C.c_void_p), ("n_steps", C.c_int32),
                ("prefill_ms", C.c_double), ("decode_ms", C.c_double), ("kv_layer", C.c_int32),
                ("kv_cols", C.c_int32), ("kv_k", C.c_void_p), ("kv_v", C.c_void_p)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_q8_quantize_ref.argtypes = [_f32p, C.c_int64, _u8p]
        L.orc_q8_quantize_x86.argtypes = [_f32p, C.c_int64, _u8p]
        L.orc_q8_dequant.argtypes = [_u8p, C.c_int64, _f32p]
        L.orc_q8_dot.restype = C.c_float
        L.orc_q8_dot.argtypes = [_u8p, _u8p, C.c_int64]
        L.orc_q8_dot_scalar.restype = C.c_float
        L.orc_q8_dot_scalar.argtypes = [_u8p, _u8p, C.c_int64]
        L.orc_q8_matmul.argtypes = [_u8p, C.c_int64, C.c_int64, _f32p, C.c_int64, _f32p, C.c_int]
        L.orc_f16_matmul.argtypes = [_u16p, C.c_int64, C.c_int64, _f32p, C.c_int64, _f32p, C.c_int, C.c_int]
        L.orc_f32_matmul.argtypes = [_f32p, C.c_int64, C.c_int64, _f32p, C.c_int64, _f32p, C.c_int, C.c_int]
        L.orc_layernorm.argtypes = [_f32p, C.c_void_p, C.c_void_p, _f32p, C.c_int64, C.c_int64, C.c_float, _f32p]
        L.orc_add_act.argtypes = [_f32p, _f32p, C.c_int64, C.c_int64, C.c_int, _f32p]
        L.orc_attn_row.argtypes = [_f32p, _f32p, _f32p, C.c_int64, C.c_int, C.c_int64, C.c_void_p, C.c_float, _f32p]
        L.orc_attn_decode_f16.argtypes = [_f32p, _u16p, _u16p, C.c_int, C.c_int, C.c_int, C.c_int64,
                                          _i32p, _i32p, C.c_float, _f32p, C.c_int]
        L.orc_attn_prefill.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, _i32p, C.c_int, C.c_int, C.c_float,
                                       _f32p, C.c_int]
        L.orc_logits_to_probs.argtypes = [C.c_int, C.c_float, C.c_float, C.c_float, _f32p, C.c_int,
                                          C.c_void_p, C.c_int, _f32p]
        L.orc_rng_next.restype = C.c_uint64
        L.orc_rng_next.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_rng_exponential.restype = C.c_float
        L.orc_rng_exponential.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_rng_exponential_n.argtypes = [C.POINTER(C.c_uint64), C.c_int64, _f32p]
        L.orc_expf_n.argtypes = [_f32p, C.c_int64, _f32p]
        L.orc_argmax_probs_over_q.restype = C.c_int
        L.orc_argmax_probs_over_q.argtypes = [_f32p, _f32p, C.c_int]
        L.orc_sample.restype = C.c_int
        L.orc_sample.argtypes = [_f32p, C.c_int, C.POINTER(C.c_uint64)]
        L.orc_pe_table.argtypes = [C.c_int, C.c_int, _f32p]
        L.orc_model_load.restype = C.c_void_p
        L.orc_model_load.argtypes = [C.c_char_p, C.c_char_p, C.c_int]
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_model_info.argtypes = [C.c_void_p, _i32p]
        L.orc_generate.restype = C.c_int
        L.orc_generate.argtypes = [C.c_void_p, C.POINTER(_Req), C.c_int, C.c_int, C.c_float, C.c_float,
                                   C.c_float, C.c_uint64, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                   C.c_void_p, C.c_uint, C.c_int, C.POINTER(_GenOut)]
        L.orc_prefill_kv.restype = C.c_int
        L.orc_prefill_kv.argtypes = [C.c_void_p, C.POINTER(_Req), C.c_int, C.c_uint, C.c_int, C.c_int,
                                     C.c_void_p, C.c_void_p, _f32p, C.POINTER(C.c_int32)]
        L.orc_first_logits.restype = C.c_int
        L.orc_first_logits.argtypes = [C.c_void_p, C.POINTER(_Req), C.c_int, C.c_uint, C.c_int, _f32p]
        _lib = L
    return _lib


def nthreads_default():
    n = os.environ.get("OMP_NUM_THREADS")
    return int(n) if n else (os.cpu_count() or 1)


# ---- thin helpers --------------------------------------------------------------------------

def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits (RNE), elementwise via the oracle's F16C conversion."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def q8_quantize_x86(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().orc_q8_quantize_x86(x.ravel(), x.size, out)
    return out


def q8_quantize_ref(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().orc_q8_quantize_ref(x.ravel(), x.size, out)
    return out


def q8_dequant(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).ravel()
    nb = blocks.size // 34
    out = np.zeros(nb * 32, np.float32)
    lib().orc_q8_dequant(blocks, nb, out)
    return out


def q8_matmul(W_blocks: np.ndarray, N: int, K: int, X: np.ndarray, nthreads=None) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    M = X.shape[0]
    Y = np.zeros((M, N), np.float32)
    lib().orc_q8_matmul(np.ascontiguousarray(W_blocks, np.uint8).ravel(), N, K, X.ravel(), M, Y, nthreads or nthreads_default())
    return Y


def f16_matmul(W16: np.ndarray, X: np.ndarray, mode: int, nthreads=None) -> np.ndarray:
    W16 = np.ascontiguousarray(W16, np.uint16)
    X = np.ascontiguousarray(X, np.float32)
    N, K = W16.shape
    Y = np.zeros((X.shape[0], N), np.float32)
    lib().orc_f16_matmul(W16, N, K, X, X.shape[0], Y, mode, nthreads or nthreads_default())
    return Y


def f32_matmul(W: np.ndarray, X: np.ndarray, mode: int, nthreads=None) -> np.ndarray:
    W = np.ascontiguousarray(W, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    N, K = W.shape
    Y = np.zeros((X.shape[0], N), np.float32)
    lib().orc_f32_matmul(W, N, K, X, X.shape[0], Y, mode, nthreads or nthreads_default())
    return Y


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def layernorm(x, r, bias, wb, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    y = np.zeros_like(x)
    r = None if r is None else np.ascontiguousarray(r, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_layernorm(x, _ptr(r), _ptr(bias), np.ascontiguousarray(wb, np.float32), rows, n, eps, y)
    return y


def add_act(a, b, act):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    y = np.zeros_like(a)
    lib().orc_add_act(a.ravel(), b.ravel(), a.size, b.size, act, y)
    return y


def attn_decode_f16(q, k16, v16, kv_begin, kv_end, scale, nthreads=None):
    """q [B][nh][hd] fp32; k16/v16 uint16 [B][nh][lstride][hd]; returns [B][nh*hd]."""
    q = np.ascontiguousarray(q, np.float32)
    B, nh, hd = q.shape
    lstride = k16.shape[2]
    out = np.zeros((B, nh * hd), np.float32)
    lib().orc_attn_decode_f16(q, np.ascontiguousarray(k16), np.ascontiguousarray(v16), B, nh, hd, lstride,
                              np.ascontiguousarray(kv_begin, np.int32), np.ascontiguousarray(kv_end, np.int32),
                              scale, out, nthreads or nthreads_default())
    return out


def attn_prefill(qkv, max_len, pad, nh, scale, nthreads=None):
    """Prefill self-attention: qkv fp32 [B][S][3*nh*hd]; returns [B][S][nh*hd]."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    B, S, three_d = qkv.shape
    D = three_d // 3
    out = np.zeros((B, S, D), np.float32)
    lib().orc_attn_prefill(qkv, B, S, max_len, np.ascontiguousarray(pad, np.int32), nh, D // nh, scale, out,
                           nthreads or nthreads_default())
    return out


def expf(x):
    """expf of this host's libm, elementwise (float32 in, float32 out)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_expf_n(x.reshape(-1), x.size, y.reshape(-1))
    return y


def logits_to_probs(cfg, logits, prev):
    logits = np.array(logits, np.float32)
    prev = None if prev is None else np.ascontiguousarray(prev, np.int32)
    probs = np.zeros_like(logits)
    lib().orc_logits_to_probs(cfg[0], cfg[1], cfg[2], cfg[3], logits, logits.size, _ptr(prev),
                              0 if prev is None else prev.size, probs)
    return logits, probs


def rng_stream(seed, n):
    s = C.c_uint64(seed if seed else 1)
    out = np.array([lib().orc_rng_next(C.byref(s)) for _ in range(n)], np.uint64)
    return out, s.value


def rng_exponential(seed, n):
    s = C.c_uint64(seed if seed else 1)
    out = np.array([lib().orc_rng_exponential(C.byref(s)) for _ in range(n)], np.float32)
    return out, s.value


def rng_exponential_n(seed, n):
    """n draws of rng_exponential from `seed` (0 -> 1), as float32."""
    s = C.c_uint64(seed if seed else 1)
    out = np.zeros(n, np.float32)
    lib().orc_rng_exponential_n(C.byref(s), n, out)
    return out


def sample(probs, seed):
    s = C.c_uint64(seed if seed else 1)
    t = lib().orc_sample(np.ascontiguousarray(probs, np.float32), len(probs), C.byref(s))
    return t, s.value


def pe_table(D, npos):
    out = np.zeros((npos, D), np.float32)
    lib().orc_pe_table(D, npos, out)
    return out


# ---- model ----------------------------------------------------------------------------------

def _reqs_struct(reqs):
    keep = []
    arr = (_Req * len(reqs))()
    for i, r in enumerate(reqs):
        ph = np.ascontiguousarray(r["phones"], np.int32)
        pr = np.ascontiguousarray(r["prompt"], np.int32)
        be = None if r.get("bert") is None else np.ascontiguousarray(r["bert"], np.float32)
        keep += [ph, pr, be]
        arr[i].phones = ph.ctypes.data
        arr[i].n_phones = ph.size
        arr[i].bert = None if be is None else be.ctypes.data
        arr[i].prompt = pr.ctypes.data
        arr[i].n_prompt = pr.size
    return arr, keep


class Model:
    def __init__(self, path):
        err = C.create_string_buffer(512)
        self.h = lib().orc_model_load(path.encode(), err, 512)
        if not self.h:
            raise RuntimeError("oracle load failed: " + err.value.decode())
        info = np.zeros(10, np.int32)
        lib().orc_model_info(self.h, info)
        (self.D, self.NH, self.HD, self.NL, self.V, self.EOS, self.PH, self.BERT, self.FFN,
         self.head_type) = [int(v) for v in info]

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    __del__ = close

    def first_logits(self, reqs, flags=0, nthreads=None):
        arr, keep = _reqs_struct(reqs)
        out = np.zeros((len(reqs), self.V), np.float32)
        rc = lib().orc_first_logits(self.h, arr, len(reqs), flags, nthreads or nthreads_default(), out)
        if rc != 0:
            raise RuntimeError("orc_first_logits failed: %d" % rc)
        return out

    def prefill_kv(self, reqs, layer, flags=0, nthreads=None):
        """(K, V [B][NH][S][HD], last-position logits [B][V]) of the prefill."""
        arr, keep = _reqs_struct(reqs)
        B = len(reqs)
        S = max(len(r["phones"]) for r in reqs) + len(reqs[0]["prompt"])
        k = np.zeros((B, self.NH, S, self.HD), np.float32)
        v = np.zeros_like(k)
        lg = np.zeros((B, self.V), np.float32)
        s_out = C.c_int32(0)
        rc = lib().orc_prefill_kv(self.h, arr, B, flags, nthreads or nthreads_default(), layer,
                                  k.ctypes.data_as(C.c_void_p), v.ctypes.data_as(C.c_void_p), lg, C.byref(s_out))
        if rc != 0:
            raise RuntimeError("orc_prefill_kv failed: %d" % rc)
        return k, v, lg

    def generate(self, reqs, sampler=(15, 1.0, 1.0, 1.35), seed_base=0, early_stop=-1, max_steps=50,
                 oracle=None, seeds=None, flags=0, nthreads=None, want_logits=False, want_probs0=False,
                 kv_layer=None):
        """kv_layer: also return that layer's K/V cache after the loop as "kv" = (K, V), each
        [B][NH][S + n_steps][HD] (the prefill's S columns, then one per decode step that ran)."""
        B = len(reqs)
        P = len(reqs[0]["prompt"])
        arr, keep = _reqs_struct(reqs)
        stride = P + max_steps
        tokens = np.zeros((B, stride), np.int32)
        tok_len = np.zeros(B, np.int32)
        lens = np.zeros(B, np.int32)
        fin = np.zeros(B, np.int32)
        sampled = np.full((max_steps, B), -1, np.int32)
        logits = np.zeros((max_steps, B, self.V), np.float32) if want_logits else None
        probs0 = np.zeros((max_steps, self.V), np.float32) if want_probs0 else None
        o = _GenOut(tokens.ctypes.data, stride, tok_len.ctypes.data, lens.ctypes.data, fin.ctypes.data,
                    sampled.ctypes.data, None if logits is None else logits.ctypes.data,
                    None if probs0 is None else probs0.ctypes.data, 0, 0.0, 0.0)
        S = max(len(r["phones"]) for r in reqs) + P
        kk = vv = None
        if kv_layer is not None:
            kk = np.zeros((B, self.NH, S + max_steps, self.HD), np.float32)
            vv = np.zeros_like(kk)
            o.kv_layer, o.kv_cols = int(kv_layer), S + max_steps
            o.kv_k, o.kv_v = kk.ctypes.data, vv.ctypes.data
        else:
            o.kv_layer, o.kv_cols = -1, 0
        orc = None if oracle is None else np.ascontiguousarray(oracle, np.int32)
        sd = None if seeds is None else np.ascontiguousarray(seeds, np.uint64)
        rc = lib().orc_generate(self.h, arr, B, sampler[0], sampler[1], sampler[2], sampler[3], seed_base,
                                early_stop, max_steps, _ptr(orc), 0 if orc is None else orc.size, _ptr(sd),
                                flags, nthreads or nthreads_default(), C.byref(o))
        if rc != 0:
            raise RuntimeError("orc_generate failed: %d" % rc)
        n = o.n_steps
        return {"tokens": [tokens[b, :tok_len[b]].copy() for b in range(B)], "lens": lens.copy(),
                "finish_seq": fin.copy(), "sampled": sampled[:n].copy(), "n_steps": n,
                "logits": None if logits is None else logits[:n], "probs0": None if probs0 is None else probs0[:n],
                "prefill_ms": o.prefill_ms, "decode_ms": o.decode_ms,
                "kv": None if kk is None else (kk[:, :, :S + n], vv[:, :, :S + n])}


# ---- reference sampler (compiled from the reference sources in this container) -------------

_ref = None


def ref_lib():
    """The reference gsv_sampler.cpp built into oracle/_ref (None when it was not built)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            return None
        L = C.CDLL(REF_PATH)
        L.ref_logits_to_probs.argtypes = [C.c_int, C.c_float, C.c_float, C.c_float, _f32p, C.c_int,
                                          C.c_void_p, C.c_int, _f32p]
        L.ref_rng_stream.restype = C.c_uint64
        L.ref_rng_stream.argtypes = [C.c_uint64, C.c_int, _u64p]
        L.ref_rng_exponential.restype = C.c_uint64
        L.ref_rng_exponential.argtypes = [C.c_uint64, C.c_int, _f32p]
        L.ref_sample.restype = C.c_int
        L.ref_sample.argtypes = [_f32p, C.c_int, C.c_uint64, C.POINTER(C.c_uint64)]
        L.ref_argmax_probs_over_q.restype = C.c_int
        L.ref_argmax_probs_over_q.argtypes = [_f32p, _f32p, C.c_int]
        _ref = L
    return _ref

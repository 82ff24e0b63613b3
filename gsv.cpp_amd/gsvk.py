"""Python binding of the gfx950 AR decoder C ABI (include/gsvk.h) over ctypes.

This is the host-side mirror of the reference's ``gsv_ar`` interface for Python callers, tests
and benchmarks. It loads ``gsv.cpp_amd/lib/libgsvk.so`` (built by ``gsv.cpp_amd/build.py``) and
raises if the library is missing: there is no fallback path. Device ops take torch tensors
(torch is only the device-memory and stream plumbing) and pass raw pointers to the kernels.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libgsvk.so")

GSVK_GEN_EOS_MASK_ALL = 1
GSVK_GEN_PROB_DUMP = 2

# every entry point declared in include/gsvk.h
EXPORTS = [
    "gsvk_last_error", "gsvk_device_count", "gsvk_parse_device", "gsvk_model_load", "gsvk_model_free",
    "gsvk_model_get_info", "gsvk_generate", "gsvk_first_logits", "gsvk_release_cache", "gsvk_kv_alloc",
    "gsvk_prefill", "gsvk_decode_step", "gsvk_kv_read", "gsvk_last_sampled", "gsvk_op_q8_dequant",
    "gsvk_op_q8_repack", "gsvk_op_q8_quantize", "gsvk_op_q8_gemv", "gsvk_op_layernorm", "gsvk_op_add_act",
    "gsvk_op_fdot", "gsvk_attn_workspace_bytes", "gsvk_op_attn_decode", "gsvk_op_ln_gemv",
    "gsvk_sample_workspace_bytes", "gsvk_op_sample", "gsvk_op_qkv_attn",
    "gsvk_qkv_attn_supported", "gsvk_op_q8_gemm", "gsvk_op_q8_gemm_ex", "gsvk_op_attn_prefill",
    "gsvk_cb_open", "gsvk_cb_add", "gsvk_cb_step", "gsvk_cb_take", "gsvk_cb_close",
    "gsvk_bert_load", "gsvk_bert_free", "gsvk_bert_get_info", "gsvk_bert_encode",
    "gsvk_op_attn_decode_noalloc", "gsvk_model_set_decode_path", "gsvk_op_dec_attn", "gsvk_op_dec_ffn",
    "gsvk_model_set_exact", "gsvk_op_attn_exact", "gsvk_op_expf_exact", "gsvk_model_set_prefill_f16",
    "gsvk_op_q8_dequant_f16", "gsvk_op_q8h_gemm", "gsvk_op_qkv_attn_exact", "gsvk_model_get_profile",
    "gsvk_model_time_decode_kernel", "gsvk_phase_stamps",
]

GSVK_DECODE_AUTO, GSVK_DECODE_GEMV, GSVK_DECODE_FUSED, GSVK_DECODE_MFMA, GSVK_DECODE_PERSIST = 0, 1, 2, 3, 4


class GsvkError(RuntimeError):
    pass


class Request(C.Structure):
    _fields_ = [("phones", C.c_void_p), ("n_phones", C.c_int32), ("bert", C.c_void_p),
                ("prompt", C.c_void_p), ("n_prompt", C.c_int32)]


class SamplerCfg(C.Structure):
    _fields_ = [("top_k", C.c_int), ("top_p", C.c_float), ("temperature", C.c_float),
                ("repetition_penalty", C.c_float)]


PROGRESS_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int)


class GenOut(C.Structure):
    _fields_ = [("tokens", C.c_void_p), ("tok_stride", C.c_int32), ("tok_len", C.c_void_p),
                ("lens", C.c_void_p), ("finish_seq", C.c_void_p), ("probs0", C.c_void_p),
                ("n_steps", C.c_int32), ("progress", PROGRESS_FN), ("progress_user", C.c_void_p),
                ("prefill_ms", C.c_double), ("decode_ms", C.c_double)]


class Profile(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("pf_build_ms", "pf_copy_ms", "pf_compute_ms", "pf_io_ms", "dec_build_ms",
                                          "dec_copy_ms", "dec_compute_ms", "dec_other_ms")] + [("steps", C.c_int)]


class ModelInfo(C.Structure):
    _fields_ = [("d_model", C.c_int), ("n_head", C.c_int), ("head_dim", C.c_int), ("n_layer", C.c_int),
                ("vocab", C.c_int), ("eos", C.c_int), ("phone_vocab", C.c_int), ("bert_dim", C.c_int),
                ("ffn_dim", C.c_int), ("head_type", C.c_int), ("text_alpha", C.c_float),
                ("audio_alpha", C.c_float), ("prompt_len", C.c_int), ("kv_batch", C.c_int),
                ("kv_lmax", C.c_int)]


class BertInfo(C.Structure):
    _fields_ = [("hidden", C.c_int), ("heads", C.c_int), ("inter", C.c_int), ("layers_used", C.c_int),
                ("vocab", C.c_int), ("max_pos", C.c_int), ("ln_eps", C.c_float), ("weight_type", C.c_int)]


_lib = None


def lib():
    """The loaded libgsvk.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GsvkError(f"{LIB_PATH} not found: build it with python gsv.cpp_amd/build.py")
        L = C.CDLL(LIB_PATH)
        vp, i64, i32, f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
        L.gsvk_last_error.restype = C.c_char_p
        L.gsvk_device_count.argtypes = [C.POINTER(C.c_int)]
        L.gsvk_parse_device.argtypes = [C.c_char_p, C.POINTER(C.c_int)]
        L.gsvk_model_load.argtypes = [C.c_char_p, i32, i32, C.POINTER(vp)]
        L.gsvk_bert_load.argtypes = [C.c_char_p, i32, i32, C.POINTER(vp)]
        L.gsvk_bert_free.argtypes = [vp]
        L.gsvk_bert_free.restype = None
        L.gsvk_bert_get_info.argtypes = [vp, C.POINTER(BertInfo)]
        L.gsvk_bert_encode.argtypes = [vp, i32, vp, vp, i32, i32, vp]
        L.gsvk_model_free.argtypes = [vp]
        L.gsvk_model_free.restype = None
        L.gsvk_model_get_info.argtypes = [vp, C.POINTER(ModelInfo)]
        L.gsvk_generate.argtypes = [vp, C.POINTER(Request), i32, C.POINTER(SamplerCfg), C.c_uint64, i32,
                                    i32, vp, i32, vp, C.c_uint, C.POINTER(GenOut)]
        L.gsvk_first_logits.argtypes = [vp, C.POINTER(Request), i32, vp]
        L.gsvk_release_cache.argtypes = [vp]
        L.gsvk_model_set_decode_path.argtypes = [vp, i32]
        L.gsvk_model_set_exact.argtypes = [vp, i32]
        L.gsvk_model_set_prefill_f16.argtypes = [vp, i32]
        L.gsvk_op_attn_exact.argtypes = [vp, vp, vp, i32, i32, i64, vp, vp, f32, vp, vp, vp, vp]
        L.gsvk_op_expf_exact.argtypes = [vp, i64, vp, vp]
        L.gsvk_op_dec_attn.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, i32, f32, i32, i32, vp, vp, vp, vp, vp,
                                       vp, i64, vp, vp, f32, vp, vp, vp, vp]
        L.gsvk_op_dec_ffn.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.gsvk_kv_alloc.argtypes = [vp, i32, i32]
        L.gsvk_prefill.argtypes = [vp, C.POINTER(Request), i32, vp, C.POINTER(C.c_int)]
        L.gsvk_decode_step.argtypes = [vp, vp, vp]
        L.gsvk_kv_read.argtypes = [vp, i32, vp, vp]
        L.gsvk_last_sampled.argtypes = [vp, i32, vp]
        L.gsvk_cb_open.argtypes = [vp, i32, i32, i32, i32, C.POINTER(SamplerCfg), i32, C.c_uint]
        L.gsvk_cb_add.argtypes = [vp, C.POINTER(Request), C.c_uint64, i32, C.POINTER(C.c_int)]
        L.gsvk_cb_step.argtypes = [vp, i32, C.POINTER(C.c_int)]
        L.gsvk_cb_take.argtypes = [vp, i32, vp, i32, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.gsvk_cb_close.argtypes = [vp]
        L.gsvk_op_q8_dequant.argtypes = [vp, i64, vp, vp]
        L.gsvk_op_q8_repack.argtypes = [vp, i64, i64, vp, vp, vp]
        L.gsvk_op_q8_quantize.argtypes = [vp, i64, i64, vp, vp, vp]
        L.gsvk_op_q8_gemv.argtypes = [vp, vp, i64, i64, vp, vp, i64, vp, i32, vp, vp]
        L.gsvk_op_layernorm.argtypes = [vp, vp, vp, vp, i64, i64, f32, vp, vp, vp, vp]
        L.gsvk_op_ln_gemv.argtypes = [vp, vp, i64, vp, vp, vp, vp, i64, vp, i32, vp, vp, vp]
        L.gsvk_op_add_act.argtypes = [vp, vp, i64, i64, i32, vp, vp]
        L.gsvk_op_fdot.argtypes = [vp, i32, i64, i64, vp, i64, vp, i32, vp]
        L.gsvk_attn_workspace_bytes.argtypes = [i32, i32, i64]
        L.gsvk_attn_workspace_bytes.restype = C.c_size_t
        L.gsvk_op_attn_decode.argtypes = [vp, vp, vp, i32, i32, i32, i64, vp, vp, i64, f32, vp, vp, vp,
                                          vp, vp, vp]
        L.gsvk_op_attn_decode_noalloc.argtypes = [vp, vp, vp, i32, i32, i32, i64, vp, vp, i64, f32, vp, vp,
                                                  vp, vp, vp]
        L.gsvk_op_qkv_attn.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, vp, vp, i64, vp, vp, f32, vp, vp,
                                       vp, vp, vp]
        L.gsvk_op_qkv_attn_exact.argtypes = L.gsvk_op_qkv_attn.argtypes
        L.gsvk_qkv_attn_supported.argtypes = [i32, i32, i64]
        L.gsvk_op_q8_gemm.argtypes = [vp, vp, i64, i64, vp, vp, i64, vp, i32, vp, vp]
        L.gsvk_op_q8_gemm_ex.argtypes = [vp, vp, i64, i64, vp, vp, i64, vp, i32, vp, vp, vp, i32, i32, vp]
        L.gsvk_op_q8_dequant_f16.argtypes = [vp, vp, i64, i64, vp, vp]
        L.gsvk_op_q8h_gemm.argtypes = [vp, i64, i64, vp, vp, i64, vp, i32, vp, vp, vp, vp]
        L.gsvk_op_attn_prefill.argtypes = [vp, i32, i32, i32, vp, i32, i32, f32, i32, vp, vp, vp, vp]
        L.gsvk_sample_workspace_bytes.argtypes = [i32]
        L.gsvk_sample_workspace_bytes.restype = C.c_size_t
        L.gsvk_op_sample.argtypes = [vp, i32, i32, vp, i32, vp, C.POINTER(SamplerCfg), vp, vp, vp, vp, vp]
        _lib = L
    return _lib


def last_error() -> str:
    return lib().gsvk_last_error().decode(errors="replace")


def check(rc: int, what: str = "gsvk call"):
    if rc != 0:
        raise GsvkError(f"{what} failed ({rc}): {last_error()}")


def device_count() -> int:
    n = C.c_int(0)
    check(lib().gsvk_device_count(C.byref(n)))
    return n.value


def parse_device(s: str) -> int:
    d = C.c_int(0)
    check(lib().gsvk_parse_device(s.encode(), C.byref(d)), "parse_device")
    return d.value


# ---- device ops on torch tensors ------------------------------------------------------------

def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def op_q8_dequant(blocks, out, stream=None):
    check(lib().gsvk_op_q8_dequant(_p(blocks), blocks.numel() // 34, _p(out), _stream(stream)), "q8_dequant")


def op_q8_repack(blocks, rows, k, qs, d, stream=None):
    check(lib().gsvk_op_q8_repack(_p(blocks), rows, k, _p(qs), _p(d), _stream(stream)), "q8_repack")


def op_q8_quantize(x, xq, xd, stream=None):
    rows, k = x.shape
    check(lib().gsvk_op_q8_quantize(_p(x), rows, k, _p(xq), _p(xd), _stream(stream)), "q8_quantize")


def op_q8_gemv(wq, wd, n, k, xq, xd, m, bias, act, y, stream=None):
    check(lib().gsvk_op_q8_gemv(_p(wq), _p(wd), n, k, _p(xq), _p(xd), m, _p(bias), act, _p(y),
                                _stream(stream)), "q8_gemv")


def op_q8_gemm(wq, wd, n, k, xq, xd, m, bias, act, y, stream=None):
    check(lib().gsvk_op_q8_gemm(_p(wq), _p(wd), n, k, _p(xq), _p(xd), m, _p(bias), act, _p(y), _stream(stream)),
          "q8_gemm")


def op_q8_gemm_ex(wq, wd, n, k, xq, xd, m, bias, act, y=None, yq=None, yd=None, tile_rows=0, tiled=False,
                  stream=None):
    check(lib().gsvk_op_q8_gemm_ex(_p(wq), _p(wd), n, k, _p(xq), _p(xd), m, _p(bias), act, _p(y), _p(yq),
                                   _p(yd), tile_rows, 1 if tiled else 0, _stream(stream)), "q8_gemm_ex")


def op_q8_dequant_f16(wq, wd, n, k, w16, stream=None):
    check(lib().gsvk_op_q8_dequant_f16(_p(wq), _p(wd), n, k, _p(w16), _stream(stream)), "q8_dequant_f16")


def op_q8h_gemm(w16, n, k, xq, xd, m, bias, act, y=None, yq=None, yd=None, stream=None):
    check(lib().gsvk_op_q8h_gemm(_p(w16), n, k, _p(xq), _p(xd), m, _p(bias), act, _p(y), _p(yq), _p(yd),
                                 _stream(stream)), "q8h_gemm")


def op_ln_gemv(wq, wd, n, res, r, ln_bias, wb, bias, act, y, ln_out=None, stream=None):
    m = res.shape[0]
    check(lib().gsvk_op_ln_gemv(_p(wq), _p(wd), n, _p(res), _p(r), _p(ln_bias), _p(wb), m, _p(bias), act,
                                _p(y), _p(ln_out), _stream(stream)), "ln_gemv")


def op_layernorm(x, r, bias, wb, eps, y, yq=None, yd=None, stream=None):
    rows, n = x.shape
    check(lib().gsvk_op_layernorm(_p(x), _p(r), _p(bias), _p(wb), rows, n, eps, _p(y), _p(yq), _p(yd),
                                  _stream(stream)), "layernorm")


def op_add_act(a, b, act, y, stream=None):
    check(lib().gsvk_op_add_act(_p(a), _p(b), a.numel(), b.numel(), act, _p(y), _stream(stream)), "add_act")


def op_fdot(w, wtype, x, y, mode, stream=None):
    n, k = w.shape
    check(lib().gsvk_op_fdot(_p(w), wtype, n, k, _p(x), x.shape[0], _p(y), mode, _stream(stream)), "fdot")


def attn_workspace_bytes(B, nh, max_keys) -> int:
    return int(lib().gsvk_attn_workspace_bytes(B, nh, max_keys))


def op_attn_decode(q, k, v, kv_begin, kv_end, max_keys, scale, out, out16=None, oq=None, od=None, ws=None,
                   stream=None):
    B, nh, hd = q.shape
    lstride = k.shape[2]
    check(lib().gsvk_op_attn_decode(_p(q), _p(k), _p(v), B, nh, hd, lstride, _p(kv_begin), _p(kv_end),
                                    max_keys, scale, _p(out), _p(out16), _p(oq), _p(od), _p(ws),
                                    _stream(stream)), "attn_decode")


def op_attn_decode_noalloc(q, k, v, kv_begin, kv_end, max_keys, scale, out, out16=None, oq=None, od=None,
                           stream=None):
    """op_attn_decode with its workspace in the library's own device array (no allocation)."""
    B, nh, hd = q.shape
    lstride = k.shape[2]
    check(lib().gsvk_op_attn_decode_noalloc(_p(q), _p(k), _p(v), B, nh, hd, lstride, _p(kv_begin),
                                            _p(kv_end), max_keys, scale, _p(out), _p(out16), _p(oq), _p(od),
                                            _stream(stream)), "attn_decode_noalloc")


def op_attn_exact(q, k, v, kv_begin, kv_end, scale, out, oq=None, od=None, stream=None):
    """Decode attention in ggml-cpu's sequential order (include/gsvk.h gsvk_op_attn_exact): q [B][nh][32]
    fp32, k, v [B][nh][lstride][32] fp16 (as int16 tensors)."""
    B, nh, hd = q.shape
    if hd != 32:
        raise ValueError("attn_exact: head_dim must be 32")
    lstride = k.shape[2]
    check(lib().gsvk_op_attn_exact(_p(q), _p(k), _p(v), B, nh, lstride, _p(kv_begin), _p(kv_end), scale, _p(out),
                                   _p(oq), _p(od), _stream(stream)), "attn_exact")


def op_expf_exact(x, y, stream=None):
    """y = expf(x) elementwise on the device with glibc's results (float32 tensors)."""
    check(lib().gsvk_op_expf_exact(_p(x), x.numel(), _p(y), _stream(stream)), "expf_exact")


def op_dec_attn(B, wq, wd, bqkv, k, v, kv_begin, col, scale, woq, wod, p1, x_out=None, res=None, parts=None,
                ln_bias=None, ln_wb=None, emb=None, pe=None, tok=None, pos=None, pos_add=0, alpha=1.0, vocab=0,
                pe_rows=0, stream=None):
    """Launch 1 of the two-launch decode layer (include/gsvk.h gsvk_op_dec_attn); k, v
    [B][16][lstride][32] fp16 (as int16 tensors)."""
    lstride = k.shape[2]
    check(lib().gsvk_op_dec_attn(B, _p(res), _p(parts), _p(ln_bias), _p(ln_wb), _p(emb), _p(pe), _p(tok), _p(pos),
                                 pos_add, alpha, vocab, pe_rows, _p(x_out), _p(wq), _p(wd), _p(bqkv), _p(k), _p(v),
                                 lstride, _p(kv_begin), _p(col), scale, _p(woq), _p(wod), _p(p1), _stream(stream)),
          "dec_attn")


def op_dec_ffn(B, res, p1, bo, ln1_wb, n1_out, w1q, w1d, b1, w2q, w2d, p2, stream=None):
    """Launch 2 of the two-launch decode layer (include/gsvk.h gsvk_op_dec_ffn)."""
    check(lib().gsvk_op_dec_ffn(B, _p(res), _p(p1), _p(bo), _p(ln1_wb), _p(n1_out), _p(w1q), _p(w1d), _p(b1), _p(w2q),
                                _p(w2d), _p(p2), _stream(stream)), "dec_ffn")


def op_attn_prefill(qkv, max_len, pad, nh, scale, out, oq=None, od=None, path=0, stream=None):
    """qkv [B][S][3*D] fp32, pad int32 [B] (device); out [B][S][D]; path 0 auto, 1 lane-per-query,
    2 matrix cores, 3 matrix cores with the weighted sum on fp16 operands (the fp16 prefill mode),
    4 matrix cores in the decoder prefill's dispatch (longest first, padding-only waves skipped)."""
    B, S, three_d = qkv.shape
    hd = three_d // 3 // nh
    check(lib().gsvk_op_attn_prefill(_p(qkv), B, S, max_len, _p(pad), nh, hd, scale, path, _p(out), _p(oq),
                                     _p(od), _stream(stream)), "attn_prefill")


def qkv_attn_supported(B, nh, max_keys) -> bool:
    return bool(lib().gsvk_qkv_attn_supported(B, nh, max_keys))


def op_qkv_attn(wq, wd, bias, res, r, ln_bias, wb, k, v, kv_begin, col, scale, out, oq=None, od=None,
                ln_out=None, stream=None, exact=False):
    """exact=True: gsvk_op_qkv_attn_exact (the attention in ggml-cpu's sequential order)."""
    B = res.shape[0]
    _, nh, lstride, _ = k.shape
    fn = lib().gsvk_op_qkv_attn_exact if exact else lib().gsvk_op_qkv_attn
    check(fn(_p(wq), _p(wd), _p(bias), _p(res), _p(r), _p(ln_bias), _p(wb), B, nh, _p(k), _p(v), lstride,
             _p(kv_begin), _p(col), scale, _p(out), _p(oq), _p(od), _p(ln_out), _stream(stream)), "qkv_attn")


def op_sample(logits, cfg, rng, tok_out, hist=None, n_hist=None, probs_out=None, ws=None, stream=None):
    """One device sampling call for logits [B][V]: cfg = (top_k, top_p, temperature, rep);
    rng [B] uint64 states (as int64 tensor) advanced in place; hist [B][stride] int32 with n_hist[b]
    tokens per row."""
    import torch
    B, V = logits.shape
    sc = SamplerCfg(int(cfg[0]), float(cfg[1]), float(cfg[2]), float(cfg[3]))
    if ws is None:
        ws = torch.empty(int(lib().gsvk_sample_workspace_bytes(V)), dtype=torch.uint8, device=logits.device)
    stride = hist.shape[1] if hist is not None else 0
    check(lib().gsvk_op_sample(_p(logits), B, V, _p(hist), stride, _p(n_hist), C.byref(sc), _p(rng), _p(tok_out),
                               _p(probs_out), _p(ws), _stream(stream)), "sample")


# ---- model ----------------------------------------------------------------------------------

def _requests(reqs):
    arr = (Request * len(reqs))()
    keep = []
    for i, r in enumerate(reqs):
        ph = np.ascontiguousarray(r["phones"], np.int32)
        pr = np.ascontiguousarray(r["prompt"], np.int32)
        be = None if r.get("bert") is None else np.ascontiguousarray(r["bert"], np.float32)
        keep += [ph, pr, be]
        arr[i].phones = ph.ctypes.data if ph.size else None
        arr[i].n_phones = ph.size
        arr[i].bert = None if be is None else be.ctypes.data
        arr[i].prompt = pr.ctypes.data if pr.size else None
        arr[i].n_prompt = pr.size
    return arr, keep


class Model:
    """A loaded AR model on one HIP device (mirror of the reference's gsv_ar)."""

    def __init__(self, path: str, device: int = 0, verbose: bool = False):
        h = C.c_void_p()
        check(lib().gsvk_model_load(path.encode(), device, int(verbose), C.byref(h)), "model_load")
        self.h = h
        self.info = self._info()

    def _info(self):
        info = ModelInfo()
        check(lib().gsvk_model_get_info(self.h, C.byref(info)), "model_get_info")
        return info

    def close(self):
        if getattr(self, "h", None):
            lib().gsvk_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def V(self):
        return self.info.vocab

    def first_logits(self, reqs):
        arr, keep = _requests(reqs)
        out = np.zeros((len(reqs), self.V), np.float32)
        check(lib().gsvk_first_logits(self.h, arr, len(reqs), out.ctypes.data), "first_logits")
        return out

    def prefill(self, reqs):
        arr, keep = _requests(reqs)
        out = np.zeros((len(reqs), self.V), np.float32)
        S = C.c_int(0)
        check(lib().gsvk_prefill(self.h, arr, len(reqs), out.ctypes.data, C.byref(S)), "prefill")
        return out, S.value

    def decode_step(self, last_tok):
        last_tok = np.ascontiguousarray(last_tok, np.int32)
        out = np.zeros((last_tok.size, self.V), np.float32)
        check(lib().gsvk_decode_step(self.h, last_tok.ctypes.data, out.ctypes.data), "decode_step")
        return out

    def kv_read(self, layer):
        info = self._info()
        shape = (info.kv_batch, info.n_head, info.kv_lmax + 1, info.head_dim)
        k = np.zeros(shape, np.uint16)
        v = np.zeros(shape, np.uint16)
        check(lib().gsvk_kv_read(self.h, layer, k.ctypes.data, v.ctypes.data), "kv_read")
        return k, v

    def release_cache(self):
        check(lib().gsvk_release_cache(self.h), "release_cache")

    def set_decode_path(self, path: int):
        """GSVK_DECODE_AUTO / _GEMV / _FUSED / _MFMA / _PERSIST (include/gsvk.h)."""
        check(lib().gsvk_model_set_decode_path(self.h, path), "set_decode_path")

    def set_prefill_f16(self, on: bool = True):
        """Prefill projections on the fp16 matrix cores (include/gsvk.h gsvk_model_set_prefill_f16)."""
        check(lib().gsvk_model_set_prefill_f16(self.h, 1 if on else 0), "set_prefill_f16")

    def profile(self):
        """The GSV_AR_PROFILE buckets of the last generate (include/gsvk.h gsvk_model_get_profile)."""
        pr = Profile()
        check(lib().gsvk_model_get_profile(self.h, C.byref(pr)), "get_profile")
        return {n: getattr(pr, n) for n, _ in Profile._fields_}

    def time_decode_kernel(self, launches: int = 50) -> float:
        """Mean duration (ms) of the persistent decode's kernel at the current step, HIP events
        around `launches` back-to-back launches (include/gsvk.h gsvk_model_time_decode_kernel)."""
        ms = C.c_float(0.0)
        check(lib().gsvk_model_time_decode_kernel(self.h, int(launches), C.byref(ms)), "time_decode_kernel")
        return float(ms.value)

    def set_exact(self, on: bool = True):
        """Exact mode (include/gsvk.h gsvk_model_set_exact): ggml-cpu's arithmetic order throughout."""
        check(lib().gsvk_model_set_exact(self.h, 1 if on else 0), "set_exact")

    # -- a batch that requests join and leave while it decodes (gsvk_cb_*) --
    def cb_open(self, capacity, max_prefill, max_steps, prompt_len, sampler=(15, 1.0, 1.0, 1.35), early_stop=-1,
                flags=0):
        cfg = SamplerCfg(*sampler)
        check(lib().gsvk_cb_open(self.h, capacity, max_prefill, max_steps, prompt_len, C.byref(cfg), early_stop,
                                 flags), "cb_open")
        self._cb_stride = prompt_len + max_steps

    def cb_add(self, req, seed, max_steps):
        arr, keep = _requests([req])
        slot = C.c_int(-1)
        check(lib().gsvk_cb_add(self.h, arr, seed, max_steps, C.byref(slot)), "cb_add")
        return slot.value

    def cb_step(self, n_steps):
        running = C.c_int(0)
        check(lib().gsvk_cb_step(self.h, n_steps, C.byref(running)), "cb_step")
        return running.value

    def cb_take(self, slot):
        """(finished, tokens, len) of the request in `slot`; a finished request leaves its row."""
        buf = np.zeros(self._cb_stride, np.int32)
        n, ln, fin = C.c_int(0), C.c_int(0), C.c_int(0)
        check(lib().gsvk_cb_take(self.h, slot, buf.ctypes.data, buf.size, C.byref(n), C.byref(ln), C.byref(fin)),
              "cb_take")
        return bool(fin.value), buf[:n.value].copy(), ln.value

    def cb_close(self):
        check(lib().gsvk_cb_close(self.h), "cb_close")

    def generate(self, reqs, sampler=(15, 1.0, 1.0, 1.35), seed_base=0, early_stop=-1, max_steps=1500,
                 oracle=None, seeds=None, flags=0, want_sampled=False, want_probs0=False):
        B = len(reqs)
        arr, keep = _requests(reqs)
        P = len(reqs[0]["prompt"])
        stride = P + max_steps
        tokens = np.zeros((B, stride), np.int32)
        tok_len = np.zeros(B, np.int32)
        lens = np.zeros(B, np.int32)
        fin = np.zeros(B, np.int32)
        probs0 = np.zeros((max(max_steps, 1), self.V), np.float32) if want_probs0 else None
        out = GenOut(tokens.ctypes.data, stride, tok_len.ctypes.data, lens.ctypes.data, fin.ctypes.data,
                     None if probs0 is None else probs0.ctypes.data, 0, PROGRESS_FN(0), None, 0.0, 0.0)
        cfg = SamplerCfg(*sampler)
        orc = None if oracle is None else np.ascontiguousarray(oracle, np.int32)
        sd = None if seeds is None else np.ascontiguousarray(seeds, np.uint64)
        if want_probs0:
            flags |= GSVK_GEN_PROB_DUMP
        check(lib().gsvk_generate(self.h, arr, B, C.byref(cfg), seed_base, early_stop, max_steps,
                                  None if orc is None else orc.ctypes.data, 0 if orc is None else orc.size,
                                  None if sd is None else sd.ctypes.data, flags, C.byref(out)), "generate")
        n = out.n_steps
        res = {"tokens": [tokens[b, :tok_len[b]].copy() for b in range(B)], "lens": lens.copy(),
               "finish_seq": fin.copy(), "n_steps": n, "prefill_ms": out.prefill_ms,
               "decode_ms": out.decode_ms}
        if want_sampled:
            s = np.zeros((max(n, 1), B), np.int32)
            check(lib().gsvk_last_sampled(self.h, n, s.ctypes.data), "last_sampled")
            res["sampled"] = s[:n]
        if want_probs0:
            res["probs0"] = probs0[:n]
        return res


class Bert:
    """A loaded BERT text encoder on one HIP device (mirror of the reference's gsv_bert)."""

    def __init__(self, path: str, device: int = 0, verbose: bool = False):
        h = C.c_void_p()
        check(lib().gsvk_bert_load(path.encode(), device, int(verbose), C.byref(h)), "bert_load")
        self.h = h
        info = BertInfo()
        check(lib().gsvk_bert_get_info(self.h, C.byref(info)), "bert_get_info")
        self.info = {k: getattr(info, k) for k, _ in BertInfo._fields_}

    def close(self):
        if self.h:
            lib().gsvk_bert_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, seqs, n_layers: int = -1, tmax: int = 0):
        """[hidden][T] float32 per sequence (token ids with [CLS]/[SEP]); all sequences in one
        call, each attending only to its own tokens."""
        lens = np.array([len(q) for q in seqs], np.int32)
        T = int(max(tmax, lens.max()))
        ids = np.zeros((len(seqs), T), np.int32)
        for b, q in enumerate(seqs):
            ids[b, :len(q)] = q
        D = self.info["hidden"]
        out = np.zeros(D * int(lens.sum()), np.float32)
        check(lib().gsvk_bert_encode(self.h, len(seqs), ids.ctypes.data, lens.ctypes.data, T, n_layers,
                                     out.ctypes.data), "bert_encode")
        res, off = [], 0
        for n in lens:
            res.append(out[off * D:(off + n) * D].reshape(D, n))
            off += int(n)
        return res

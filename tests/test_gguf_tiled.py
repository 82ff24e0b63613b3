"""The pre-swizzled GGUF (gsv.cpp_amd/gguf_tiled.py): the round trip to the Q8_0 block form is
byte-identical, the tiled tensors hold the documented order, and the loader checks the tiled
contract before touching a device. (The GPU side, tests/test_gpu_tiled.py: a model loaded from
either form computes the same bits.)"""
import struct

import numpy as np
import pytest

import gguf_tiled as GT
import gsvk
import synth_model as sm


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiled")
    src = sm.write_model(str(d / "ar.gguf"), n_layer=2)
    tiled = str(d / "ar.tiled.gguf")
    back = str(d / "ar.back.gguf")
    assert GT.main([src, tiled]) == 0
    assert GT.main(["--back", tiled, back]) == 0
    return {"src": src, "tiled": tiled, "back": back, "dir": d}


def test_round_trip_is_byte_identical(files):
    assert open(files["back"], "rb").read() == open(files["src"], "rb").read()


def test_tiled_tensors_hold_the_documented_order(files):
    src = {t["name"]: t for t in GT.read(files["src"]).tensors}
    til = GT.read(files["tiled"])
    names = [t["name"] for t in til.tensors]
    assert "transformer.block1.ffn2_w" not in names and "transformer.block1.ffn2_w.qt" in names
    assert "ar.predict" in names and "ar.text_emb" in names          # everything else unchanged
    assert dict(til.kvs)[GT.KEY_LAYOUT][-4:] == struct.pack("<I", 1)
    tt = {t["name"]: t for t in til.tensors}
    rng = np.random.default_rng(5)
    for base in ("transformer.block0.qkv_w", "transformer.block1.out_w", "transformer.block0.ffn2_w"):
        k, n = src[base]["ne"]
        nblk = k // 32
        blocks = np.frombuffer(src[base]["data"], np.uint8).reshape(n, nblk, 34)
        qt = np.frombuffer(tt[base + ".qt"]["data"], np.uint8)
        dt = np.frombuffer(tt[base + ".dt"]["data"], "<u2")
        assert tt[base + ".qt"]["ne"] == [k, n] and tt[base + ".dt"]["ne"] == [k // 32, n]
        for _ in range(200):
            r, blk, h = int(rng.integers(n)), int(rng.integers(nblk)), int(rng.integers(2))
            T, i = r // 32, r % 32
            chunk = (T * nblk + blk) * 1024 + (32 * h + i) * 16
            assert bytes(qt[chunk:chunk + 16]) == bytes(blocks[r, blk, 2 + 16 * h:2 + 16 * h + 16])
            assert int(dt[(T * nblk + blk) * 32 + i]) == int(blocks[r, blk, 0]) | (int(blocks[r, blk, 1]) << 8)


def test_tiling_twice_or_untiling_a_plain_file_is_refused(files):
    with pytest.raises(ValueError, match="already"):
        GT.tile(GT.read(files["tiled"]))
    with pytest.raises(ValueError, match="not pre-swizzled"):
        GT.untile(GT.read(files["src"]))


def _load_error(path):
    with pytest.raises(gsvk.GsvkError) as e:
        gsvk.Model(path)
    return str(e.value)


def test_loader_checks_the_tiled_contract_before_the_device(files):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present: the load would succeed")
    # a valid tiled file passes every check and fails only for want of a device (7)
    assert "(7)" in _load_error(files["tiled"])
    g = GT.read(files["tiled"])
    # a scale tensor missing
    g1 = GT.Gguf(g.version, g.kvs, g.alignment, [t for t in g.tensors if t["name"] != "transformer.block1.out_w.dt"])
    p1 = str(files["dir"] / "no_dt.gguf")
    GT.write(p1, g1)
    msg = _load_error(p1)
    assert "(4)" in msg and "transformer.block1.out_w.dt" in msg
    # quants stored with the wrong type
    g2 = GT.Gguf(g.version, g.kvs, g.alignment,
                 [dict(t, type=GT.GGML_F16, data=t["data"] * 2) if t["name"] == "transformer.block0.qkv_w.qt" else t
                  for t in g.tensors])
    p2 = str(files["dir"] / "bad_type.gguf")
    GT.write(p2, g2)
    msg = _load_error(p2)
    assert "(4)" in msg and "transformer.block0.qkv_w.qt" in msg
    # an unknown layout number
    kvs = [(k, raw[:-4] + struct.pack("<I", 7)) if k == GT.KEY_LAYOUT else (k, raw) for k, raw in g.kvs]
    p3 = str(files["dir"] / "layout7.gguf")
    GT.write(p3, GT.Gguf(g.version, kvs, g.alignment, g.tensors))
    msg = _load_error(p3)
    assert "(4)" in msg and "gsvk.q8_layout" in msg

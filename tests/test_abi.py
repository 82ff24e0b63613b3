"""CPU checks of the C ABI library: it loads, exports every entry point include/gsvk.h declares
and the gsv_ar class of include/gsv_ar.h, and its host-side logic (device strings, GGUF contract
validation, argument errors) behaves without a GPU."""
import os
import re
import subprocess

import numpy as np
import pytest

import gsvk
import synth_model as sm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsvk_\w+)\s*\(", text)))


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", gsvk.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_exports_every_declared_entry_point():
    declared = _declared("gsvk.h")
    exported = _exported()
    missing = [f for f in declared if f not in exported]
    assert not missing, missing
    assert sorted(gsvk.EXPORTS) == declared
    gsvk.lib()   # resolves every argtypes binding


def test_library_exports_the_gsv_ar_class():
    exported = _exported()
    for member in ("4load", "8generate", "12first_logits", "13release_cache", "10hidden_dim", "10vocab_size",
                   "3eos", "8bert_dim", "19prompt_len_expected"):
        assert any(f"6gsv_ar{member}" in s for s in exported), member
    assert any(s.startswith("_ZN6gsv_arD") for s in exported)   # destructor


def test_device_strings():
    assert gsvk.parse_device("") == 0
    assert gsvk.parse_device("gpu") == 0
    assert gsvk.parse_device("vulkan") == 0
    assert gsvk.parse_device("hip:2") == 2
    assert gsvk.parse_device("gpu:1") == 1
    assert gsvk.parse_device("3") == 3
    for bad in ("cpu", "CPU", "tpu"):
        with pytest.raises(gsvk.GsvkError):
            gsvk.parse_device(bad)


@pytest.fixture(scope="module")
def bad_models(tmp_path_factory):
    """Small files that break the GGUF contract in the ways src/gsv_ar.cpp:586, 632-637 reject."""
    d = tmp_path_factory.mktemp("bad")
    good = sm.write_model(str(d / "good.gguf"), n_layer=1)
    raw = open(good, "rb").read()
    out = {"good": good}
    # a missing tensor: rename one in the directory
    p = str(d / "missing.gguf")
    open(p, "wb").write(raw.replace(b"transformer.block0.norm2_b", b"transformer.block0.norm2_X"))
    out["missing"] = p
    # text embedding stored as F16 (the loader requires F32)
    p = str(d / "f16emb.gguf")
    import struct
    i = raw.find(b"ar.text_emb")
    j = i + len(b"ar.text_emb")
    nd = struct.unpack_from("<I", raw, j)[0]
    tpos = j + 4 + 8 * nd
    bad = bytearray(raw)
    struct.pack_into("<I", bad, tpos, 1)
    open(p, "wb").write(bytes(bad))
    out["f16emb"] = p
    p = str(d / "trunc.gguf")
    open(p, "wb").write(raw[: len(raw) // 3])
    out["trunc"] = p
    p = str(d / "notgguf.gguf")
    open(p, "wb").write(b"NOPE" + raw[4:100])
    out["notgguf"] = p
    return out


@pytest.mark.parametrize("case,code,needle", [
    ("missing", 4, "missing tensor transformer.block0.norm2_b"),
    ("f16emb", 4, "ar.text_emb"),
    ("trunc", 4, "extends past the end"),
    ("notgguf", 4, "not a GGUF file"),
])
def test_load_rejects_contract_violations(bad_models, case, code, needle):
    with pytest.raises(gsvk.GsvkError) as e:
        gsvk.Model(bad_models[case])
    assert f"({code})" in str(e.value) and needle in str(e.value)


def test_load_without_device_reports_nodev(bad_models):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    with pytest.raises(gsvk.GsvkError) as e:
        gsvk.Model(bad_models["good"])
    assert "(7)" in str(e.value)


def test_missing_file():
    with pytest.raises(gsvk.GsvkError) as e:
        gsvk.Model("/nonexistent/ar.gguf")
    assert "(3)" in str(e.value)


def test_op_argument_errors_need_no_device():
    # shape checks run on the host before any launch
    L = gsvk.lib()
    rc = L.gsvk_op_q8_gemv(None, None, 16, 100, None, None, 1, None, 0, None, None)
    assert rc == 1 and "null pointer" in gsvk.last_error()
    rc = L.gsvk_op_attn_decode(None, None, None, 1, 16, 64, 10, None, None, 10, 1.0, None, None, None, None,
                               None, None)
    assert rc == 1
    assert gsvk.attn_workspace_bytes(16, 16, 1000) > 0


def test_attn_noalloc_rejects_shapes_beyond_its_scratch():
    # 4096 x 16 rows of 4096 keys need 35 MB of split partials, more than the 8 MiB array; the
    # size check runs on the host before any device call
    L = gsvk.lib()
    assert gsvk.attn_workspace_bytes(4096, 16, 4096) > (8 << 20)
    rc = L.gsvk_op_attn_decode_noalloc(None, None, None, 4096, 16, 32, 4096, None, None, 4096, 1.0, None,
                                       None, None, None, None)
    assert rc == 1 and "scratch" in gsvk.last_error()


def test_phase_stamps_need_the_stamps_build():
    """gsvk_phase_stamps: the default library is built without the persistent decode's phase stamps
    and says so (GSVK_ERR_STATE, no device call); a buffer below 256 x 1024 values is refused."""
    import ctypes as C
    L = gsvk.lib()
    buf = np.zeros(256 * 1024, np.int64)
    assert L.gsvk_phase_stamps(C.c_void_p(buf.ctypes.data), C.c_size_t(buf.size)) == 6
    assert b"phase stamps" in L.gsvk_last_error()
    assert L.gsvk_phase_stamps(C.c_void_p(buf.ctypes.data), C.c_size_t(100)) == 1

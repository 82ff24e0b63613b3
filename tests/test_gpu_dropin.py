"""Drop-in check of the gsv_ar interface: the reference's own AR benchmark
(tests/bench_ar_width.cpp), compiled unchanged against include/gsv_ar.h and linked with
libgsvk.so (oracle/Makefile, target dropin), loads the model and runs teacher-forced batched
generation at B = 1, 2, 4, 8 on the GPU."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "bench_ar_width")

pytestmark = pytest.mark.gpu


def test_reference_caller_runs_unchanged(gpu, small_model_path):
    if not os.path.exists(BIN):
        pytest.skip("oracle/_ref/bench_ar_width was not built (the reference tree was absent at build time)")
    # device string "vulkan" is the reference's default; it selects HIP device 0 here
    p = subprocess.run([BIN, small_model_path, "vulkan", "48"], capture_output=True, text=True, timeout=180)
    print(p.stdout)
    assert p.returncode == 0, p.stderr
    assert "unexpected lens" not in p.stderr
    assert re.search(r"ar: D=512 V=1025 bert=1024 eos=1024", p.stdout)
    rows = [l.split() for l in p.stdout.splitlines() if re.match(r"^[1248]\s+\d", l)]
    assert [int(r[0]) for r in rows] == [1, 2, 4, 8]
    for r in rows:
        assert float(r[-1]) > 0.0   # tok/s

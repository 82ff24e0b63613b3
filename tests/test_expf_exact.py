"""The device exponential of exact mode (gsv.cpp_amd/csrc/expf_exact.h) against this host's libm
expf, the function the oracle's and ggml-cpu's flash-attention softmax call: compiled for the host
with g++ (FMA as on the reference's x86-64 build) and compared bit for bit on every third float
bit pattern (NaNs aside); the full sweep of all 2^32 patterns is the same program with step 1."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def expf_check(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("expf") / "expf_check")
    subprocess.run(["g++", "-std=c++17", "-O3", "-mfma", "-ffp-contract=off", "-pthread",
                    "-I" + os.path.join(ROOT, "gsv.cpp_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "expf_check.cpp"), "-o", exe, "-lm"], check=True)
    return exe


def test_expf_restatement_matches_libm(expf_check):
    r = subprocess.run([expf_check, "3"], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert r.stdout.startswith("checked 14")   # 4278190082 / 3 non-NaN patterns
    assert " 0 differ" in r.stdout


def test_oracle_expf_is_libm_on_known_values():
    """The oracle's elementwise expf: exact at 0, the known rounding of e, the limits (the largest
    float whose exponential is finite)."""
    x = np.array([0.0, -0.0, 1.0, -np.inf, np.inf, -200.0, 100.0, float.fromhex('0x1.62e42ep6')], np.float32)
    y = O.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.float32(np.e)
    assert y[3] == 0.0 and y[4] == np.inf and y[5] == 0.0 and y[6] == np.inf
    assert np.isfinite(y[7]) and y[7] > 3.4e38

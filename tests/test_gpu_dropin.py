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


def test_profile_buckets(gpu, small_model_path):
    """GSV_AR_PROFILE's buckets (src/gsv_ar.cpp:18-42): the reference caller prints the reference's
    three report lines, and the buckets of a generate add up: the prefill's device phases are
    positive, the decode's compute is the step loop's wall time, steps the steps that ran."""
    import synth_model as sm
    if os.path.exists(BIN):
        env = dict(os.environ, GSV_AR_PROFILE="1")
        p = subprocess.run([BIN, small_model_path, "vulkan", "16"], capture_output=True, text=True, timeout=180,
                           env=env)
        assert p.returncode == 0, p.stderr
        assert re.search(r"\[prof:decode\] prefill\(build/copy/compute/io\) = [\d.]+/[\d.]+/[\d.]+/[\d.]+ ms", p.stdout)
        assert re.search(r"\[prof:decode\] steps=\d+ build=[\d.]+ms copy=[\d.]+ms compute=[\d.]+ms other=[\d.]+ms", p.stdout)
        assert "[prof:decode] host per-step: mask=" in p.stdout
    g = gpu.Model(small_model_path)
    try:
        reqs = sm.synth_requests(77, 3, 16, [10, 20, 5])
        r = g.generate(reqs, sampler=(15, 1.0, 1.0, 1.35), max_steps=12, seeds=[1, 2, 3], flags=1)
        pr = g.profile()
    finally:
        g.close()
    assert pr["steps"] == r["n_steps"] == 12
    assert pr["pf_compute_ms"] > 0 and pr["pf_copy_ms"] >= 0 and pr["pf_io_ms"] >= 0 and pr["pf_build_ms"] >= 0
    assert pr["pf_copy_ms"] + pr["pf_compute_ms"] + pr["pf_io_ms"] <= r["prefill_ms"] + 1e-3
    assert abs(pr["dec_compute_ms"] - r["decode_ms"]) < 1e-9
    assert pr["dec_build_ms"] > 0 and pr["dec_copy_ms"] > 0 and pr["dec_other_ms"] > 0


def test_generate_ticks_the_engine_progress_counters(gpu, small_model_path):
    """gsv_ar::generate sets the engine's /progress counters (src/gsv_ar.cpp:761-763): stage 2 with
    the step budget as total, one tick per decode step, seen from the calling program (the
    counters are one object per process). tests/dropin/gsv_ar_progress_check.cpp, built by
    oracle/Makefile (target progresscheck)."""
    binp = os.path.join(ROOT, "tests", "dropin", "gsv_ar_progress_check")
    if not os.path.exists(binp):
        pytest.skip("tests/dropin/gsv_ar_progress_check was not built")
    p = subprocess.run([binp, small_model_path], capture_output=True, text=True, timeout=180)
    print(p.stdout, p.stderr)
    assert p.returncode == 0, p.stderr
    line = [l for l in p.stdout.splitlines() if l.startswith("progress ")]
    stage, cur, total, generated = (int(x) for x in line[0].split()[1:])
    assert stage == 2 and total == 17
    # every step that ran ticked once: the generated tokens, plus the step that chose EOS if any
    assert generated <= cur <= min(17, generated + 1)

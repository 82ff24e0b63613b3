"""The GEMV-chain decode step replayed on the CPU under AddressSanitizer (tests/native/hostemu).

The library's kernels (fused QKV + attention, the layer GEMVs, the F16 head with its LayerNorm
stage, the sampler) are compiled for the host with a stand-in HIP runtime that runs each
workgroup's threads as fibers and resolves barriers and wave exchanges with wave64 semantics.
Every buffer has the exact size the runtime allocates for the shape, so any access outside one is
reported with its kernel and line. The shape is the one whose GPU run faulted (batch 32, the
batch-16 request shape: prompts up to 400 rows, a cache for 500 steps, lstride = S + 509, the
first steps); a planted mistake (the K cache one step short for the last head) must be reported.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CXX = "/opt/rocm/llvm/bin/clang++"
EXE = os.path.join(ROOT, "_build", "hostemu", "decode_replay")

pytestmark = pytest.mark.skipif(not os.path.exists(CXX) or shutil.which("make") is None,
                                reason="needs the ROCm clang++ for the host build")


@pytest.fixture(scope="module")
def replay():
    r = subprocess.run(["make", "-s", "-j8", "-C", os.path.join(HERE, "native", "hostemu")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return EXE


def _run(exe, args, plant=False):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    if plant:
        env["EMU_PLANT"] = "1"
    return subprocess.run([exe] + [str(a) for a in args], capture_output=True, text=True, env=env, timeout=900)


def test_gemv_decode_batch32_in_bounds(replay):
    """Batch 32, step 7, layers 0 and 23 (the cache's first and last layer), the head and the
    next step's sampler: no access outside any buffer."""
    r = _run(replay, [32, 400, 500, 7, 0, 23])
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "replay done: no access outside the buffers" in r.stdout


def test_planted_cache_overflow_is_reported(replay):
    """The same replay with the K cache one step short for the last (sequence, head) pair of the
    last layer: AddressSanitizer reports the append of the fused QKV + attention kernel."""
    r = _run(replay, [32, 400, 500, 7, 23], plant=True)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr and "k_qkv_attn" in r.stderr, r.stderr[-4000:]


CHECK = os.path.join(ROOT, "_build", "hostemu", "exact_attn_check")


@pytest.mark.parametrize("args", [(3, 300, 40, 1), (4, 700, 650, 2), (5, 1200, 1100, 3)])
def test_exact_fused_kernel_equals_the_two_launches(replay, args):
    """Exact mode's fused decode kernel (QKV + K/V append + ggml-order attention in chunks of 256
    keys) against the QKV GEMV + one-wave exact attention it replaces, on the CPU under
    AddressSanitizer: outputs, Q8_0 copies and appended K/V equal to the bit, no access outside a
    buffer; rows of 1 key (only the new one) up to 1101 keys (5 chunks)."""
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    r = subprocess.run([CHECK] + [str(a) for a in args], capture_output=True, text=True, env=env, timeout=900)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "equal to the bit" in r.stdout

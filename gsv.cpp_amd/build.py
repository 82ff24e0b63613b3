"""Build the gfx950 library gsv.cpp_amd/lib/libgsvk.so (HIP kernels + C ABI + the gsv_ar class).

    python gsv.cpp_amd/build.py            # compile every source, link the library
    python gsv.cpp_amd/build.py --phase-stamps   # the same with the persistent decode's phase
                                                 # stamps (lib/libgsvk_stamps.so, for profiling)

Every HIP source is compiled for gfx950 only, without FMA contraction (the kernels write their
FMAs explicitly) and with packed FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(ROOT, "_build", "gsvk")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libgsvk.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", os.path.join(ROCM, "bin", "hipcc"))
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
DEVICE = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          # matrix-core results in ordinary VGPRs: the kernels scale or reduce them with vector
          # instructions right away, and the AGPR form would add a copy per value
          "-mllvm", "-amdgpu-mfma-vgpr-form=1"]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str, build_dir: str = BUILD, extra: tuple = ()) -> tuple[str, str]:
    obj = os.path.join(build_dir, src + ".o")
    cmd = [HIPCC] + COMMON + list(extra) + DEVICE + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC] + COMMON + ["-x", "c++", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{msg}")
    return obj, msg


def build(verbose: bool = False, phase_stamps: bool = False) -> str:
    build_dir = BUILD + ("_stamps" if phase_stamps else "")
    lib = os.path.join(LIB_DIR, "libgsvk_stamps.so") if phase_stamps else LIB
    extra = ("-DGSVK_PHASE_STAMPS",) if phase_stamps else ()
    os.makedirs(build_dir, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    objs = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        for obj, msg in ex.map(lambda f: _compile(f, build_dir, extra), srcs):
            objs.append(obj)
            if msg.strip() and verbose:
                print(msg, file=sys.stderr)
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True, phase_stamps="--phase-stamps" in sys.argv[1:]))

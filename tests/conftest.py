"""Shared test setup: import paths, the gpu marker, synthetic-model fixtures.

CPU tests (-m "not gpu") exercise the oracle against golden vectors and closed forms, the host
logic and the C ABI library's exports. GPU tests (-m gpu) are the parity tests proper: they call
the HIP library through its C ABI and compare with the oracle on the same seeded inputs.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "gsv.cpp_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

FIXTURE_DIR = os.environ.get("GSV_FIXTURE_DIR", os.path.join(ROOT, "_fixtures"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def small_model_path():
    """2-layer synthetic model (full width), F16 head."""
    import synth_model
    return synth_model.cached_model(FIXTURE_DIR, n_layer=2)


@pytest.fixture(scope="session")
def model4_path():
    """4-layer synthetic model, F16 head."""
    import synth_model
    return synth_model.cached_model(FIXTURE_DIR, n_layer=4)


@pytest.fixture(scope="session")
def model24_path():
    """The 24-layer synthetic model of the benchmark workloads, F16 head."""
    import synth_model
    return synth_model.cached_model(FIXTURE_DIR, n_layer=24)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import gsvk
    return gsvk

"""Shared pytest configuration: the `gpu` marker and import paths for the bindings and oracle."""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in (os.path.join(REPO, "scicompute-attention_amd", "python"), REPO,
            os.path.join(REPO, "tests")):
    if sub not in sys.path:
        sys.path.insert(0, sub)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def hip():
    """The kernel library; on a GPU test it must load and see a device (no fallback)."""
    import sca_amd

    lib = sca_amd.hip_lib()
    if not sca_amd.gpu_available():
        raise RuntimeError("GPU test started but no HIP device is visible")
    return lib

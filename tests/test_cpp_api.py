"""Runs the C++ API test program (tests/cpp/test_host_api.cpp, built into
scicompute-attention_amd/lib/test_host_api by the package build)."""

from __future__ import annotations

import os
import subprocess

import pytest

from sca_amd import hip as HIP

BINARY = os.path.join(HIP.LIB_DIR, "test_host_api")


def run(group: str, timeout: int) -> None:
    assert os.path.exists(BINARY), "build the package first (scicompute-attention_amd/build.py)"
    proc = subprocess.run([BINARY, group], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_cpp_api_cpu_cases():
    run("cpu", 120)


@pytest.mark.gpu
def test_cpp_api_gpu_cases(hip):
    run("gpu", 110)

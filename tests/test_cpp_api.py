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


@pytest.mark.gpu
def test_rollout_engine_example(hip, tmp_path):
    """The serving-loop example runs end to end through the public API on the GPU."""
    import json
    exe = os.path.join(HIP.LIB_DIR, "rollout_engine")
    if not os.path.exists(exe):
        pytest.fail("rollout_engine is not built (run scicompute-attention_amd/build.py)")
    out = tmp_path / "rollout.json"
    proc = subprocess.run([exe, "--requests", "8", "--max-new", "4", "--min-prompt", "64",
                           "--json", str(out)], capture_output=True, text=True, timeout=120)
    print(proc.stdout, proc.stderr, flush=True)
    assert proc.returncode == 0
    res = json.loads(out.read_text())
    assert res["generated_tokens"] == 32 and res["prefill_ms"] > 0
    assert res["decode_attend_gbps"] > 0

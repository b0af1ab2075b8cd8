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
    """The 36-layer serving-loop example runs end to end through the public API on the GPU, and
    its outputs match the FP64 oracle: sampled (layer, sequence) pairs of the prefill and of the
    first and last decode step, recomputed from the inputs the example fed that layer."""
    import json

    import numpy as np

    import oracle.oracle as orc
    from attn_util import check_attention, to_float

    exe = os.path.join(HIP.LIB_DIR, "rollout_engine")
    if not os.path.exists(exe):
        pytest.fail("rollout_engine is not built (run scicompute-attention_amd/build.py)")
    out = tmp_path / "rollout.json"
    dump = tmp_path / "dump"
    dump.mkdir()
    proc = subprocess.run([exe, "--requests", "8", "--max-new", "4", "--min-prompt", "64",
                           "--layers", "36", "--json", str(out), "--dump", str(dump)],
                          capture_output=True, text=True, timeout=120)
    print(proc.stdout, proc.stderr, flush=True)
    assert proc.returncode == 0
    res = json.loads(out.read_text())
    assert res["layers"] == 36 and res["generated_tokens"] == 32
    assert res["prefill_attention_ms"] > 0 and res["decode_attend_gbps"] > 0
    assert res["decode_tokens_per_s"] > 0
    man = json.loads((dump / "manifest.json").read_text())
    assert man["layers"] == [0, 18, 35] and man["seqs"] == [0, 1]
    arrays = man["arrays"]

    def load(tag):
        bits = np.fromfile(dump / f"{tag}.f16", dtype=np.uint16).reshape(arrays[tag])
        return to_float(bits, "f16")

    rng = np.random.default_rng(3)
    checked = 0
    for layer in man["layers"]:
        for seq in man["seqs"]:
            for phase in ("prefill", "decode0", f"decode{man['max_new'] - 1}"):
                tag = f"{phase}_l{layer}_s{seq}"
                q, k, v, o = (load(f"{tag}_{x}") for x in ("q", "k", "v", "out"))
                L, Hq, D = q.shape
                causal = phase == "prefill"
                # Prefill: 24 query positions (the last included) in every head; decode: all.
                pos = np.unique(np.append(rng.integers(0, L, size=24), L - 1)) if causal \
                    else np.arange(L)
                rows = (np.arange(Hq)[:, None] * L + pos[None, :]).reshape(-1)
                ref, _ = orc.reference_attention(q.transpose(1, 0, 2)[None],
                                                 k.transpose(1, 0, 2)[None],
                                                 v.transpose(1, 0, 2)[None], causal, rows=rows)
                got = o.transpose(1, 0, 2)[:, pos].reshape(-1, D)
                check_attention(got, ref, "f16", tag, abs_gate=True)
                checked += 1
    assert checked == 18

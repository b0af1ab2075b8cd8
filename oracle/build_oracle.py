"""Builds the CPU oracle (test infrastructure only).

  * ``oracle/_build/liboracle.so`` - the C restatement in sca_oracle.c (gcc, OpenMP)
  * ``oracle/_ref/libsca_ref.so``   - the reference's own host sources (CPU STUB mode), compiled
    directly from /root/reference with g++ plus the trace driver ref/ref_driver.cpp. Built only
    when /root/reference is present; the outputs never enter the repository history.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(ORACLE_DIR, "_build")
REF_OUT_DIR = os.path.join(ORACLE_DIR, "_ref")
REFERENCE = os.environ.get("SCA_REFERENCE_DIR", "/root/reference")

# Host translation units of the reference's CPU (STUB) build: src/CMakeLists.txt:6-45.
REF_SOURCES = [
    "api/status.cpp",
    "api/api_validate.cpp",
    "api/attention_api.cpp",
    "kv_cache/kv_cache.cpp",
    "kv_cache/block_manager.cpp",
    "kv_cache/paged_kv_cache.cpp",
    "runtime/capability.cpp",
    "runtime/workspace.cpp",
    "runtime/dispatcher.cpp",
    "runtime/backend_lookup.cpp",
    "runtime/scratch_pool.cpp",
    "backends/naive/naive_backend.cpp",
    "backends/tiled/tiled_backend.cpp",
    "backends/flash/flash_backend.cpp",
    "backends/decode/decode_backend.cpp",
    "backends/paged/paged_backend.cpp",
    "runtime/device_probe_stub.cpp",
    "kv_cache/kv_cache_kernels_stub.cpp",
    "backends/backends_stub.cpp",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError("oracle build failed: " + " ".join(cmd))


def build_oracle() -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    out = os.path.join(BUILD_DIR, "liboracle.so")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-Wall",
          os.path.join(ORACLE_DIR, "sca_oracle.c"), "-o", out, "-lm"])
    return out


def build_reference(workers: int = 8) -> str | None:
    src_root = os.path.join(REFERENCE, "src")
    if not os.path.isdir(src_root):
        return None
    os.makedirs(REF_OUT_DIR, exist_ok=True)
    flags = ["-std=c++20", "-O1", "-fPIC", "-w", "-DSCI_ATTENTION_INFRA_STUB=1",
             "-I" + os.path.join(REFERENCE, "include"), "-I" + src_root,
             "-I" + os.path.join(REFERENCE, "stub", "include")]
    jobs, objects = [], []
    for rel in REF_SOURCES + ["__driver__"]:
        if rel == "__driver__":
            src = os.path.join(ORACLE_DIR, "ref", "ref_driver.cpp")
            obj = os.path.join(REF_OUT_DIR, "ref_driver.o")
        else:
            src = os.path.join(src_root, rel)
            obj = os.path.join(REF_OUT_DIR, rel.replace("/", "_") + ".o")
        objects.append(obj)
        jobs.append(["g++", *flags, "-c", src, "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, j) for j in jobs]:
            fut.result()
    out = os.path.join(REF_OUT_DIR, "libsca_ref.so")
    _run(["g++", "-shared", "-fPIC", *objects, "-o", out, "-pthread"])
    for obj in objects:
        os.remove(obj)
    return out


if __name__ == "__main__":
    print(build_oracle())
    print(build_reference())

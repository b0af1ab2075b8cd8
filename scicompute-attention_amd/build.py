"""Builds the native libraries of the stack in-tree.

Outputs (all under ``scicompute-attention_amd/lib/``):
  * ``libsca_hip.so``  - gfx950 HIP kernels + their C ABI (include/sca_hip.h)
  * ``libsca_calib.so`` - calibration kernels timed by bench.py (not part of the library)
  * ``libsca_host.so`` - the C++ host layer (sca:: API, dispatcher, KV cache) + the ctypes-facing
    C ABI (include/sca_capi.h); links libsca_hip.so

Every HIP translation unit is compiled for gfx950 only, with packed-FP32 instructions disabled.
Object files are compiled in parallel; nothing is cached between calls.
"""

from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
SRC_DIR = os.path.join(PKG_DIR, "src")
LIB_DIR = os.path.join(PKG_DIR, "lib")
OBJ_DIR = os.path.join(PKG_DIR, "_build")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
CXX = os.environ.get("CXX", "g++")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms are kept out of every code object.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE_DIR,
    "-I" + CSRC_DIR,
]

# Per-file additions. The flash kernel never produces NaN from finite inputs (masked logits are
# -inf, fully masked rows are handled explicitly), so NaN-preserving max operations are not needed.
FILE_FLAGS = {"flash_fwd.hip": ["-fno-honor-nans"]}

HOST_FLAGS = [
    "-std=c++20",
    "-O2",
    "-fPIC",
    "-Wall",
    "-Wextra",
    "-Wno-unused-parameter",
    "-fvisibility=hidden",
    "-I" + INCLUDE_DIR,
    "-I" + SRC_DIR,
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that is expected.
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError("build step failed: " + " ".join(cmd))
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def _compile_all(jobs: list[list[str]], workers: int) -> None:
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, job) for job in jobs]:
            fut.result()


def build_hip(workers: int) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))
    objects = []
    jobs = []
    for src in sources:
        obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
        objects.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o",
                     obj])
    _compile_all(jobs, workers)
    out = os.path.join(LIB_DIR, "libsca_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", *objects, "-o",
          tmp])
    os.replace(tmp, out)
    return out


def build_host(workers: int) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(SRC_DIR, "**", "*.cpp"), recursive=True))
    objects = []
    jobs = []
    for src in sources:
        rel = os.path.relpath(src, SRC_DIR).replace(os.sep, "_")
        obj = os.path.join(OBJ_DIR, "host_" + rel + ".o")
        objects.append(obj)
        jobs.append([CXX, *HOST_FLAGS, "-c", src, "-o", obj])
    _compile_all(jobs, workers)
    out = os.path.join(LIB_DIR, "libsca_host.so")
    tmp = out + ".tmp"
    _run([CXX, "-shared", "-fPIC", *objects, "-o", tmp, "-L" + LIB_DIR, "-lsca_hip",
          "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined", "-pthread"])
    os.replace(tmp, out)
    return out


def build_cpp_tests() -> str:
    """The C++ API test program (tests/cpp/test_host_api.cpp), linked against libsca_host.so."""
    src = os.path.join(REPO_DIR, "tests", "cpp", "test_host_api.cpp")
    out = os.path.join(LIB_DIR, "test_host_api")
    tmp = out + ".tmp"
    _run([CXX, "-std=c++20", "-O1", "-Wall", "-I" + INCLUDE_DIR, src, "-o", tmp, "-L" + LIB_DIR,
          "-lsca_host", "-lsca_hip", "-Wl,-rpath,$ORIGIN", "-pthread"])
    os.replace(tmp, out)
    return out


def build_examples() -> list[str]:
    """Example programs (examples/*.cpp), linked against libsca_host.so."""
    outs = []
    for src in sorted(glob.glob(os.path.join(PKG_DIR, "examples", "*.cpp"))):
        out = os.path.join(LIB_DIR, os.path.splitext(os.path.basename(src))[0])
        tmp = out + ".tmp"
        _run([CXX, "-std=c++20", "-O2", "-Wall", "-I" + INCLUDE_DIR, src, "-o", tmp, "-L" + LIB_DIR,
              "-lsca_host", "-lsca_hip", "-Wl,-rpath,$ORIGIN", "-pthread"])
        os.replace(tmp, out)
        outs.append(out)
    return outs


def build_calib() -> str:
    """Calibration kernels for bench.py (calib/*.hip) in lib/libsca_calib.so; not part of the
    attention library."""
    out = os.path.join(LIB_DIR, "libsca_calib.so")
    tmp = out + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", *sorted(glob.glob(os.path.join(PKG_DIR, "calib", "*.hip"))),
          "-o", tmp])
    os.replace(tmp, out)
    return out


def build(workers: int | None = None) -> list[str]:
    workers = workers or min(8, os.cpu_count() or 4)
    if os.path.isdir(OBJ_DIR):
        shutil.rmtree(OBJ_DIR)
    outputs = [build_hip(workers), build_calib()]
    if glob.glob(os.path.join(SRC_DIR, "**", "*.cpp"), recursive=True):
        outputs.append(build_host(workers))
        if os.path.exists(os.path.join(REPO_DIR, "tests", "cpp", "test_host_api.cpp")):
            outputs.append(build_cpp_tests())
        outputs.extend(build_examples())
    return outputs


if __name__ == "__main__":
    for path in build():
        print(path)

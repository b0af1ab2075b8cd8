"""The C-ABI libraries load and export every function their headers declare (no GPU calls)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

import sca_amd
from sca_amd import hip as HIP
from sca_amd import host as H

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")

HEADERS = {
    "sca_hip.h": ("SCA_HIP_API", "libsca_hip.so"),
    "sca_capi.h": ("SCA_CAPI", "libsca_host.so"),
}


def declared(header: str, macro: str) -> list[str]:
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = "\n".join(ln for ln in text.splitlines() if not ln.lstrip().startswith("#"))
    names = re.findall(rf"{macro}\s+[^;(]*?\b(\w+)\s*\(", text)
    return sorted(set(names))


def exported(lib: str) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(HIP.LIB_DIR, lib)],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_every_declared_symbol_is_exported(header):
    macro, lib = HEADERS[header]
    names = declared(header, macro)
    assert len(names) > 20, names
    missing = [n for n in names if n not in exported(lib)]
    assert not missing, f"{lib} lacks {missing}"


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_every_declared_symbol_resolves_through_ctypes(header):
    macro, _ = HEADERS[header]
    lib = HIP.hip_lib() if header == "sca_hip.h" else H.host_lib()
    for name in declared(header, macro):
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_libraries_are_gfx950_only_and_fail_loudly_when_missing(tmp_path, monkeypatch):
    # The kernel library carries gfx950 code objects and no other target.
    out = subprocess.run(["strings", os.path.join(HIP.LIB_DIR, "libsca_hip.so")],
                         capture_output=True, text=True).stdout
    assert "gfx950" in out
    assert not re.search(r"gfx9[0-4]\d\b|gfx1\d{3}\b", out)
    # With the library directory pointing nowhere, loading raises instead of falling back.
    monkeypatch.setattr(HIP, "LIB_DIR", str(tmp_path))
    monkeypatch.setattr(HIP, "_LIB", None, raising=False)
    with pytest.raises(Exception):
        HIP.hip_lib()


def test_host_library_metadata_without_gpu():
    assert H.host_lib().sca_version().decode() == "0.1.0"
    assert H.host_lib().sca_build_flavor().decode() == "mi355x-hip-gfx950"
    assert sca_amd.hip_lib().sca_hip_last_error_string() is not None

"""ctypes bindings of the MI355X attention stack.

Two native libraries are loaded from ``scicompute-attention_amd/lib`` (built in-tree by
``scicompute-attention_amd/build.py``):

* ``libsca_hip.so``  - gfx950 kernels behind the C ABI of ``include/sca_hip.h``;
* ``libsca_host.so`` - the C++ host layer (sca:: API, dispatcher, KV cache) behind the C ABI of
  ``include/sca_capi.h``.

There is no fallback: if a library is missing, importing the corresponding binding raises.
Device memory is managed through the C ABI (``DeviceBuffer``); host data is numpy.
"""

from __future__ import annotations

from .hip import (  # noqa: F401
    HipError,
    DeviceBuffer,
    Event,
    FlashParams,
    DecodeParams,
    KvShape,
    DTYPE_F32,
    DTYPE_F16,
    DTYPE_BF16,
    hip_lib,
    gpu_available,
    device_probe,
    synchronize,
)

from . import host  # noqa: E402,F401  (libsca_host.so is loaded lazily by host.host_lib())

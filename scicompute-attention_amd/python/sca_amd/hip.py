"""ctypes binding of ``libsca_hip.so`` (include/sca_hip.h)."""

from __future__ import annotations

import ctypes
import os

import numpy as np

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
# SCA_LIB_DIR points the bindings at another build of the same libraries (measurement only).
LIB_DIR = os.environ.get("SCA_LIB_DIR") or os.path.join(PKG_ROOT, "lib")

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
COPY_H2D, COPY_D2H, COPY_D2D = 1, 2, 3

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p


class HipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class DeviceProbe(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch_name", ctypes.c_char * 64),
        ("major", ctypes.c_int),
        ("minor", ctypes.c_int),
        ("cu_count", ctypes.c_int),
        ("wave_size", ctypes.c_int),
        ("clock_khz", ctypes.c_int),
        ("memory_clock_khz", ctypes.c_int),
        ("memory_bus_width_bits", ctypes.c_int),
        ("lds_per_cu", ctypes.c_ulonglong),
        ("lds_per_block", ctypes.c_ulonglong),
        ("regs_per_cu", ctypes.c_ulonglong),
        ("max_threads_per_cu", ctypes.c_ulonglong),
        ("l2_bytes", ctypes.c_ulonglong),
        ("total_mem_bytes", ctypes.c_ulonglong),
        ("free_mem_bytes", ctypes.c_ulonglong),
        ("gpu_available", ctypes.c_int),
        ("binary_has_gfx950", ctypes.c_int),
    ]


class FlashParams(ctypes.Structure):
    _fields_ = [
        ("q", c_vp), ("k", c_vp), ("v", c_vp), ("out", c_vp), ("lse", c_vp),
        ("batch", c_i64), ("num_heads", c_i64), ("num_kv_heads", c_i64),
        ("seq_q", c_i64), ("seq_kv", c_i64), ("head_dim", c_i64),
        ("q_sb", c_i64), ("q_sh", c_i64), ("q_ss", c_i64),
        ("k_sb", c_i64), ("k_sh", c_i64), ("k_ss", c_i64),
        ("v_sb", c_i64), ("v_sh", c_i64), ("v_ss", c_i64),
        ("o_sb", c_i64), ("o_sh", c_i64), ("o_ss", c_i64),
        ("scale", ctypes.c_float), ("causal", c_i32), ("dtype", c_i32),
        ("diagonal", c_i64),
    ]


class FlashVarlenParams(ctypes.Structure):
    _fields_ = [
        ("q", c_vp), ("k", c_vp), ("v", c_vp), ("out", c_vp),
        ("cu_seqlens_q", c_vp), ("cu_seqlens_kv", c_vp), ("tiles", c_vp),
        ("num_seqs", c_i64), ("num_tiles", c_i64), ("max_seq_kv", c_i64),
        ("num_heads", c_i64), ("num_kv_heads", c_i64), ("head_dim", c_i64),
        ("q_sh", c_i64), ("q_ss", c_i64), ("k_sh", c_i64), ("k_ss", c_i64),
        ("v_sh", c_i64), ("v_ss", c_i64), ("o_sh", c_i64), ("o_ss", c_i64),
        ("scale", ctypes.c_float), ("causal", c_i32), ("dtype", c_i32),
    ]


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("q", c_vp), ("k", c_vp), ("v", c_vp), ("out", c_vp),
        ("partial_m", c_vp), ("partial_l", c_vp), ("partial_o", c_vp),
        ("batch", c_i64), ("num_heads", c_i64), ("num_kv_heads", c_i64),
        ("seq_kv", c_i64), ("head_dim", c_i64), ("num_splits", c_i64),
        ("q_sb", c_i64), ("q_sh", c_i64),
        ("k_sb", c_i64), ("k_sh", c_i64), ("k_ss", c_i64),
        ("v_sb", c_i64), ("v_sh", c_i64), ("v_ss", c_i64),
        ("o_sb", c_i64), ("o_sh", c_i64),
        ("scale", ctypes.c_float), ("dtype", c_i32),
        ("page_table", c_vp), ("block_size", c_i64), ("max_blocks_per_seq", c_i64),
        ("num_kv_blocks", c_i64), ("seq_lens", c_vp), ("batch_order", c_vp),
        ("slot_waves", c_i32),
    ]


class KvShape(ctypes.Structure):
    _fields_ = [("num_blocks", c_i64), ("block_size", c_i64), ("num_kv_heads", c_i64),
                ("head_dim", c_i64)]


_LIB = None


def hip_lib() -> ctypes.CDLL:
    """Loads libsca_hip.so (raises if it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = os.path.join(LIB_DIR, "libsca_hip.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run scicompute-attention_amd/build.py first")
    lib = ctypes.CDLL(path)
    lib.sca_hip_last_error_string.restype = ctypes.c_char_p
    lib.sca_hip_probe_device.argtypes = [ctypes.c_int, ctypes.POINTER(DeviceProbe)]
    lib.sca_hip_mem_get_info.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)] * 2
    lib.sca_hip_get_device_count.argtypes = [ctypes.POINTER(ctypes.c_int)]
    lib.sca_hip_malloc.argtypes = [ctypes.POINTER(c_vp), ctypes.c_size_t]
    lib.sca_hip_free.argtypes = [c_vp]
    lib.sca_hip_memcpy.argtypes = [c_vp, c_vp, ctypes.c_size_t, ctypes.c_int]
    lib.sca_hip_memcpy_async.argtypes = [c_vp, c_vp, ctypes.c_size_t, ctypes.c_int, c_vp]
    lib.sca_hip_zero_async.argtypes = [c_vp, ctypes.c_size_t, c_vp]
    lib.sca_hip_stream_create.argtypes = [ctypes.POINTER(c_vp)]
    lib.sca_hip_stream_destroy.argtypes = [c_vp]
    lib.sca_hip_stream_synchronize.argtypes = [c_vp]
    lib.sca_hip_event_create.argtypes = [ctypes.POINTER(c_vp)]
    lib.sca_hip_event_destroy.argtypes = [c_vp]
    lib.sca_hip_event_record.argtypes = [c_vp, c_vp]
    lib.sca_hip_event_synchronize.argtypes = [c_vp]
    lib.sca_hip_event_elapsed_ms.argtypes = [ctypes.POINTER(ctypes.c_float), c_vp, c_vp]
    lib.sca_hip_flash_lds_bytes.argtypes = [c_i32, c_i64]
    lib.sca_hip_flash_lds_bytes.restype = c_i64
    lib.sca_hip_flash_tile.argtypes = [c_i32] + [ctypes.POINTER(c_i32)] * 4
    lib.sca_hip_flash_fwd.argtypes = [ctypes.POINTER(FlashParams), c_vp]
    lib.sca_hip_flash_varlen_tiles.argtypes = [c_vp, c_vp, c_i64, c_i32, c_vp]
    lib.sca_hip_flash_varlen_tiles.restype = c_i64
    lib.sca_hip_flash_varlen_supported.argtypes = [c_i32]
    lib.sca_hip_flash_fwd_varlen.argtypes = [ctypes.POINTER(FlashVarlenParams), c_vp]
    lib.sca_hip_decode_partial_elements.argtypes = [c_i64] * 4
    lib.sca_hip_decode_partial_elements.restype = c_i64
    lib.sca_hip_decode_splitk.argtypes = [ctypes.POINTER(DecodeParams), c_vp]
    lib.sca_hip_decode_splitk_paged.argtypes = [ctypes.POINTER(DecodeParams), c_vp]
    lib.sca_hip_decode_splitk_noalloc.argtypes = [ctypes.POINTER(DecodeParams), c_vp]
    lib.sca_hip_kv_append.argtypes = [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64,
                                      ctypes.POINTER(KvShape), c_i64, c_vp]
    lib.sca_hip_kv_reset_blocks.argtypes = [c_vp, c_vp, c_vp, c_i64, ctypes.POINTER(KvShape),
                                            c_i64, c_vp]
    lib.sca_hip_kv_gather.argtypes = [c_vp, c_vp, c_i64, c_vp, ctypes.POINTER(KvShape), c_i64,
                                      c_vp]
    _LIB = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        raise HipError(rc, hip_lib().sca_hip_last_error_string().decode())


def device_probe(device: int = 0) -> DeviceProbe:
    out = DeviceProbe()
    check(hip_lib().sca_hip_probe_device(device, ctypes.byref(out)))
    return out


def gpu_available() -> bool:
    n = ctypes.c_int(0)
    check(hip_lib().sca_hip_get_device_count(ctypes.byref(n)))
    return n.value > 0


def synchronize() -> None:
    check(hip_lib().sca_hip_device_synchronize())


class DeviceBuffer:
    """An owning device allocation made through sca_hip_malloc."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = c_vp()
        check(hip_lib().sca_hip_malloc(ctypes.byref(ptr), max(self.nbytes, 1)))
        self.ptr = ptr.value

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    @classmethod
    def zeros(cls, nbytes: int) -> "DeviceBuffer":
        buf = cls(nbytes)
        check(hip_lib().sca_hip_zero_async(buf.ptr, max(buf.nbytes, 1), None))
        return buf

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        check(hip_lib().sca_hip_memcpy(self.ptr, arr.ctypes.data, arr.nbytes, COPY_H2D))

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dtype)
        if n:
            check(hip_lib().sca_hip_memcpy(out.ctypes.data, self.ptr, out.nbytes, COPY_D2H))
        return out

    def free(self) -> None:
        if self.ptr:
            check(hip_lib().sca_hip_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                hip_lib().sca_hip_free(self.ptr)
                self.ptr = None
        except Exception:
            pass


class Event:
    def __init__(self):
        ev = c_vp()
        check(hip_lib().sca_hip_event_create(ctypes.byref(ev)))
        self.ev = ev.value

    def record(self, stream=None) -> None:
        check(hip_lib().sca_hip_event_record(self.ev, stream))

    def synchronize(self) -> None:
        check(hip_lib().sca_hip_event_synchronize(self.ev))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        check(hip_lib().sca_hip_event_elapsed_ms(ctypes.byref(ms), self.ev, end.ev))
        return float(ms.value)

    def __del__(self):
        try:
            hip_lib().sca_hip_event_destroy(self.ev)
        except Exception:
            pass


def flash_fwd(params: FlashParams, stream=None) -> None:
    check(hip_lib().sca_hip_flash_fwd(ctypes.byref(params), stream))


def flash_varlen_tiles(cu_q: np.ndarray, cu_kv: np.ndarray, causal: bool) -> np.ndarray:
    """Work list (rows of (sequence, row tile), longest first) for a packed launch."""
    cu_q = np.ascontiguousarray(cu_q, np.int32)
    cu_kv = np.ascontiguousarray(cu_kv, np.int32)
    lib = hip_lib()
    n = lib.sca_hip_flash_varlen_tiles(cu_q.ctypes.data, cu_kv.ctypes.data, len(cu_q) - 1,
                                       int(causal), None)
    if n < 0:
        check(int(-n))
    out = np.zeros(2 * n, np.int32)
    lib.sca_hip_flash_varlen_tiles(cu_q.ctypes.data, cu_kv.ctypes.data, len(cu_q) - 1,
                                   int(causal), out.ctypes.data)
    return out.reshape(n, 2)


def flash_fwd_varlen(params: FlashVarlenParams, stream=None) -> None:
    check(hip_lib().sca_hip_flash_fwd_varlen(ctypes.byref(params), stream))


def decode_splitk(params: DecodeParams, stream=None) -> None:
    check(hip_lib().sca_hip_decode_splitk(ctypes.byref(params), stream))


def decode_splitk_paged(params: DecodeParams, stream=None) -> None:
    check(hip_lib().sca_hip_decode_splitk_paged(ctypes.byref(params), stream))


def decode_splitk_noalloc(params: DecodeParams, stream=None) -> None:
    """The allocation-free decode entry point: partial_m/l/o and batch_order must be None."""
    check(hip_lib().sca_hip_decode_splitk_noalloc(ctypes.byref(params), stream))

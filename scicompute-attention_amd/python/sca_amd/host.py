"""ctypes binding of ``libsca_host.so`` (include/sca_capi.h): the sca:: C++ API from Python.

Names follow the reference's C++ API (``attention``, ``flash_attention``, ``decode_attention``,
``paged_attention``, ``AttentionDispatcher.select/explain``, ``BlockManager``, ``PagedKVCache``,
``Workspace`` ...). Failures raise ``ScaError`` whose ``code`` is the attention status code
(2001..2010) and whose message is the library's "[SCA-<code>] ..." text.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os

import numpy as np

from . import hip as _hip

c_i64, c_i32, c_u64, c_vp, c_f = ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_float
c_char_p = ctypes.c_char_p

BACKENDS = {"auto": 0, "naive": 1, "tiled": 2, "flash": 3, "decode": 4, "paged": 5}
LAYOUTS = {"bhsd": 0, "bshd": 1}
DTYPES = {"f32": 0, "f16": 1, "bf16": 2, "i32": 4, "u8": 8}
ELEM = {"f32": 4, "f16": 2, "bf16": 2, "i32": 4, "u8": 1}
HOST, GPU = 0, 1


class ScaError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code
        self.message = message


class ScaConfig(ctypes.Structure):
    _fields_ = [
        ("backend", c_i32), ("layout", c_i32), ("causal", c_i32), ("return_lse", c_i32),
        ("scale", c_f), ("softcap", c_f), ("sliding_window", c_i64), ("num_splits", c_i64),
        ("allow_fallback", c_i32), ("reserved", c_i32),
        ("cu_seqlens_q", c_vp), ("cu_seqlens_kv", c_vp), ("stream", c_vp),
    ]


class ScaShape(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seq_q", c_i64), ("seq_kv", c_i64), ("num_heads", c_i64),
                ("num_kv_heads", c_i64), ("head_dim", c_i64)]


class ScaKvConfig(ctypes.Structure):
    _fields_ = [("num_layers", c_i64), ("num_kv_heads", c_i64), ("head_dim", c_i64),
                ("block_size", c_i64), ("num_blocks", c_i64), ("max_num_seqs", c_i64),
                ("dtype", c_i32), ("layout", c_i32)]


class ScaStats(ctypes.Structure):
    _fields_ = [("used_backend", c_i32), ("tile", c_i32 * 4), ("workspace_bytes", c_u64),
                ("kv_bytes", c_u64), ("num_splits", c_i64), ("materialized_score_bytes", c_i64),
                ("note", ctypes.c_char * 256)]


class ScaKvStats(ctypes.Structure):
    _fields_ = [("num_blocks", c_i64), ("used_blocks", c_i64), ("free_blocks", c_i64),
                ("num_appends", c_i64), ("num_resets", c_i64), ("peak_bytes", c_u64),
                ("bytes", c_u64)]


class ScaPagedParams(ctypes.Structure):
    _fields_ = [("page_table", c_vp), ("seq_lens", c_vp), ("num_seqs", c_i64),
                ("block_size", c_i64), ("max_blocks_per_seq", c_i64), ("layer", c_i64)]


_LIB = None

# (name, restype, argtypes)
_SIGS = [
    ("sca_last_error", c_char_p, []),
    ("sca_version", c_char_p, []),
    ("sca_build_flavor", c_char_p, []),
    ("sca_status_name", c_char_p, [ctypes.c_int]),
    ("sca_to_sci_code", ctypes.c_int, [ctypes.c_int]),
    ("sca_make_status", ctypes.c_int, [ctypes.c_int, c_char_p, c_char_p, ctypes.c_size_t]),
    ("sca_extract_code", ctypes.c_int, [c_char_p]),
    ("sca_backend_name", c_char_p, [ctypes.c_int]),
    ("sca_layout_name", c_char_p, [ctypes.c_int]),
    ("sca_parse_backend", ctypes.c_int, [c_char_p, ctypes.POINTER(c_i32)]),
    ("sca_supported_head_dim_index", ctypes.c_int, [c_i64]),
    ("sca_tile_smem_bytes_flash", c_i64, [c_i32, c_i64, c_i32, c_i32, c_i32, c_i32]),
    ("sca_flash_lds_bytes", c_i64, [c_i64, c_i64]),
    ("sca_validate", ctypes.c_int, [ctypes.POINTER(ScaConfig), ctypes.POINTER(ScaShape), c_char_p,
                                    ctypes.c_size_t]),
    ("sca_effective_scale", c_f, [ctypes.POINTER(ScaConfig), ctypes.POINTER(ScaShape)]),
    ("sca_validate_varlen", ctypes.c_int, [c_vp, c_i64, ctypes.POINTER(c_i64)]),
    ("sca_select", ctypes.c_int, [ctypes.POINTER(ScaConfig), ctypes.POINTER(ScaShape),
                                  ctypes.POINTER(c_i32), c_i32 * 4, ctypes.POINTER(c_u64),
                                  c_char_p, ctypes.c_size_t]),
    ("sca_explain", None, [ctypes.POINTER(ScaConfig), ctypes.POINTER(ScaShape), c_char_p,
                           ctypes.c_size_t]),
    ("sca_recommend_tile", None, [ctypes.POINTER(ScaConfig), ctypes.POINTER(ScaShape), c_i32 * 4]),
    ("sca_decode_splits", c_i64, [ctypes.POINTER(ScaShape), c_i64]),
    ("sca_paged_decode_plan", ctypes.c_int, [c_vp, c_i64, c_i64, c_i64, c_i64,
                                              ctypes.POINTER(c_i64), ctypes.POINTER(c_i32)]),
    ("sca_compute_slot_mapping", ctypes.c_int, [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    ("sca_kv_cache_bytes", ctypes.c_int, [ctypes.POINTER(ScaKvConfig), ctypes.POINTER(c_u64)]),
    ("sca_max_blocks_for_budget", c_i64, [ctypes.POINTER(ScaKvConfig), c_u64]),
    ("sca_tensor_new", c_vp, [ctypes.POINTER(c_i64), c_i32, c_i32, c_i32]),
    ("sca_tensor_wrap", c_vp, [c_vp, ctypes.POINTER(c_i64), c_i32, c_i32, c_i32]),
    ("sca_tensor_free", None, [c_vp]),
    ("sca_tensor_data", c_vp, [c_vp]),
    ("sca_tensor_nbytes", c_u64, [c_vp]),
    ("sca_tensor_ndims", c_i32, [c_vp]),
    ("sca_tensor_dim", c_i64, [c_vp, c_i32]),
    ("sca_tensor_upload", ctypes.c_int, [c_vp, c_vp, c_u64]),
    ("sca_tensor_download", ctypes.c_int, [c_vp, c_vp, c_u64]),
    ("sca_run_attention", ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, ctypes.POINTER(ScaConfig),
                                         ctypes.POINTER(c_vp), ctypes.POINTER(c_vp),
                                         ctypes.POINTER(ScaStats)]),
    ("sca_run_flash_varlen", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64,
                                            ctypes.POINTER(ScaConfig), ctypes.POINTER(c_vp),
                                            ctypes.POINTER(ScaStats)]),
    ("sca_explain_tensors", None, [c_vp, c_vp, c_vp, ctypes.POINTER(ScaConfig), c_char_p,
                                   ctypes.c_size_t]),
    ("sca_pkv_create", c_vp, [ctypes.POINTER(ScaKvConfig), c_i32]),
    ("sca_pkv_destroy", None, [c_vp]),
    ("sca_pkv_append", ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp]),
    ("sca_pkv_append_batch", ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp]),
    ("sca_pkv_reserve", ctypes.c_int, [c_vp, c_i64, c_i64, c_vp]),
    ("sca_pkv_reserve_batch", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    ("sca_pkv_write_layer", ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_vp]),
    ("sca_pkv_append_batch_all_layers", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp]),
    ("sca_pkv_reset", ctypes.c_int, [c_vp, c_i64, c_vp]),
    ("sca_pkv_sync", ctypes.c_int, [c_vp, c_vp]),
    ("sca_pkv_force_sync", ctypes.c_int, [c_vp, c_vp]),
    ("sca_pkv_page_table_device", c_vp, [c_vp]),
    ("sca_pkv_page_table_host", None, [c_vp, c_vp]),
    ("sca_pkv_seq_len", c_i64, [c_vp, c_i64]),
    ("sca_pkv_block_count", c_i64, [c_vp, c_i64]),
    ("sca_pkv_max_blocks_per_seq", c_i64, [c_vp]),
    ("sca_pkv_revision", c_u64, [c_vp]),
    ("sca_pkv_synced_revision", c_u64, [c_vp]),
    ("sca_pkv_stats", None, [c_vp, ctypes.POINTER(ScaKvStats)]),
    ("sca_pkv_layer_k", c_vp, [c_vp, c_i64]),
    ("sca_pkv_layer_v", c_vp, [c_vp, c_i64]),
    ("sca_pkv_blocks", c_vp, [c_vp]),
    ("sca_pkv_gather", ctypes.c_int, [c_vp, c_i32, c_i64, c_vp, c_i64, c_vp, ctypes.POINTER(c_vp)]),
    ("sca_run_paged", ctypes.c_int, [c_vp, c_vp, ctypes.POINTER(ScaPagedParams),
                                     ctypes.POINTER(ScaConfig), ctypes.POINTER(c_vp),
                                     ctypes.POINTER(ScaStats)]),
    ("sca_bm_create", c_vp, [c_i64, c_i64, c_i64, c_i32]),
    ("sca_bm_destroy", None, [c_vp]),
    ("sca_bm_allocate", ctypes.c_int, [c_vp, c_i64, c_vp]),
    ("sca_bm_free", None, [c_vp, c_vp, c_i64]),
    ("sca_bm_append_to_table", ctypes.c_int, [c_vp, c_i64, c_vp, c_i64]),
    ("sca_bm_reset_seq", ctypes.c_int, [c_vp, c_i64]),
    ("sca_bm_sync", ctypes.c_int, [c_vp, c_vp]),
    ("sca_bm_num_free", c_i64, [c_vp]),
    ("sca_bm_num_total", c_i64, [c_vp]),
    ("sca_bm_failures", c_i64, [c_vp]),
    ("sca_bm_double_frees", c_i64, [c_vp]),
    ("sca_bm_revision", c_u64, [c_vp]),
    ("sca_bm_synced_revision", c_u64, [c_vp]),
    ("sca_bm_table", None, [c_vp, c_vp]),
    ("sca_bm_table_device", ctypes.c_int, [c_vp, c_vp]),
    ("sca_ws_create", c_vp, [c_u64, c_i32]),
    ("sca_ws_destroy", None, [c_vp]),
    ("sca_ws_slice", ctypes.c_int, [c_vp, c_u64, c_u64, c_u64, ctypes.POINTER(c_u64)]),
    ("sca_ws_reset", ctypes.c_int, [c_vp]),
    ("sca_ws_peak", c_u64, [c_vp]),
    ("sca_ws_slices", c_u64, [c_vp]),
    ("sca_gpu_empty_cache", c_u64, []),
    ("sca_gpu_cached_bytes", c_u64, []),
    ("sca_gpu_allocated_bytes", c_u64, []),
    ("sca_release_scratch", ctypes.c_int, []),
    ("sca_scratch_high_water_bytes", c_u64, []),
    ("sca_gpu_available", ctypes.c_int, []),
    ("sca_device_cu_count", ctypes.c_int, []),
    ("sca_synchronize", ctypes.c_int, []),
]


def host_lib() -> ctypes.CDLL:
    """Loads libsca_host.so (and through it libsca_hip.so); raises when it was not built."""
    global _LIB
    if _LIB is None:
        _hip.hip_lib()  # load the kernel library first, from the same directory
        path = os.path.join(_hip.LIB_DIR, "libsca_host.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: run scicompute-attention_amd/build.py")
        lib = ctypes.CDLL(path)
        for name, res, args in _SIGS:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def _raise(code: int):
    if code != 0:
        raise ScaError(code, host_lib().sca_last_error().decode())


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(c_vp)


# ---- configuration ------------------------------------------------------------------------------

@dataclasses.dataclass
class AttentionConfig:
    backend: str = "auto"
    layout: str = "bhsd"
    causal: bool = False
    return_lse: bool = False
    scale: float = 0.0
    softcap: float = 0.0
    sliding_window: int = 0
    num_splits: int = 0
    allow_fallback: bool = False
    cu_seqlens_q: np.ndarray | None = None
    cu_seqlens_kv: np.ndarray | None = None
    stream: int | None = None

    def to_c(self) -> ScaConfig:
        c = ScaConfig()
        c.backend = BACKENDS[self.backend] if isinstance(self.backend, str) else int(self.backend)
        c.layout = LAYOUTS[self.layout] if isinstance(self.layout, str) else int(self.layout)
        c.causal = int(self.causal)
        c.return_lse = int(self.return_lse)
        c.scale = self.scale
        c.softcap = self.softcap
        c.sliding_window = self.sliding_window
        c.num_splits = self.num_splits
        c.allow_fallback = int(self.allow_fallback)
        self._keep = []
        for name in ("cu_seqlens_q", "cu_seqlens_kv"):
            arr = getattr(self, name)
            if arr is not None:
                arr = np.ascontiguousarray(arr, dtype=np.int32)
                self._keep.append(arr)
                setattr(c, name, arr.ctypes.data)
        c.stream = self.stream
        return c


@dataclasses.dataclass
class AttentionShape:
    batch: int = 0
    seq_q: int = 0
    seq_kv: int = 0
    num_heads: int = 0
    num_kv_heads: int = 0
    head_dim: int = 0

    def to_c(self) -> ScaShape:
        return ScaShape(self.batch, self.seq_q, self.seq_kv, self.num_heads, self.num_kv_heads,
                        self.head_dim)


@dataclasses.dataclass
class KVCacheConfig:
    num_layers: int = 1
    num_kv_heads: int = 1
    head_dim: int = 128
    block_size: int = 16
    num_blocks: int = 0
    max_num_seqs: int = 1
    dtype: str = "f16"
    layout: int = 0

    def to_c(self) -> ScaKvConfig:
        return ScaKvConfig(self.num_layers, self.num_kv_heads, self.head_dim, self.block_size,
                           self.num_blocks, self.max_num_seqs, DTYPES[self.dtype], self.layout)


def _stats(s: ScaStats) -> dict:
    return {"used_backend": s.used_backend, "tile": tuple(s.tile),
            "workspace_bytes": s.workspace_bytes, "kv_bytes": s.kv_bytes,
            "num_splits": s.num_splits, "materialized_score_bytes": s.materialized_score_bytes,
            "note": s.note.decode()}


# ---- tensors ------------------------------------------------------------------------------------

class Tensor:
    """sci::Tensor handle. ``Tensor.from_numpy(storage, dtype, device)`` uploads a storage array
    (uint16 bits for f16/bf16)."""

    def __init__(self, handle, dtype: str):
        if not handle:
            raise ScaError(1, host_lib().sca_last_error().decode())
        self.handle = handle
        self.dtype = dtype

    @classmethod
    def empty(cls, shape, dtype: str, device: int = GPU) -> "Tensor":
        dims = (c_i64 * len(shape))(*shape)
        return cls(host_lib().sca_tensor_new(dims, len(shape), DTYPES[dtype], device), dtype)

    @classmethod
    def from_numpy(cls, arr: np.ndarray, dtype: str, device: int = GPU) -> "Tensor":
        arr = np.ascontiguousarray(arr)
        t = cls.empty(arr.shape, dtype, device)
        assert arr.nbytes == t.nbytes, (arr.nbytes, t.nbytes)
        host_lib().sca_tensor_upload(t.handle, _ptr(arr), arr.nbytes)
        return t

    @property
    def nbytes(self) -> int:
        return host_lib().sca_tensor_nbytes(self.handle)

    @property
    def shape(self) -> tuple:
        lib = host_lib()
        return tuple(lib.sca_tensor_dim(self.handle, i) for i in range(lib.sca_tensor_ndims(self.handle)))

    @property
    def data_ptr(self) -> int:
        return host_lib().sca_tensor_data(self.handle)

    def numpy(self, np_dtype=None) -> np.ndarray:
        np_dtype = np_dtype or {"f32": np.float32, "f16": np.uint16, "bf16": np.uint16,
                                "i32": np.int32, "u8": np.uint8}[self.dtype]
        out = np.empty(self.shape, dtype=np_dtype)
        host_lib().sca_tensor_download(self.handle, _ptr(out), out.nbytes)
        return out

    def free(self):
        if getattr(self, "handle", None):
            host_lib().sca_tensor_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # interpreter shutdown
            pass


@dataclasses.dataclass
class AttentionResult:
    out: Tensor
    lse: Tensor | None
    stats: dict


_ENTRY = {"attention": 0, "flash_attention": 1, "decode_attention": 2, "decode": 3,
          "naive_attention": 4, "tiled_attention": 5}


def _run(entry: str, q: Tensor, k: Tensor, v: Tensor, cfg: AttentionConfig | None) -> AttentionResult:
    cfg = cfg or AttentionConfig()
    c = cfg.to_c()
    out, lse, st = c_vp(), c_vp(), ScaStats()
    rc = host_lib().sca_run_attention(_ENTRY[entry], q.handle, k.handle, v.handle,
                                      ctypes.byref(c), ctypes.byref(out), ctypes.byref(lse),
                                      ctypes.byref(st))
    _raise(rc)
    lse_t = Tensor(lse.value, "f32") if lse.value else None
    return AttentionResult(Tensor(out.value, q.dtype), lse_t, _stats(st))


def attention(q, k, v, cfg=None):
    return _run("attention", q, k, v, cfg)


def flash_attention(q, k, v, cfg=None):
    return _run("flash_attention", q, k, v, cfg)


def decode_attention(q, k, v, cfg=None):
    return _run("decode_attention", q, k, v, cfg)


def decode(q, k, v, cfg=None):
    return _run("decode", q, k, v, cfg)


def naive_attention(q, k, v, cfg=None):
    return _run("naive_attention", q, k, v, cfg)


def tiled_attention(q, k, v, cfg=None):
    return _run("tiled_attention", q, k, v, cfg)


def flash_attention_varlen(q, k, v, num_seqs, cu_q, cu_kv, max_q, max_kv, cfg=None):
    cfg = cfg or AttentionConfig()
    c = cfg.to_c()
    cu_q = np.ascontiguousarray(cu_q, dtype=np.int32)
    cu_kv = np.ascontiguousarray(cu_kv, dtype=np.int32)
    out, st = c_vp(), ScaStats()
    rc = host_lib().sca_run_flash_varlen(q.handle, k.handle, v.handle, num_seqs, _ptr(cu_q),
                                         _ptr(cu_kv), max_q, max_kv, ctypes.byref(c),
                                         ctypes.byref(out), ctypes.byref(st))
    _raise(rc)
    return AttentionResult(Tensor(out.value, q.dtype), None, _stats(st))


def explain_attention(q, k, v, cfg=None) -> str:
    cfg = cfg or AttentionConfig()
    c = cfg.to_c()
    buf = ctypes.create_string_buffer(4096)
    host_lib().sca_explain_tensors(q.handle, k.handle, v.handle, ctypes.byref(c), buf, 4096)
    return buf.value.decode()


# ---- dispatcher / validation ---------------------------------------------------------------------

def validate(cfg: AttentionConfig, shape: AttentionShape):
    """(code, detail) of sca::Validate."""
    c, s = cfg.to_c(), shape.to_c()
    buf = ctypes.create_string_buffer(2048)
    code = host_lib().sca_validate(ctypes.byref(c), ctypes.byref(s), buf, 2048)
    return code, buf.value.decode()


def effective_scale(cfg: AttentionConfig, shape: AttentionShape) -> float:
    c, s = cfg.to_c(), shape.to_c()
    return host_lib().sca_effective_scale(ctypes.byref(c), ctypes.byref(s))


def validate_varlen(cu, batch):
    cu = np.ascontiguousarray(cu, dtype=np.int32)
    mx = c_i64(-1)
    code = host_lib().sca_validate_varlen(_ptr(cu) if cu.size else None, batch, ctypes.byref(mx))
    msg = host_lib().sca_last_error().decode() if code else ""
    return code, mx.value, msg


def select(cfg: AttentionConfig, shape: AttentionShape) -> dict:
    c, s = cfg.to_c(), shape.to_c()
    backend, tile, ws = c_i32(), (c_i32 * 4)(), c_u64()
    buf = ctypes.create_string_buffer(4096)
    host_lib().sca_select(ctypes.byref(c), ctypes.byref(s), ctypes.byref(backend), tile,
                          ctypes.byref(ws), buf, 4096)
    return {"backend": backend.value, "tile": tuple(tile), "workspace": ws.value,
            "reason": buf.value.decode()}


def explain(cfg: AttentionConfig, shape: AttentionShape) -> str:
    c, s = cfg.to_c(), shape.to_c()
    buf = ctypes.create_string_buffer(4096)
    host_lib().sca_explain(ctypes.byref(c), ctypes.byref(s), buf, 4096)
    return buf.value.decode()


def decode_splits(shape: AttentionShape, cu_count: int) -> int:
    s = shape.to_c()
    return host_lib().sca_decode_splits(ctypes.byref(s), cu_count)


def paged_decode_plan(lengths, num_heads: int, num_kv_heads: int, cu_count: int):
    """(splits, slot_waves) of the paged MFMA decode kernel for a batch of host-side lengths:
    the plan the paged backend applies when it attends the cache's own page table."""
    lens = np.ascontiguousarray(lengths, dtype=np.int64)
    splits, waves = c_i64(0), c_i32(0)
    _raise(host_lib().sca_paged_decode_plan(_ptr(lens) if lens.size else None, lens.size,
                                            num_heads, num_kv_heads, cu_count,
                                            ctypes.byref(splits), ctypes.byref(waves)))
    return int(splits.value), int(waves.value)


def compute_slot_mapping(row, seq_start, num_tokens, block_size, max_blocks):
    row = np.ascontiguousarray(row, dtype=np.int32)
    out = np.zeros(max(num_tokens, 0), dtype=np.int32)
    rc = host_lib().sca_compute_slot_mapping(_ptr(row) if row.size else None, seq_start, num_tokens,
                                             block_size, max_blocks, _ptr(out))
    _raise(rc)
    return out


def kv_cache_bytes(cfg: KVCacheConfig) -> int:
    c = cfg.to_c()
    out = c_u64()
    _raise(host_lib().sca_kv_cache_bytes(ctypes.byref(c), ctypes.byref(out)))
    return out.value


def max_blocks_for_budget(cfg: KVCacheConfig, budget: int) -> int:
    c = cfg.to_c()
    return host_lib().sca_max_blocks_for_budget(ctypes.byref(c), budget)


# ---- BlockManager / PagedKVCache / Workspace ------------------------------------------------------

class BlockManager:
    def __init__(self, num_blocks, max_num_seqs, max_blocks_per_seq, device=HOST, _borrowed=None):
        lib = host_lib()
        self._owned = _borrowed is None
        self.h = _borrowed or lib.sca_bm_create(num_blocks, max_num_seqs, max_blocks_per_seq, device)
        if not self.h:
            raise ScaError(lib.sca_extract_code(lib.sca_last_error()), lib.sca_last_error().decode())
        self.max_num_seqs = max_num_seqs
        self.max_blocks_per_seq = max_blocks_per_seq

    def allocate(self, count):
        out = np.zeros(max(count, 0), dtype=np.int32)
        _raise(host_lib().sca_bm_allocate(self.h, count, _ptr(out)))
        return out

    def free(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        host_lib().sca_bm_free(self.h, _ptr(ids) if ids.size else None, ids.size)

    def append_to_table(self, seq, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        _raise(host_lib().sca_bm_append_to_table(self.h, seq, _ptr(ids) if ids.size else None,
                                                 ids.size))

    def reset_seq(self, seq):
        _raise(host_lib().sca_bm_reset_seq(self.h, seq))

    def sync(self, stream=None):
        _raise(host_lib().sca_bm_sync(self.h, stream))

    def table(self) -> np.ndarray:
        out = np.empty(self.max_num_seqs * self.max_blocks_per_seq, dtype=np.int32)
        host_lib().sca_bm_table(self.h, _ptr(out))
        return out

    def table_device(self) -> np.ndarray:
        out = np.empty(self.max_num_seqs * self.max_blocks_per_seq, dtype=np.int32)
        _raise(host_lib().sca_bm_table_device(self.h, _ptr(out)))
        return out

    def state(self) -> dict:
        lib = host_lib()
        return {"num_free": lib.sca_bm_num_free(self.h), "failures": lib.sca_bm_failures(self.h),
                "double_frees": lib.sca_bm_double_frees(self.h),
                "revision": lib.sca_bm_revision(self.h),
                "synced_revision": lib.sca_bm_synced_revision(self.h),
                "table": self.table().tolist()}

    def __del__(self):
        if getattr(self, "_owned", False) and getattr(self, "h", None):
            try:
                host_lib().sca_bm_destroy(self.h)
            except Exception:
                pass
            self.h = None


class PagedKVCache:
    def __init__(self, cfg: KVCacheConfig, device=GPU):
        lib = host_lib()
        self.cfg = cfg
        c = cfg.to_c()
        self.h = lib.sca_pkv_create(ctypes.byref(c), device)
        if not self.h:
            msg = lib.sca_last_error()
            raise ScaError(lib.sca_extract_code(msg), msg.decode())

    def append_tokens(self, seq, layer, k_new: Tensor, v_new: Tensor, stream=None):
        _raise(host_lib().sca_pkv_append(self.h, seq, layer, k_new.handle, v_new.handle, stream))

    def append_batch(self, seq_ids, layer, k_new: Tensor, v_new: Tensor, stream=None):
        """One token per entry of seq_ids ([n, H_kv, D] device tensors), in order."""
        ids = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int64))
        _raise(host_lib().sca_pkv_append_batch(self.h, ids.ctypes.data, ids.size, layer,
                                               k_new.handle, v_new.handle, stream))

    def reserve(self, seq, num_tokens, stream=None):
        _raise(host_lib().sca_pkv_reserve(self.h, seq, num_tokens, stream))

    def reserve_batch(self, seq_ids, stream=None):
        ids = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int64))
        _raise(host_lib().sca_pkv_reserve_batch(self.h, ids.ctypes.data, ids.size, stream))

    def write_layer(self, layer, k_new: Tensor, v_new: Tensor, stream=None):
        _raise(host_lib().sca_pkv_write_layer(self.h, layer, k_new.handle, v_new.handle, stream))

    def append_batch_all_layers(self, seq_ids, k_layers: Tensor, v_layers: Tensor, stream=None):
        ids = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int64))
        _raise(host_lib().sca_pkv_append_batch_all_layers(self.h, ids.ctypes.data, ids.size,
                                                          k_layers.handle, v_layers.handle, stream))

    def reset_seq(self, seq, stream=None):
        _raise(host_lib().sca_pkv_reset(self.h, seq, stream))

    def sync_page_table(self, stream=None):
        _raise(host_lib().sca_pkv_sync(self.h, stream))

    def force_sync_page_table(self, stream=None):
        _raise(host_lib().sca_pkv_force_sync(self.h, stream))

    @property
    def page_table_device_ptr(self) -> int:
        return host_lib().sca_pkv_page_table_device(self.h)

    @property
    def max_blocks_per_seq(self) -> int:
        return host_lib().sca_pkv_max_blocks_per_seq(self.h)

    def page_table_host(self) -> np.ndarray:
        out = np.empty((self.cfg.max_num_seqs, self.max_blocks_per_seq), dtype=np.int32)
        host_lib().sca_pkv_page_table_host(self.h, _ptr(out))
        return out

    def page_table_device(self) -> np.ndarray:
        out = np.empty((self.cfg.max_num_seqs, self.max_blocks_per_seq), dtype=np.int32)
        _hip.check(_hip.hip_lib().sca_hip_device_synchronize())
        _hip.check(_hip.hip_lib().sca_hip_memcpy(_ptr(out), self.page_table_device_ptr,
                                                  out.nbytes, _hip.COPY_D2H))
        return out

    def seq_length(self, seq) -> int:
        return host_lib().sca_pkv_seq_len(self.h, seq)

    def logical_block_count(self, seq) -> int:
        return host_lib().sca_pkv_block_count(self.h, seq)

    @property
    def revision(self) -> int:
        return host_lib().sca_pkv_revision(self.h)

    @property
    def synced_revision(self) -> int:
        return host_lib().sca_pkv_synced_revision(self.h)

    def stats(self) -> dict:
        s = ScaKvStats()
        host_lib().sca_pkv_stats(self.h, ctypes.byref(s))
        return {f: getattr(s, f) for f, _ in ScaKvStats._fields_}

    def layer_ptrs(self, layer=0):
        lib = host_lib()
        return lib.sca_pkv_layer_k(self.h, layer), lib.sca_pkv_layer_v(self.h, layer)

    def blocks(self) -> BlockManager:
        return BlockManager(0, self.cfg.max_num_seqs, self.max_blocks_per_seq,
                            _borrowed=host_lib().sca_pkv_blocks(self.h))

    def gather(self, is_key: bool, layer: int, block_ids_dev: int, n: int) -> Tensor:
        out = c_vp()
        _raise(host_lib().sca_pkv_gather(self.h, int(is_key), layer, block_ids_dev, n, None,
                                         ctypes.byref(out)))
        return Tensor(out.value, self.cfg.dtype)

    def __del__(self):
        if getattr(self, "h", None):
            try:
                host_lib().sca_pkv_destroy(self.h)
            except Exception:
                pass
            self.h = None


def paged_attention(q: Tensor, kv: PagedKVCache, params: dict | None = None, cfg=None):
    cfg = cfg or AttentionConfig()
    c = cfg.to_c()
    out, st = c_vp(), ScaStats()
    if params is None:
        p_ptr = None
    else:
        p = ScaPagedParams(params.get("page_table"), params.get("seq_lens"),
                           params.get("num_seqs", 0), params.get("block_size", 16),
                           params.get("max_blocks_per_seq", 0), params.get("layer", 0))
        p_ptr = ctypes.byref(p)
    _raise(host_lib().sca_run_paged(q.handle, kv.h, p_ptr, ctypes.byref(c), ctypes.byref(out),
                                    ctypes.byref(st)))
    return AttentionResult(Tensor(out.value, q.dtype), None, _stats(st))


class Workspace:
    def __init__(self, nbytes, device=HOST):
        lib = host_lib()
        self.h = lib.sca_ws_create(nbytes, device)
        if not self.h:
            msg = lib.sca_last_error()
            raise ScaError(lib.sca_extract_code(msg), msg.decode())

    def slice(self, offset, nbytes, align=256) -> int:
        rel = c_u64()
        _raise(host_lib().sca_ws_slice(self.h, offset, nbytes, align, ctypes.byref(rel)))
        return rel.value

    def reset(self):
        _raise(host_lib().sca_ws_reset(self.h))

    @property
    def peak(self):
        return host_lib().sca_ws_peak(self.h)

    @property
    def slices(self):
        return host_lib().sca_ws_slices(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            try:
                host_lib().sca_ws_destroy(self.h)
            except Exception:
                pass
            self.h = None


# ---- status helpers ------------------------------------------------------------------------------

def status_name(code: int) -> str:
    return host_lib().sca_status_name(code).decode()


def make_status(code: int, detail: str):
    buf = ctypes.create_string_buffer(4096)
    sci = host_lib().sca_make_status(code, detail.encode(), buf, 4096)
    return sci, buf.value.decode()


def extract_code(message: str) -> int:
    return host_lib().sca_extract_code(message.encode())


def to_sci_code(code: int) -> int:
    return host_lib().sca_to_sci_code(code)


def backend_name(kind: int) -> str:
    return host_lib().sca_backend_name(kind).decode()


def layout_name(layout: int) -> str:
    return host_lib().sca_layout_name(layout).decode()


def parse_backend(name: str):
    out = c_i32(-1)
    ok = host_lib().sca_parse_backend(name.encode(), ctypes.byref(out))
    return out.value if ok else None


def supported_head_dim_index(d: int) -> int:
    return host_lib().sca_supported_head_dim_index(d)

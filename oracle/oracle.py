"""Python face of the CPU oracle. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (the naive restatement is also the timed CPU baseline). The product path
never imports it.

Wraps ``oracle/_build/liboracle.so`` (the C restatement in sca_oracle.c) and, when it was built in
this container, ``oracle/_ref/libsca_ref.so`` (the reference's own host code, CPU STUB mode).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p
c_sz = ctypes.c_size_t
c_char_p = ctypes.c_char_p


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(ORACLE_DIR, "_build", "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run oracle/build_oracle.py")
        L = ctypes.CDLL(path)
        L.oracle_random_floats.argtypes = [c_vp, c_sz, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        L.oracle_float_to_half_bits.argtypes = [ctypes.c_float]
        L.oracle_float_to_half_bits.restype = ctypes.c_uint16
        L.oracle_half_bits_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_half_bits_to_float.restype = ctypes.c_float
        L.oracle_float_to_bf16_bits.argtypes = [ctypes.c_float]
        L.oracle_float_to_bf16_bits.restype = ctypes.c_uint16
        L.oracle_bf16_bits_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_bits_to_float.restype = ctypes.c_float
        L.oracle_encode.argtypes = [c_vp, c_sz, ctypes.c_int, c_vp, c_vp]
        L.oracle_reference_attention.argtypes = [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64,
                                                 c_i64, ctypes.c_int, ctypes.c_double, c_vp, c_i64,
                                                 c_vp, c_vp, ctypes.c_int]
        L.oracle_naive_attention_f32.argtypes = [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64,
                                                 c_i64, c_i64, ctypes.c_int, ctypes.c_float, c_vp,
                                                 c_vp, c_vp, ctypes.c_int]
        L.oracle_splitk_decode.argtypes = [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64,
                                           c_i64, ctypes.c_double, c_vp, c_vp, c_vp, c_vp, c_vp]
        L.oracle_splits_for.argtypes = [c_i64, c_i64]
        L.oracle_splits_for.restype = c_i64
        L.oracle_partial_elements.argtypes = [c_i64] * 4
        L.oracle_partial_elements.restype = c_i64
        L.oracle_compute_slot_mapping.argtypes = [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp,
                                                  ctypes.c_char_p, c_sz]
        L.oracle_kv_cache_bytes.argtypes = [c_i64] * 7
        L.oracle_kv_cache_bytes.restype = c_i64
        L.oracle_max_blocks_for_budget.argtypes = [c_i64] * 5 + [ctypes.c_uint64]
        L.oracle_max_blocks_for_budget.restype = c_i64
        L.oracle_bm_create.argtypes = [c_i64] * 3
        L.oracle_bm_create.restype = c_vp
        L.oracle_bm_destroy.argtypes = [c_vp]
        L.oracle_bm_allocate.argtypes = [c_vp, c_i64, c_vp, ctypes.c_char_p, c_sz]
        L.oracle_bm_free.argtypes = [c_vp, c_vp, c_i64]
        L.oracle_bm_append_to_table.argtypes = [c_vp, c_i64, c_vp, c_i64, ctypes.c_char_p, c_sz]
        L.oracle_bm_reset_seq.argtypes = [c_vp, c_i64, ctypes.c_char_p, c_sz]
        L.oracle_bm_sync.argtypes = [c_vp]
        for name in ("num_free", "failures", "double_frees"):
            getattr(L, f"oracle_bm_{name}").argtypes = [c_vp]
            getattr(L, f"oracle_bm_{name}").restype = c_i64
        for name in ("revision", "synced_revision"):
            getattr(L, f"oracle_bm_{name}").argtypes = [c_vp]
            getattr(L, f"oracle_bm_{name}").restype = ctypes.c_uint64
        L.oracle_bm_table.argtypes = [c_vp, c_vp]
        L.oracle_bm_free_list.argtypes = [c_vp, c_vp]
        L.oracle_bm_free_list.restype = c_i64
        L.oracle_pkv_create.argtypes = [c_i64] * 4
        L.oracle_pkv_create.restype = c_vp
        L.oracle_pkv_destroy.argtypes = [c_vp]
        L.oracle_pkv_append.argtypes = [c_vp, c_i64, c_i64, c_i64, c_vp, ctypes.c_char_p, c_sz]
        L.oracle_pkv_reset.argtypes = [c_vp, c_i64, ctypes.c_char_p, c_sz]
        L.oracle_pkv_sync.argtypes = [c_vp]
        L.oracle_pkv_seq_len.argtypes = [c_vp, c_i64]
        L.oracle_pkv_seq_len.restype = c_i64
        L.oracle_pkv_block_count.argtypes = [c_vp, c_i64]
        L.oracle_pkv_block_count.restype = c_i64
        L.oracle_pkv_page_table.argtypes = [c_vp, c_vp]
        L.oracle_pkv_stats.argtypes = [c_vp, c_vp]
        L.oracle_pkv_blocks.argtypes = [c_vp]
        L.oracle_pkv_blocks.restype = c_vp
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(c_vp) if a is not None else None


# ---- generation / encoding (tests/common/test_utils.hpp:24-131) ------------------------------------
def random_floats(n: int, seed: int, low: float = -1.0, high: float = 1.0) -> np.ndarray:
    out = np.empty(int(n), dtype=np.float32)
    lib().oracle_random_floats(_ptr(out), out.size, ctypes.c_uint32(seed & 0xFFFFFFFF), low, high)
    return out


def encode(values: np.ndarray, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """dtype 'f16' or 'bf16' -> (uint16 storage bits, float32 dequantised values)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if dtype == "f32":
        return values.view(np.uint32).copy(), values.copy()
    bits = np.empty(values.shape, dtype=np.uint16)
    deq = np.empty(values.shape, dtype=np.float32)
    lib().oracle_encode(_ptr(values), values.size, 1 if dtype == "f16" else 2, _ptr(bits), _ptr(deq))
    return bits, deq


def decode_bits(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Storage bits -> float32 (exact)."""
    bits = np.ascontiguousarray(bits)
    if dtype == "f16":
        return bits.view(np.float16).astype(np.float32)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float32)


# ---- attention ------------------------------------------------------------------------------------
def reference_attention(q, k, v, causal: bool, scale: float | None = None, rows=None,
                        threads: int = 0):
    """FP64 oracle (test_utils.hpp:229-285). q [B,Hq,Sq,D], k/v [B,Hkv,Skv,D] float32 (BHSD).

    Returns (out [n_rows, D] float64, lse [n_rows] float64) for the requested flat rows
    (b*Hq + h)*Sq + i (all rows when None)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    if rows is None:
        n_rows = B * Hq * Sq
        rows_arr = None
    else:
        rows_arr = np.ascontiguousarray(rows, dtype=np.int64)
        n_rows = rows_arr.size
    out = np.empty((n_rows, D), dtype=np.float64)
    lse = np.empty(n_rows, dtype=np.float64)
    lib().oracle_reference_attention(_ptr(q), _ptr(k), _ptr(v), B, Hq, Hkv, Sq, Skv, D,
                                     1 if causal else 0, float(scale or 0.0), _ptr(rows_arr),
                                     n_rows, _ptr(out), _ptr(lse), threads)
    return out, lse


def naive_attention(q, k, v, causal: bool, scale: float | None = None, threads: int = 1):
    """FP32 three-pass restatement (attention_naive.cu:41-135): (out float32 BHSD, lse)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    sc = float(scale) if scale else float(np.float32(1.0 / np.sqrt(np.float64(D))))
    scores = np.empty(B * Hq * Sq * Skv, dtype=np.float32)
    out = np.empty_like(q)
    lse = np.empty((B, Hq, Sq), dtype=np.float32)
    lib().oracle_naive_attention_f32(_ptr(q), _ptr(k), _ptr(v), B, Hq, Hkv, Sq, Skv, D,
                                     1 if causal else 0, sc, _ptr(scores), _ptr(out), _ptr(lse),
                                     threads)
    return out, lse


def naive_attention_into(q, k, v, causal, scale, scores, out, lse, threads):
    """Same as naive_attention with caller-provided buffers (for timing)."""
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    lib().oracle_naive_attention_f32(_ptr(q), _ptr(k), _ptr(v), B, Hq, Hkv, Sq, Skv, D,
                                     1 if causal else 0, float(scale), _ptr(scores), _ptr(out),
                                     _ptr(lse), threads)


def splitk_decode(q, k, v, splits: int, scale: float | None = None, seq_lens=None):
    """Split-K model (decode_splitk.cu:66-182). q [B,Hq,1,D]; k/v [B,Hkv,Skv,D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, Hq, _, D = q.shape
    _, Hkv, Skv, _ = k.shape
    lens = None if seq_lens is None else np.ascontiguousarray(seq_lens, dtype=np.int32)
    out = np.empty((B, Hq, D), dtype=np.float64)
    pm = np.empty(B * Hq * splits, dtype=np.float64)
    pl = np.empty_like(pm)
    po = np.empty((B * Hq * splits, D), dtype=np.float64)
    lib().oracle_splitk_decode(_ptr(q), _ptr(k), _ptr(v), B, Hq, Hkv, Skv, D, splits,
                               float(scale or 0.0), _ptr(lens), _ptr(out), _ptr(pm), _ptr(pl),
                               _ptr(po))
    return out, pm, pl, po


def paged_gather(pool: np.ndarray, page_row: np.ndarray, length: int, block_size: int,
                 num_blocks: int):
    """Contiguous view of one sequence in a block-major pool (page_table.cuh:18-36).

    pool [num_blocks, block_size, Hkv, D]; returns ([Hkv, length, D], valid[length]) where tokens
    whose logical block is unmapped (< 0 or >= num_blocks, or beyond the row) are invalid."""
    j = np.arange(length)
    logical = j // block_size
    phys = np.full(length, -1, dtype=np.int64)
    in_row = logical < page_row.size
    phys[in_row] = page_row[logical[in_row]]
    valid = (phys >= 0) & (phys < num_blocks)
    rows = np.where(valid, phys * block_size + j % block_size, 0)
    flat = pool.reshape(num_blocks * block_size, pool.shape[2], pool.shape[3])
    kv = flat[rows].transpose(1, 0, 2).copy()
    kv[:, ~valid, :] = 0.0
    return kv, valid


# ---- integer helpers ------------------------------------------------------------------------------
def splits_for(seq_kv: int, sm_count: int) -> int:
    return int(lib().oracle_splits_for(seq_kv, sm_count))


def partial_elements(b: int, h: int, s: int, d: int) -> int:
    return int(lib().oracle_partial_elements(b, h, s, d))


def compute_slot_mapping(row, seq_start, num_tokens, block_size, max_blocks):
    row = np.ascontiguousarray(row, dtype=np.int32)
    slots = np.empty(max(int(num_tokens), 1), dtype=np.int32)
    msg = ctypes.create_string_buffer(512)
    rc = lib().oracle_compute_slot_mapping(_ptr(row), seq_start, num_tokens, block_size, max_blocks,
                                           _ptr(slots), msg, 512)
    return rc, slots[: max(int(num_tokens), 0)], msg.value.decode()


def kv_cache_bytes(layers, heads, d, bs, nb, max_seqs, elem_bytes) -> int:
    return int(lib().oracle_kv_cache_bytes(layers, heads, d, bs, nb, max_seqs, elem_bytes))


def max_blocks_for_budget(layers, heads, d, bs, elem_bytes, budget) -> int:
    return int(lib().oracle_max_blocks_for_budget(layers, heads, d, bs, elem_bytes, budget))


class BlockManager:
    """Restatement of sca::BlockManager (block_manager.cpp:11-144)."""

    def __init__(self, num_blocks, max_num_seqs, max_blocks_per_seq):
        self.h = lib().oracle_bm_create(num_blocks, max_num_seqs, max_blocks_per_seq)
        if not self.h:
            raise ValueError("invalid BlockManager arguments")
        self.shape = (max_num_seqs, max_blocks_per_seq)

    def allocate(self, count):
        out = np.empty(max(int(count), 1), dtype=np.int32)
        msg = ctypes.create_string_buffer(512)
        rc = lib().oracle_bm_allocate(self.h, count, _ptr(out), msg, 512)
        return rc, (out[:count].tolist() if rc == 0 else []), msg.value.decode()

    def free(self, ids):
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        lib().oracle_bm_free(self.h, _ptr(arr), arr.size)

    def append_to_table(self, seq, ids):
        arr = None if ids is None else np.ascontiguousarray(ids, dtype=np.int32)
        msg = ctypes.create_string_buffer(512)
        n = 0 if arr is None else arr.size
        rc = lib().oracle_bm_append_to_table(self.h, seq, _ptr(arr), n, msg, 512)
        return rc, msg.value.decode()

    def reset_seq(self, seq):
        msg = ctypes.create_string_buffer(512)
        rc = lib().oracle_bm_reset_seq(self.h, seq, msg, 512)
        return rc, msg.value.decode()

    def sync(self):
        return int(lib().oracle_bm_sync(self.h))

    def state(self) -> dict:
        L = lib()
        table = np.empty(self.shape[0] * self.shape[1], dtype=np.int32)
        L.oracle_bm_table(self.h, _ptr(table))
        return {
            "num_free": int(L.oracle_bm_num_free(self.h)),
            "failures": int(L.oracle_bm_failures(self.h)),
            "double_frees": int(L.oracle_bm_double_frees(self.h)),
            "revision": int(L.oracle_bm_revision(self.h)),
            "synced_revision": int(L.oracle_bm_synced_revision(self.h)),
            "table": table.tolist(),
        }

    def __del__(self):
        try:
            lib().oracle_bm_destroy(self.h)
        except Exception:
            pass


class PagedKV:
    """Restatement of sca::PagedKVCache host state (paged_kv_cache.cpp:13-211)."""

    def __init__(self, num_blocks, block_size, max_num_seqs, num_layers=1):
        self.h = lib().oracle_pkv_create(num_blocks, block_size, max_num_seqs, num_layers)
        if not self.h:
            raise ValueError("invalid PagedKV arguments")
        self.num_blocks = num_blocks
        self.max_num_seqs = max_num_seqs

    def append(self, seq, num_tokens, layer=0):
        slots = np.empty(max(int(num_tokens), 1), dtype=np.int32)
        msg = ctypes.create_string_buffer(512)
        rc = lib().oracle_pkv_append(self.h, seq, layer, num_tokens, _ptr(slots), msg, 512)
        return rc, (slots[:num_tokens].tolist() if rc == 0 else []), msg.value.decode()

    def reset(self, seq):
        msg = ctypes.create_string_buffer(512)
        return lib().oracle_pkv_reset(self.h, seq, msg, 512), msg.value.decode()

    def sync(self):
        return int(lib().oracle_pkv_sync(self.h))

    def seq_len(self, seq):
        return int(lib().oracle_pkv_seq_len(self.h, seq))

    def block_count(self, seq):
        return int(lib().oracle_pkv_block_count(self.h, seq))

    def page_table(self) -> np.ndarray:
        out = np.empty(self.max_num_seqs * self.num_blocks, dtype=np.int32)
        lib().oracle_pkv_page_table(self.h, _ptr(out))
        return out.reshape(self.max_num_seqs, self.num_blocks)

    def stats(self) -> dict:
        out = np.empty(6, dtype=np.int64)
        lib().oracle_pkv_stats(self.h, _ptr(out))
        keys = ("used_blocks", "free_blocks", "num_appends", "num_resets", "revision",
                "synced_revision")
        return dict(zip(keys, (int(x) for x in out)))

    def __del__(self):
        try:
            lib().oracle_pkv_destroy(self.h)
        except Exception:
            pass


# ---- the reference's own host code (oracle/_ref), when built here --------------------------------
class RefCfg(ctypes.Structure):
    _fields_ = [("backend", c_i32), ("layout", c_i32), ("causal", c_i32), ("return_lse", c_i32),
                ("scale", ctypes.c_float), ("softcap", ctypes.c_float),
                ("sliding_window", c_i64), ("num_splits", c_i64), ("allow_fallback", c_i32),
                ("has_cu_seqlens_q", c_i32), ("has_cu_seqlens_kv", c_i32)]


class RefShape(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seq_q", c_i64), ("seq_kv", c_i64), ("num_heads", c_i64),
                ("num_kv_heads", c_i64), ("head_dim", c_i64)]


def ref_lib():
    """The reference's host library (STUB build) or None when it was not built here."""
    global _REF
    if _REF is not None:
        return _REF
    path = os.path.join(ORACLE_DIR, "_ref", "libsca_ref.so")
    if not os.path.exists(path):
        return None
    R = ctypes.CDLL(path)
    P = ctypes.POINTER
    R.ref_validate.argtypes = [P(RefCfg), P(RefShape), ctypes.c_char_p, c_sz]
    R.ref_effective_scale.argtypes = [P(RefCfg), P(RefShape)]
    R.ref_effective_scale.restype = ctypes.c_float
    R.ref_validate_varlen.argtypes = [c_vp, c_i64, P(c_i64), ctypes.c_char_p, c_sz]
    R.ref_select.argtypes = [P(RefCfg), P(RefShape), P(c_i32), P(c_i32), P(ctypes.c_uint64),
                             ctypes.c_char_p, c_sz]
    R.ref_explain.argtypes = [P(RefCfg), P(RefShape), ctypes.c_char_p, c_sz]
    R.ref_make_status.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_char_p, c_sz]
    R.ref_status_name.argtypes = [ctypes.c_int]
    R.ref_status_name.restype = ctypes.c_char_p
    R.ref_to_sci_code.argtypes = [ctypes.c_int]
    R.ref_extract_code.argtypes = [ctypes.c_char_p]
    R.ref_backend_name.argtypes = [ctypes.c_int]
    R.ref_backend_name.restype = ctypes.c_char_p
    R.ref_layout_name.argtypes = [ctypes.c_int]
    R.ref_layout_name.restype = ctypes.c_char_p
    R.ref_parse_backend.argtypes = [ctypes.c_char_p, P(c_i32)]
    R.ref_supported_head_dim_index.argtypes = [c_i64]
    R.ref_tile_smem_bytes_flash.argtypes = [c_i32, c_i64, c_i32, c_i32, c_i32, c_i32]
    R.ref_tile_smem_bytes_flash.restype = c_i64
    R.ref_compute_slot_mapping.argtypes = [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp,
                                           ctypes.c_char_p, c_sz]
    R.ref_kv_cache_bytes.argtypes = [c_i64] * 6 + [c_i32, ctypes.c_char_p, c_sz]
    R.ref_kv_cache_bytes.restype = c_i64
    R.ref_max_blocks_for_budget.argtypes = [c_i64] * 4 + [c_i32, ctypes.c_uint64]
    R.ref_max_blocks_for_budget.restype = c_i64
    R.ref_splits_for.argtypes = [c_i64, c_i64]
    R.ref_splits_for.restype = c_i64
    R.ref_partial_elements.argtypes = [c_i64] * 4
    R.ref_partial_elements.restype = c_i64
    R.ref_bm_create.argtypes = [c_i64, c_i64, c_i64, ctypes.c_char_p, c_sz]
    R.ref_bm_create.restype = c_vp
    R.ref_bm_destroy.argtypes = [c_vp]
    R.ref_bm_allocate.argtypes = [c_vp, c_i64, c_vp, ctypes.c_char_p, c_sz]
    R.ref_bm_free.argtypes = [c_vp, c_vp, c_i64]
    R.ref_bm_append_to_table.argtypes = [c_vp, c_i64, c_vp, c_i64, ctypes.c_char_p, c_sz]
    R.ref_bm_reset_seq.argtypes = [c_vp, c_i64, ctypes.c_char_p, c_sz]
    R.ref_bm_sync.argtypes = [c_vp]
    for name in ("num_free", "failures", "double_frees"):
        getattr(R, f"ref_bm_{name}").argtypes = [c_vp]
        getattr(R, f"ref_bm_{name}").restype = c_i64
    for name in ("revision", "synced_revision"):
        getattr(R, f"ref_bm_{name}").argtypes = [c_vp]
        getattr(R, f"ref_bm_{name}").restype = ctypes.c_uint64
    R.ref_bm_table.argtypes = [c_vp, c_vp]
    R.ref_ws_create.argtypes = [ctypes.c_uint64, ctypes.c_char_p, c_sz]
    R.ref_ws_create.restype = c_vp
    R.ref_ws_destroy.argtypes = [c_vp]
    R.ref_ws_slice.argtypes = [c_vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                               P(ctypes.c_uint64), ctypes.c_char_p, c_sz]
    R.ref_ws_reset.argtypes = [c_vp]
    R.ref_ws_peak.argtypes = [c_vp]
    R.ref_ws_peak.restype = ctypes.c_uint64
    R.ref_ws_slices.argtypes = [c_vp]
    R.ref_ws_slices.restype = ctypes.c_uint64
    _REF = R
    return R


class RefBlockManager:
    """sca::BlockManager of the reference itself (STUB build)."""

    def __init__(self, num_blocks, max_num_seqs, max_blocks_per_seq):
        R = ref_lib()
        msg = ctypes.create_string_buffer(512)
        self.h = R.ref_bm_create(num_blocks, max_num_seqs, max_blocks_per_seq, msg, 512)
        if not self.h:
            raise ValueError(msg.value.decode())
        self.shape = (max_num_seqs, max_blocks_per_seq)

    def allocate(self, count):
        out = np.empty(max(int(count), 1), dtype=np.int32)
        msg = ctypes.create_string_buffer(512)
        rc = ref_lib().ref_bm_allocate(self.h, count, _ptr(out), msg, 512)
        return rc, (out[:count].tolist() if rc == 0 else []), msg.value.decode()

    def free(self, ids):
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        ref_lib().ref_bm_free(self.h, _ptr(arr), arr.size)

    def append_to_table(self, seq, ids):
        arr = None if ids is None else np.ascontiguousarray(ids, dtype=np.int32)
        msg = ctypes.create_string_buffer(512)
        n = 0 if arr is None else arr.size
        rc = ref_lib().ref_bm_append_to_table(self.h, seq, _ptr(arr), n, msg, 512)
        return rc, msg.value.decode()

    def reset_seq(self, seq):
        msg = ctypes.create_string_buffer(512)
        rc = ref_lib().ref_bm_reset_seq(self.h, seq, msg, 512)
        return rc, msg.value.decode()

    def sync(self):
        before = int(ref_lib().ref_bm_synced_revision(self.h))
        ref_lib().ref_bm_sync(self.h)
        after = int(ref_lib().ref_bm_synced_revision(self.h))
        rev = int(ref_lib().ref_bm_revision(self.h))
        return 1 if (before != rev and after == rev) else 0

    def state(self) -> dict:
        R = ref_lib()
        table = np.empty(self.shape[0] * self.shape[1], dtype=np.int32)
        R.ref_bm_table(self.h, _ptr(table))
        return {
            "num_free": int(R.ref_bm_num_free(self.h)),
            "failures": int(R.ref_bm_failures(self.h)),
            "double_frees": int(R.ref_bm_double_frees(self.h)),
            "revision": int(R.ref_bm_revision(self.h)),
            "synced_revision": int(R.ref_bm_synced_revision(self.h)),
            "table": table.tolist(),
        }

    def __del__(self):
        try:
            ref_lib().ref_bm_destroy(self.h)
        except Exception:
            pass

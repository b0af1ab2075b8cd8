"""Helpers shared by the GPU parity tests: input generation, kernel calls through the C ABI,
and the tolerance definitions.

Tolerance (written here once, used by every attention parity test):
  * primary gate (the hot-path contract): rel = max|out - ref| / max|ref| over the checked rows,
    rel <= 2e-3 for fp16 and <= 1.6e-2 for bf16 (ref = FP64 oracle on the dequantised inputs);
  * secondary gate (the reference's own table, tests/common/test_utils.hpp:293-299), applied to
    the U(-1,1) reference-style cases: max-abs <= 5e-3 / mean-abs <= 5e-4 (fp16),
    2e-2 / 2e-3 (bf16), 1e-4 / 1e-6 (fp32).
"""

from __future__ import annotations

import ctypes

import numpy as np

import oracle.oracle as orc
import sca_amd
from sca_amd import hip as H

REL_TOL = {"f16": 2e-3, "bf16": 1.6e-2, "f32": 1e-5}
ABS_TOL = {"f16": (5e-3, 5e-4), "bf16": (2e-2, 2e-3), "f32": (1e-4, 1e-6)}
DTYPE_ID = {"f32": H.DTYPE_F32, "f16": H.DTYPE_F16, "bf16": H.DTYPE_BF16}
ELEM_BYTES = {"f32": 4, "f16": 2, "bf16": 2}


def uniform(shape, seed, low=-1.0, high=1.0) -> np.ndarray:
    """xorshift32 U(low, high) values exactly as the reference's RandomFloats."""
    n = int(np.prod(shape))
    return orc.random_floats(n, seed, low, high).reshape(shape)


def normal(shape, seed, std=1.0) -> np.ndarray:
    """N(0, std^2) from numpy's PCG64 with a recorded seed."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def quantize(x: np.ndarray, dtype: str):
    """(storage array for the device, dequantised float32 values)."""
    bits, deq = orc.encode(x, dtype)
    return bits.reshape(x.shape), deq.reshape(x.shape)


def to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    return orc.decode_bits(bits, dtype)


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(got.astype(np.float64) - ref))) if ref.size else 0.0
    return err / scale if scale > 0 else err


def abs_err(got: np.ndarray, ref: np.ndarray):
    d = np.abs(got.astype(np.float64) - ref)
    return float(d.max()), float(d.mean())


def bhsd_strides(seq, heads, d):
    return heads * seq * d, seq * d, d


def bshd_strides(seq, heads, d):
    return seq * heads * d, d, heads * d


def run_flash(qb, kb, vb, dtype, causal, *, B, Hq, Hkv, Sq, Skv, D, layout="bhsd",
              want_lse=False, scale=None):
    """Runs sca_hip_flash_fwd on storage arrays; returns (out float32 [B,Hq,Sq,D], lse)."""
    strides = bhsd_strides if layout == "bhsd" else bshd_strides
    dq = H.DeviceBuffer.from_array(qb)
    dk = H.DeviceBuffer.from_array(kb)
    dv = H.DeviceBuffer.from_array(vb)
    dout = H.DeviceBuffer(B * Hq * Sq * D * ELEM_BYTES[dtype])
    dlse = H.DeviceBuffer(B * Hq * Sq * 4) if want_lse else None
    p = H.FlashParams()
    p.q, p.k, p.v, p.out = dq.ptr, dk.ptr, dv.ptr, dout.ptr
    p.lse = dlse.ptr if dlse else None
    p.batch, p.num_heads, p.num_kv_heads = B, Hq, Hkv
    p.seq_q, p.seq_kv, p.head_dim = Sq, Skv, D
    p.q_sb, p.q_sh, p.q_ss = strides(Sq, Hq, D)
    p.k_sb, p.k_sh, p.k_ss = strides(Skv, Hkv, D)
    p.v_sb, p.v_sh, p.v_ss = strides(Skv, Hkv, D)
    p.o_sb, p.o_sh, p.o_ss = bhsd_strides(Sq, Hq, D)
    p.scale = scale if scale else float(np.float32(1.0 / np.sqrt(np.float64(D))))
    p.causal = 1 if causal else 0
    p.dtype = DTYPE_ID[dtype]
    p.diagonal = (Skv - Sq) if causal else 0
    H.flash_fwd(p)
    sca_amd.synchronize()
    out = to_float(dout.download(np.uint16), dtype).reshape(B, Hq, Sq, D)
    lse = dlse.download(np.float32).reshape(B, Hq, Sq) if dlse else None
    return out, lse


def bhsd_to_bshd(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


def check_attention(got, ref, dtype, tag, abs_gate=False):
    rel = rel_err(got, ref)
    assert rel <= REL_TOL[dtype], f"{tag}: rel err {rel:.3e} > {REL_TOL[dtype]:.1e}"
    if abs_gate:
        mx, mean = abs_err(got, ref)
        amax, amean = ABS_TOL[dtype]
        assert mx <= amax and mean <= amean, f"{tag}: abs err max {mx:.3e} mean {mean:.3e}"
    assert np.all(np.isfinite(got)), f"{tag}: non-finite output"
    return rel


def decode_params(dq, dk, dv, dout, parts, *, B, Hq, Hkv, Skv, D, splits, dtype, scale=None,
                  q_strides=None, k_strides=None, o_strides=None):
    p = H.DecodeParams()
    p.q, p.k, p.v, p.out = dq.ptr, dk.ptr, dv.ptr, dout.ptr
    if parts is not None:
        base = B * Hq * splits
        p.partial_m = parts.ptr
        p.partial_l = parts.ptr + base * 4
        p.partial_o = parts.ptr + 2 * base * 4
    p.batch, p.num_heads, p.num_kv_heads = B, Hq, Hkv
    p.seq_kv, p.head_dim, p.num_splits = Skv, D, splits
    qs = q_strides or (Hq * D, D)
    ks = k_strides or (Hkv * Skv * D, Skv * D, D)
    os_ = o_strides or (Hq * D, D)
    p.q_sb, p.q_sh = qs
    p.k_sb, p.k_sh, p.k_ss = ks
    p.v_sb, p.v_sh, p.v_ss = ks
    p.o_sb, p.o_sh = os_
    p.scale = scale if scale else float(np.float32(1.0 / np.sqrt(np.float64(D))))
    p.dtype = DTYPE_ID[dtype]
    return p


def run_decode(qb, kb, vb, dtype, *, B, Hq, Hkv, Skv, D, splits, seq_lens=None, slot_waves=0):
    """Contiguous split-K decode: q [B,Hq,1,D], k/v [B,Hkv,Skv,D] storage arrays. slot_waves:
    0 = library default, 1 = one wave per KV-head slot, 4 = four waves per slot."""
    dq = H.DeviceBuffer.from_array(qb)
    dk = H.DeviceBuffer.from_array(kb)
    dv = H.DeviceBuffer.from_array(vb)
    dout = H.DeviceBuffer(B * Hq * D * ELEM_BYTES[dtype])
    parts = H.DeviceBuffer(4 * sca_amd.hip_lib().sca_hip_decode_partial_elements(B, Hq, splits, D))
    p = decode_params(dq, dk, dv, dout, parts, B=B, Hq=Hq, Hkv=Hkv, Skv=Skv, D=D, splits=splits,
                      dtype=dtype)
    lens_buf = None
    if seq_lens is not None:
        lens_buf = H.DeviceBuffer.from_array(np.asarray(seq_lens, dtype=np.int32))
        p.seq_lens = lens_buf.ptr
    p.slot_waves = slot_waves
    H.decode_splitk(p)
    sca_amd.synchronize()
    raw = dout.download(np.uint32 if dtype == "f32" else np.uint16)
    return to_float(raw, dtype).reshape(B, Hq, D)

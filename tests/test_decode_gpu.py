"""Split-K decode parity on the GPU through sca_hip_decode_splitk, against the FP64 oracle.

Case lists follow tests/kernel/test_decode_correctness.cu:74-147 (seeds: q=seed, k=seed+101,
v=seed+202) and tests/kernel/test_numerics.cu, plus BASELINE config C4 at full size.
"""

import numpy as np
import pytest

import oracle.oracle as orc
import sca_amd
from sca_amd import hip as H
from attn_util import (check_attention, decode_params, normal, quantize, run_decode, uniform)

pytestmark = pytest.mark.gpu


def _case(dtype, B, Hq, Hkv, Skv, D, splits, seed, abs_gate=True, seq_lens=None, slot_waves=0):
    q = uniform((B, Hq, 1, D), seed)
    k = uniform((B, Hkv, Skv, D), seed + 101)
    v = uniform((B, Hkv, Skv, D), seed + 202)
    qb, qd = quantize(q, dtype) if dtype != "f32" else (q.view(np.uint32), q)
    kb, kd = quantize(k, dtype) if dtype != "f32" else (k.view(np.uint32), k)
    vb, vd = quantize(v, dtype) if dtype != "f32" else (v.view(np.uint32), v)
    out = run_decode(qb, kb, vb, dtype, B=B, Hq=Hq, Hkv=Hkv, Skv=Skv, D=D, splits=splits,
                     seq_lens=seq_lens, slot_waves=slot_waves)
    tag = (f"decode {dtype} B={B} Hq={Hq} Hkv={Hkv} Skv={Skv} D={D} splits={splits} seed={seed} "
           f"slot_waves={slot_waves}")
    print(tag, flush=True)
    if seq_lens is None:
        ref, _ = orc.reference_attention(qd, kd, vd, True)
    else:
        ref = np.concatenate([orc.reference_attention(qd[b:b + 1], kd[b:b + 1, :, :L],
                                                      vd[b:b + 1, :, :L], True)[0]
                              for b, L in enumerate(seq_lens)])
    check_attention(out.reshape(-1, D), ref, dtype, tag, abs_gate=abs_gate)
    return out


@pytest.mark.parametrize("splits", [1, 2, 3, 4, 8, 16])
def test_every_split_count(hip, splits):
    for i, skv in enumerate([1, 127, 1024, 4096]):
        _case("f16", 1, 8, 8, skv, 128, splits, 70000 + 4 * splits + i)


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_gqa_across_split_counts(hip, group):
    for j, splits in enumerate([1, 4, 16]):
        _case("f16", 1, 8 * group, 8, 2048, 128, splits, 71000 + 3 * group + j)


@pytest.mark.parametrize("d", [32, 64, 96, 128, 160, 192, 256])
def test_bf16_every_head_dim(hip, d):
    _case("bf16", 1, 4, 2, 512, d, 4, 72000 + d)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_fp32(hip, d):
    _case("f32", 2, 8, 2, 300, d, 3, 73000 + d)


def test_odd_group_sizes(hip):
    _case("f16", 2, 6, 2, 777, 128, 5, 74001)   # group 3
    _case("bf16", 1, 5, 1, 333, 64, 2, 74002)   # group 5 (MQA-like)


def test_ragged_seq_lens_and_empty_splits(hip):
    # per-batch lengths, including lengths shorter than the split count (empty splits)
    _case("f16", 4, 8, 2, 600, 128, 16, 75001, seq_lens=[600, 3, 1, 257])


def test_split_count_invariance(hip):
    B, Hq, Hkv, Skv, D = 2, 16, 4, 3000, 128
    q, k, v = normal((B, Hq, 1, D), 1), normal((B, Hkv, Skv, D), 2), normal((B, Hkv, Skv, D), 3)
    qb, qd = quantize(q, "f16")
    kb, kd = quantize(k, "f16")
    vb, vd = quantize(v, "f16")
    outs = [run_decode(qb, kb, vb, "f16", B=B, Hq=Hq, Hkv=Hkv, Skv=Skv, D=D, splits=s)
            for s in (1, 2, 7, 16, 64)]
    for o in outs[1:]:
        assert float(np.max(np.abs(o - outs[0]))) <= 2e-3


def test_uniform_logits_give_mean_of_v(hip):
    D, Skv = 128, 512
    v = uniform((1, 4, Skv, D), 80 + 2)
    vb, vd = quantize(v, "f16")
    out = run_decode(np.zeros((1, 4, 1, D), np.uint16), np.zeros((1, 4, Skv, D), np.uint16), vb,
                     "f16", B=1, Hq=4, Hkv=4, Skv=Skv, D=D, splits=4)
    assert float(np.max(np.abs(out - vd.mean(axis=2)))) <= 1e-3


def test_baseline_c4_full_size(hip):
    # C4: B=16, Hq=32, Hkv=8, D=128, S_kv=4096, fp16, N(0,1); splits as the MI355X table picks
    B, Hq, Hkv, Skv, D = 16, 32, 8, 4096, 128
    q, k, v = normal((B, Hq, 1, D), 4001), normal((B, Hkv, Skv, D), 4002), \
        normal((B, Hkv, Skv, D), 4003)
    qb, qd = quantize(q, "f16")
    kb, kd = quantize(k, "f16")
    vb, vd = quantize(v, "f16")
    for splits in (8, 4):
        out = run_decode(qb, kb, vb, "f16", B=B, Hq=Hq, Hkv=Hkv, Skv=Skv, D=D, splits=splits)
        ref, _ = orc.reference_attention(qd, kd, vd, False)
        check_attention(out.reshape(-1, D), ref, "f16", f"C4 splits={splits}")


def test_rejects_bad_arguments(hip):
    p = H.DecodeParams()
    with pytest.raises(H.HipError):
        H.decode_splitk(p)
    buf = H.DeviceBuffer(4096)
    p = decode_params(buf, buf, buf, buf, None, B=1, Hq=8, Hkv=3, Skv=4, D=128, splits=1,
                      dtype="f16")
    with pytest.raises(H.HipError) as exc:
        H.decode_splitk(p)
    assert exc.value.code == 2005
    p = decode_params(buf, buf, buf, buf, None, B=1, Hq=8, Hkv=8, Skv=4, D=48, splits=1,
                      dtype="f16")
    with pytest.raises(H.HipError) as exc:
        H.decode_splitk(p)
    assert exc.value.code == 2001


def test_groups_wider_than_one_mfma_tile(hip):
    # 16 query heads share one MFMA tile: group 32 takes two chunks, group 24 a partial second
    _case("f16", 2, 32, 1, 700, 128, 3, 77001)
    _case("bf16", 1, 24, 1, 515, 64, 2, 77002)
    _case("bf16", 2, 16, 1, 95, 128, 1, 77003)


@pytest.mark.parametrize("slot_waves", [1, 4])
def test_contiguous_slot_layouts(hip, slot_waves):
    """Both MFMA work splits on contiguous KV: one wave per KV-head slot (workgroups of four
    slots, the last one partly empty when the slot count is not a multiple of four) and four
    waves per slot; ragged lengths, empty splits and a group wider than one MFMA tile."""
    _case("f16", 3, 24, 6, 1500, 128, 3, 76001, slot_waves=slot_waves)
    _case("bf16", 2, 8, 8, 700, 64, 1, 76002, slot_waves=slot_waves)
    _case("f16", 4, 8, 2, 600, 128, 16, 76003, seq_lens=[600, 3, 1, 257], slot_waves=slot_waves)
    _case("bf16", 1, 32, 1, 900, 128, 2, 76004, slot_waves=slot_waves)

"""The allocation-free decode entry point (sca_hip_decode_splitk_noalloc) against the entry point
with caller-provided scratch (sca_hip_decode_splitk / _paged): bit-identical outputs on calls in
a row through the C ABI, the later ones smaller, with the static scratch reused in between."""

import numpy as np
import pytest

import sca_amd
from sca_amd import hip as H
from attn_util import ELEM_BYTES, check_attention, decode_params, quantize, to_float, uniform
from test_paged_gpu import build_pool, reference

pytestmark = pytest.mark.gpu

# (lengths seed, batch, Hq, Hkv, D, dtype, splits, block size, max length); the first case
# ranks its 300 sequences through the static batch-order scratch.
CASES = [
    (1, 300, 16, 4, 128, "f16", 4, 16, 600),
    (2, 20, 32, 8, 64, "bf16", 6, 16, 3000),
    (3, 3, 8, 8, 128, "bf16", 1, 8, 200),
]


def _paged_params(case, with_scratch):
    seed, S, Hq, Hkv, D, dtype, splits, bs, max_len = case
    rng = np.random.default_rng(seed)
    lengths = [int(x) for x in rng.integers(1, max_len + 1, size=S)]
    nb, mb, table, kb, kd, vb, vd = build_pool(lengths, bs, Hkv, D, dtype, seed)
    qb, qd = quantize(uniform((S, Hq, 1, D), seed + 5), dtype)
    bufs = dict(q=H.DeviceBuffer.from_array(qb), k=H.DeviceBuffer.from_array(kb),
                v=H.DeviceBuffer.from_array(vb), t=H.DeviceBuffer.from_array(table),
                l=H.DeviceBuffer.from_array(np.asarray(lengths, np.int32)),
                o=H.DeviceBuffer(S * Hq * D * ELEM_BYTES[dtype]))
    parts = None
    if with_scratch:
        n = sca_amd.hip_lib().sca_hip_decode_partial_elements(S, Hq, splits, D)
        bufs["parts"] = parts = H.DeviceBuffer(4 * n)
        bufs["order"] = H.DeviceBuffer(8 * S)
    p = decode_params(bufs["q"], bufs["k"], bufs["v"], bufs["o"], parts, B=S, Hq=Hq, Hkv=Hkv,
                      Skv=nb * bs, D=D, splits=splits, dtype=dtype, k_strides=(0, D, Hkv * D))
    p.page_table, p.block_size, p.max_blocks_per_seq, p.num_kv_blocks = bufs["t"].ptr, bs, mb, nb
    p.seq_lens = bufs["l"].ptr
    p.batch_order = bufs["order"].ptr if with_scratch else None
    ref = (qd, kd, vd, table, lengths, bs, nb)
    return p, bufs, ref


def _out(bufs, case):
    _, S, Hq, _, D, dtype, *_ = case
    return to_float(bufs["o"].download(np.uint16), dtype).reshape(S, Hq, D)


def test_noalloc_matches_the_scratch_entry_point_on_calls_in_a_row(hip):
    for case in CASES:
        print(f"no-alloc case {case}", flush=True)
        p_ref, b_ref, ref = _paged_params(case, with_scratch=True)
        p_na, b_na, _ = _paged_params(case, with_scratch=False)
        H.decode_splitk_paged(p_ref)
        H.decode_splitk_noalloc(p_na)
        sca_amd.synchronize()
        want, got = _out(b_ref, case), _out(b_na, case)
        assert np.array_equal(got, want), f"{case}: differs from the scratch entry point"
        o = reference(*ref)
        check_attention(got.reshape(-1, case[4]), o, case[5], f"no-alloc {case}")


def test_noalloc_contiguous_then_smaller(hip):
    for S, Hq, Hkv, Skv, D, splits, dtype, seed in [(8, 32, 8, 4096, 128, 16, "bf16", 7),
                                                   (2, 8, 2, 300, 64, 3, "f16", 8)]:
        print(f"no-alloc contiguous B={S} Skv={Skv} splits={splits}", flush=True)
        qb, _ = quantize(uniform((S, Hq, 1, D), seed), dtype)
        kb, _ = quantize(uniform((S, Hkv, Skv, D), seed + 1), dtype)
        vb, _ = quantize(uniform((S, Hkv, Skv, D), seed + 2), dtype)
        dq, dk, dv = (H.DeviceBuffer.from_array(x) for x in (qb, kb, vb))
        outs = []
        for scratch in (True, False):
            dout = H.DeviceBuffer(S * Hq * D * ELEM_BYTES[dtype])
            parts = H.DeviceBuffer(4 * sca_amd.hip_lib().sca_hip_decode_partial_elements(
                S, Hq, splits, D)) if scratch else None
            p = decode_params(dq, dk, dv, dout, parts, B=S, Hq=Hq, Hkv=Hkv, Skv=Skv, D=D,
                              splits=splits, dtype=dtype)
            (H.decode_splitk if scratch else H.decode_splitk_noalloc)(p)
            sca_amd.synchronize()
            outs.append(dout.download(np.uint16))
        assert np.array_equal(outs[0], outs[1])


def test_noalloc_rejects_scratch_arguments_and_oversized_partials(hip):
    case = CASES[1]
    p, bufs, _ = _paged_params(case, with_scratch=True)
    with pytest.raises(H.HipError) as e:
        H.decode_splitk_noalloc(p)  # caller scratch is refused, not silently ignored
    assert e.value.code == 2008
    p, bufs, _ = _paged_params(case, with_scratch=False)
    p.num_splits = 65535  # 20*32*65535*66*4 B of partials: beyond the 16 MiB maximum
    with pytest.raises(H.HipError) as e:
        H.decode_splitk_noalloc(p)
    assert e.value.code == 2008 and "static scratch" in str(e.value)

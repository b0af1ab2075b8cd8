"""Flash prefill parity on the GPU, through the C ABI (sca_hip_flash_fwd), against the FP64 oracle.

Case lists follow the reference's tests/kernel/test_flash_correctness.cu:123-214 and
tests/kernel/test_numerics.cu:77-110 (seeds included), plus the BASELINE configurations at full size
(checked on sampled rows) with size-independent properties.
"""

import numpy as np
import pytest

import oracle.oracle as orc
import sca_amd
from sca_amd import hip as H
from attn_util import (DTYPE_ID, bhsd_to_bshd, check_attention, normal, quantize, run_flash, to_float,
                       uniform)

pytestmark = pytest.mark.gpu

HEAD_DIMS = [32, 64, 96, 128, 160, 192, 256]


def _case(dtype, causal, B, Hq, Hkv, Sq, Skv, D, seed, abs_gate=True, want_lse=False):
    # reference seeds: q=seed, k=seed+7919, v=seed+104729 (test_flash_correctness.cu:39-41)
    q = uniform((B, Hq, Sq, D), seed)
    k = uniform((B, Hkv, Skv, D), seed + 7919)
    v = uniform((B, Hkv, Skv, D), seed + 104729)
    qb, qd = quantize(q, dtype)
    kb, kd = quantize(k, dtype)
    vb, vd = quantize(v, dtype)
    out, lse = run_flash(qb, kb, vb, dtype, causal, B=B, Hq=Hq, Hkv=Hkv, Sq=Sq, Skv=Skv, D=D,
                         want_lse=want_lse)
    ref, ref_lse = orc.reference_attention(qd, kd, vd, causal)
    tag = f"flash {dtype} causal={causal} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Skv={Skv} D={D} seed={seed}"
    print(tag, flush=True)
    check_attention(out.reshape(-1, D), ref, dtype, tag, abs_gate=abs_gate)
    if want_lse:
        err = float(np.max(np.abs(lse.reshape(-1).astype(np.float64) - ref_lse)))
        assert err <= 1e-2, f"{tag}: LSE err {err}"
    return out


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_dtypes_and_head_dims(hip, dtype, causal):
    seed = 20000 + (0 if dtype == "f16" else 14) + (7 if causal else 0)
    for i, d in enumerate(HEAD_DIMS):
        _case(dtype, causal, 1, 8, 8, 128, 128, d, seed + i)


@pytest.mark.parametrize("seq", [1, 7, 63, 64, 65, 127, 128, 129, 1024])
def test_non_tile_multiples(hip, seq):
    for j, causal in enumerate([False, True]):
        _case("f16", causal, 1, 8, 8, seq, seq, 128, 30000 + 2 * seq + j)


@pytest.mark.parametrize("skv", [192, 256, 257, 320, 448, 449])
def test_key_tile_counts(hip, skv):
    # 3 to 8 key tiles of 64: every parity of the last step within the paired-barrier steps of
    # the 128-row kernel, with and without a partial tail tile; causal is bottom-right aligned
    for j, causal in enumerate([False, True]):
        _case("bf16", causal, 1, 4, 2, 96, skv, 128, 31000 + 2 * skv + j)
        _case("f16", causal, 1, 4, 4, 64, skv, 64, 32000 + 2 * skv + j)


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_gqa_groups(hip, group):
    _case("f16", True, 2, 8 * group, 8, 96, 160, 128, 40000 + group)


def test_lse_matches_logsumexp(hip):
    _case("f16", False, 1, 4, 2, 64, 64, 64, 50123, want_lse=True)
    _case("bf16", True, 2, 8, 2, 100, 300, 128, 50124, want_lse=True)


@pytest.mark.parametrize("sq,skv,D,dtype", [(320, 320, 128, "f16"), (448, 512, 64, "bf16"),
                                            (577, 700, 128, "bf16"), (64, 64, 128, "f16")])
def test_causal_two_group_pairs(hip, sq, skv, D, dtype):
    # Small causal grids run complementary 64-row tiles in two wave groups: odd tile counts
    # leave a middle tile split between the groups, skv > sq moves the diagonal, and the long
    # tile's two halves and the short tile are written by different waves (output and LSE).
    _case(dtype, True, 1, 4, 2, sq, skv, D, 51000 + sq + D, want_lse=True)


@pytest.mark.parametrize("B,Hq,Hkv,sq,skv,D,dtype", [
    (2, 8, 2, 193, 450, 64, "bf16"),    # GQA group 4, two batches, ragged rows and keys
    (1, 8, 8, 1, 700, 128, "f16"),      # one query row far below the diagonal
    (1, 2, 1, 1473, 1473, 128, "f16"),  # 24 row tiles with a 1-row tail, 12 pairs
    (3, 4, 4, 130, 130, 64, "f16"),     # three tiles: one pair and a lone middle tile
    (1, 2, 2, 2100, 2100, 128, "f16"),  # 33 tiles: the lone middle tile runs both phases alone
    (1, 2, 1, 1500, 2000, 64, "bf16"),  # diagonal moved by 500 keys, long two-phase pairs
    (1, 2, 2, 380, 380, 128, "bf16"),   # 6 tiles: pairs at the single/two-phase boundary
])
def test_causal_two_group_pairs_shapes(hip, B, Hq, Hkv, sq, skv, D, dtype):
    _case(dtype, True, B, Hq, Hkv, sq, skv, D, 52000 + sq + skv + D, want_lse=True)


def test_bshd_layout_equals_bhsd(hip):
    B, Hq, Hkv, S, D = 2, 8, 4, 200, 128
    q, k, v = uniform((B, Hq, S, D), 7), uniform((B, Hkv, S, D), 8), uniform((B, Hkv, S, D), 9)
    qb, _ = quantize(q, "f16")
    kb, _ = quantize(k, "f16")
    vb, _ = quantize(v, "f16")
    a, _ = run_flash(qb, kb, vb, "f16", True, B=B, Hq=Hq, Hkv=Hkv, Sq=S, Skv=S, D=D)
    b, _ = run_flash(bhsd_to_bshd(qb), bhsd_to_bshd(kb), bhsd_to_bshd(vb), "f16", True, B=B,
                     Hq=Hq, Hkv=Hkv, Sq=S, Skv=S, D=D, layout="bshd")
    assert np.array_equal(a, b), "BSHD and BHSD inputs must give bit-identical outputs"


@pytest.mark.parametrize("magnitude", [0.0, 1.0, 10.0, 1e2, 1e4])
def test_extreme_logits_stay_finite(hip, magnitude):
    # test_numerics.cu:29-75: Q/K ~ U(-mag, mag), V ~ U(-1,1), fp16, H=4, S=64, D=128
    seed = 1234 + int(magnitude)
    q = uniform((1, 4, 64, 128), seed, -magnitude, magnitude)
    k = uniform((1, 4, 64, 128), seed + 1, -magnitude, magnitude)
    v = uniform((1, 4, 64, 128), seed + 2)
    qb, qd = quantize(q, "f16")
    kb, kd = quantize(k, "f16")
    vb, vd = quantize(v, "f16")
    out, _ = run_flash(qb, kb, vb, "f16", False, B=1, Hq=4, Hkv=4, Sq=64, Skv=64, D=128)
    ref, _ = orc.reference_attention(qd, kd, vd, False)
    assert np.all(np.isfinite(out))
    err = float(np.max(np.abs(out.reshape(-1, 128) - ref)))
    assert err <= 5e-3, f"magnitude={magnitude}: max abs err {err}"


def test_uniform_rows_and_long_sequence(hip):
    # all-equal logits (magnitude 0) => mean of the visible V rows; causal Sq=1 sees everything
    for sq, skv, d, causal, seed in [(1, 1, 64, False, 77), (1, 1024, 128, True, 78)]:
        v = uniform((1, 4, skv, d), seed + 2)
        vb, vd = quantize(v, "f16")
        zeros = np.zeros((1, 4, sq, d), np.uint16)
        kz = np.zeros((1, 4, skv, d), np.uint16)
        out, _ = run_flash(zeros, kz, vb, "f16", causal, B=1, Hq=4, Hkv=4, Sq=sq, Skv=skv, D=d)
        expect = vd.mean(axis=2, keepdims=True).repeat(sq, axis=2)
        assert float(np.max(np.abs(out - expect))) <= 2e-3
    # long sequence, causal, bottom-right aligned: Sq=512, Skv=8192 (test_numerics.cu:104-107)
    _case("f16", True, 1, 4, 4, 512, 8192, 128, 4242, abs_gate=False)


def _sample_rows(B, H, S, n, seed):
    rng = np.random.default_rng(seed)
    rows = set(rng.integers(0, B * H * S, size=n).tolist())
    for b in range(B):
        for h in (0, H - 1):
            for i in (0, 1, S - 1, S // 2):
                rows.add((b * H + h) * S + i)
    return np.array(sorted(rows), dtype=np.int64)


@pytest.mark.parametrize("causal", [True, False])
def test_baseline_c2_full_size(hip, causal):
    # C2: B=1, H=8, D=128, S=4096, fp16, N(0,1) inputs
    B, H, S, D = 1, 8, 4096, 128
    q, k, v = normal((B, H, S, D), 2001), normal((B, H, S, D), 2002), normal((B, H, S, D), 2003)
    qb, qd = quantize(q, "f16")
    kb, kd = quantize(k, "f16")
    vb, vd = quantize(v, "f16")
    out, lse = run_flash(qb, kb, vb, "f16", causal, B=B, Hq=H, Hkv=H, Sq=S, Skv=S, D=D,
                         want_lse=True)
    # Causal: every one of the 32,768 rows against the FP64 oracle (the pair kernel's tile
    # pairing and the XCD order decide which workgroup computes which rows, so a sample could
    # miss a misplaced tile); non-causal: a sample of rows.
    rows = None if causal else _sample_rows(B, H, S, 96, 7)
    ref, ref_lse = orc.reference_attention(qd, kd, vd, causal, rows=rows)
    got = out.reshape(-1, D) if rows is None else out.reshape(-1, D)[rows]
    got_lse = lse.reshape(-1) if rows is None else lse.reshape(-1)[rows]
    check_attention(got, ref, "f16", f"C2 causal={causal}")
    assert float(np.max(np.abs(got_lse - ref_lse))) <= 1e-2
    # size-independent property: V = constant c  =>  every output row is exactly c
    ones = np.full((B, H, S, D), 0x3C00, np.uint16)  # fp16 1.0
    o1, _ = run_flash(qb, kb, ones, "f16", causal, B=B, Hq=H, Hkv=H, Sq=S, Skv=S, D=D)
    assert float(np.max(np.abs(o1 - 1.0))) <= 1e-3, "constant V must give back the constant"


def test_baseline_c3_gqa_bf16_full_size(hip):
    # C3: B=4, Hq=32, Hkv=8, D=128, S=8192, causal, bf16, N(0, 0.5^2)
    B, Hq, Hkv, S, D = 4, 32, 8, 8192, 128
    q, k, v = normal((B, Hq, S, D), 3001, 0.5), normal((B, Hkv, S, D), 3002, 0.5), \
        normal((B, Hkv, S, D), 3003, 0.5)
    qb, qd = quantize(q, "bf16")
    del q
    kb, kd = quantize(k, "bf16")
    vb, vd = quantize(v, "bf16")
    out, _ = run_flash(qb, kb, vb, "bf16", True, B=B, Hq=Hq, Hkv=Hkv, Sq=S, Skv=S, D=D)
    rows = _sample_rows(B, Hq, S, 64, 11)
    ref, _ = orc.reference_attention(qd, kd, vd, True, rows=rows)
    check_attention(out.reshape(-1, D)[rows], ref, "bf16", "C3 GQA bf16")
    # Every row of one whole (batch, KV head) group: batch 1, KV head 3 = query heads 12..15,
    # 4 x 8,192 rows. Its group index 1*8 + 3 = 11 puts it on XCD slot 3 of the XCD order.
    b, h_kv, gsz = 1, 3, Hq // Hkv
    heads = np.arange(h_kv * gsz, (h_kv + 1) * gsz)
    rows = ((b * Hq + heads)[:, None] * S + np.arange(S)[None, :]).reshape(-1)
    ref, _ = orc.reference_attention(qd, kd, vd, True, rows=rows)
    check_attention(out.reshape(-1, D)[rows], ref, "bf16", "C3 GQA bf16, group (1, 3) all rows")


@pytest.mark.parametrize("seq", [1, 7, 63, 1000])
def test_baseline_c3_ragged_tail(hip, seq):
    B, Hq, Hkv, D = 1, 32, 8, 128
    q, k, v = normal((B, Hq, seq, D), 3100 + seq, 0.5), normal((B, Hkv, seq, D), 3200 + seq, 0.5), \
        normal((B, Hkv, seq, D), 3300 + seq, 0.5)
    qb, qd = quantize(q, "bf16")
    kb, kd = quantize(k, "bf16")
    vb, vd = quantize(v, "bf16")
    out, _ = run_flash(qb, kb, vb, "bf16", True, B=B, Hq=Hq, Hkv=Hkv, Sq=seq, Skv=seq, D=D)
    ref, _ = orc.reference_attention(qd, kd, vd, True)
    check_attention(out.reshape(-1, D), ref, "bf16", f"C3 ragged S={seq}")


def _varlen_case(dtype, causal, lens_q, lens_kv, Hq, Hkv, D, seed):
    """One packed launch (sca_hip_flash_fwd_varlen) checked sequence by sequence."""
    import sca_amd
    from sca_amd import hip as H
    from attn_util import to_float
    Tq, Tkv = int(sum(lens_q)), int(sum(lens_kv))
    q = uniform((Tq, Hq, D), seed)
    k = uniform((Tkv, Hkv, D), seed + 7919)
    v = uniform((Tkv, Hkv, D), seed + 104729)
    (qb, qd), (kb, kd), (vb, vd) = quantize(q, dtype), quantize(k, dtype), quantize(v, dtype)
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_kv = np.concatenate([[0], np.cumsum(lens_kv)]).astype(np.int32)
    tiles = H.flash_varlen_tiles(cu_q, cu_kv, causal)
    bufs = [H.DeviceBuffer.from_array(a) for a in (qb, kb, vb, cu_q, cu_kv, tiles)]
    dout = H.DeviceBuffer.zeros(Tq * Hq * D * 2)
    p = H.FlashVarlenParams()
    p.q, p.k, p.v, p.out = bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, dout.ptr
    p.cu_seqlens_q, p.cu_seqlens_kv, p.tiles = bufs[3].ptr, bufs[4].ptr, bufs[5].ptr
    p.num_seqs, p.num_tiles, p.max_seq_kv = len(lens_q), len(tiles), int(max(lens_kv))
    p.num_heads, p.num_kv_heads, p.head_dim = Hq, Hkv, D
    p.q_sh, p.q_ss, p.k_sh, p.k_ss = D, Hq * D, D, Hkv * D
    p.v_sh, p.v_ss, p.o_sh, p.o_ss = D, Hkv * D, D, Hq * D
    p.scale = float(np.float32(1.0 / np.sqrt(D)))
    p.causal = int(causal)
    p.dtype = H.DTYPE_F16 if dtype == "f16" else H.DTYPE_BF16
    H.flash_fwd_varlen(p)
    sca_amd.synchronize()
    out = to_float(dout.download(np.uint16), dtype).reshape(Tq, Hq, D)
    tag = f"varlen {dtype} causal={causal} lens_q={list(lens_q)[:6]} D={D}"
    print(tag, flush=True)
    for s in range(len(lens_q)):
        sq = slice(cu_q[s], cu_q[s + 1])
        skv = slice(cu_kv[s], cu_kv[s + 1])
        ref, _ = orc.reference_attention(qd[sq].transpose(1, 0, 2)[None],
                                         kd[skv].transpose(1, 0, 2)[None],
                                         vd[skv].transpose(1, 0, 2)[None], causal)
        got = out[sq].transpose(1, 0, 2).reshape(-1, D)
        check_attention(got, ref.reshape(-1, D), dtype, f"{tag} seq {s}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_one_launch(hip, D, causal):
    lens_q = [1, 7, 63, 1000, 64, 65, 129, 300]
    lens_kv = [1, 7, 63, 1000, 64, 65, 129, 300] if causal else [5, 700, 63, 1000, 64, 1, 200, 301]
    _varlen_case("f16", causal, lens_q, lens_kv, 8, 8, D, 61000 + D + int(causal))
    # GQA, bf16, S_kv > S_q (bottom-right diagonal per sequence)
    _varlen_case("bf16", causal, [96, 3, 257], [160, 40, 400], 8, 2, D, 62000 + D + int(causal))


@pytest.mark.parametrize("causal", [False, True])
def test_kv_extent_beyond_2gib_falls_back(hip, causal):
    """K/V rows so far apart that a launch's K/V extent passes 2 GiB: the DMA-based kernels
    address K/V with 32-bit buffer offsets, so the launcher takes the register kernel instead,
    whose results must match the oracle like any other."""
    Sq = Skv = 1024
    D, dtype = 128, "f16"
    # (Skv + 256) rows of this stride exceed 2^31 bytes (the pair kernel's check; the wide
    # kernel's, with 512 rows of overrun, too).
    row = ((1 << 31) // (2 * (Skv + 256)) + 8) // 8 * 8
    q = uniform((1, 1, Sq, D), 51)
    k = uniform((1, 1, Skv, D), 52)
    v = uniform((1, 1, Skv, D), 53)
    (qb, qd), (kb, kd), (vb, vd) = quantize(q, dtype), quantize(k, dtype), quantize(v, dtype)
    nbytes = ((Skv - 1) * row + D) * 2
    L = sca_amd.hip_lib()
    dk, dv = H.DeviceBuffer(nbytes), H.DeviceBuffer(nbytes)
    for dst, src in ((dk, kb), (dv, vb)):
        rows = np.ascontiguousarray(src.reshape(Skv, D))
        for j in range(Skv):
            H.check(L.sca_hip_memcpy(dst.ptr + j * row * 2, rows[j].ctypes.data, D * 2, H.COPY_H2D))
    dq = H.DeviceBuffer.from_array(qb)
    dout = H.DeviceBuffer(Sq * D * 2)
    p = H.FlashParams()
    p.q, p.k, p.v, p.out, p.lse = dq.ptr, dk.ptr, dv.ptr, dout.ptr, None
    p.batch, p.num_heads, p.num_kv_heads = 1, 1, 1
    p.seq_q, p.seq_kv, p.head_dim = Sq, Skv, D
    p.q_sb, p.q_sh, p.q_ss = Sq * D, Sq * D, D
    p.k_sb, p.k_sh, p.k_ss = Skv * row, Skv * row, row
    p.v_sb, p.v_sh, p.v_ss = Skv * row, Skv * row, row
    p.o_sb, p.o_sh, p.o_ss = Sq * D, Sq * D, D
    p.scale = float(np.float32(1.0 / np.sqrt(np.float64(D))))
    p.causal = 1 if causal else 0
    p.dtype = DTYPE_ID[dtype]
    p.diagonal = 0
    H.flash_fwd(p)
    sca_amd.synchronize()
    out = to_float(dout.download(np.uint16), dtype).reshape(Sq, D)
    ref, _ = orc.reference_attention(qd, kd, vd, causal)
    check_attention(out, ref, dtype, f"2 GiB extent causal={causal}", abs_gate=True)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,dtype", [
    (2, 8, 4, 300, 128, "f16"),    # 8 (batch, KV head) groups of 2 heads: XCD order, wide kernel
    (2, 16, 4, 130, 64, "bf16"),   # groups of 4, two row tiles
    (1, 64, 8, 200, 128, "bf16"),  # groups of 8
    (4, 8, 2, 257, 96, "f16"),     # groups of 4, register-staged kernel (head dim 96)
    (1, 16, 8, 900, 128, "f16"),   # small causal grid: pair kernel with groups of 2
    (3, 12, 4, 150, 64, "f16"),    # 12 groups: not a multiple of 8, plain order
])
def test_xcd_group_order(hip, B, Hq, Hkv, S, D, dtype):
    """Workgroups are dealt to XCDs by (batch, KV head) group when the group count divides by
    eight; every (row tile, head) must still be computed exactly once."""
    for j, causal in enumerate([False, True]):
        _case(dtype, causal, B, Hq, Hkv, S, S, D, 88000 + 97 * Hq + S + j)

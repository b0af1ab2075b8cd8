"""Paged decode parity on the GPU through sca_hip_decode_splitk_paged, against the FP64 oracle
applied to the page-table gather of the block-major pool (page_table.cuh:18-36).

Case lists follow tests/kernel/test_paged_correctness.cu:134-166, with a seeded random
permutation as the block table (the reference's own tests only ever see ascending LIFO ids).
"""

import numpy as np
import pytest

import oracle.oracle as orc
import sca_amd
from sca_amd import hip as H
from attn_util import check_attention, decode_params, normal, quantize, uniform, to_float, \
    ELEM_BYTES

pytestmark = pytest.mark.gpu


def build_pool(lengths, bs, Hkv, D, dtype, seed, slack=3, gen="uniform"):
    """Block-major pool [num_blocks, bs, Hkv, D] with a permuted block table per sequence."""
    rng = np.random.default_rng(seed)
    need = [(L + bs - 1) // bs for L in lengths]
    num_blocks = sum(need) + slack
    perm = rng.permutation(num_blocks).astype(np.int32)
    max_blocks = max(max(need), 1) + 2
    table = np.full((len(lengths), max_blocks), -1, np.int32)
    pos = 0
    for s, n in enumerate(need):
        table[s, :n] = perm[pos:pos + n]
        pos += n
    shape = (num_blocks, bs, Hkv, D)
    if gen == "uniform":
        k, v = uniform(shape, seed + 11), uniform(shape, seed + 22)
    else:
        k, v = normal(shape, seed + 11), normal(shape, seed + 22)
    kb, kd = quantize(k, dtype)
    vb, vd = quantize(v, dtype)
    return num_blocks, max_blocks, table, kb, kd, vb, vd


def run_paged(qb, kb, vb, table, lengths, dtype, *, Hq, Hkv, D, bs, num_blocks, splits,
              pass_lens=True, longest_first=True, slot_waves=0):
    S = len(lengths)
    max_blocks = table.shape[1]
    dq = H.DeviceBuffer.from_array(qb)
    dk = H.DeviceBuffer.from_array(kb)
    dv = H.DeviceBuffer.from_array(vb)
    dt = H.DeviceBuffer.from_array(table)
    dl = H.DeviceBuffer.from_array(np.asarray(lengths, np.int32))
    dout = H.DeviceBuffer(S * Hq * D * ELEM_BYTES[dtype])
    parts = H.DeviceBuffer(4 * sca_amd.hip_lib().sca_hip_decode_partial_elements(S, Hq, splits, D))
    p = decode_params(dq, dk, dv, dout, parts, B=S, Hq=Hq, Hkv=Hkv, Skv=num_blocks * bs, D=D,
                      splits=splits, dtype=dtype, k_strides=(0, D, Hkv * D))
    p.page_table = dt.ptr
    p.block_size = bs
    p.max_blocks_per_seq = max_blocks
    p.num_kv_blocks = num_blocks
    p.seq_lens = dl.ptr if pass_lens else None
    order = H.DeviceBuffer(8 * S)
    p.batch_order = order.ptr if longest_first else None
    p.slot_waves = slot_waves
    H.decode_splitk_paged(p)
    sca_amd.synchronize()
    return to_float(dout.download(np.uint16), dtype).reshape(S, Hq, D)


def reference(qd, kd, vd, table, lengths, bs, num_blocks):
    outs = []
    for s, L in enumerate(lengths):
        kc, valid = orc.paged_gather(kd, table[s], L, bs, num_blocks)
        vc, _ = orc.paged_gather(vd, table[s], L, bs, num_blocks)
        kc, vc = kc[:, valid], vc[:, valid]
        o, _ = orc.reference_attention(qd[s:s + 1], kc[None], vc[None], True)
        outs.append(o)
    return np.concatenate(outs)


def _case(lengths, bs, Hq, Hkv, D, dtype, seed, splits=16, gen="uniform", longest_first=True,
          slot_waves=0):
    nb, mb, table, kb, kd, vb, vd = build_pool(lengths, bs, Hkv, D, dtype, seed, gen=gen)
    q = uniform((len(lengths), Hq, 1, D), seed) if gen == "uniform" else \
        normal((len(lengths), Hq, 1, D), seed)
    qb, qd = quantize(q, dtype)
    out = run_paged(qb, kb, vb, table, lengths, dtype, Hq=Hq, Hkv=Hkv, D=D, bs=bs, num_blocks=nb,
                    splits=splits, longest_first=longest_first, slot_waves=slot_waves)
    ref = reference(qd, kd, vd, table, lengths, bs, nb)
    tag = (f"paged {dtype} lens={lengths[:4]} bs={bs} Hq={Hq} Hkv={Hkv} D={D} splits={splits} "
           f"longest_first={longest_first} slot_waves={slot_waves}")
    print(tag, flush=True)
    check_attention(out.reshape(-1, D), ref, dtype, tag)


# slot_waves: 0 = the paged default (one wave per KV-head slot), 4 = four waves share a slot's
# key tiles (the plan's choice for ragged batches with few slots per CU).
@pytest.mark.parametrize("slot_waves", [0, 4])
@pytest.mark.parametrize("bs", [1, 8, 16, 32])
def test_every_block_size(hip, bs, slot_waves):
    _case([257], bs, 8, 8, 128, "f16", 80000 + bs, slot_waves=slot_waves)


@pytest.mark.parametrize("group", [1, 2, 4])
def test_gqa_and_lengths(hip, group):
    for j, L in enumerate([33, 129, 512]):
        _case([L], 16, 8 * group, 8, 64, "f16", 81000 + 3 * group + j)


def test_many_ragged_sequences_bf16(hip):
    rng = np.random.default_rng(5)
    lengths = rng.integers(1, 3000, size=12).tolist()
    _case(lengths, 16, 32, 8, 128, "bf16", 82001, gen="normal")
    _case(lengths, 16, 32, 8, 128, "bf16", 82002, splits=1, gen="normal")
    _case(lengths, 16, 32, 8, 128, "bf16", 82003, splits=3, gen="normal", longest_first=False)
    _case(lengths + [0, 5], 16, 32, 8, 64, "f16", 82004, splits=4)
    _case(lengths, 16, 32, 8, 128, "bf16", 82005, splits=6, gen="normal", slot_waves=4)
    _case(lengths + [0, 5], 16, 32, 8, 64, "f16", 82006, splits=3, slot_waves=4,
          longest_first=False)
    _case(lengths, 16, 64, 4, 128, "bf16", 82007, splits=2, gen="normal", slot_waves=1)


def test_slot_waves_outside_0_1_4_rejected(hip):
    lengths = [40]
    nb, mb, table, kb, kd, vb, vd = build_pool(lengths, 16, 2, 64, "f16", 82101)
    qb, _ = quantize(uniform((1, 8, 1, 64), 82101), "f16")
    for bad in (2, 3, 8, -1):
        with pytest.raises(H.HipError, match="slot_waves"):
            run_paged(qb, kb, vb, table, lengths, "f16", Hq=8, Hkv=2, D=64, bs=16, num_blocks=nb,
                      splits=2, slot_waves=bad)


def test_unmapped_pages_contribute_nothing(hip):
    # a -1 hole and an out-of-pool id in the middle of the table: those tokens are skipped
    lengths = [160]
    bs, Hq, Hkv, D = 16, 8, 2, 128
    nb, mb, table, kb, kd, vb, vd = build_pool(lengths, bs, Hkv, D, "f16", 83001)
    table[0, 3] = -1
    table[0, 5] = nb + 7
    q = uniform((1, Hq, 1, D), 83001)
    qb, qd = quantize(q, "f16")
    out = run_paged(qb, kb, vb, table, lengths, "f16", Hq=Hq, Hkv=Hkv, D=D, bs=bs, num_blocks=nb,
                    splits=4)
    ref = reference(qd, kd, vd, table, lengths, bs, nb)
    check_attention(out.reshape(-1, D), ref, "f16", "paged holes")


def test_null_seq_lens_uses_pool_upper_bound(hip):
    # without seq_lens every mapped page of the row is attended in full (decode_splitk.cu:102)
    lengths = [40]
    bs, Hq, Hkv, D = 16, 4, 4, 64
    nb, mb, table, kb, kd, vb, vd = build_pool(lengths, bs, Hkv, D, "f16", 84001)
    q = uniform((1, Hq, 1, D), 84001)
    qb, qd = quantize(q, "f16")
    out = run_paged(qb, kb, vb, table, lengths, "f16", Hq=Hq, Hkv=Hkv, D=D, bs=bs, num_blocks=nb,
                    splits=4, pass_lens=False)
    full = 3 * bs  # 3 mapped pages
    ref = reference(qd, kd, vd, table, [full], bs, nb)
    check_attention(out.reshape(-1, D), ref, "f16", "paged null seq_lens")


@pytest.mark.parametrize("bs,D", [(1, 64), (16, 128), (32, 64)])
def test_nan_outside_attended_rows_is_never_used(hip, bs, D):
    # Every pool row that no sequence attends (free blocks, the tail of each last page) holds
    # NaN bits: tiles that straddle a sequence's end or an unmapped page must not let them in.
    lengths = [37, 1, 100, 16 * 5 + 3]
    Hq, Hkv = 8, 2
    nb, mb, table, kb, kd, vb, vd = build_pool(lengths, bs, Hkv, D, "bf16", 85001 + bs)
    table[2, 1] = -1
    used = np.zeros((nb, bs), bool)
    for s, L in enumerate(lengths):
        for t in range(L):
            page = table[s, t // bs]
            if 0 <= page < nb:
                used[page, t % bs] = True
    kb = kb.copy()
    vb = vb.copy()
    kb[~used] = 0x7FC0
    vb[~used] = 0x7FC0
    q = uniform((len(lengths), Hq, 1, D), 85001)
    qb, qd = quantize(q, "bf16")
    ref = reference(qd, kd, vd, table, lengths, bs, nb)
    for splits, waves in ((1, 0), (3, 0), (1, 4), (3, 4)):
        out = run_paged(qb, kb, vb, table, lengths, "bf16", Hq=Hq, Hkv=Hkv, D=D, bs=bs,
                        num_blocks=nb, splits=splits, slot_waves=waves)
        check_attention(out.reshape(-1, D), ref, "bf16",
                        f"paged NaN pool bs={bs} D={D} splits={splits} slot_waves={waves}")


def test_large_ragged_batch_ranked_through_scratch(hip):
    # more than 256 sequences: the longest-first order comes from the batch_order scratch
    rng = np.random.default_rng(86001)
    lengths = rng.integers(0, 90, size=300).tolist()
    _case(lengths, 16, 8, 2, 64, "f16", 86001, splits=2)
    _case(lengths, 16, 8, 2, 64, "f16", 86002, splits=3, longest_first=False)
    _case(lengths, 16, 8, 2, 64, "f16", 86003, splits=2, slot_waves=4)



def _bf16_normal(rng, shape):
    """bf16 bit patterns of N(0, 1) samples (upper half of the fp32 word)."""
    f = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
    return (f.view(np.uint32) >> 16).astype(np.uint16).reshape(shape)


def _bf16_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_c5_full_size_against_fp32(hip):
    """C5 at its full shape (64 sequences, L ~ U[512, 16384], bs 16, Hq 32, Hkv 8, D 128, bf16,
    permuted block table, 2.2 GB pool), run twice: 12 splits with one wave per KV-head slot (the
    pool-sized split count) and 3 splits with four waves per slot (the length-aware plan on a
    256-CU MI355X). Each sequence
    is checked against an fp32 softmax(q k^T * scale) v over the rows its block table gathers
    (page_table.cuh:18-36), within the bf16 tolerance of the other paged cases (max abs error
    <= 1.6e-2 of max |ref|)."""
    S, bs, Hq, Hkv, D, splits = 64, 16, 32, 8, 128, 12
    rng = np.random.default_rng(5005)
    lengths = rng.integers(512, 16384 + 1, size=S).astype(np.int64)
    need = (lengths + bs - 1) // bs
    nb = int(need.sum()) + 64
    perm = rng.permutation(nb).astype(np.int32)
    table = np.full((S, int(need.max())), -1, np.int32)
    pos = 0
    for s in range(S):
        table[s, :need[s]] = perm[pos:pos + need[s]]
        pos += need[s]
    kb = _bf16_normal(rng, (nb * bs, Hkv, D))
    vb = _bf16_normal(rng, (nb * bs, Hkv, D))
    qb = _bf16_normal(rng, (S, Hq, 1, D))
    runs = {}
    for sp, waves in ((splits, 1), (3, 4)):
        print(f"paged C5 full size: seqs={S} pool blocks={nb} splits={sp} slot_waves={waves}",
              flush=True)
        runs[(sp, waves)] = run_paged(qb, kb, vb, table, lengths.tolist(), "bf16", Hq=Hq,
                                      Hkv=Hkv, D=D, bs=bs, num_blocks=nb, splits=sp,
                                      slot_waves=waves)

    scale = np.float32(1.0 / np.sqrt(D))
    qf = _bf16_to_f32(qb).reshape(S, Hkv, Hq // Hkv, D)  # query heads grouped by KV head
    ref = np.empty((S, Hq, D), np.float64)
    for s in range(S):
        L = int(lengths[s])
        idx = (table[s, :need[s]].astype(np.int64)[:, None] * bs + np.arange(bs)).reshape(-1)[:L]
        ks = _bf16_to_f32(kb[idx]).transpose(1, 0, 2)  # [Hkv, L, D]
        vs = _bf16_to_f32(vb[idx]).transpose(1, 0, 2)
        sc = np.matmul(qf[s], ks.transpose(0, 2, 1)) * scale  # [Hkv, group, L]
        sc -= sc.max(axis=-1, keepdims=True)
        w = np.exp(sc)
        w /= w.sum(axis=-1, keepdims=True)
        ref[s] = np.matmul(w, vs).reshape(Hq, D)
    for (sp, waves), got in runs.items():
        check_attention(got.reshape(-1, D), ref.reshape(-1, D), "bf16",
                        f"paged C5 full size splits={sp} slot_waves={waves}")


@pytest.mark.parametrize("bs,L,splits", [(2, 9001, 2), (2, 9001, 3), (1, 5000, 1), (4, 20001, 2),
                                         (16, 40000, 1)])
@pytest.mark.parametrize("D,dtype,slot_waves", [(128, "bf16", 0), (128, "bf16", 4),
                                                (96, "f16", 0)])
def test_splits_spanning_several_page_segments(hip, bs, L, splits, D, dtype, slot_waves):
    """Splits longer than one staged page-id segment (2048 pages), starting on and off a page
    boundary: the segment loop restages the page ids of every segment. D=128 bf16 runs the MFMA
    kernel (one or four waves per KV-head slot), D=96 the VALU kernel."""
    print(f"paged multi-segment bs={bs} L={L} splits={splits} D={D} {dtype} "
          f"slot_waves={slot_waves}", flush=True)
    _case([L, 3], bs, 8, 2, D, dtype, 87000 + bs + splits + D, splits=splits,
          slot_waves=slot_waves)

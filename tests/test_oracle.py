"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Every oracle function is checked against something other than its own formula: the reference's
own outputs (golden fixtures recorded from the reference's host code), known answers from the
reference's tests, an independent library implementation (torch), or a closed form that a
plausible mistake (dropped term, wrong sign or index, transposed operand) would violate.
CPU only."""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

import oracle.oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# ---- input generation / encoding ----------------------------------------------------------------

def test_xorshift32_known_answers():
    # Marsaglia's xorshift32 (13, 17, 5) from state 1 yields 270369, then 67634689.
    u = orc.random_floats(2, 1, 0.0, 1.0).astype(np.float64)
    assert np.float32(270369 / 4294967295.0) == np.float32(u[0])
    assert np.float32(67634689 / 4294967295.0) == np.float32(u[1])
    # seed 0 is mapped to 1
    assert np.array_equal(orc.random_floats(8, 0), orc.random_floats(8, 1))


def test_random_floats_range_and_moments():
    x = orc.random_floats(200_000, 12345, -2.0, 3.0).astype(np.float64)
    assert x.min() >= -2.0 and x.max() <= 3.0
    assert abs(x.mean() - 0.5) < 0.02
    assert abs(x.var() - 25.0 / 12.0) < 0.03


def test_fp16_encoder_matches_ieee_rne_outside_subnormals():
    x = np.concatenate([orc.random_floats(100_000, 7, -70000.0, 70000.0),
                        orc.random_floats(100_000, 8, -1.0, 1.0),
                        np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, 2.0 ** -14,
                                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32)])
    bits, deq = orc.encode(x, "f16")
    ref = torch.from_numpy(x).to(torch.float16)
    normal = np.abs(x) >= 2.0 ** -14
    assert np.array_equal(bits[normal], ref.numpy().view(np.uint16)[normal])
    # The reference's encoder flushes results that would be fp16-subnormal to signed zero.
    tiny = np.array([1e-6, -3e-7, 2.0 ** -15], dtype=np.float32)
    tb, td = orc.encode(tiny, "f16")
    assert tb.tolist() == [0x0000, 0x8000, 0x0000]
    assert np.array_equal(deq, orc.decode_bits(bits, "f16"))


def test_bf16_encoder_matches_torch_rne():
    x = np.concatenate([orc.random_floats(200_000, 9, -1e30, 1e30),
                        orc.random_floats(100_000, 10, -1.0, 1.0),
                        np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -0.0], dtype=np.float32)])
    bits, deq = orc.encode(x, "bf16")
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, ref)
    assert np.array_equal(deq, orc.decode_bits(bits, "bf16"))


# ---- attention ----------------------------------------------------------------------------------

def _torch_attention(q, k, v, causal, scale=None):
    """Independent FP64 attention via torch with an explicit bottom-right causal mask."""
    qt, kt, vt = (torch.from_numpy(np.asarray(a, dtype=np.float64)) for a in (q, k, v))
    B, Hq, Sq, D = qt.shape
    Hkv, Skv = kt.shape[1], kt.shape[2]
    g = Hq // Hkv
    kt = kt.repeat_interleave(g, dim=1)
    vt = vt.repeat_interleave(g, dim=1)
    sc = scale if scale else 1.0 / math.sqrt(D)
    s = torch.einsum("bhid,bhjd->bhij", qt, kt) * sc
    if causal:
        i = torch.arange(Sq)[:, None]
        j = torch.arange(Skv)[None, :]
        s = s.masked_fill(j > i + (Skv - Sq), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    out = torch.softmax(s, dim=-1) @ vt
    return out.reshape(-1, D).numpy(), lse.reshape(-1).numpy()


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,causal", [
    (1, 2, 2, 5, 5, 32, False), (2, 4, 2, 7, 19, 64, True), (1, 8, 1, 1, 33, 128, True),
    (2, 6, 3, 17, 17, 96, True), (1, 2, 1, 3, 40, 256, False)])
def test_reference_attention_matches_torch(B, Hq, Hkv, Sq, Skv, D, causal):
    q = orc.random_floats(B * Hq * Sq * D, 1).reshape(B, Hq, Sq, D)
    k = orc.random_floats(B * Hkv * Skv * D, 2).reshape(B, Hkv, Skv, D)
    v = orc.random_floats(B * Hkv * Skv * D, 3).reshape(B, Hkv, Skv, D)
    out, lse = orc.reference_attention(q, k, v, causal)
    ref_out, ref_lse = _torch_attention(q, k, v, causal)
    np.testing.assert_allclose(out, ref_out, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse, rtol=0, atol=1e-12)
    rows = np.array([0, B * Hq * Sq - 1, (B * Hq * Sq) // 2])
    sub, sub_lse = orc.reference_attention(q, k, v, causal, rows=rows)
    np.testing.assert_array_equal(sub, out[rows])
    np.testing.assert_array_equal(sub_lse, lse[rows])


def test_reference_attention_closed_forms():
    D, S = 64, 37
    v = orc.random_floats(S * D, 5).reshape(1, 1, S, D)
    k = orc.random_floats(S * D, 6).reshape(1, 1, S, D)
    zero_q = np.zeros((1, 1, S, D), dtype=np.float32)
    # q = 0: every visible key has the same logit, so out = mean of the visible values and
    # lse = log(#visible) (causal: row i sees i + 1 keys).
    out, lse = orc.reference_attention(zero_q, k, v, False)
    np.testing.assert_allclose(out, np.tile(v[0, 0].astype(np.float64).mean(0), (S, 1)), atol=1e-12)
    np.testing.assert_allclose(lse, np.full(S, math.log(S)), atol=1e-12)
    out, lse = orc.reference_attention(zero_q, k, v, True)
    csum = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    np.testing.assert_allclose(out, csum, atol=1e-12)
    np.testing.assert_allclose(lse, np.log(np.arange(1, S + 1)), atol=1e-12)
    # One key: the output is that key's value row whatever q is.
    q1 = orc.random_floats(D, 9).reshape(1, 1, 1, D)
    out, lse = orc.reference_attention(q1, k[:, :, :1], v[:, :, :1], False)
    np.testing.assert_allclose(out[0], v[0, 0, 0], atol=1e-12)
    assert abs(lse[0] - float(np.dot(q1[0, 0, 0].astype(np.float64), k[0, 0, 0]) / 8.0)) < 1e-12
    # Explicit scale and GQA head mapping h_kv = h // group: heads 2,3 of a 4:2 layout use kv 1.
    q4 = orc.random_floats(4 * 3 * D, 11).reshape(1, 4, 3, D)
    k2 = orc.random_floats(2 * 5 * D, 12).reshape(1, 2, 5, D)
    v2 = orc.random_floats(2 * 5 * D, 13).reshape(1, 2, 5, D)
    full, _ = orc.reference_attention(q4, k2, v2, False, scale=0.3)
    part, _ = orc.reference_attention(q4[:, 2:4], k2[:, 1:2], v2[:, 1:2], False, scale=0.3)
    np.testing.assert_array_equal(full.reshape(4, 3, D)[2:4].reshape(-1, D), part)


def test_naive_f32_matches_fp64_and_masks_with_minus_infinity():
    B, H, S, D = 1, 4, 48, 64
    q = orc.random_floats(B * H * S * D, 21).reshape(B, H, S, D)
    k = orc.random_floats(B * H * S * D, 22).reshape(B, H, S, D)
    v = orc.random_floats(B * H * S * D, 23).reshape(B, H, S, D)
    for causal in (False, True):
        out, lse = orc.naive_attention(q, k, v, causal)
        ref, ref_lse = orc.reference_attention(q, k, v, causal)
        assert np.abs(out.reshape(-1, D) - ref).max() < 2e-6
        assert np.abs(lse.reshape(-1) - ref_lse).max() < 2e-5
    # Row 0 under the causal mask sees exactly key 0.
    out, _ = orc.naive_attention(q, k, v, True)
    np.testing.assert_allclose(out[0, :, 0], v[0, :, 0], atol=1e-6)


@pytest.mark.parametrize("splits", [1, 2, 3, 4, 8, 16, 64])
def test_splitk_model_is_split_invariant(splits):
    B, Hq, Hkv, S, D = 2, 8, 2, 50, 64
    q = orc.random_floats(B * Hq * D, 31).reshape(B, Hq, 1, D)
    k = orc.random_floats(B * Hkv * S * D, 32).reshape(B, Hkv, S, D)
    v = orc.random_floats(B * Hkv * S * D, 33).reshape(B, Hkv, S, D)
    out, pm, pl, po = orc.splitk_decode(q, k, v, splits)
    ref, _ = orc.reference_attention(q, k, v, False)
    np.testing.assert_allclose(out.reshape(-1, D), ref, atol=1e-12)
    # Splits beyond the length are empty: m = -inf, l = 0.
    if splits > S:
        assert np.isneginf(pm.reshape(B * Hq, splits)[:, -1]).all()
        assert (pl.reshape(B * Hq, splits)[:, -1] == 0).all()
    # Ragged lengths equal a contiguous call on the truncated keys.
    lens = [7, 50]
    out2, *_ = orc.splitk_decode(q, k, v, splits, seq_lens=lens)
    for b, L in enumerate(lens):
        r, _ = orc.reference_attention(q[b:b + 1], k[b:b + 1, :, :L], v[b:b + 1, :, :L], False)
        np.testing.assert_allclose(out2[b], r, atol=1e-12)


def test_paged_gather_against_fancy_indexing():
    nb, bs, H, D = 12, 4, 2, 32
    pool = orc.random_floats(nb * bs * H * D, 41).reshape(nb, bs, H, D)
    row = np.array([5, 0, 11, -1, 3], dtype=np.int32)
    kv, valid = orc.paged_gather(pool, row, 18, bs, nb)
    for j in range(18):
        page = row[j // bs] if j // bs < row.size else -1
        if 0 <= page < nb:
            assert valid[j]
            np.testing.assert_array_equal(kv[:, j], pool[page, j % bs])
        else:
            assert not valid[j] and not kv[:, j].any()


# ---- integer helpers vs the reference's own outputs ----------------------------------------------

def test_integer_helpers_match_reference_goldens():
    kv = load("kv_helpers.json")
    for c in kv["splits_for"]:
        assert orc.splits_for(c["seq_kv"], c["sms"]) == c["value"], c
    for c in kv["partial_elements"]:
        assert orc.partial_elements(*c["args"]) == c["value"]
    for c in kv["slot_mapping"]:
        rc, slots, msg = orc.compute_slot_mapping(c["row"], c["start"], c["n"], c["bs"],
                                                  c["max_blocks"])
        assert rc == c["code"], c
        if rc == 0:
            assert slots.tolist() == c["slots"]
        else:
            assert f"[SCA-{rc}] {msg}" == c["message"]
    esize = {0: 4, 1: 2, 2: 2, 4: 4}
    for c in kv["kv_cache_bytes"]:
        layers, heads, d, bs, nb, seqs, dtype = c["cfg"]
        got = orc.kv_cache_bytes(layers, heads, d, bs, nb, seqs, esize[dtype])
        if c["value"] > 0 and dtype in (0, 1, 2):
            assert got == c["value"], c
        elif dtype in (0, 1, 2):
            assert got <= 0, c
    for c in kv["max_blocks_for_budget"]:
        layers, heads, d, bs, dtype, budget = c["args"]
        assert orc.max_blocks_for_budget(layers, heads, d, bs, esize[dtype], budget) == c["value"]


@pytest.mark.parametrize("index", range(5))
def test_oracle_block_manager_matches_reference_trace(index):
    trace = load("block_manager_traces.json")[index]
    bm = orc.BlockManager(*trace["create"])
    for op, want in zip(trace["ops"], trace["results"]):
        kind = op["op"]
        if kind == "allocate":
            rc, ids, msg = bm.allocate(op["count"])
            assert (rc, ids) == (want["rc"], want["ids"]), op
            assert (f"[SCA-{rc}] {msg}" if rc else msg) == want["msg"], op
        elif kind == "free":
            bm.free(op["ids"])
        elif kind == "append_to_table":
            rc, msg = bm.append_to_table(op["seq"], op["ids"] or None)
            assert rc == want["rc"], op
            assert not rc or f"[SCA-{rc}] {msg}" == want["msg"], op
        elif kind == "reset_seq":
            rc, msg = bm.reset_seq(op["seq"])
            assert rc == want["rc"], op
            assert not rc or f"[SCA-{rc}] {msg}" == want["msg"], op
        else:
            bm.sync()
        assert bm.state() == want["state"], op


def test_oracle_paged_kv_reference_known_answers():
    """test_paged_kv.cpp:44-123 of the reference (block_size 8, head_dim 32, f16)."""
    c = orc.PagedKV(num_blocks=8, block_size=8, max_num_seqs=4)
    assert c.append(0, 3)[0] == 0
    assert c.append(1, 3)[0] == 0
    assert c.append(0, 6)[0] == 0
    assert (c.seq_len(0), c.seq_len(1), c.block_count(0), c.block_count(1)) == (9, 3, 2, 1)
    st = c.stats()
    assert (st["used_blocks"], st["free_blocks"], st["num_appends"]) == (3, 5, 3)
    # LIFO allocation from a fresh pool: seq 0 gets page 0, seq 1 page 1, seq 0 then page 2.
    pt = c.page_table()
    assert pt[0, :3].tolist() == [0, 2, -1] and pt[1, :2].tolist() == [1, -1]

    c = orc.PagedKV(num_blocks=2, block_size=8, max_num_seqs=4)
    assert c.append(0, 16)[0] == 0 and c.stats()["free_blocks"] == 0
    rc, _, msg = c.append(1, 8)
    assert rc == 2007 and "needs 1 more blocks but only 0 are free" in msg
    assert (c.seq_len(1), c.block_count(1), c.seq_len(0), c.stats()["free_blocks"]) == (0, 0, 16, 0)

    c = orc.PagedKV(num_blocks=2, block_size=8, max_num_seqs=4)
    assert c.append(0, 8)[0] == 0
    assert c.reset(0)[0] == 0
    st = c.stats()
    assert (c.seq_len(0), st["free_blocks"], st["num_resets"]) == (0, 2, 1)
    assert c.append(1, 8)[0] == 0
    assert (c.seq_len(1), c.stats()["free_blocks"]) == (8, 1)


def test_oracle_paged_kv_slots_are_page_times_block_plus_offset():
    c = orc.PagedKV(num_blocks=16, block_size=4, max_num_seqs=3)
    lens = [0, 0, 0]
    rng = np.random.default_rng(3)
    for _ in range(40):
        s = int(rng.integers(0, 3))
        n = int(rng.integers(1, 6))
        rc, slots, _ = c.append(s, n)
        if rc:
            continue
        row = c.page_table()[s]
        for t, slot in enumerate(slots):
            pos = lens[s] + t
            assert slot == row[pos // 4] * 4 + pos % 4
        lens[s] += n
        assert c.seq_len(s) == lens[s]
        assert c.block_count(s) == -(-lens[s] // 4)


# ---- PagedKVCache restatement: properties the allocator's specification fixes -------------------
# (paged_kv_cache.cpp:52-201 over block_manager.cpp:11-144: LIFO free list, all-or-nothing
# allocation, table rows as long as the pool, revision bumped by every successful append or reset)

def _pkv_snapshot(c, seqs):
    return (c.page_table().copy(), [c.seq_len(s) for s in range(seqs)],
            [c.block_count(s) for s in range(seqs)], c.stats())


def test_oracle_paged_kv_failed_append_leaves_state_unchanged():
    """An append the pool cannot serve changes nothing: table, lengths, counters, revision, and
    the free list itself (the next allocation hands out the ids an untouched twin hands out)."""
    bs = 4
    a = orc.PagedKV(num_blocks=10, block_size=bs, max_num_seqs=3)
    b = orc.PagedKV(num_blocks=10, block_size=bs, max_num_seqs=3)
    for c in (a, b):
        assert c.append(0, 13)[0] == 0      # 4 blocks
        assert c.append(1, 9)[0] == 0       # 3 blocks
        assert c.reset(0)[0] == 0           # 4 back on the stack
        assert c.append(2, 5)[0] == 0       # 2 blocks: 5 used, 5 free
    before = _pkv_snapshot(a, 3)
    rc, slots, msg = a.append(0, 6 * bs)    # needs 6 blocks, 5 are free
    assert rc == 2007 and slots == [] and "needs 6 more blocks but only 5 are free" in msg
    rc, _, _ = a.append(1, 6 * bs)          # seq 1 holds 9 tokens in 3 blocks: needs 6 more
    assert rc == 2007
    after = _pkv_snapshot(a, 3)
    assert np.array_equal(before[0], after[0]) and before[1:] == after[1:]
    assert a.append(0, 5 * bs)[0] == 0 and b.append(0, 5 * bs)[0] == 0
    assert np.array_equal(a.page_table(), b.page_table())
    assert a.stats() == b.stats()


def test_oracle_paged_kv_reset_returns_blocks_lifo_in_row_order():
    """ResetSeq pushes the sequence's blocks back in row order, so the next allocation pops
    them in reverse row order."""
    c = orc.PagedKV(num_blocks=12, block_size=2, max_num_seqs=3)
    # interleave two sequences so seq 0's row is not contiguous: 0,1 | 2 | 3,4 | 5 ...
    assert c.append(0, 4)[0] == 0           # seq 0: blocks 0, 1
    assert c.append(1, 2)[0] == 0           # seq 1: block 2
    assert c.append(0, 3)[0] == 0           # seq 0: 7 tokens -> 4 blocks: + 3, 4
    assert c.append(1, 1)[0] == 0           # seq 1: 3 tokens -> 2 blocks: + 5
    row0 = c.page_table()[0, :4].tolist()
    assert row0 == [0, 1, 3, 4]
    assert c.reset(0)[0] == 0
    assert c.page_table()[0].tolist() == [-1] * 12 and c.seq_len(0) == 0
    # free stack (top last): 11 10 9 8 7 6 | 0 1 3 4  -> pops 4, 3, 1, 0, then 6, 7, ...
    assert c.append(2, 2 * 6)[0] == 0
    assert c.page_table()[2, :6].tolist() == [4, 3, 1, 0, 6, 7]


def test_oracle_paged_kv_revision_counts_successful_appends_and_resets_only():
    c = orc.PagedKV(num_blocks=4, block_size=4, max_num_seqs=2)
    assert c.stats()["revision"] == 1 and c.stats()["synced_revision"] == 1
    want = 1
    ops = [("a", 0, 3, 0), ("a", 0, 1, 0), ("r", 1, 0, 0),         # reset of an empty seq counts
           ("a", 1, 20, 2007), ("a", 2, 1, 2005), ("r", 5, 0, 2005),  # failures do not
           ("a", 1, 8, 0), ("r", 0, 0, 0), ("a", 1, 9, 2007)]
    for kind, seq, n, rc_want in ops:
        rc = c.append(seq, n)[0] if kind == "a" else c.reset(seq)[0]
        assert rc == rc_want, (kind, seq, n)
        if rc == 0:
            want += 1
        assert c.stats()["revision"] == want, (kind, seq, n)
    assert c.stats()["synced_revision"] == 1
    c.sync()
    assert c.stats()["synced_revision"] == want
    st = c.stats()
    assert (st["num_appends"], st["num_resets"]) == (3, 2)


def test_oracle_paged_kv_block_conservation_over_a_random_trace():
    """After every operation: used blocks = sum ceil(len/bs); every row lists exactly its
    blocks, then -1; no block is owned twice; used + free = pool."""
    nb, bs, seqs = 40, 4, 5
    c = orc.PagedKV(num_blocks=nb, block_size=bs, max_num_seqs=seqs)
    rng = np.random.default_rng(77)
    for _ in range(400):
        s = int(rng.integers(0, seqs))
        if rng.random() < 0.15:
            assert c.reset(s)[0] == 0
        else:
            c.append(s, int(rng.integers(1, 11)))
        lens = [c.seq_len(i) for i in range(seqs)]
        need = [-(-L // bs) for L in lens]
        st = c.stats()
        assert st["used_blocks"] == sum(need) and st["used_blocks"] + st["free_blocks"] == nb
        pt = c.page_table()
        owned = []
        for i in range(seqs):
            assert c.block_count(i) == need[i]
            assert (pt[i, :need[i]] >= 0).all() and (pt[i, need[i]:] == -1).all()
            owned += pt[i, :need[i]].tolist()
        assert len(owned) == len(set(owned)) and all(0 <= b < nb for b in owned)


def test_oracle_paged_kv_one_sequence_can_own_the_whole_pool():
    """Rows are as long as the pool (paged_kv_cache.cpp:24-26), so a row never fills before the
    pool does: the table-full rollback is unreachable and the first failure is capacity."""
    nb, bs = 6, 3
    c = orc.PagedKV(num_blocks=nb, block_size=bs, max_num_seqs=2)
    assert c.append(0, nb * bs)[0] == 0
    assert c.block_count(0) == nb and c.stats()["free_blocks"] == 0
    assert sorted(c.page_table()[0].tolist()) == list(range(nb))
    rc, _, msg = c.append(0, 1)
    assert rc == 2007 and "needs 1 more blocks but only 0 are free" in msg
    assert c.seq_len(0) == nb * bs

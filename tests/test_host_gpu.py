"""The sca:: host API end to end on the GPU (libsca_host.so -> libsca_hip.so), against the FP64
oracle: dispatcher-routed attention, varlen prefill, decode, and the paged KV cache driven the way
a serving loop drives it (prompt appends, per-step token appends, page-table sync, paged decode).
Host-visible KV state is compared bit-exactly with the oracle's restatement of the reference's
PagedKVCache."""

from __future__ import annotations

import numpy as np
import pytest

import oracle.oracle as orc
from attn_util import check_attention, quantize, to_float, uniform
from sca_amd import host as H

pytestmark = pytest.mark.gpu


def tensor(bits, dtype):
    return H.Tensor.from_numpy(bits, dtype)


def out_float(res, dtype):
    return to_float(res.out.numpy(), dtype)


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_dispatches_to_flash(hip, layout, causal):
    B, Hq, Hkv, S, D, dtype = 2, 8, 2, 300, 128, "f16"
    q, k, v = uniform((B, Hq, S, D), 1), uniform((B, Hkv, S, D), 2), uniform((B, Hkv, S, D), 3)
    (qb, qd), (kb, kd), (vb, vd) = quantize(q, dtype), quantize(k, dtype), quantize(v, dtype)
    if layout == "bshd":
        qb, kb, vb = (np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (qb, kb, vb))
    cfg = H.AttentionConfig(layout=layout, causal=causal, return_lse=True)
    res = H.attention(tensor(qb, dtype), tensor(kb, dtype), tensor(vb, dtype), cfg)
    assert res.stats["used_backend"] == H.BACKENDS["flash"]
    assert res.stats["workspace_bytes"] == 0 and res.stats["materialized_score_bytes"] == 0
    assert res.out.shape == (B, Hq, S, D)  # always BHSD
    ref, ref_lse = orc.reference_attention(qd, kd, vd, causal)
    check_attention(out_float(res, dtype).reshape(-1, D), ref, dtype, "attention", abs_gate=True)
    lse = res.lse.numpy().reshape(-1)
    assert np.abs(lse - ref_lse).max() < 1e-2


def test_flash_varlen_ragged_c3_tail(hip):
    """C3's ragged tail S in {1, 7, 63, 1000} (causal, bf16, Hq 32, Hkv 8, D 128) packed."""
    lens = [1, 7, 63, 1000]
    Hq, Hkv, D, dtype = 32, 8, 128, "bf16"
    T = sum(lens)
    q, k, v = uniform((T, Hq, D), 11), uniform((T, Hkv, D), 12), uniform((T, Hkv, D), 13)
    (qb, qd), (kb, kd), (vb, vd) = quantize(q, dtype), quantize(k, dtype), quantize(v, dtype)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    res = H.flash_attention_varlen(tensor(qb, dtype), tensor(kb, dtype), tensor(vb, dtype),
                                   len(lens), cu, cu, max(lens), max(lens),
                                   H.AttentionConfig(causal=True))
    out = out_float(res, dtype)
    for s, L in enumerate(lens):
        a, b = cu[s], cu[s + 1]
        ref, _ = orc.reference_attention(qd[a:b].transpose(1, 0, 2)[None],
                                         kd[a:b].transpose(1, 0, 2)[None],
                                         vd[a:b].transpose(1, 0, 2)[None], True)
        got = out[a:b].transpose(1, 0, 2).reshape(-1, D)
        check_attention(got, ref, dtype, f"varlen seq {s} (S={L})")


def test_varlen_rejects_sequences_outside_the_packed_tensors(hip):
    t = tensor(np.zeros((8, 4, 64), np.uint16), "f16")
    with pytest.raises(H.ScaError) as e:
        H.flash_attention_varlen(t, t, t, 2, [0, 4, 9], [0, 4, 9], 5, 5)
    assert e.value.code == 2005


def test_decode_auto_splits_and_explicit_configs(hip):
    B, Hq, Hkv, S, D, dtype = 4, 32, 8, 4096, 128, "f16"
    q, k, v = uniform((B, Hq, 1, D), 21), uniform((B, Hkv, S, D), 22), uniform((B, Hkv, S, D), 23)
    (qb, qd), (kb, kd), (vb, vd) = quantize(q, dtype), quantize(k, dtype), quantize(v, dtype)
    tq, tk, tv = tensor(qb, dtype), tensor(kb, dtype), tensor(vb, dtype)
    ref, _ = orc.reference_attention(qd, kd, vd, False)
    auto = H.attention(tq, tk, tv)
    assert auto.stats["used_backend"] == H.BACKENDS["decode"]
    assert auto.stats["num_splits"] == H.decode_splits(H.AttentionShape(B, 1, S, Hq, Hkv, D),
                                                       H.host_lib().sca_device_cu_count())
    base = out_float(auto, dtype)
    check_attention(base.reshape(-1, D), ref, dtype, "decode auto", abs_gate=True)
    for splits in (1, 3, 16, 64, 500):
        res = H.decode(tq, tk, tv, H.AttentionConfig(num_splits=splits))
        assert res.stats["num_splits"] == min(splits, 64)
        check_attention(out_float(res, dtype).reshape(-1, D), ref, dtype, f"decode splits={splits}")
    with pytest.raises(H.ScaError) as e:
        H.decode_attention(tensor(np.zeros((1, 8, 2, 64), np.uint16), "f16"),
                           tensor(np.zeros((1, 8, 300, 64), np.uint16), "f16"),
                           tensor(np.zeros((1, 8, 300, 64), np.uint16), "f16"))
    assert e.value.code == 2009


def test_explicit_reference_only_backends_fail_loudly(hip):
    t = tensor(np.zeros((1, 2, 64, 64), np.uint16), "f16")
    for fn in (H.naive_attention, H.tiled_attention):
        with pytest.raises(H.ScaError) as e:
            fn(t, t, t)
        assert e.value.code == 2009 and "not built for MI355X" in e.value.message
    with pytest.raises(H.ScaError):
        H.attention(t, t, t, H.AttentionConfig(backend="naive"))


# ---- paged KV cache ------------------------------------------------------------------------------

class Serving:
    """A PagedKVCache plus the host copies of what was appended (for the oracle)."""

    def __init__(self, num_blocks, bs, seqs, Hkv, D, dtype):
        self.cfg = H.KVCacheConfig(1, Hkv, D, bs, num_blocks, seqs, dtype)
        self.cache = H.PagedKVCache(self.cfg)
        self.mirror = orc.PagedKV(num_blocks, bs, seqs)
        self.k = [np.zeros((0, Hkv, D), np.float32) for _ in range(seqs)]
        self.v = [np.zeros((0, Hkv, D), np.float32) for _ in range(seqs)]
        self.dtype, self.Hkv, self.D = dtype, Hkv, D

    def append(self, seq, n, seed):
        k = uniform((n, self.Hkv, self.D), seed)
        v = uniform((n, self.Hkv, self.D), seed + 1)
        (kb, kd), (vb, vd) = quantize(k, self.dtype), quantize(v, self.dtype)
        want_rc, _, want_msg = self.mirror.append(seq, n)
        try:
            self.cache.append_tokens(seq, 0, tensor(kb, self.dtype), tensor(vb, self.dtype))
            rc = 0
        except H.ScaError as e:
            rc, msg = e.code, e.message
            assert f"[SCA-{rc}] {want_msg}" == msg
        assert rc == want_rc
        if rc == 0:
            self.k[seq] = np.concatenate([self.k[seq], kd])
            self.v[seq] = np.concatenate([self.v[seq], vd])
        return rc

    def reset(self, seq):
        assert self.mirror.reset(seq)[0] == 0
        self.cache.reset_seq(seq)
        self.k[seq] = self.k[seq][:0]
        self.v[seq] = self.v[seq][:0]

    def check_state(self):
        pt = self.cache.page_table_host()
        assert np.array_equal(pt, self.mirror.page_table())
        for s in range(self.cfg.max_num_seqs):
            assert self.cache.seq_length(s) == self.mirror.seq_len(s)
            assert self.cache.logical_block_count(s) == self.mirror.block_count(s)
        st, ms = self.cache.stats(), self.mirror.stats()
        for key in ("used_blocks", "free_blocks", "num_appends", "num_resets"):
            assert st[key] == ms[key], key
        assert self.cache.revision == ms["revision"]

    def check_device_table(self):
        self.cache.sync_page_table()
        assert self.cache.synced_revision == self.cache.revision
        assert np.array_equal(self.cache.page_table_device(), self.cache.page_table_host())


def test_paged_cache_state_matches_reference_restatement(hip):
    rng = np.random.default_rng(5)
    srv = Serving(num_blocks=40, bs=8, seqs=5, Hkv=2, D=64, dtype="f16")
    for step in range(120):
        r = rng.random()
        seq = int(rng.integers(0, 5))
        if r < 0.75:
            srv.append(seq, int(rng.integers(1, 20)), 1000 + step)
        else:
            srv.reset(seq)
        srv.check_state()
        if step % 7 == 0:
            srv.check_device_table()
    srv.check_device_table()
    # Every stored token reads back bit-exactly through the page table.
    pt = srv.cache.page_table_host()
    k_ptr, _ = srv.cache.layer_ptrs(0)
    for s in range(5):
        n = srv.cache.logical_block_count(s)
        if n == 0:
            continue
        ids = tensor(pt[s, :n].copy(), "i32")
        got = srv.cache.gather(True, 0, ids.data_ptr, n).numpy()
        flat = to_float(got, "f16").reshape(n * 8, 2, 64)[: len(srv.k[s])]
        assert np.array_equal(flat, srv.k[s])


def test_batched_append_equals_per_sequence_appends(hip):
    # One AppendTokensBatch per decode step (ids may repeat) leaves exactly the state of one
    # AppendTokens call per entry, and the same tokens in the same slots.
    rng = np.random.default_rng(11)
    seqs, bs, Hkv, D = 6, 8, 2, 64
    a = Serving(num_blocks=60, bs=bs, seqs=seqs, Hkv=Hkv, D=D, dtype="bf16")
    b = Serving(num_blocks=60, bs=bs, seqs=seqs, Hkv=Hkv, D=D, dtype="bf16")
    for s in range(seqs):
        n = int(rng.integers(1, 9))
        assert a.append(s, n, 500 + s) == 0 and b.append(s, n, 500 + s) == 0
    for step in range(25):
        ids = rng.integers(0, seqs, size=int(rng.integers(1, 9)))
        k = uniform((len(ids), Hkv, D), 900 + step)
        v = uniform((len(ids), Hkv, D), 950 + step)
        (kb, _), (vb, _) = quantize(k, "bf16"), quantize(v, "bf16")
        a.cache.append_batch(ids, 0, tensor(kb, "bf16"), tensor(vb, "bf16"))
        for i, s in enumerate(ids):
            b.cache.append_tokens(int(s), 0, tensor(kb[i:i + 1].copy(), "bf16"),
                                  tensor(vb[i:i + 1].copy(), "bf16"))
        assert np.array_equal(a.cache.page_table_host(), b.cache.page_table_host())
        for s in range(seqs):
            assert a.cache.seq_length(s) == b.cache.seq_length(s)
            assert a.cache.logical_block_count(s) == b.cache.logical_block_count(s)
        assert a.cache.revision == b.cache.revision
        sa, sb = a.cache.stats(), b.cache.stats()
        for key in ("used_blocks", "free_blocks", "num_appends", "num_resets"):
            assert sa[key] == sb[key], key
    pt = a.cache.page_table_host()
    for s in range(seqs):
        n = a.cache.logical_block_count(s)
        ids = tensor(pt[s, :n].copy(), "i32")
        ga = a.cache.gather(True, 0, ids.data_ptr, n).numpy()
        gb = b.cache.gather(True, 0, ids.data_ptr, n).numpy()
        L = a.cache.seq_length(s)
        assert np.array_equal(ga.reshape(n * bs, -1)[:L], gb.reshape(n * bs, -1)[:L])
        va = a.cache.gather(False, 0, ids.data_ptr, n).numpy()
        vb_ = b.cache.gather(False, 0, ids.data_ptr, n).numpy()
        assert np.array_equal(va.reshape(n * bs, -1)[:L], vb_.reshape(n * bs, -1)[:L])
    # A batch the pool cannot hold changes nothing.
    before = (a.cache.page_table_host().copy(), a.cache.revision,
              [a.cache.seq_length(s) for s in range(seqs)])
    free = a.cache.stats()["free_blocks"]
    big = np.repeat(np.arange(seqs), (free + 2) * bs // seqs + bs)
    z = tensor(np.zeros((len(big), Hkv, D), np.uint16), "bf16")
    with pytest.raises(H.ScaError) as e:
        a.cache.append_batch(big, 0, z, z)
    assert e.value.code == 2007
    assert np.array_equal(a.cache.page_table_host(), before[0]) and a.cache.revision == before[1]
    assert [a.cache.seq_length(s) for s in range(seqs)] == before[2]


def test_paged_cache_errors_leave_state_unchanged(hip):
    srv = Serving(num_blocks=2, bs=8, seqs=4, Hkv=1, D=32, dtype="f16")
    assert srv.append(0, 16, 1) == 0
    assert srv.append(1, 8, 2) == 2007
    srv.check_state()
    with pytest.raises(H.ScaError):
        srv.cache.append_tokens(9, 0, tensor(np.zeros((1, 1, 32), np.uint16), "f16"),
                                tensor(np.zeros((1, 1, 32), np.uint16), "f16"))
    with pytest.raises(H.ScaError):
        srv.cache.append_tokens(0, 3, tensor(np.zeros((1, 1, 32), np.uint16), "f16"),
                                tensor(np.zeros((1, 1, 32), np.uint16), "f16"))
    srv.check_state()
    srv.reset(0)
    srv.check_state()
    assert srv.append(1, 8, 3) == 0
    srv.check_state()
    srv.check_device_table()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_serving_loop_paged_decode(hip, dtype):
    """Prompt appends, then decode steps: append one token per sequence, sync, paged decode."""
    Hq, Hkv, D, bs, seqs = 32, 8, 128, 16, 6
    rng = np.random.default_rng(9)
    prompts = [int(x) for x in rng.integers(1, 700, size=seqs)]
    srv = Serving(num_blocks=sum(-(-(p + 8) // bs) for p in prompts) + 4, bs=bs, seqs=seqs,
                  Hkv=Hkv, D=D, dtype=dtype)
    for s in rng.permutation(seqs):
        srv.append(int(s), prompts[s], 50 + int(s))
    for step in range(4):
        for s in range(seqs):
            assert srv.append(s, 1, 900 + 10 * step + s) == 0
        srv.cache.sync_page_table()
        lens = np.array([srv.cache.seq_length(s) for s in range(seqs)], np.int32)
        q = uniform((seqs, Hq, 1, D), 77 + step)
        qb, qd = quantize(q, dtype)
        dl = tensor(lens, "i32")
        res = H.paged_attention(tensor(qb, dtype), srv.cache,
                                {"seq_lens": dl.data_ptr, "num_seqs": seqs, "block_size": bs},
                                H.AttentionConfig())
        assert res.stats["used_backend"] == H.BACKENDS["paged"]
        # the cache's host lengths drive the length-aware plan (a ragged batch of six sequences
        # gets four waves per KV-head slot)
        splits, waves = H.paged_decode_plan(lens, Hq, Hkv, H.host_lib().sca_device_cu_count())
        assert waves == 4 and res.stats["num_splits"] == splits, res.stats
        assert "four waves per head slot" in res.stats["note"], res.stats["note"]
        out = out_float(res, dtype)
        for s in range(seqs):
            ref, _ = orc.reference_attention(qd[s:s + 1], srv.k[s].transpose(1, 0, 2)[None],
                                             srv.v[s].transpose(1, 0, 2)[None], False)
            check_attention(out[s].reshape(-1, D), ref, dtype, f"step {step} seq {s}")
    srv.check_state()


def test_reserved_multi_layer_appends(hip):
    # ReserveTokens / ReserveTokensBatch leave the allocator state of the equivalent AppendTokens /
    # AppendTokensBatch calls, and each WriteReservedLayer lands its rows in its own layer only.
    rng = np.random.default_rng(21)
    layers, seqs, bs, Hkv, D, dt = 3, 5, 8, 2, 64, "bf16"
    cfg = H.KVCacheConfig(layers, Hkv, D, bs, 64, seqs, dt)
    a, b = H.PagedKVCache(cfg), H.PagedKVCache(H.KVCacheConfig(1, Hkv, D, bs, 64, seqs, dt))
    hist = [[np.zeros((0, Hkv, D), np.uint16) for _ in range(seqs)] for _ in range(layers)]
    vhist = [[np.zeros((0, Hkv, D), np.uint16) for _ in range(seqs)] for _ in range(layers)]

    # c gets the same tokens through the one-call form (every layer's rows stacked).
    c = H.PagedKVCache(cfg)

    def write_all(ids, n_rows, seed):
        ks, vs = [], []
        for layer in range(layers):
            kb, _ = quantize(uniform((n_rows, Hkv, D), seed + 2 * layer), dt)
            vb, _ = quantize(uniform((n_rows, Hkv, D), seed + 2 * layer + 1), dt)
            a.write_layer(layer, tensor(kb, dt), tensor(vb, dt))
            ks.append(kb)
            vs.append(vb)
            for i, s in enumerate(ids):
                hist[layer][s] = np.concatenate([hist[layer][s], kb[i:i + 1]])
                vhist[layer][s] = np.concatenate([vhist[layer][s], vb[i:i + 1]])
        c.append_batch_all_layers(ids, tensor(np.stack(ks), dt), tensor(np.stack(vs), dt))
        return kb, vb

    z = lambda n: tensor(np.zeros((n, Hkv, D), np.uint16), dt)  # noqa: E731
    # Prompts: one reservation per sequence, written layer by layer.
    for s in range(seqs):
        n = int(rng.integers(1, 30))
        a.reserve(s, n)
        write_all([s] * n, n, 1000 + 10 * s)
        b.append_tokens(s, 0, z(n), z(n))
    # Decode steps: one batch reservation (ids may repeat), then every layer.
    for step in range(12):
        ids = [int(x) for x in rng.integers(0, seqs, size=int(rng.integers(1, 7)))]
        a.reserve_batch(ids)
        write_all(ids, len(ids), 5000 + 10 * step)
        b.append_batch(ids, 0, z(len(ids)), z(len(ids)))
        assert np.array_equal(a.page_table_host(), b.page_table_host())
        assert a.revision == b.revision
        for s in range(seqs):
            assert a.seq_length(s) == b.seq_length(s)
        sa, sb = a.stats(), b.stats()
        for key in ("used_blocks", "free_blocks", "num_appends", "num_resets"):
            assert sa[key] == sb[key], key
    pt = a.page_table_host()
    # (Revisions differ by design: a batch counts one per entry, ReserveTokens one per call.)
    assert np.array_equal(c.page_table_host(), pt)
    for layer in range(layers):
        for s in range(seqs):
            n, L = a.logical_block_count(s), a.seq_length(s)
            assert c.seq_length(s) == L
            ids = tensor(pt[s, :n].copy(), "i32")
            for cache in (a, c):
                gk = cache.gather(True, layer, ids.data_ptr, n).numpy().reshape(n * bs, Hkv, D)[:L]
                gv = cache.gather(False, layer, ids.data_ptr, n).numpy().reshape(n * bs, Hkv, D)[:L]
                assert np.array_equal(gk, hist[layer][s]), (layer, s)
                assert np.array_equal(gv, vhist[layer][s]), (layer, s)
    # The one-call form checks its shapes before anything changes.
    before = (c.page_table_host().copy(), c.revision)
    with pytest.raises(H.ScaError):
        c.append_batch_all_layers([0, 1], tensor(np.zeros((layers - 1, 2, Hkv, D), np.uint16), dt),
                                  tensor(np.zeros((layers - 1, 2, Hkv, D), np.uint16), dt))
    assert np.array_equal(c.page_table_host(), before[0]) and c.revision == before[1]
    # Misuse is rejected without touching the state.
    before = (a.page_table_host().copy(), a.revision)
    a.append_tokens(0, 0, z(1), z(1))  # ends the last reservation
    b.append_tokens(0, 0, z(1), z(1))
    with pytest.raises(H.ScaError):
        a.write_layer(1, z(1), z(1))
    a.reserve_batch([1, 2])
    with pytest.raises(H.ScaError):
        a.write_layer(1, z(3), z(3))  # rows differ from the reservation
    with pytest.raises(H.ScaError):
        a.write_layer(layers, z(2), z(2))
    b.append_batch([1, 2], 0, z(2), z(2))
    free = a.stats()["free_blocks"]
    with pytest.raises(H.ScaError) as e:
        a.reserve_batch(np.repeat([3], (free + 1) * bs + bs))
    assert e.value.code == 2007
    assert np.array_equal(a.page_table_host(), b.page_table_host()) and a.revision == b.revision
    assert not np.array_equal(before[0], a.page_table_host()) or before[1] != a.revision

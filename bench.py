"""Benchmark of the MI355X attention hot path (one GPU).

Workloads (inputs synthetic, seeded, resident in HBM before timing):
  * C2  flash prefill fp16, B=1, H=8, D=128, S=4096, causal (the headline `value`) and
        non-causal;
  * C5  paged decode bf16, 64 sequences with lengths U[512,16384], block size 16, block-major pool
        with a seeded permuted block table, H_q=32, H_kv=8, D=128; each step appends one token per
        sequence (host block bookkeeping + the append kernel), then attends; the attend kernel is
        timed;
  * C4  split-K decode fp16, B=16, H_q=32, H_kv=8, D=128, S_kv=4096.
A step of C2 is one flash launch over the whole batch. Kernel time is measured with HIP events
recorded on the launch stream around the K timed launches; the algorithmic work per launch
(FLOPs or bytes) divided by the average launch time gives the achieved rate.

The CPU baseline is the naive three-pass FP32 restatement of the reference's naive backend
(oracle/sca_oracle.c, attention_naive.cu:41-135) timed on a bounded sample of C2 (one head)
on the host cores.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "scicompute-attention_amd", "python"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import sca_amd  # noqa: E402
from sca_amd import hip as H  # noqa: E402

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E


def causal_flops(B, H_, S, D):
    return 4 * B * H_ * D * (S * (S + 1) // 2)


def f16_bits(rng, shape):
    return rng.standard_normal(size=shape, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(rng, shape, chunk=1 << 24, std=1.0):
    """Seeded N(0, std^2) bf16 bits; large tensors tile one random chunk (the values do not
    change the amount of work)."""
    n = int(np.prod(shape))
    m = min(n, chunk)
    x = (rng.standard_normal(size=m, dtype=np.float32) * np.float32(std)).view(np.uint32)
    bits = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    if m < n:
        bits = np.resize(bits, n)
    return bits.reshape(shape)


def dispatcher_splits(batch, Hq, Hkv, seq_kv, D):
    """The split count the host dispatcher picks for this decode shape on this device."""
    from sca_amd import host as SH
    cus = H.device_probe(0).cu_count
    return SH.decode_splits(SH.AttentionShape(batch, 1, seq_kv, Hq, Hkv, D), cus)


def paged_plan(lengths, Hq, Hkv):
    """(splits, slot_waves) the paged backend plans for these host-side lengths on this device."""
    from sca_amd import host as SH
    return SH.paged_decode_plan(lengths, Hq, Hkv, H.device_probe(0).cu_count)


def prewarm(launch, seconds):
    """Untimed launches for `seconds`: the device's clocks ramp up under sustained load, so each
    timed leg starts from the operating point a busy device runs at."""
    if seconds <= 0:
        return
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(20):
            launch()
        sca_amd.synchronize()


def time_launches(launch, steps, warmup):
    for _ in range(warmup):
        launch()
    sca_amd.synchronize()
    start, stop = H.Event(), H.Event()
    start.record()
    for _ in range(steps):
        launch()
    stop.record()
    stop.synchronize()
    sca_amd.synchronize()
    return start.elapsed_ms(stop) / steps


def launch_percentiles(launch, runs=50):
    """P50/P90/P99 of single launches (HIP events around each launch), in ms."""
    events = [(H.Event(), H.Event()) for _ in range(runs)]
    for a, b in events:
        a.record()
        launch()
        b.record()
    events[-1][1].synchronize()
    ms = np.sort([a.elapsed_ms(b) for a, b in events])
    return {"p50": float(np.percentile(ms, 50)), "p90": float(np.percentile(ms, 90)),
            "p99": float(np.percentile(ms, 99))}


# ---- C2: flash prefill -------------------------------------------------------------------------
def bench_flash(steps, warmup, causal, B=1, Hh=8, S=4096, D=128, prewarm_s=0.0):
    rng = np.random.default_rng(2024)
    dq = H.DeviceBuffer.from_array(f16_bits(rng, (B, Hh, S, D)))
    dk = H.DeviceBuffer.from_array(f16_bits(rng, (B, Hh, S, D)))
    dv = H.DeviceBuffer.from_array(f16_bits(rng, (B, Hh, S, D)))
    dout = H.DeviceBuffer(B * Hh * S * D * 2)
    p = H.FlashParams()
    p.q, p.k, p.v, p.out, p.lse = dq.ptr, dk.ptr, dv.ptr, dout.ptr, None
    p.batch, p.num_heads, p.num_kv_heads, p.seq_q, p.seq_kv, p.head_dim = B, Hh, Hh, S, S, D
    p.q_sb, p.q_sh, p.q_ss = Hh * S * D, S * D, D
    p.k_sb, p.k_sh, p.k_ss = p.q_sb, p.q_sh, p.q_ss
    p.v_sb, p.v_sh, p.v_ss = p.q_sb, p.q_sh, p.q_ss
    p.o_sb, p.o_sh, p.o_ss = p.q_sb, p.q_sh, p.q_ss
    p.scale = float(np.float32(1.0 / np.sqrt(D)))
    p.causal = 1 if causal else 0
    p.dtype = H.DTYPE_F16
    p.diagonal = 0
    prewarm(lambda: H.flash_fwd(p), prewarm_s)
    ms = time_launches(lambda: H.flash_fwd(p), steps, warmup)
    flops = causal_flops(B, Hh, S, D) if causal else 4 * B * Hh * S * S * D
    pct = launch_percentiles(lambda: H.flash_fwd(p))
    return {"ms": ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12,
            "bytes": 4 * B * Hh * S * D * 2, "pct": pct}


# ---- C3: GQA causal prefill (reported next to the headline) -----------------------------------
def bench_flash_gqa(steps, warmup, B=4, Hq=32, Hkv=8, S=8192, D=128, prewarm_s=0.0):
    """C3: bf16 Q/K/V ~ N(0, 0.5^2), causal, group 4; flash through the C ABI."""
    rng = np.random.default_rng(2025)
    dq = H.DeviceBuffer.from_array(bf16_bits(rng, (B, Hq, S, D), std=0.5))
    dk = H.DeviceBuffer.from_array(bf16_bits(rng, (B, Hkv, S, D), std=0.5))
    dv = H.DeviceBuffer.from_array(bf16_bits(rng, (B, Hkv, S, D), std=0.5))
    dout = H.DeviceBuffer(B * Hq * S * D * 2)
    p = H.FlashParams()
    p.q, p.k, p.v, p.out, p.lse = dq.ptr, dk.ptr, dv.ptr, dout.ptr, None
    p.batch, p.num_heads, p.num_kv_heads, p.seq_q, p.seq_kv, p.head_dim = B, Hq, Hkv, S, S, D
    p.q_sb, p.q_sh, p.q_ss = Hq * S * D, S * D, D
    p.k_sb, p.k_sh, p.k_ss = Hkv * S * D, S * D, D
    p.v_sb, p.v_sh, p.v_ss = p.k_sb, p.k_sh, p.k_ss
    p.o_sb, p.o_sh, p.o_ss = p.q_sb, p.q_sh, p.q_ss
    p.scale = float(np.float32(1.0 / np.sqrt(D)))
    p.causal = 1
    p.dtype = H.DTYPE_BF16
    p.diagonal = 0
    prewarm(lambda: H.flash_fwd(p), prewarm_s)
    ms = time_launches(lambda: H.flash_fwd(p), steps, warmup)
    flops = causal_flops(B, Hq, S, D)
    return {"ms": ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12}


# ---- C4: split-K decode --------------------------------------------------------------------------
def bench_decode(steps, warmup, B=16, Hq=32, Hkv=8, S=4096, D=128, splits=None, prewarm_s=0.0,
                 slot_waves=0):
    if splits is None:
        splits = dispatcher_splits(B, Hq, Hkv, S, D)
    rng = np.random.default_rng(4004)
    dq = H.DeviceBuffer.from_array(f16_bits(rng, (B, Hq, 1, D)))
    dk = H.DeviceBuffer.from_array(f16_bits(rng, (B, Hkv, S, D)))
    dv = H.DeviceBuffer.from_array(f16_bits(rng, (B, Hkv, S, D)))
    dout = H.DeviceBuffer(B * Hq * D * 2)
    parts = H.DeviceBuffer(4 * sca_amd.hip_lib().sca_hip_decode_partial_elements(B, Hq, splits, D))
    p = H.DecodeParams()
    p.q, p.k, p.v, p.out = dq.ptr, dk.ptr, dv.ptr, dout.ptr
    base = B * Hq * splits
    p.partial_m, p.partial_l, p.partial_o = parts.ptr, parts.ptr + 4 * base, parts.ptr + 8 * base
    p.batch, p.num_heads, p.num_kv_heads, p.seq_kv, p.head_dim, p.num_splits = B, Hq, Hkv, S, D, splits
    p.q_sb, p.q_sh = Hq * D, D
    p.k_sb, p.k_sh, p.k_ss = Hkv * S * D, S * D, D
    p.v_sb, p.v_sh, p.v_ss = p.k_sb, p.k_sh, p.k_ss
    p.o_sb, p.o_sh = Hq * D, D
    p.scale = float(np.float32(1.0 / np.sqrt(D)))
    p.dtype = H.DTYPE_F16
    p.slot_waves = slot_waves
    prewarm(lambda: H.decode_splitk(p), prewarm_s)
    ms = time_launches(lambda: H.decode_splitk(p), steps, warmup)
    nbytes = 2 * B * Hkv * S * D * 2 + 2 * B * Hq * D * 2
    return {"ms": ms, "bytes": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9, "splits": splits}


# ---- C5: paged decode ------------------------------------------------------------------------------
def bench_paged(steps, num_seqs=64, bs=16, Hq=32, Hkv=8, D=128, splits=None, lo=512, hi=16384,
                prewarm_s=0.0, slot_waves=None):
    rng = np.random.default_rng(5005)
    lengths = rng.integers(lo, hi + 1, size=num_seqs).astype(np.int64)
    final = lengths + steps
    need = (final + bs - 1) // bs
    num_blocks = int(need.sum()) + 64
    perm = rng.permutation(num_blocks).astype(np.int32)
    max_blocks = int(need.max())
    if splits is None or slot_waves is None:
        # The paged backend's length-aware plan over the starting lengths (the cache's host
        # lengths when the host layer attends its own page table).
        plan_splits, plan_waves = paged_plan(lengths, Hq, Hkv)
        splits = plan_splits if splits is None else splits
        slot_waves = plan_waves if slot_waves is None else slot_waves
    table = np.full((num_seqs, max_blocks), -1, np.int32)
    pos = 0
    for s in range(num_seqs):
        table[s, : need[s]] = perm[pos: pos + need[s]]
        pos += need[s]
    row_elems = Hkv * D
    pool_shape = (num_blocks, bs, Hkv, D)
    dk = H.DeviceBuffer.from_array(bf16_bits(rng, pool_shape))
    dv = H.DeviceBuffer.from_array(bf16_bits(rng, pool_shape))
    dt = H.DeviceBuffer.from_array(table)
    dq = H.DeviceBuffer.from_array(bf16_bits(rng, (num_seqs, Hq, 1, D)))
    dout = H.DeviceBuffer(num_seqs * Hq * D * 2)
    parts = H.DeviceBuffer(4 * sca_amd.hip_lib().sca_hip_decode_partial_elements(num_seqs, Hq,
                                                                                  splits, D))
    new_k = H.DeviceBuffer.from_array(bf16_bits(rng, (num_seqs, Hkv, D)))
    new_v = H.DeviceBuffer.from_array(bf16_bits(rng, (num_seqs, Hkv, D)))
    shape = H.KvShape()
    shape.num_blocks, shape.block_size, shape.num_kv_heads, shape.head_dim = num_blocks, bs, Hkv, D
    p = H.DecodeParams()
    p.q, p.k, p.v, p.out = dq.ptr, dk.ptr, dv.ptr, dout.ptr
    base = num_seqs * Hq * splits
    p.partial_m, p.partial_l, p.partial_o = parts.ptr, parts.ptr + 4 * base, parts.ptr + 8 * base
    p.batch, p.num_heads, p.num_kv_heads = num_seqs, Hq, Hkv
    p.seq_kv, p.head_dim, p.num_splits = num_blocks * bs, D, splits
    p.q_sb, p.q_sh = Hq * D, D
    p.k_sb, p.k_sh, p.k_ss = 0, D, row_elems
    p.v_sb, p.v_sh, p.v_ss = 0, D, row_elems
    p.o_sb, p.o_sh = Hq * D, D
    p.scale = float(np.float32(1.0 / np.sqrt(D)))
    p.dtype = H.DTYPE_BF16
    p.page_table, p.block_size, p.max_blocks_per_seq = dt.ptr, bs, max_blocks
    p.num_kv_blocks = num_blocks
    p.slot_waves = slot_waves
    dorder = H.DeviceBuffer(num_seqs * 8)
    p.batch_order = dorder.ptr
    L = sca_amd.hip_lib()
    # Every step's slots and lengths are computed up front and uploaded once, so the steps are
    # enqueued back to back, as in a decode loop over many layers: step t appends one token per
    # sequence at position lengths + t, then attends over lengths + t + 1 tokens. Two untimed
    # warmup steps attend over the starting lengths first.
    all_lens = np.stack([lengths] * 2 + [lengths + t + 1 for t in range(steps)]).astype(np.int32)
    all_slots = np.stack([table[np.arange(num_seqs), (lengths + t) // bs].astype(np.int64) * bs
                          + (lengths + t) % bs for t in range(steps)]).astype(np.int32)
    dlens_all = H.DeviceBuffer.from_array(all_lens)
    dslots_all = H.DeviceBuffer.from_array(all_slots)
    p.seq_lens = dlens_all.ptr  # the starting lengths
    prewarm(lambda: H.decode_splitk_paged(p), prewarm_s)
    events = [(H.Event(), H.Event()) for _ in range(steps)]
    total_bytes = 0
    for step in range(steps + 2):
        timed = step >= 2
        if timed:
            t = step - 2
            H.check(L.sca_hip_kv_append(dk.ptr, dv.ptr, new_k.ptr, new_v.ptr,
                                        dslots_all.ptr + 4 * t * num_seqs, num_seqs, shape, 2,
                                        None))
            cur = all_lens[step].astype(np.int64)
            total_bytes += int(cur.sum()) * Hkv * D * 2 * 2 + int(((cur + bs - 1) // bs).sum()) * 4 \
                + 2 * num_seqs * Hq * D * 2
        p.seq_lens = dlens_all.ptr + 4 * step * num_seqs
        if timed:
            events[step - 2][0].record()
        H.decode_splitk_paged(p)
        if timed:
            events[step - 2][1].record()
    events[-1][1].synchronize()
    total_ms = sum(a.elapsed_ms(b) for a, b in events)
    ms = total_ms / steps
    nbytes = total_bytes / steps
    return {"ms": ms, "bytes": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9, "splits": splits,
            "slot_waves": slot_waves, "num_blocks": num_blocks, "pool_bytes": 2 * num_blocks * bs * row_elems * 2,
            "mean_len": float(lengths.mean())}


# ---- C5 through the host layer (PagedKVCache + sca::paged_attention) ------------------------------
class C5HostLoop:
    """C5 as a serving loop drives it, through the public host API (include/sca_capi.h).

    Fill: the page-sized appends of all sequences go through PagedKVCache::AppendTokens in a
    seeded random order, so every sequence's pages are scattered over the pool; each append
    takes its K and V rows from a bank of `bank` distinct seeded pages (a partial last page takes
    the first rows of one). Step t: one AppendTokensBatch appends one token to every sequence
    (token rows from a bank of 8 seeded [num_seqs, H_kv, D] tensors), SyncPageTable uploads the
    changed entries, then sca::paged_attention attends with seq_lens including the new token.
    `log` records every append (sequence, bank page or step token, rows) so a checker can rebuild
    each sequence's K/V rows and the allocator trace."""

    def __init__(self, steps, num_seqs=64, bs=16, Hq=32, Hkv=8, D=128, lo=512, hi=16384,
                 seed=5006, bank=64):
        from sca_amd import host as SH
        self.SH = SH
        self.num_seqs, self.bs, self.Hq, self.Hkv, self.D = num_seqs, bs, Hq, Hkv, D
        rng = np.random.default_rng(seed)
        self.lengths = rng.integers(lo, hi + 1, size=num_seqs).astype(np.int64)
        self.num_blocks = int(((self.lengths + steps + bs - 1) // bs).sum()) + 64
        self.cache = SH.PagedKVCache(SH.KVCacheConfig(1, Hkv, D, bs, self.num_blocks, num_seqs,
                                                      "bf16"))
        self.bank_k = bf16_bits(rng, (bank, bs, Hkv, D))
        self.bank_v = bf16_bits(rng, (bank, bs, Hkv, D))
        self.tok_k = bf16_bits(rng, (8, num_seqs, Hkv, D))
        self.tok_v = bf16_bits(rng, (8, num_seqs, Hkv, D))
        self.q_bits = bf16_bits(rng, (num_seqs, Hq, 1, D))
        dev_k = [SH.Tensor.from_numpy(self.bank_k[i], "bf16") for i in range(bank)]
        dev_v = [SH.Tensor.from_numpy(self.bank_v[i], "bf16") for i in range(bank)]
        order = np.concatenate([np.full((L + bs - 1) // bs, s) for s, L in enumerate(self.lengths)])
        rng.shuffle(order)
        filled = np.zeros(num_seqs, np.int64)
        self.log = []  # ("page", seq, bank index, rows) or ("token", seq, step)
        tails = {}
        for i, s in enumerate(order):
            n = int(min(bs, self.lengths[s] - filled[s]))
            j = (i * 7919) % bank
            if n == bs:
                self.cache.append_tokens(int(s), 0, dev_k[j], dev_v[j])
            else:
                key = (j, n)
                if key not in tails:
                    tails[key] = (SH.Tensor.from_numpy(np.ascontiguousarray(self.bank_k[j, :n]), "bf16"),
                                  SH.Tensor.from_numpy(np.ascontiguousarray(self.bank_v[j, :n]), "bf16"))
                self.cache.append_tokens(int(s), 0, *tails[key])
            self.log.append(("page", int(s), j, n))
            filled[s] += n
        self.q = SH.Tensor.from_numpy(self.q_bits, "bf16")
        self.toks = [(SH.Tensor.from_numpy(self.tok_k[i], "bf16"),
                      SH.Tensor.from_numpy(self.tok_v[i], "bf16")) for i in range(8)]
        self.lens_dev = H.DeviceBuffer(num_seqs * 4)
        self.ids = np.arange(num_seqs)
        self.cur = self.lengths.copy()
        self.t = 0

    def append_step(self):
        """AppendTokensBatch (one token per sequence) and SyncPageTable."""
        tk, tv = self.toks[self.t % 8]
        self.cache.append_batch(self.ids, 0, tk, tv)
        self.cache.sync_page_table()
        for s in range(self.num_seqs):
            self.log.append(("token", s, self.t))
        self.cur = self.cur + 1
        self.lens_dev.upload(self.cur.astype(np.int32))
        self.t += 1

    def attend(self):
        """sca::paged_attention over every sequence (seq_lens include this step's token)."""
        return self.SH.paged_attention(self.q, self.cache,
                                       {"seq_lens": self.lens_dev.ptr, "num_seqs": self.num_seqs,
                                        "block_size": self.bs})

    def rows(self, seq):
        """The K and V rows (bf16 bits, [L, H_kv, D]) sequence `seq` holds, in order."""
        ks, vs = [], []
        for e in self.log:
            if e[1] != seq:
                continue
            if e[0] == "page":
                ks.append(self.bank_k[e[2], :e[3]])
                vs.append(self.bank_v[e[2], :e[3]])
            else:
                ks.append(self.tok_k[e[2] % 8, seq][None])
                vs.append(self.tok_v[e[2] % 8, seq][None])
        return np.concatenate(ks), np.concatenate(vs)

    def step_bytes(self):
        """Algorithmic bytes of the attend call: K+V once per KV head, page-table entries, Q+O."""
        cur, bs = self.cur, self.bs
        return int(cur.sum()) * self.Hkv * self.D * 2 * 2 + int(((cur + bs - 1) // bs).sum()) * 4 + \
            2 * self.num_seqs * self.Hq * self.D * 2


def bench_paged_host(steps):
    """C5 through the public host API (C5HostLoop). The attend call is timed with HIP events
    around the API call (dispatcher and allocation included); append + sync are timed the same
    way, separately."""
    loop = C5HostLoop(steps)
    start, mid, stop = H.Event(), H.Event(), H.Event()
    t_attend = t_append = 0.0
    total_bytes = 0
    splits = None
    for step in range(steps + 2):  # two untimed warmup steps
        timed = step >= 2
        start.record()
        loop.append_step()
        mid.record()
        res = loop.attend()
        stop.record()
        stop.synchronize()
        splits = res.stats.get("num_splits")
        del res
        if timed:
            t_append += start.elapsed_ms(mid)
            t_attend += mid.elapsed_ms(stop)
            total_bytes += loop.step_bytes()
    ms = t_attend / steps
    nbytes = total_bytes / steps
    return {"ms": ms, "gbps": nbytes / (ms * 1e-3) / 1e9, "append_sync_ms": t_append / steps,
            "splits": splits, "num_blocks": loop.num_blocks}


# ---- copy calibration ------------------------------------------------------------------------------
def bench_page_probe(steps, warmup, num_seqs=64, bs=16, Hkv=8, D=128, lo=512, hi=16384):
    """The paged decode's read pattern alone (lib/libsca_calib.so): C5's starting pool (same
    seed, lengths and permuted page table as the paged leg; 12 splits), K and V head slices
    of every page read once, nothing computed. Reported per in-flight depth (32-token tiles per
    wave, 16 KB each); the best is the practical ceiling for the paged decode kernel. Sequences
    run longest first, as the decode kernel runs a ragged batch."""
    import ctypes
    rng = np.random.default_rng(5005)
    lengths = rng.integers(lo, hi + 1, size=num_seqs).astype(np.int64)
    need = (lengths + bs - 1) // bs
    num_blocks = int(need.sum()) + 64
    perm = rng.permutation(num_blocks).astype(np.int32)
    max_blocks = int(need.max())
    table = np.full((num_seqs, max_blocks), -1, np.int32)
    pos = 0
    for s in range(num_seqs):
        table[s, : need[s]] = perm[pos: pos + need[s]]
        pos += need[s]
    splits = 12  # the one-wave-per-slot kernel's pool-sized split count for C5 on 256 CUs
    # Longest sequences first, as the decode kernel schedules a ragged batch.
    order = np.argsort(-lengths, kind="stable")
    table, lengths = np.ascontiguousarray(table[order]), lengths[order]
    page = bs * Hkv * D * 2
    dk = H.DeviceBuffer(num_blocks * page)
    dv = H.DeviceBuffer(num_blocks * page)
    dt = H.DeviceBuffer.from_array(table)
    dl = H.DeviceBuffer.from_array(lengths.astype(np.int32))
    sink = H.DeviceBuffer(64)
    lib = ctypes.CDLL(os.path.join(sca_amd.hip.LIB_DIR, "libsca_calib.so"))
    c_vp, c_int = ctypes.c_void_p, ctypes.c_int
    lib.sca_calib_page_read.argtypes = [c_vp, c_vp, c_vp, c_vp] + [c_int] * 6 + [c_vp, c_vp]
    nbytes = int(lengths.sum()) * Hkv * D * 2 * 2
    # mode 0: K and V to registers, 4 rows x 256 B per load; mode 3: the decode kernel's own
    # pattern (V through LDS with global_load_lds, K as MFMA fragments of 16 rows x 64 B).
    variants = [(0, d) for d in (1, 2, 3, 4)] + [(3, d) for d in (1, 2)]
    out = {"bytes_read": nbytes, "splits": splits, "runs": {}}
    for mode, depth in variants:
        ms = time_launches(lambda: H.check(lib.sca_calib_page_read(
            dk.ptr, dv.ptr, dt.ptr, dl.ptr, num_seqs, Hkv, max_blocks, splits, depth, mode,
            sink.ptr, None)), steps, warmup)
        out["runs"][f"mode{mode}_depth{depth}"] = {"ms": ms, "gbps": nbytes / (ms * 1e-3) / 1e9}
    best = max((r for k, r in out["runs"].items() if k.startswith("mode0")), key=lambda r: r["gbps"])
    own = max((r for k, r in out["runs"].items() if k.startswith("mode3")), key=lambda r: r["gbps"])
    out["gbps"], out["ms"] = best["gbps"], best["ms"]
    out["decode_pattern_gbps"] = own["gbps"]
    return out


def bench_copy(steps, warmup, mib=256):
    """A plain copy of known size (the block gather kernel over ids 0..n-1): the reference point
    that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes, and the practical HBM
    copy rate."""
    bs, Hkv, D = 16, 8, 128
    page = bs * Hkv * D * 2
    n = mib * (1 << 20) // page
    src = H.DeviceBuffer(n * page)
    dst = H.DeviceBuffer(n * page)
    ids = H.DeviceBuffer.from_array(np.arange(n, dtype=np.int32))
    shape = H.KvShape()
    shape.num_blocks, shape.block_size, shape.num_kv_heads, shape.head_dim = n, bs, Hkv, D
    L = sca_amd.hip_lib()
    ms = time_launches(lambda: H.check(L.sca_hip_kv_gather(src.ptr, ids.ptr, n, dst.ptr, shape, 2,
                                                             None)), steps, warmup)
    nbytes = 2 * n * page
    return {"ms": ms, "bytes_read": n * page, "bytes_written": n * page,
            "gbps": nbytes / (ms * 1e-3) / 1e9}


# ---- CPU baseline ------------------------------------------------------------------------------------
def cpu_baseline(max_seconds=12.0):
    import oracle.oracle as orc  # the CPU restatement is the timed baseline

    threads = host_threads()
    S, D = 4096, 128
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 1, S, D), dtype=np.float32)
    k = rng.standard_normal((1, 1, S, D), dtype=np.float32)
    v = rng.standard_normal((1, 1, S, D), dtype=np.float32)
    scores = np.empty(S * S, np.float32)
    out = np.empty_like(q)
    lse = np.empty((1, 1, S), np.float32)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    runs, t0 = 0, time.perf_counter()
    while True:
        orc.naive_attention_into(q, k, v, True, scale, scores, out, lse, threads)
        runs += 1
        if time.perf_counter() - t0 >= max_seconds or runs >= 50:
            break
    secs = (time.perf_counter() - t0) / runs
    flops = causal_flops(1, 1, S, D)
    # C1 (the reference's CPU configuration): B=1, H=8, D=64, S=128, fp32, non-causal; P50 of
    # 100 runs after 20 warmup runs, on one thread and on all of them.
    c1 = {}
    S1, D1, H1 = 128, 64, 8
    q1 = rng.standard_normal((1, H1, S1, D1), dtype=np.float32)
    k1 = rng.standard_normal((1, H1, S1, D1), dtype=np.float32)
    v1 = rng.standard_normal((1, H1, S1, D1), dtype=np.float32)
    sc1 = np.empty(S1 * S1 * H1, np.float32)
    o1 = np.empty_like(q1)
    l1 = np.empty((1, H1, S1), np.float32)
    scale1 = float(np.float32(1.0 / np.sqrt(D1)))
    for nt in sorted({1, threads}):
        times = []
        for r in range(120):
            t1 = time.perf_counter()
            orc.naive_attention_into(q1, k1, v1, False, scale1, sc1, o1, l1, nt)
            if r >= 20:
                times.append(time.perf_counter() - t1)
        p50 = float(np.percentile(times, 50))
        c1[f"threads_{nt}"] = {"p50_ms": round(p50 * 1e3, 4),
                               "gflops": round(4 * H1 * S1 * S1 * D1 / p50 / 1e9, 2)}
    return {"value": flops / secs / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"naive 3-pass FP32 restatement (attention_naive.cu:41-135) on one head of "
                      f"C2 (B=1,H=1,S=4096,D=128,causal), {runs} runs, {secs * 1e3:.1f} ms/run, "
                      f"algorithmic causal FLOPs, {threads} threads",
            "host": host_cores(),
            "c1": c1}


def host_cores():
    """What the host reports: nproc (affinity-aware), std::thread::hardware_concurrency (the
    online CPUs, as os.cpu_count), the affinity mask, and the CPU share one GPU job is given."""
    try:
        nproc = int(subprocess.run(["nproc"], capture_output=True, text=True, timeout=10).stdout)
    except (OSError, ValueError, subprocess.SubprocessError):
        nproc = None
    share = os.environ.get("OMP_NUM_THREADS")
    return {"nproc": nproc, "hardware_concurrency": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0)),
            "job_cpu_share": int(share) if share and share.isdigit() else None}


def host_threads():
    """All the cores this process may use: the affinity mask, capped by the per-job CPU share
    the GPU box sets in OMP_NUM_THREADS (16 per GPU on this pool)."""
    n = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(n, 1)


# PCI device ids that rocm-smi may report in place of a product name.
PCI_NAMES = {"0x75a3": "AMD Instinct MI355X", "0x75a0": "AMD Instinct MI350X"}


def device_name(probe):
    """The device's marketing name: HIP's, else rocm-smi's product name (a PCI device id is
    translated, or dropped), else None."""
    name = probe.name.decode().strip()
    if name:
        return name
    if "rocprof" in os.environ.get("LD_PRELOAD", ""):
        # under the profiler a helper program would start with the GPU already initialised
        return None
    try:
        out = subprocess.run(["rocm-smi", "--showproductname", "--json"], capture_output=True,
                             text=True, timeout=30).stdout
        for card in json.loads(out).values():
            for key in ("Card Series", "Card series", "Card Model", "Card model", "Card SKU",
                        "Marketing Name", "Device Name"):
                val = str(card.get(key, "")).strip()
                if val.lower() in PCI_NAMES:
                    return PCI_NAMES[val.lower()]
                if val and val.upper() != "N/A" and not val.lower().startswith("0x"):
                    return val
    except (OSError, ValueError, subprocess.SubprocessError, AttributeError):
        pass
    return None


def load_traffic(name):
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--paged-steps", type=int, default=128)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prewarm", type=float, default=0.5,
                    help="seconds of untimed launches of each leg's own work before it is timed")
    ap.add_argument("--only", default="all",
                    help="comma list of prefill, gqa, paged, paged_host, decode, copy, "
                         "page_probe (default: all but copy and page_probe)")
    args = ap.parse_args()
    parts = ({"prefill", "gqa", "paged", "paged_host", "decode"} if args.only == "all"
             else set(args.only.split(",")))
    unknown = parts - {"prefill", "gqa", "paged", "paged_host", "decode", "copy", "page_probe"}
    if unknown:
        ap.error(f"unknown --only part(s): {sorted(unknown)}")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(this build has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    if not sca_amd.gpu_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    probe = sca_amd.device_probe(0)

    res = {}
    if "prefill" in parts:
        res["c2_causal"] = bench_flash(args.steps, args.warmup, True, prewarm_s=args.prewarm)
        res["c2_noncausal"] = bench_flash(args.steps, args.warmup, False, prewarm_s=args.prewarm)
    if "gqa" in parts:
        res["c3_gqa"] = bench_flash_gqa(max(5, args.steps // 5), 3, prewarm_s=args.prewarm)
    if "paged" in parts:
        res["c5_paged"] = bench_paged(args.paged_steps, prewarm_s=args.prewarm)
    if "paged_host" in parts:
        res["c5_host"] = bench_paged_host(args.paged_steps)
    if "decode" in parts:
        res["c4_decode"] = bench_decode(args.steps, args.warmup, prewarm_s=args.prewarm)
    if "copy" in parts:
        res["copy"] = bench_copy(args.steps, args.warmup)
    if "page_probe" in parts:
        res["page_probe"] = bench_page_probe(args.steps, args.warmup)

    line = {
        "metric": "prefill TFLOP/s (causal S=4096) + paged decode HBM GB/s, 1xMI355X",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (seeded N(0,1))",
        "device": {"name": device_name(probe), "arch": probe.arch_name.decode(),
                   "cus": probe.cu_count},
    }
    if "c2_causal" in res:
        c = res["c2_causal"]
        line.update({"value": round(c["tflops"], 2), "unit": "TFLOP/s",
                     "ms_per_step": round(c["ms"], 4)})
        line["config"] = {"workload": "C2 flash prefill fp16 causal B=1 H=8 D=128 S=4096",
                          "batch": 1, "heads": 8, "head_dim": 128, "seq_len": 4096,
                          "causal": True}
        line["roofline"] = {"bound": "mfma", "achieved": round(c["tflops"], 2),
                            "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(c["tflops"] / PEAK_FP16_TFLOPS, 4),
                            "traffic": load_traffic("flash_c2_causal")}
        n = res["c2_noncausal"]
        line["prefill_noncausal"] = {"value": round(n["tflops"], 2), "unit": "TFLOP/s",
                                     "ms": round(n["ms"], 4),
                                     "frac": round(n["tflops"] / PEAK_FP16_TFLOPS, 4),
                                     "launch_ms_pct": {k: round(v, 4) for k, v in n["pct"].items()}}
        line["launch_ms_pct"] = {k: round(v, 4) for k, v in c["pct"].items()}
    if "c3_gqa" in res:
        g = res["c3_gqa"]
        line["gqa_prefill_c3"] = {
            "value": round(g["tflops"], 2), "unit": "TFLOP/s", "dtype": "bf16",
            "ms": round(g["ms"], 4), "frac": round(g["tflops"] / PEAK_FP16_TFLOPS, 4),
            "workload": "C3 GQA causal flash prefill bf16 B=4 Hq=32 Hkv=8 D=128 S=8192, "
                        "N(0, 0.5^2)"}
    if "c5_paged" in res:
        pg = res["c5_paged"]
        line["paged_decode"] = {
            "value": round(pg["gbps"], 1), "unit": "GB/s", "dtype": "bf16",
            "ms_per_step": round(pg["ms"], 4), "steps": args.paged_steps,
            "splits": pg["splits"], "slot_waves": pg["slot_waves"],
            "workload": "C5 paged decode bf16, 64 seqs L~U[512,16384], bs=16, Hq=32, Hkv=8, "
                        "D=128, permuted block table, append 1 token/seq per step; the K/V "
                        "pool repeats one seeded 16M-element random chunk (values do not change "
                        "the work)",
            "roofline": {"bound": "hbm", "achieved": round(pg["gbps"], 1), "peak": PEAK_HBM_GBPS,
                         "unit": "GB/s", "frac": round(pg["gbps"] / PEAK_HBM_GBPS, 4),
                         "traffic": load_traffic("paged_c5")},
        }
    if "c5_host" in res:
        hp = res["c5_host"]
        line["paged_decode_host_api"] = {
            "value": round(hp["gbps"], 1), "unit": "GB/s", "dtype": "bf16",
            "ms_per_step": round(hp["ms"], 4), "append_batch_and_sync_ms": round(hp["append_sync_ms"], 4),
            "splits": hp["splits"],
            "workload": "C5 through PagedKVCache (pages scattered by interleaved appends) and "
                        "sca::paged_attention; API-inclusive attend time; one AppendTokensBatch "
                        "+ sparse page-table sync per step timed separately"}
    if "c4_decode" in res:
        d = res["c4_decode"]
        line["splitk_decode"] = {"value": round(d["gbps"], 1), "unit": "GB/s", "dtype": "f16",
                                 "ms": round(d["ms"], 4), "splits": d["splits"],
                                 "frac": round(d["gbps"] / PEAK_HBM_GBPS, 4)}
    if "copy" in res:
        line["copy_calibration"] = {k: round(v, 4) if isinstance(v, float) else v
                                    for k, v in res["copy"].items()}
    if "page_probe" in res:
        pr = res["page_probe"]
        line["page_read_calibration"] = {
            "gbps": round(pr["gbps"], 1), "ms": round(pr["ms"], 4),
            "decode_pattern_gbps": round(pr["decode_pattern_gbps"], 1), "splits": pr["splits"],
            "bytes_read": pr["bytes_read"],
            "runs": {k: {"gbps": round(r["gbps"], 1), "ms": round(r["ms"], 4)}
                     for k, r in pr["runs"].items()},
            "what": "C5's starting K/V pages read once in the paged decode's order, nothing "
                    "computed (lib/libsca_calib.so): gbps = best coalesced pattern, "
                    "decode_pattern_gbps = the decode kernel's own load pattern"}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()

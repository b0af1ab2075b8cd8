"""C5 as BASELINE.json defines it, checked end to end: 64 sequences with lengths ~ U[512, 16384],
block size 16, H_q 32, H_kv 8, D 128, bf16; the pool filled through PagedKVCache::AppendTokens in
a seeded interleaved order (scattered pages), then 128 steps of AppendTokensBatch (one token per
sequence) + SyncPageTable + sca::paged_attention. This is the loop bench.py times
(bench.C5HostLoop, the `paged_decode_host_api` leg).

At steps 0, 63 and 127:
  * the host page table, lengths and block counts equal those of the oracle's PagedKVCache
    restatement (oracle/sca_oracle.c over paged_kv_cache.cpp:52-201) driven by the same trace
    (AppendTokensBatch is one AppendTokens per sequence, in order);
  * the longest and the shortest sequence and four seeded others are checked against the FP64
    oracle (test_utils.hpp:229-285) over the rows each sequence holds, within the bf16 gate
    (max|out - ref| <= 1.6e-2 * max|ref|).
"""

import numpy as np
import pytest

import bench
import oracle.oracle as orc
from attn_util import check_attention, to_float

pytestmark = pytest.mark.gpu


def test_c5_append_then_attend_128_steps(hip):
    steps = 128
    loop = bench.C5HostLoop(steps)
    S, bs, Hq, Hkv, D = loop.num_seqs, loop.bs, loop.Hq, loop.Hkv, loop.D
    print(f"C5 loop: {S} sequences, pool {loop.num_blocks} blocks", flush=True)
    pk = orc.PagedKV(loop.num_blocks, bs, S)
    for e in loop.log:
        rc = pk.append(e[1], e[3])[0]
        assert rc == 0
    rng = np.random.default_rng(31)
    others = [int(x) for x in rng.choice(S, size=6, replace=False)]
    pick = [int(np.argmax(loop.lengths)), int(np.argmin(loop.lengths))]
    pick += [s for s in others if s not in pick][:4]
    q = to_float(loop.q_bits, "bf16").reshape(S, Hq, 1, D)
    for t in range(steps):
        loop.append_step()
        for s in range(S):
            assert pk.append(s, 1)[0] == 0
        if t not in (0, 63, 127):
            continue
        res = loop.attend()
        out = to_float(res.out.numpy(np.uint16), "bf16").reshape(S, Hq, D)
        host = loop.cache.page_table_host()
        assert np.array_equal(host, pk.page_table()), f"step {t}: page table"
        for s in range(S):
            assert loop.cache.seq_length(s) == pk.seq_len(s) == loop.lengths[s] + t + 1
            assert loop.cache.logical_block_count(s) == pk.block_count(s)
        dev = loop.cache.page_table_device()
        assert np.array_equal(dev, host), f"step {t}: device page table"
        for s in pick:
            kb, vb = loop.rows(s)
            assert kb.shape[0] == loop.lengths[s] + t + 1
            k = to_float(kb, "bf16").transpose(1, 0, 2)[None]
            v = to_float(vb, "bf16").transpose(1, 0, 2)[None]
            ref, _ = orc.reference_attention(q[s:s + 1], k, v, False)
            check_attention(out[s].reshape(-1, D), ref, "bf16", f"C5 step {t} seq {s}")
        print(f"step {t}: table, lengths and sequences {pick} checked", flush=True)

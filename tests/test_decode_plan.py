"""The length-aware plan of the paged MFMA decode kernel (sca_paged_decode_plan), on the CPU.

The expected (splits, slot_waves) pairs are the fastest settings measured on an MI355X (256 CUs)
for these batches in 48-step bf16 decode loops (H_q 32, H_kv 8, D 128, bs 16): each row names
the measured rate of the chosen setting and of the best alternative."""

import numpy as np
import pytest

from sca_amd import host as H

CUS = 256


def lengths_uniform_random(n, lo, hi, seed=5005):
    return np.random.default_rng(seed).integers(lo, hi + 1, size=n).astype(np.int64)


@pytest.mark.parametrize("name,lengths,want", [
    # C5: ragged, 64 x 8 slots = two per CU -> four waves per slot, 3 splits (5.74 TB/s;
    # one wave per slot at its best split count, 12: 5.61)
    ("c5", lengths_uniform_random(64, 512, 16384), (3, 4)),
    # uniform 64 x 8448: one wave per slot, one workgroup per CU (5.89 TB/s; four waves: 5.58)
    ("uniform64", np.full(64, 8448), (2, 1)),
    # uniform 32 x 16384: 4 splits, one wave per slot (5.88 TB/s; four waves: 5.65)
    ("uniform32", np.full(32, 16384), (4, 1)),
    # 16 ragged sequences: four waves per slot, 12 splits (4.98 TB/s; one wave per slot: 4.26)
    ("ragged16", lengths_uniform_random(16, 512, 16384), (12, 4)),
    # 128 ragged sequences (four slots per CU): one wave per slot, 6 splits (5.57 TB/s)
    ("ragged128", lengths_uniform_random(128, 128, 8192), (6, 1)),
    # mildly ragged (longest 5/4 of the mean): four waves per slot, 3 splits (5.55 TB/s; one
    # wave per slot at one workgroup per CU: 5.41)
    ("mild64", lengths_uniform_random(64, 6000, 10000), (3, 4)),
    # 256 ragged sequences: one wave per slot, 3 splits (5.56 TB/s; four waves: 5.54 at 1)
    ("ragged256", lengths_uniform_random(256, 512, 4096), (3, 1)),
])
def test_plan_picks_the_measured_setting(name, lengths, want):
    assert H.paged_decode_plan(lengths, 32, 8, CUS) == want, name


def test_plan_bounds():
    # each split keeps at least 512 keys of the longest sequence
    assert H.paged_decode_plan(np.full(64, 300), 32, 8, CUS) == (1, 1)
    assert H.paged_decode_plan(np.full(4, 1500), 32, 8, CUS) == (3, 1)
    # the split count never exceeds the table's cap of 64
    assert H.paged_decode_plan([100000], 32, 8, CUS) == (64, 1)
    assert H.paged_decode_plan([100000, 1], 8, 8, CUS) == (64, 4)
    # no lengths known: one split, library default
    assert H.paged_decode_plan(np.zeros(8), 32, 8, CUS) == (1, 0)
    # a KV head with more than 16 query heads takes one slot per 16 of them: 32 heads over one KV
    # head fill twice the slots of 16, so half the splits reach the same occupancy
    lens = lengths_uniform_random(200, 512, 16384)
    assert H.paged_decode_plan(lens, 16, 1, CUS) == (8, 4)
    assert H.paged_decode_plan(lens, 32, 1, CUS) == (4, 4)


def test_plan_for_every_batch_is_within_bounds():
    rng = np.random.default_rng(1)
    for _ in range(200):
        n = int(rng.integers(1, 600))
        lens = rng.integers(0, 40000, size=n)
        hkv = int(rng.choice([1, 2, 4, 8]))
        hq = hkv * int(rng.choice([1, 2, 4, 8, 32]))
        splits, waves = H.paged_decode_plan(lens, hq, hkv, CUS)
        assert 1 <= splits <= 64
        if lens.max() == 0:
            assert (splits, waves) == (1, 0)
        else:
            assert waves in (1, 4)
            assert splits <= max(1, -(-int(lens.max()) // 512))


def test_plan_rejects_invalid_heads():
    with pytest.raises(Exception):
        H.paged_decode_plan([10], 6, 4, CUS)
    with pytest.raises(Exception):
        H.paged_decode_plan([], 32, 8, CUS)


@pytest.mark.parametrize("B,S,want", [
    (16, 4096, 8),    # C4: 128 slots -> four workgroups per CU (5.97 TB/s)
    (64, 4096, 1),    # a slot per CU or more runs unsplit, no combine (6.07 TB/s vs 5.65 at 8)
    (128, 2048, 1),   # (6.02 vs 5.64 at 4)
    (32, 4096, 1),    # (5.74 vs 5.42 at 8)
    (8, 32768, 8),    # at most 8 splits (5.95 vs 5.47 at 64)
    (4, 16384, 8),    # (5.84 vs 5.66 at 32)
    (1, 65536, 32),   # unless fewer leave CUs idle (5.60 vs 5.22 at 64)
    (24, 4096, 6),    # four workgroups per CU
    (1, 2048, 4),     # each split keeps 512 keys
])
def test_contiguous_decode_splits(B, S, want):
    assert H.decode_splits(H.AttentionShape(B, 1, S, 32, 8, 128), CUS) == want


@pytest.mark.parametrize("B,S,want", [(4, 16384, 32), (16, 4096, 8), (64, 4096, 1), (1, 1024, 2)])
def test_contiguous_decode_splits_valu_head_dim(B, S, want):
    # head_dim 96 runs the VALU kernel: splits until every CU holds four workgroups, no cap at
    # 8, and at least min_tokens_per_split keys per split (the 1 x 1024 case)
    assert H.decode_splits(H.AttentionShape(B, 1, S, 32, 8, 96), CUS) == want

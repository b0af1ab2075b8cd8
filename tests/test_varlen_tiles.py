"""The work list of the one-launch varlen prefill (host code of libsca_hip.so; no GPU needed)."""

import numpy as np
import pytest

from sca_amd import hip as H


def _keys(sq, skv, t, causal):
    last = min(sq, (t + 1) * 128) - 1 + (skv - sq)
    return min(skv, last + 1) if causal else skv


@pytest.mark.parametrize("causal", [False, True])
def test_tiles_cover_every_row_tile_once_longest_first(causal):
    rng = np.random.default_rng(3)
    lens_q = rng.integers(1, 900, size=17)
    lens_kv = lens_q + (rng.integers(0, 300, size=17) if causal else rng.integers(-50, 300, size=17).clip(-lens_q + 1))
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_kv = np.concatenate([[0], np.cumsum(lens_kv)]).astype(np.int32)
    tiles = H.flash_varlen_tiles(cu_q, cu_kv, causal)
    want = {(s, t) for s in range(17) for t in range((int(lens_q[s]) + 127) // 128)}
    got = [tuple(map(int, x)) for x in tiles]
    assert sorted(got) == sorted(want) and len(got) == len(want)
    keys = [_keys(int(lens_q[s]), int(lens_kv[s]), t, causal) for s, t in got]
    assert all(a >= b for a, b in zip(keys, keys[1:]))


def test_tiles_reject_invalid_lengths():
    cu = np.array([0, 10, 20], np.int32)
    with pytest.raises(Exception):
        H.flash_varlen_tiles(cu, np.array([0, 5, 30], np.int32), True)  # causal S_kv < S_q
    with pytest.raises(Exception):
        H.flash_varlen_tiles(cu, np.array([0, 0, 10], np.int32), False)  # S_kv = 0

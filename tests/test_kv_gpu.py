"""KV cache data movement on the GPU (sca_hip_kv_append / reset_blocks / gather), checked as
round trips over the block-major layout (kv_cache_kernels.cu:17-86 semantics)."""

import numpy as np
import pytest

import sca_amd
from sca_amd import hip as H

pytestmark = pytest.mark.gpu


def _shape(nb, bs, hkv, d):
    s = H.KvShape()
    s.num_blocks, s.block_size, s.num_kv_heads, s.head_dim = nb, bs, hkv, d
    return s


@pytest.mark.parametrize("bs", [1, 8, 16, 32, 64])
@pytest.mark.parametrize("elem", [2, 4])
def test_append_gather_reset_round_trip(hip, bs, elem):
    L = sca_amd.hip_lib()
    nb, hkv, d = 6, 2, 64
    row = hkv * d * elem
    rng = np.random.default_rng(bs * 10 + elem)
    dtype = np.uint16 if elem == 2 else np.uint32
    layer_k = H.DeviceBuffer.zeros(nb * bs * row)
    layer_v = H.DeviceBuffer.zeros(nb * bs * row)
    T = 3 * bs + 1
    slots = rng.permutation(nb * bs)[:T].astype(np.int32)
    slots[1] = -1                # skipped
    slots[2] = nb * bs + 5       # block beyond the pool: skipped
    k_new = rng.integers(1, 60000, size=(T, hkv, d)).astype(dtype)
    v_new = rng.integers(1, 60000, size=(T, hkv, d)).astype(dtype)
    dk, dv = H.DeviceBuffer.from_array(k_new), H.DeviceBuffer.from_array(v_new)
    ds = H.DeviceBuffer.from_array(slots)
    shape = _shape(nb, bs, hkv, d)
    H.check(L.sca_hip_kv_append(layer_k.ptr, layer_v.ptr, dk.ptr, dv.ptr, ds.ptr, T, shape, elem,
                                None))
    ids = np.arange(nb, dtype=np.int32)[::-1].copy()
    dids = H.DeviceBuffer.from_array(ids)
    out = H.DeviceBuffer(nb * bs * row)
    H.check(L.sca_hip_kv_gather(layer_k.ptr, dids.ptr, nb, out.ptr, shape, elem, None))
    sca_amd.synchronize()
    got = out.download(dtype).reshape(nb, bs, hkv, d)[::-1].reshape(nb * bs, hkv, d)
    expect = np.zeros((nb * bs, hkv, d), dtype)
    for t, s in enumerate(slots):
        if 0 <= s < nb * bs:
            expect[s] = k_new[t]
    assert np.array_equal(got, expect)
    # reset two blocks (plus an invalid id): only those become zero
    rid = np.array([1, 4, -3], np.int32)
    drid = H.DeviceBuffer.from_array(rid)
    H.check(L.sca_hip_kv_reset_blocks(layer_k.ptr, layer_v.ptr, drid.ptr, 3, shape, elem, None))
    vk = layer_v.download(dtype).reshape(nb, bs, hkv, d)
    kk = layer_k.download(dtype).reshape(nb, bs, hkv, d)
    e = expect.reshape(nb, bs, hkv, d).copy()
    e[[1, 4]] = 0
    assert np.array_equal(kk, e)
    assert not np.any(vk[[1, 4]])
    # gather with an invalid id yields zero rows
    gid = H.DeviceBuffer.from_array(np.array([0, 99], np.int32))
    out2 = H.DeviceBuffer(2 * bs * row)
    H.check(L.sca_hip_kv_gather(layer_k.ptr, gid.ptr, 2, out2.ptr, shape, elem, None))
    g2 = out2.download(dtype).reshape(2, bs, hkv, d)
    assert np.array_equal(g2[0], e[0]) and not np.any(g2[1])

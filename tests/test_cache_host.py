"""Host-side cache logic on the CPU: growth, layouts, masks, state round trip.

The reference's cache-surface invariants (engine/tests/test_shared_kv.py:19-37,
64-79) are mirrored: views follow writes, growth keeps the earlier contents,
limits raise "Decode context limit exhausted", a failed call invalidates.
"""

import numpy as np
import pytest
import torch

from rec_amd import MixedQuantizedKVCache, QuantizedKV, QuantizedKVCache, to_logical
from rec_amd.cache import BLOCK, _alloc


def _block_v8(codes_logical):
    """Independent blocked layout for int8 V: [B][H][T/64][128][64]."""
    B, H, T, D = codes_logical.shape
    x = codes_logical.reshape(B, H, T // 64, 64, D).transpose(0, 1, 2, 4, 3)
    return np.ascontiguousarray(x).reshape(B, H, T // 64, D * 64)


def _block_v4(q):
    """uint4 V codes q[B][H][T][128] (0..15) -> [B][H][T/64][128][32] bytes."""
    B, H, T, D = q.shape
    x = q.reshape(B, H, T // 64, 64, D).transpose(0, 1, 2, 4, 3)  # [.., d, t]
    packed = x[..., 0::2] | (x[..., 1::2] << 4)
    return np.ascontiguousarray(packed).reshape(B, H, T // 64, D * 32).astype(np.uint8)


def test_to_logical_int8_blocked_roundtrip():
    rng = np.random.default_rng(0)
    logical = rng.integers(-127, 128, size=(2, 3, 128, 128), dtype=np.int8)
    blocked = torch.from_numpy(_block_v8(logical))
    scales = torch.from_numpy(rng.standard_normal((2, 3, 128)).astype(np.float16))
    kv = QuantizedKV(blocked, scales, None, 8, 100, True)
    c, s, z = to_logical(kv)
    np.testing.assert_array_equal(c.numpy(), logical[:, :, :100])
    np.testing.assert_array_equal(s.numpy(), scales.numpy()[:, :, :100])
    assert z is None


def test_to_logical_int4_blocked_roundtrip():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(1, 2, 192, 128), dtype=np.uint8)
    blocked = torch.from_numpy(_block_v4(q))
    sc = rng.standard_normal((1, 2, 3, 4, 64)).astype(np.float16)
    zp = rng.integers(0, 16, size=(1, 2, 3, 4, 64)).astype(np.float16)
    kv = QuantizedKV(blocked, torch.from_numpy(sc), torch.from_numpy(zp), 4, 150, True)
    c, s, z = to_logical(kv)
    expect = q[..., 0::2] | (q[..., 1::2] << 4)
    np.testing.assert_array_equal(c.numpy(), expect[:, :, :150])
    # scale of token t, group g lives at [t // 64][g][t % 64]
    t, g = 130, 3
    assert s.numpy()[0, 1, t, g] == sc[0, 1, t // 64, g, t % 64]
    assert z.numpy()[0, 0, t, g] == zp[0, 0, t // 64, g, t % 64]


def test_alloc_shapes():
    k = _alloc(1, 4, 256, 8, False, "cpu")
    v = _alloc(1, 4, 256, 4, True, "cpu")
    assert k[0].shape == (1, 4, 256, 128) and k[1].shape == (1, 4, 256) and k[2] is None
    assert v[0].shape == (1, 4, 4, 128 * 32) and v[1].shape == (1, 4, 4, 4, 64) and v[2].shape == v[1].shape
    assert QuantizedKV(*v, 4, 0, True).capacity == 256
    assert QuantizedKV(*k, 8, 0, False).capacity == 256


def test_growth_keeps_contents_and_step_rounding():
    c = QuantizedKVCache(32, 8, 4)
    c._reserve(1, 2, 5, "cpu")
    assert c.capacity == 256
    c.keys[0][0, 1, 3] = 7
    c.values[1][0, 0, 0, 2, 5] = 1.5
    c._reserve(1, 2, 300, "cpu")
    assert c.capacity == 512
    assert c.keys[0][0, 1, 3, 0] == 7
    assert c.values[1][0, 0, 0, 2, 5] == 1.5
    c._reserve(1, 2, 512, "cpu")
    assert c.capacity == 512


def test_limits_and_invalidation():
    c = QuantizedKVCache(32, 8, 8, max_tokens=100)
    c._reserve(1, 1, 10, "cpu")
    assert c.capacity == 128  # one allocation, rounded to 64-token blocks
    with pytest.raises(ValueError, match="Decode context limit exhausted"):
        c._reserve(1, 1, 101, "cpu")
    c._usable = False
    with pytest.raises(RuntimeError, match="invalidated"):
        c._check_usable()


def test_constructor_validation_and_mixed_defaults():
    m = MixedQuantizedKVCache()
    assert (m.key_bits, m.value_bits, m.group_size, m.bits) == (8, 4, 32, 8)
    with pytest.raises(ValueError):
        QuantizedKVCache(64, 8, 4)
    with pytest.raises(ValueError):
        QuantizedKVCache(32, 3, 8)


def test_mask_trim_state():
    c = QuantizedKVCache(32, 8, 8)
    assert c.empty() and c.size() == 0 and c.make_mask(1) is None
    assert c.make_mask(5) == "causal"
    c._reserve(1, 1, 10, "cpu")
    c.offset = 10
    m = c.make_mask(3, return_array=True)
    assert m.shape == (3, 13) and bool(m[0, 10]) and not bool(m[0, 11]) and bool(m[2, 12])
    assert c.is_trimmable() and c.trim(4) == 4 and c.offset == 6
    st = c.state
    d = QuantizedKVCache(32, 4, 4)
    d.state = st
    assert (d.offset, d.key_bits, d.value_bits, d.capacity) == (6, 8, 8, 256)
    assert d.keys[0] is c.keys[0]
    assert d.meta_state == ("256", "6", "32", "8", "8")
    assert c.nbytes == 256 * 128 * 2 + 256 * 2 * 2

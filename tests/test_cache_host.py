"""Host-side cache logic on the CPU: growth, layouts, masks, state round trip.

The reference's cache-surface invariants (engine/tests/test_shared_kv.py:19-37,
64-79) are mirrored: views follow writes, growth keeps the earlier contents,
limits raise "Decode context limit exhausted", a failed call invalidates.
"""

import numpy as np
import pytest
import torch

from rec_amd import MixedQuantizedKVCache, QuantizedKV, QuantizedKVCache, to_logical
from rec_amd.cache import _alloc


def _pos(t):
    # tokens 16j + 4kg + i of a 32-token block sit at positions 8kg + 4j + i
    j, kg, i = t // 16, (t // 4) % 4, t % 4
    return 8 * kg + 4 * j + i


def _store_k(logical, bits):
    """Independent loop construction of the K code layouts.

    int8: [nb][2 halves][32 tokens][64 bytes].  int4 (64 packed bytes per
    token, byte L = half L // 32, byte b = L % 32 of the half):
    [nb][32 tokens][4 runs of 8 bytes][2 halves][8 bytes].
    """
    B, H, T, W = logical.shape  # W = 128 (int8) or 64 packed bytes (int4)
    w = W // 2
    out = np.zeros((B, H, T // 32, 2 * 32 * w), logical.dtype)
    for t in range(T):
        if bits == 8:
            for m in range(2):
                out[:, :, t // 32, m * 32 * w + (t % 32) * w : m * 32 * w + (t % 32) * w + w] = logical[:, :, t, m * w : (m + 1) * w]
        else:
            for L in range(64):
                m, b = L // 32, L % 32
                out[:, :, t // 32, (t % 32) * 64 + (b // 8) * 16 + m * 8 + b % 8] = logical[:, :, t, L]
    return out


def _store_v8(logical):
    """int8 V codes: dim d = 16 n + c at position p = 8 kg + e sits in byte
    [n // 2][c][kg][n % 2][e] of its 4096-byte block."""
    B, H, T, D = logical.shape
    out = np.zeros((B, H, T // 32, D * 32), np.int8)
    for t in range(T):
        p = _pos(t % 32)
        for d in range(D):
            n, c = d // 16, d % 16
            out[:, :, t // 32, (n // 2) * 1024 + (c * 4 + p // 8) * 16 + (n % 2) * 8 + p % 8] = logical[:, :, t, d]
    return out


def _store_v4(q):
    """uint4 V codes q[B][H][T][128] (0..15) -> 2048-byte blocks.

    Dim d = 16 n + c at position p = 8 kg + e sits in byte
    [n // 4][c][kg][n % 4][e // 2], low nibble = even e.
    """
    B, H, T, D = q.shape
    out = np.zeros((B, H, T // 32, D * 16), np.uint8)
    for t in range(T):
        p = _pos(t % 32)
        for d in range(D):
            n, c = d // 16, d % 16
            byte = (n // 4) * 1024 + (c * 4 + p // 8) * 16 + (n % 4) * 4 + (p % 8) // 2
            out[:, :, t // 32, byte] |= (q[:, :, t, d] << (4 * (p % 2))).astype(np.uint8)
    return out


def _store_scales(logical, groups=None):
    if groups is None:  # (B, H, T) -> (B, H, nb, 32)
        B, H, T = logical.shape
        out = np.zeros((B, H, T // 32, 32), logical.dtype)
        for t in range(T):
            out[:, :, t // 32, _pos(t % 32)] = logical[:, :, t]
        return out
    B, H, T, G = logical.shape
    out = np.zeros((B, H, T // 32, G, 32), logical.dtype)
    order = [0, 4, 1, 5, 2, 6, 3, 7]  # positions held by the 8 slots of each run
    for t in range(T):
        p = _pos(t % 32)
        slot = (p // 8) * 8 + order.index(p % 8)
        out[:, :, t // 32, :, slot] = logical[:, :, t, :]
    return out


def test_block_pos_is_a_permutation_keeping_pairs():
    from rec_amd.cache import block_pos

    ps = [block_pos(t) for t in range(32)]
    assert sorted(ps) == list(range(32))
    assert all(ps[t] == _pos(t) for t in range(32))
    assert all(block_pos(t ^ 1) == ps[t] ^ 1 for t in range(32))


def test_to_logical_int8_roundtrip():
    rng = np.random.default_rng(0)
    kl = rng.integers(-127, 128, size=(2, 3, 96, 128), dtype=np.int8)
    vl = rng.integers(-127, 128, size=(2, 3, 96, 128), dtype=np.int8)
    sl = rng.standard_normal((2, 3, 96)).astype(np.float16)
    k = QuantizedKV(torch.from_numpy(_store_k(kl, 8)), torch.from_numpy(_store_scales(sl)), None, 8, 70, False)
    v = QuantizedKV(torch.from_numpy(_store_v8(vl)), torch.from_numpy(_store_scales(sl)), None, 8, 70, True)
    c, s, z = to_logical(k)
    np.testing.assert_array_equal(c.numpy(), kl[:, :, :70])
    np.testing.assert_array_equal(s.numpy(), sl[:, :, :70])
    assert z is None
    c, s, _ = to_logical(v)
    np.testing.assert_array_equal(c.numpy(), vl[:, :, :70])


def test_to_logical_int4_roundtrip():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(1, 2, 64, 128), dtype=np.uint8)
    packed = q[..., 0::2] | (q[..., 1::2] << 4)
    sc = rng.standard_normal((1, 2, 64, 4)).astype(np.float16)
    zp = rng.integers(0, 16, size=(1, 2, 64, 4)).astype(np.float16)
    k = QuantizedKV(torch.from_numpy(_store_k(packed, 4)), torch.from_numpy(_store_scales(sc, 4)),
                    torch.from_numpy(_store_scales(zp, 4)), 4, 50, False)
    v = QuantizedKV(torch.from_numpy(_store_v4(q)), torch.from_numpy(_store_scales(sc, 4)),
                    torch.from_numpy(_store_scales(zp, 4)), 4, 50, True)
    for kv in (k, v):
        c, s, z = to_logical(kv)
        np.testing.assert_array_equal(c.numpy(), packed[:, :, :50])
        np.testing.assert_array_equal(s.numpy(), sc[:, :, :50])
        np.testing.assert_array_equal(z.numpy(), zp[:, :, :50])


def test_alloc_shapes():
    k = _alloc(1, 4, 256, 8, False, "cpu")
    v = _alloc(1, 4, 256, 4, True, "cpu")
    assert k[0].shape == (1, 4, 8, 32 * 128) and k[1].shape == (1, 4, 8, 32) and k[2] is None
    assert v[0].shape == (1, 4, 8, 32 * 64) and v[1].shape == (1, 4, 8, 4, 32) and v[2].shape == v[1].shape
    assert QuantizedKV(*v, 4, 0, True).capacity == 256
    assert QuantizedKV(*k, 8, 0, False).capacity == 256


def test_growth_keeps_contents_and_step_rounding():
    c = QuantizedKVCache(32, 8, 4)
    c._reserve(1, 2, 5, "cpu")
    assert c.capacity == 256
    c.keys[0][0, 1, 3, 5] = 7
    c.values[1][0, 0, 0, 2, 5] = 1.5
    c._reserve(1, 2, 300, "cpu")
    assert c.capacity == 512
    assert c.keys[0][0, 1, 3, 5] == 7
    assert c.values[1][0, 0, 0, 2, 5] == 1.5
    c._reserve(1, 2, 512, "cpu")
    assert c.capacity == 512


def test_limits_and_invalidation():
    c = QuantizedKVCache(32, 8, 8, max_tokens=100)
    c._reserve(1, 1, 10, "cpu")
    assert c.capacity == 128  # one allocation, rounded to 32-token blocks
    with pytest.raises(ValueError, match="Decode context limit exhausted"):
        c._reserve(1, 1, 101, "cpu")
    c._usable = False
    with pytest.raises(RuntimeError, match="invalidated"):
        c._check_usable()


def test_constructor_validation_and_mixed_defaults():
    m = MixedQuantizedKVCache()  # the reference's defaults: group 64 affine, 8-bit K, 4-bit V
    assert (m.key_bits, m.value_bits, m.group_size, m.bits, m.affine) == (8, 4, 64, 8, True)
    m32 = MixedQuantizedKVCache(32)
    assert (m32.key_bits, m32.value_bits, m32.affine) == (8, 4, False)
    with pytest.raises(NotImplementedError):
        QuantizedKVCache(64, 8, 8)
    with pytest.raises(ValueError):
        QuantizedKVCache(48, 8, 4)
    with pytest.raises(ValueError):
        QuantizedKVCache(32, 3, 8)


def _store_affine_scales(sc, bi):
    """(B, H, T, 2) scales and biases -> [nb][scale, bias][2 groups][32 slots],
    each run of 8 positions stored as 0, 4, 1, 5, 2, 6, 3, 7."""
    B, H, T, G = sc.shape
    out = np.zeros((B, H, T // 32, 2, G, 32), sc.dtype)
    order = [0, 4, 1, 5, 2, 6, 3, 7]
    for t in range(T):
        p = _pos(t % 32)
        slot = (p // 8) * 8 + order.index(p % 8)
        out[:, :, t // 32, 0, :, slot] = sc[:, :, t]
        out[:, :, t // 32, 1, :, slot] = bi[:, :, t]
    return out


def test_to_logical_affine_roundtrip():
    rng = np.random.default_rng(2)
    kq = rng.integers(0, 256, size=(1, 2, 64, 128), dtype=np.uint8)
    vq = rng.integers(0, 16, size=(1, 2, 64, 128), dtype=np.uint8)
    vpacked = vq[..., 0::2] | (vq[..., 1::2] << 4)
    sc = torch.randn((1, 2, 64, 2)).to(torch.bfloat16)
    bi = torch.randn((1, 2, 64, 2)).to(torch.bfloat16)
    sb = torch.from_numpy(_store_affine_scales(sc.view(torch.int16).numpy(), bi.view(torch.int16).numpy()))
    sb = sb.view(torch.bfloat16)
    k = QuantizedKV(torch.from_numpy(_store_k(kq, 8)), sb, None, 8, 50, False, True)
    v = QuantizedKV(torch.from_numpy(_store_v4(vq)), sb, None, 4, 50, True, True)
    assert (k.code, v.code) == (0x108, 0x104)
    for kv, codes in ((k, kq), (v, vpacked)):
        c, s, b = to_logical(kv)
        np.testing.assert_array_equal(c.numpy(), codes[:, :, :50])
        assert torch.equal(s, sc[:, :, :50]) and torch.equal(b, bi[:, :, :50])
    ka = _alloc(1, 4, 64, 8, False, "cpu", True)
    va = _alloc(1, 4, 64, 4, True, "cpu", True)
    assert ka[0].shape == (1, 4, 2, 4096) and ka[1].shape == (1, 4, 2, 2, 2, 32) and ka[2] is None
    assert va[0].shape == (1, 4, 2, 2048) and va[1].dtype == torch.bfloat16
    # fp16 scales and biases: the fp16 affine codes of the C ABI
    k16 = QuantizedKV(torch.from_numpy(_store_k(kq, 8)), sb.view(torch.float16), None, 8, 50, False, True)
    v16 = QuantizedKV(torch.from_numpy(_store_v4(vq)), sb.view(torch.float16), None, 4, 50, True, True)
    assert (k16.code, v16.code) == (0x208, 0x204)


def test_affine_scales_take_the_keys_dtype():
    """The reference allocates the affine scales and biases in the keys' dtype
    (model.py:57-58): fp16 keys give fp16, bf16 keys bf16; fp32 keys bf16 (the
    kernels read 16-bit scales).  Growth keeps the first allocation's dtype."""
    from rec_amd import MixedQuantizedKVCache
    from rec_amd.cache import affine_meta_dtype

    assert affine_meta_dtype(torch.float16) == torch.float16
    assert affine_meta_dtype(torch.bfloat16) == torch.bfloat16
    assert affine_meta_dtype(torch.float32) == torch.bfloat16
    c = MixedQuantizedKVCache()
    c._reserve(1, 2, 10, "cpu", torch.float16)
    assert c.keys[1].dtype == torch.float16 and c.values[1].dtype == torch.float16
    c._reserve(1, 2, 1000, "cpu", torch.bfloat16)  # growth: the dtype stays
    assert c.capacity == 1024 and c.keys[1].dtype == torch.float16
    st = c.state
    assert st[0][1].dtype == torch.float16
    k, v = c.keys_and_values()
    assert (k.code, v.code) == (0x208, 0x204)
    d = QuantizedKVCache(32, 8, 8)  # int8 / uint4 scales are fp16 whatever the keys
    d._reserve(1, 1, 10, "cpu", torch.bfloat16)
    assert d.keys[1].dtype == torch.float16


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


def test_make_cache_full_attention_layers():
    """make_cache builds what Model.make_cache does for full-attention layers
    (model.py:347-360): MixedQuantizedKVCache(kv_group_size, kv_key_bits,
    kv_value_bits), the reference's defaults 64 / 8 / 4 (model.py:35-37)."""
    from rec_amd import make_cache

    caches = make_cache(["full_attention"] * 3, max_tokens=4096)
    assert len(caches) == 3 and len({id(c) for c in caches}) == 3
    for c in caches:
        assert type(c) is MixedQuantizedKVCache
        assert (c.group_size, c.key_bits, c.value_bits) == (64, 8, 4)
        assert c.offset == 0
    c = make_cache(["full_attention"], kv_group_size=32, kv_key_bits=8, kv_value_bits=4)[0]
    assert (c.group_size, c.key_bits, c.value_bits) == (32, 8, 4)
    with pytest.raises(NotImplementedError):  # the affine format is 8-bit keys with 4-bit values
        make_cache(["full_attention"], kv_key_bits=4)
    assert make_cache([]) == []

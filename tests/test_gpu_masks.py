"""Mask arrays on the attention entry points (model.py:122-128): boolean and
additive (0 / -inf) arrays whose pattern is every key, causal, or causal
over the last `window` keys run on the kernels' own masking and match the
oracle under the same array; the string form gives the same bytes."""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import (FixedKVCache, KVStorage, MixedQuantizedKVCache, QuantizedKVCache, attend,
                     quantized_attention_with_sinks, scaled_dot_product_attention, synthetic)
from tests.gpu_util import (SCALE, assert_cache_equal, assert_close, dequant, f32, oracle_quantize, oracle_xhat,
                            prefill_side)

pytestmark = pytest.mark.gpu


def keep_pattern(L, T, window=0):
    q = np.arange(T - L, T)[:, None]
    k = np.arange(T)[None]
    m = q >= k
    return m & (q < k + window) if window else m


def quantized_cache(bits, T, seed):
    c = QuantizedKVCache(32, *bits)
    k = synthetic.kv((1, 2, T, 128), seed, kind="outliers", frac=0.02)
    v = synthetic.kv((1, 2, T, 128), seed + 1, kind="outliers", frac=0.02)
    kq, vq = c.update_and_fetch(k, v)
    kh = dequant(bits[0], *oracle_quantize(f32(k), bits[0]))
    vh = dequant(bits[1], *oracle_quantize(f32(v), bits[1]))
    return kq, vq, kh, vh


@pytest.mark.parametrize("form", ["bool", "bool4d", "additive"])
def test_int8_prefill_mask_arrays(gpu, form):
    L, T = 40, 300
    kq, vq, kh, vh = quantized_cache((8, 8), T, 11)
    q = synthetic.query(1, 16, L, 12, dtype=torch.bfloat16)
    sinks = torch.randn(16, device="cuda")
    keep = keep_pattern(L, T)
    if form == "bool":
        mask = torch.from_numpy(keep).cuda()
    elif form == "bool4d":
        mask = torch.from_numpy(keep).cuda()[None, None]
    else:
        mask = torch.zeros((L, T), device="cuda").masked_fill(~torch.from_numpy(keep).cuda(), float("-inf"))
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, mask, sinks, 32, 8, 8, out_dtype=torch.float32)
    ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks), keep)
    assert_close(f32(out), ref, form)
    same = quantized_attention_with_sinks(q, kq, vq, SCALE, "causal", sinks, 32, 8, 8, out_dtype=torch.float32)
    assert torch.equal(out, same)


def test_decode_all_keys_mask_arrays(gpu):
    T = 777
    kq, vq, kh, vh = quantized_cache((8, 4), T, 21)
    q = synthetic.query(1, 16, 1, 22)
    outs = [quantized_attention_with_sinks(q, kq, vq, SCALE, m, None, 32, 8, 4, out_dtype=torch.float32)
            for m in (None, torch.ones((1, T), dtype=torch.bool, device="cuda"), torch.zeros((1, 1, 1, T), device="cuda"))]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert_close(f32(outs[0]), O.attention(f32(q), kh, vh, SCALE), "decode")
    with pytest.raises(NotImplementedError):  # a window at one query runs on the matrix cores: bf16/f16 only
        quantized_attention_with_sinks(q.float(), kq, vq, SCALE, torch.from_numpy(keep_pattern(1, T, 100)).cuda(),
                                       None, 32, 8, 4)


WINDOW_FORMATS = {
    "i8_i8": lambda: QuantizedKVCache(32, 8, 8),
    "u4_u4": lambda: QuantizedKVCache(32, 4, 4),
    "i8_u4": lambda: QuantizedKVCache(32, 8, 4),
    "affine": lambda: MixedQuantizedKVCache(),
}
WINDOW_CASES = [
    # format, L, T, window, splits (0 = automatic), query dtype
    ("u4_u4", 33, 500, 64, 0, torch.float16),
    ("i8_i8", 100, 2000, 300, 7, torch.bfloat16),   # splits before the window start stay empty
    ("i8_u4", 40, 1500, 97, 0, torch.float16),
    ("affine", 64, 1200, 200, 0, torch.bfloat16),
    ("i8_i8", 64, 9000, 8500, 0, torch.bfloat16),   # every row sees > 8192 keys: the plain P·V
    ("i8_i8", 1, 3000, 200, 0, torch.bfloat16),     # one query: the last 200 tokens
    ("u4_u4", 1, 5000, 4000, 5, torch.float16),
    ("affine", 1, 777, 33, 0, torch.bfloat16),
]


@pytest.mark.parametrize("case", WINDOW_CASES, ids=lambda c: "{}_L{}_T{}_W{}_sp{}_{}".format(*c[:5], str(c[5])[6:]))
def test_quantized_window_mask(gpu, case):
    """A sliding-window pattern over a quantized cache runs on the prefill
    kernel's own window masking, tiles dequantized on chip (one query too),
    and matches the oracle under the same boolean array."""
    fmt, L, T, W, splits, dtype = case
    cache = WINDOW_FORMATS[fmt]()
    k = synthetic.kv((1, 2, T, 128), 31 + W, kind="outliers", frac=0.02)
    v = synthetic.kv((1, 2, T, 128), 32 + W, kind="outliers", frac=0.02)
    kq, vq = cache.update_and_fetch(k, v)
    q = synthetic.query(1, 16, L, 33 + L, dtype=dtype)
    sinks = torch.randn(16, device="cuda")
    keep = keep_pattern(L, T, W)
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, torch.from_numpy(keep).cuda(), sinks, cache.group_size,
                                         cache.key_bits, cache.value_bits, out_dtype=torch.float32,
                                         splits=splits or None)
    torch.cuda.synchronize()
    kh, vh = prefill_side(oracle_xhat(kq), kq, dtype), prefill_side(oracle_xhat(vq), vq, dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks), keep)
    assert_close(f32(out), ref, f"{case}")


def test_attend_one_query_window(gpu):
    """attend() with one new token under a window pattern appends the token,
    then attends over the last W cached tokens (the unfused path)."""
    T, W = 1000, 150
    cache = QuantizedKVCache(32, 8, 8)
    k = synthetic.kv((1, 2, T + 1, 128), 51, kind="outliers", frac=0.02)
    v = synthetic.kv((1, 2, T + 1, 128), 52, kind="outliers", frac=0.02)
    cache.update_and_fetch(k[:, :, :T], v[:, :, :T])
    q = synthetic.query(1, 16, 1, 53, dtype=torch.bfloat16)
    keep = keep_pattern(1, T + 1, W)
    out = attend(q, k[:, :, T:], v[:, :, T:], cache, SCALE, torch.from_numpy(keep).cuda(), None,
                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert cache.offset == T + 1
    kq, vq = cache.keys_and_values()
    assert_cache_equal(kq, oracle_quantize(f32(k), 8))
    ref = O.attention(f32(q), oracle_xhat(kq), oracle_xhat(vq), SCALE, None, keep)
    assert_close(f32(out), ref, "attend window")


def test_attend_refuses_f32_matrix_core_queries_before_append(gpu):
    """A float32 chunk, or one float32 query under a window over a quantized
    cache, is refused before the new tokens touch the cache."""
    cache = QuantizedKVCache(32, 8, 8)
    k = synthetic.kv((1, 2, 103, 128), 61)
    v = synthetic.kv((1, 2, 103, 128), 62)
    cache.update_and_fetch(k[:, :, :100], v[:, :, :100])
    q3 = synthetic.query(1, 16, 3, 63, dtype=torch.float32)
    with pytest.raises(NotImplementedError):
        attend(q3, k[:, :, 100:], v[:, :, 100:], cache, SCALE, "causal")
    assert cache.offset == 100
    q1 = synthetic.query(1, 16, 1, 64, dtype=torch.float32)
    with pytest.raises(NotImplementedError):
        attend(q1, k[:, :, 100:101], v[:, :, 100:101], cache, SCALE, torch.from_numpy(keep_pattern(1, 101, 50)).cuda())
    assert cache.offset == 100
    out = attend(q1, k[:, :, 100:101], v[:, :, 100:101], cache, SCALE, "causal", out_dtype=torch.float32)
    assert cache.offset == 101 and torch.isfinite(out).all()


def test_bf16_decode_window_mask(gpu):
    """One query over a bf16 cache with a window pattern attends over the last W keys."""
    T, W = 1000, 129
    cache = FixedKVCache(KVStorage(1, T, 2), 0)
    k = synthetic.kv((1, 2, T, 128), 41, dtype=torch.bfloat16)
    v = synthetic.kv((1, 2, T, 128), 42, dtype=torch.bfloat16)
    kk, vv = cache.update_and_fetch(k, v)
    q = synthetic.query(1, 16, 1, 43, dtype=torch.bfloat16)
    keep = keep_pattern(1, T, W)
    out = scaled_dot_product_attention(q, kk, vv, SCALE, torch.from_numpy(keep).cuda(), None, out_dtype=torch.float32)
    ref = O.attention(f32(q), f32(k), f32(v), SCALE, None, keep)
    assert_close(f32(out), ref, "bf16 window decode")

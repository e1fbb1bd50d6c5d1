"""Mask arrays on the attention entry points (model.py:122-128).

Host arrays (NumPy, CPU tensors) holding every key, causal, or causal over
the last `window` keys take the kernels' own masking; every other array --
any array on the GPU, which is never inspected on the host -- is added to the
scores as a bias inside the kernels.  Each case matches the oracle under the
same array: random boolean masks, padding masks of a two-sequence batch with
unequal lengths, finite additive masks, per-group-member masks, in decode and
prefill, over the quantized and bf16 caches."""

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
    # the device array ran as a bias; the string and the host array run the causal kernel
    same = quantized_attention_with_sinks(q, kq, vq, SCALE, "causal", sinks, 32, 8, 8, out_dtype=torch.float32)
    host = quantized_attention_with_sinks(q, kq, vq, SCALE, mask.cpu(), sinks, 32, 8, 8, out_dtype=torch.float32)
    assert torch.equal(host, same)
    torch.testing.assert_close(out, same, rtol=1e-6, atol=1e-6)


def test_decode_all_keys_mask_arrays(gpu):
    T = 777
    kq, vq, kh, vh = quantized_cache((8, 4), T, 21)
    q = synthetic.query(1, 16, 1, 22)
    outs = [quantized_attention_with_sinks(q, kq, vq, SCALE, m, None, 32, 8, 4, out_dtype=torch.float32)
            for m in (None, torch.ones((1, T), dtype=torch.bool), torch.zeros((1, 1, 1, T)),
                      torch.ones((1, T), dtype=torch.bool, device="cuda"), torch.zeros((1, 1, 1, T), device="cuda"))]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])  # host arrays: the plain decode
    for o in outs[3:]:  # device arrays: a zero bias
        torch.testing.assert_close(o, outs[0], rtol=1e-6, atol=1e-6)
    assert_close(f32(outs[0]), O.attention(f32(q), kh, vh, SCALE), "decode")
    # one query under a window (host pattern or device array): the decode
    # kernel with the window as a bias, any query dtype
    keep = keep_pattern(1, T, 100)
    for m in (keep, torch.from_numpy(keep).cuda()):
        out = quantized_attention_with_sinks(q.float(), kq, vq, SCALE, m, None, 32, 8, 4, out_dtype=torch.float32)
        assert_close(f32(out), O.attention(f32(q), kh, vh, SCALE, None, keep), "f32 query, window as a bias")


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
    kh, vh = oracle_xhat(kq), oracle_xhat(vq)
    if L > 1:  # the prefill rounds 4-bit and affine values to the query dtype; one query decodes exactly
        kh, vh = prefill_side(kh, kq, dtype), prefill_side(vh, vq, dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks), keep)
    assert_close(f32(out), ref, f"{case}")
    # the same pattern from the host: the window kernel (chunks) or the decode with a window bias (one query)
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, keep, sinks, cache.group_size, cache.key_bits,
                                         cache.value_bits, out_dtype=torch.float32, splits=splits or None)
    assert_close(f32(out), ref, f"{case}, host mask")


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


def test_attend_f32_queries_under_masks(gpu):
    """A float32 chunk under a window pattern (a decode per query, the window
    its bias row), then one float32 query under a window (the window a bias)
    and a plain float32 decode step."""
    cache = QuantizedKVCache(32, 8, 8)
    k = synthetic.kv((1, 2, 105, 128), 61)
    v = synthetic.kv((1, 2, 105, 128), 62)
    cache.update_and_fetch(k[:, :, :100], v[:, :, :100])
    q3 = synthetic.query(1, 16, 3, 63, dtype=torch.float32)
    keep3 = keep_pattern(3, 103, 20)
    out = attend(q3, k[:, :, 100:103], v[:, :, 100:103], cache, SCALE, keep3)
    assert cache.offset == 103 and out.dtype == torch.float32
    kq, vq = cache.keys_and_values()
    assert_close(f32(out), O.attention(f32(q3), oracle_xhat(kq), oracle_xhat(vq), SCALE, None, keep3), "f32 chunk")
    q1 = synthetic.query(1, 16, 1, 64, dtype=torch.float32)
    keep = keep_pattern(1, 104, 50)
    out = attend(q1, k[:, :, 103:104], v[:, :, 103:104], cache, SCALE, keep, out_dtype=torch.float32)
    assert cache.offset == 104
    kq, vq = cache.keys_and_values()
    assert_close(f32(out), O.attention(f32(q1), oracle_xhat(kq), oracle_xhat(vq), SCALE, None, keep), "f32 window")
    out = attend(q1, k[:, :, 104:105], v[:, :, 104:105], cache, SCALE, "causal", out_dtype=torch.float32)
    assert cache.offset == 105 and torch.isfinite(out).all()


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


# ---------------------------------------------------------------------------
# general masks: a bias added to the scores inside the kernels

MASK_FORMATS = {
    "i8": lambda: QuantizedKVCache(32, 8, 8),
    "u4": lambda: QuantizedKVCache(32, 4, 4),
    "i8u4": lambda: QuantizedKVCache(32, 8, 4),
    "affine": lambda: MixedQuantizedKVCache(),
}


def general_masks(B, Hkv, G, L, T, seed):
    """name -> (mask array, the same array for the oracle)."""
    g = torch.Generator().manual_seed(seed)
    rnd = torch.rand(L, T, generator=g) > 0.35                        # random keep pattern (a row may lose every key)
    lengths = [T, T - 37]                                             # two sequences of unequal length, right padding
    pad = torch.zeros(B, 1, 1, T, dtype=torch.bool)
    for b in range(B):
        pad[b, ..., : lengths[b % 2]] = True
    left = torch.zeros(B, 1, L, T, dtype=torch.bool)                  # left padding plus causal
    q = torch.arange(T - L, T)[:, None]
    k = torch.arange(T)[None]
    for b in range(B):
        left[b, 0] = (q >= k) & (k >= 13 * b)
    add = torch.randn(L, T, generator=g) * 2.0                        # finite additive
    grp = torch.rand(G, L, T, generator=g) > 0.5                      # per group member (3-D, model.py broadcasting)
    per_kv = torch.randn(B, Hkv, L, T, generator=g).clamp(-3, 3)      # per sequence and KV head, additive
    return {"random": rnd, "padding": pad, "left_padding_causal": left, "additive": add, "group": grp,
            "per_kv_head": per_kv}


MASK_CASES = [
    # format, B, Hq, Hkv, L, T, q dtype
    ("i8", 2, 16, 2, 1, 300, torch.bfloat16),
    ("u4", 2, 8, 1, 1, 5000, torch.float16),
    ("affine", 2, 16, 2, 1, 777, torch.float32),
    ("i8u4", 2, 16, 2, 1, 64, torch.bfloat16),
    ("i8", 2, 16, 2, 24, 400, torch.bfloat16),
    ("u4", 2, 8, 1, 40, 1500, torch.float16),
    ("affine", 2, 16, 2, 33, 260, torch.bfloat16),
    ("i8u4", 2, 12, 4, 17, 2100, torch.bfloat16),
]


@pytest.mark.parametrize("case", MASK_CASES, ids=lambda c: "{}_B{}_Hq{}_Hkv{}_L{}_T{}_{}".format(*c[:6], str(c[6])[6:]))
@pytest.mark.parametrize("name", ["random", "padding", "left_padding_causal", "additive", "group", "per_kv_head"])
def test_general_masks_quantized(gpu, case, name):
    fmt, B, Hq, Hkv, L, T, qdt = case
    G = Hq // Hkv
    cache = MASK_FORMATS[fmt]()
    k = synthetic.kv((B, Hkv, T, 128), 700 + T, kind="outliers", frac=0.02)
    v = synthetic.kv((B, Hkv, T, 128), 701 + T, kind="outliers", frac=0.02)
    kq, vq = cache.update_and_fetch(k, v)
    q = synthetic.query(B, Hq, L, 702 + L, dtype=qdt)
    sinks = torch.randn(Hq, device="cuda")
    mask = general_masks(B, Hkv, G, L, T, 703)[name]
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, mask.cuda(), sinks, cache.group_size, cache.key_bits,
                                         cache.value_bits, out_dtype=torch.float32)
    torch.cuda.synchronize()
    kh, vh = oracle_xhat(kq), oracle_xhat(vq)
    if L > 1:
        kh, vh = prefill_side(kh, kq, qdt), prefill_side(vh, vq, qdt)
    ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks), mask.numpy())
    assert_close(f32(out), ref, f"{name} {case}")


BF16_MASK_CASES = [
    # B, Hq, Hkv, L, T, q dtype, splits
    (2, 16, 2, 1, 300, torch.bfloat16, None),
    (2, 8, 1, 1, 3000, torch.float32, 7),
    (2, 16, 2, 24, 400, torch.bfloat16, None),
    (2, 12, 4, 60, 1000, torch.float16, None),
]


@pytest.mark.parametrize("case", BF16_MASK_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_L{}_T{}_{}_sp{}".format(
    *c[:5], str(c[5])[6:], c[6]))
@pytest.mark.parametrize("name", ["random", "padding", "left_padding_causal", "additive", "group", "per_kv_head"])
def test_general_masks_bf16(gpu, case, name):
    B, Hq, Hkv, L, T, qdt, splits = case
    G = Hq // Hkv
    k = synthetic.kv((B, Hkv, T, 128), 710 + T, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 711 + T, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, L, 712 + L, dtype=qdt)
    sinks = torch.randn(Hq, device="cuda")
    mask = general_masks(B, Hkv, G, L, T, 713)[name]
    out = scaled_dot_product_attention(q, k, v, SCALE, mask.cuda(), sinks, out_dtype=torch.float32, splits=splits)
    torch.cuda.synchronize()
    ref = O.attention(f32(q), f32(k), f32(v), SCALE, f32(sinks), mask.numpy())
    assert_close(f32(out), ref, f"{name} {case}")


def test_attend_with_padding_mask_decode_and_chunk(gpu):
    """attend() with a device padding mask: a chunk, then decode steps, over a
    two-sequence int8 cache whose second sequence is 50 tokens shorter (its
    rows past its length masked out); the cache bytes are those of the plain
    append, and each output matches the oracle under the same mask."""
    B, Hq, Hkv, P, L = 2, 16, 2, 200, 30
    cache = QuantizedKVCache(32, 8, 8)
    n = P + L + 3
    k = synthetic.kv((B, Hkv, n, 128), 721, kind="outliers", frac=0.02)
    v = synthetic.kv((B, Hkv, n, 128), 722, kind="outliers", frac=0.02)
    sinks = torch.randn(Hq, device="cuda")
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    short = torch.ones(B, 1, 1, n, dtype=torch.bool)
    short[1, ..., P - 50 : P] = False  # sequence 1: 50 pad tokens at the end of its prefix
    kh = dequant(8, *oracle_quantize(f32(k), 8))
    vh = dequant(8, *oracle_quantize(f32(v), 8))
    pos = P
    for step_len in (L, 1, 1, 1):
        T = pos + step_len
        qi = torch.arange(T - step_len, T)[:, None]
        m = short[..., :T] & (qi >= torch.arange(T)[None])  # padding and causal, (B, 1, step_len, T)
        q = synthetic.query(B, Hq, step_len, 730 + pos, dtype=torch.bfloat16)
        out = attend(q, k[:, :, pos:T], v[:, :, pos:T], cache, SCALE, m.cuda(), sinks, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert cache.offset == T
        sk = f32(sinks) if step_len == 1 else O.sink_logits(f32(sinks), "bfloat16")
        ref = O.attention(f32(q), kh[:, :, :T], vh[:, :, :T], SCALE, sk, m.numpy())
        assert_close(f32(out), ref, f"step at {pos} of {step_len}")
        pos = T
    kq, vq = cache.keys_and_values()
    assert_cache_equal(kq, oracle_quantize(f32(k), 8))

"""Mask arrays on the attention entry points (model.py:122-128): boolean and
additive (0 / -inf) arrays whose pattern is every key, causal, or causal
over the last `window` keys run on the kernels' own masking and match the
oracle under the same array; the string form gives the same bytes."""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import (FixedKVCache, KVStorage, QuantizedKVCache, quantized_attention_with_sinks,
                     scaled_dot_product_attention, synthetic)
from tests.gpu_util import SCALE, assert_close, dequant, f32, oracle_quantize

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
    with pytest.raises(NotImplementedError):  # a window over a quantized cache at one query
        quantized_attention_with_sinks(q, kq, vq, SCALE, torch.from_numpy(keep_pattern(1, T, 100)).cuda(), None,
                                       32, 8, 4)


def test_uint4_prefill_window_mask(gpu):
    """A sliding-window pattern over a 4-bit cache runs on the bf16 prefill's
    window masking (the cache is dequantized to bf16 first)."""
    L, T, W = 33, 500, 64
    kq, vq, kh, vh = quantized_cache((4, 4), T, 31)
    q = synthetic.query(1, 16, L, 32, dtype=torch.float16)
    keep = keep_pattern(L, T, W)
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, torch.from_numpy(keep).cuda(), None, 32, 4, 4,
                                         out_dtype=torch.float32)
    ref = O.attention(f32(q), O.bf16_rn(kh), O.bf16_rn(vh), SCALE, None, keep)
    assert_close(f32(out), ref, "window")


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

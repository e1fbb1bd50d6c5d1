"""Outputs stored in the query dtype by the kernels themselves.

Every decode and prefill entry point takes an output dtype (fp32, bf16,
fp16); the kernel that finishes the attention (the split merge, or the
attention kernel of a one-split plan) rounds the fp32 result to nearest even.
The 16-bit outputs must equal the fp32 output of the same call rounded by
torch, bit for bit, on every path: quantized decode (split and one-split),
bf16-cache decode (split, one-workgroup, ring), prefill (tiled, split,
few-query) over the quantized and bf16 caches.
"""

import pytest
import torch

from rec_amd import (FixedKVCache, FixedSlidingKVCache, KVStorage, MixedQuantizedKVCache, QuantizedKVCache,
                     quantized_attention_with_sinks, scaled_dot_product_attention, synthetic)
from tests.gpu_util import SCALE

pytestmark = pytest.mark.gpu

ODT = [torch.bfloat16, torch.float16]


def same_rounding(o32, o16, what):
    ref = o32.to(o16.dtype)
    assert o16.dtype == ref.dtype and o16.shape == ref.shape
    assert torch.equal(o16.view(torch.int16), ref.view(torch.int16)), f"{what}: 16-bit output is not the fp32 one rounded"


@pytest.mark.parametrize("odt", ODT)
@pytest.mark.parametrize("fmt,T,L,splits", [
    ("i8", 3000, 1, None), ("i8", 100, 1, 1), ("u4", 700, 1, 5), ("affine", 2049, 1, None),
    ("i8", 3000, 20, None), ("i8", 300, 64, None), ("affine", 5000, 4, None), ("u4", 1000, 40, 3),
])
def test_quantized_paths_store_the_query_dtype(gpu, odt, fmt, T, L, splits):
    cache = {"i8": lambda: QuantizedKVCache(32, 8, 8), "u4": lambda: QuantizedKVCache(32, 4, 4),
             "affine": lambda: MixedQuantizedKVCache()}[fmt]()
    k = synthetic.kv((1, 4, T, 128), 601, kind="outliers", frac=0.02)
    v = synthetic.kv((1, 4, T, 128), 602, kind="outliers", frac=0.02)
    kq, vq = cache.update_and_fetch(k, v)
    q = synthetic.query(1, 32, L, 603, dtype=torch.bfloat16)
    sinks = torch.randn(32, device="cuda")
    mask = "causal" if L > 1 else None
    args = (q, kq, vq, SCALE, mask, sinks, cache.group_size, cache.key_bits, cache.value_bits)
    o32 = quantized_attention_with_sinks(*args, out_dtype=torch.float32, splits=splits)
    o16 = quantized_attention_with_sinks(*args, out_dtype=odt, splits=splits)
    same_rounding(o32, o16, f"{fmt} T={T} L={L}")
    assert quantized_attention_with_sinks(*args, splits=splits).dtype == q.dtype  # default: the query dtype


@pytest.mark.parametrize("odt", ODT)
@pytest.mark.parametrize("T,L,splits", [(513, 1, None), (1024, 1, None), (5000, 1, None), (700, 1, 4),
                                        (3000, 24, None), (600, 300, None)])
def test_bf16_paths_store_the_query_dtype(gpu, odt, T, L, splits):
    k = synthetic.kv((2, 2, T, 128), 611, dtype=torch.bfloat16)
    v = synthetic.kv((2, 2, T, 128), 612, dtype=torch.bfloat16)
    q = synthetic.query(2, 16, L, 613, dtype=torch.bfloat16)
    sinks = torch.randn(16, device="cuda")
    mask = "causal" if L > 1 else None
    o32 = scaled_dot_product_attention(q, k, v, SCALE, mask, sinks, out_dtype=torch.float32, splits=splits)
    o16 = scaled_dot_product_attention(q, k, v, SCALE, mask, sinks, out_dtype=odt, splits=splits)
    same_rounding(o32, o16, f"bf16 T={T} L={L}")


def test_attend_returns_the_query_dtype_without_a_cast(gpu):
    """attend() over each cache returns the query dtype, equal to its fp32
    output rounded (fused decode steps, ring steps, chunks)."""
    from rec_amd import attend

    B, Hq, Hkv = 1, 32, 4
    k = synthetic.kv((B, Hkv, 700, 128), 621, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, 700, 128), 622, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    makers = [lambda: QuantizedKVCache(32, 8, 8), lambda: MixedQuantizedKVCache(),
              lambda: FixedKVCache(KVStorage(1, 1024, Hkv), 0),
              lambda: FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=513)]
    for make in makers:
        a, b = make(), make()
        pos = 0
        for L in (600, 1, 1, 60, 1):
            q = synthetic.query(B, Hq, L, 630 + pos, dtype=torch.bfloat16)
            mask = "causal" if L > 1 else None
            o16 = attend(q, k[:, :, pos : pos + L], v[:, :, pos : pos + L], a, SCALE, mask, sinks)
            o32 = attend(q, k[:, :, pos : pos + L], v[:, :, pos : pos + L], b, SCALE, mask, sinks,
                         out_dtype=torch.float32)
            assert o16.dtype == torch.bfloat16
            same_rounding(o32, o16, f"{type(a).__name__} step at {pos} of {L}")
            pos += L

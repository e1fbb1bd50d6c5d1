"""Chunks of float32 queries (L > 1) on every cache.

The reference's prefill SDPA takes float32 queries and dequantizes the cache
to float32 for them (model.py:191-203, 211).  Here each query row runs as one
decode over the keys it sees (the decode kernels attend with float32 queries
over the exact dequantized values): causal limits, a sliding window and mask
arrays (as each query's bias row) must give the oracle's output over the
unrounded x̂, with float32 sinks, as they do for a chunk of bf16 queries.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import (FixedKVCache, FixedSlidingKVCache, KVStorage, MixedQuantizedKVCache, QuantizedKVCache, attend,
                     quantized_attention_with_sinks, scaled_dot_product_attention, synthetic)
from tests.gpu_util import SCALE, assert_close, f32, oracle_xhat

pytestmark = pytest.mark.gpu


def keep_pattern(L, T, window=0):
    q = np.arange(T - L, T)[:, None]
    k = np.arange(T)[None]
    m = q >= k
    return m & (q < k + window) if window else m


CACHES = {"int8": lambda: QuantizedKVCache(32, 8, 8), "uint4": lambda: QuantizedKVCache(32, 4, 4),
          "k8v4": lambda: QuantizedKVCache(32, 8, 4), "affine": lambda: MixedQuantizedKVCache()}


@pytest.mark.parametrize("fmt", list(CACHES))
@pytest.mark.parametrize("P,L,sinks", [(300, 5, True), (7, 9, False), (2000, 3, True)])
def test_f32_chunk_through_attend(gpu, fmt, P, L, sinks):
    """attend() appends the chunk, then each float32 query attends causally
    over the cache (the first P + i + 1 tokens for query i)."""
    B, Hq, Hkv = 1, 16, 2
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 31 + P, kind="outliers", frac=0.02)
    v = synthetic.kv((B, Hkv, T, 128), 32 + P, kind="outliers", frac=0.02)
    q = synthetic.query(B, Hq, L, 33 + L, dtype=torch.float32)
    s = torch.randn(Hq, device="cuda") * 2 if sinks else None
    cache = CACHES[fmt]()
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", s)
    assert out.dtype == torch.float32 and out.shape == (B, Hq, L, 128)
    torch.cuda.synchronize()
    kq, vq = cache.keys_and_values()
    ref = O.attention(f32(q), oracle_xhat(kq), oracle_xhat(vq), SCALE, None if s is None else f32(s), "causal")
    assert_close(f32(out), ref, f"{fmt} P={P} L={L}")


@pytest.mark.parametrize("fmt", ["int8", "uint4", "affine"])
def test_f32_chunk_mask_arrays(gpu, fmt):
    """A random boolean mask on the GPU (each query's bias row), a per-sequence
    padding mask of a two-sequence batch, and a host window pattern."""
    B, Hq, Hkv, T, L = 2, 8, 2, 260, 6
    k = synthetic.kv((B, Hkv, T, 128), 41, kind="outliers", frac=0.02)
    v = synthetic.kv((B, Hkv, T, 128), 42, kind="outliers", frac=0.02)
    q = synthetic.query(B, Hq, L, 43, dtype=torch.float32)
    sinks = torch.randn(Hq, device="cuda")
    cache = CACHES[fmt]()
    kq, vq = cache.update_and_fetch(k, v)
    bits, group = (kq.bits, vq.bits), 64 if kq.affine else 32
    kh, vh = oracle_xhat(kq), oracle_xhat(vq)
    rng = np.random.default_rng(44)
    keep = rng.random((L, T)) < 0.6
    keep[:, 0] = True
    pad = np.ones((B, 1, L, T), dtype=bool)
    pad[1, :, :, 200:] = False  # the second sequence holds 200 tokens
    for what, host in (("random", keep), ("padding", pad), ("window", keep_pattern(L, T, 50))):
        m = torch.from_numpy(host)
        mask = m if what == "window" else m.cuda()
        out = quantized_attention_with_sinks(q, kq, vq, SCALE, mask, sinks, group, *bits)
        ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks), host)
        assert_close(f32(out), ref, f"{fmt} {what}")


def test_f32_chunk_bf16_caches(gpu):
    """FixedKVCache (causal, an additive mask) and the sliding ring (its
    window) under float32 queries."""
    B, Hq, Hkv, P, L = 1, 32, 4, 700, 6
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 51, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 52, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, L, 53, dtype=torch.float32)
    sinks = torch.randn(Hq, device="cuda")
    cache = FixedKVCache(KVStorage(1, 4096, Hkv, batch=B), 0)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", sinks)
    torch.cuda.synchronize()
    assert_close(f32(out), O.attention(f32(q), f32(k), f32(v), SCALE, f32(sinks), "causal"), "FixedKVCache")
    kk, vv = cache.storage.layer(0, T)[:, 0], cache.storage.layer(0, T)[:, 1]
    add = torch.randn((L, T), device="cuda").clamp(min=-3.0)
    out = scaled_dot_product_attention(q, kk, vv, SCALE, add, sinks)
    ref = O.attention(f32(q), f32(k), f32(v), SCALE, f32(sinks), f32(add))
    assert_close(f32(out), ref, "additive mask")

    W = 40
    ring = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W)
    ring.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], ring, SCALE, None, sinks)
    torch.cuda.synchronize()
    lo = P - W
    ref = O.attention(f32(q), f32(k[:, :, lo:]), f32(v[:, :, lo:]), SCALE, f32(sinks),
                      keep_pattern(L, T - lo, W))
    assert_close(f32(out), ref, "sliding ring chunk")

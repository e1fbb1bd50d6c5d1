"""GQA ratios above 8 query heads per KV head.

One launch holds at most 8 query heads of a KV head (its matrix-core
columns); larger ratios run the heads of each KV head in groups of 8 and put
the outputs back in head order.  Each case must match the oracle, which has
no such limit (model.py:111-116 repeats the KV heads for any ratio): decode
and chunks over the quantized caches, sinks, a per-head mask array, the bf16
caches and the sliding ring.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import (FixedKVCache, FixedSlidingKVCache, KVStorage, QuantizedKVCache, attend,
                     quantized_attention_with_sinks, synthetic)
from tests.gpu_util import SCALE, assert_close, f32, oracle_xhat, prefill_side, q_sinks

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,Hq,Hkv", [((8, 8), 64, 4), ((4, 4), 24, 2), ((8, 4), 40, 2)],
                         ids=["int8_G16", "uint4_G12", "k8v4_G20"])
def test_large_gqa_quantized(gpu, bits, Hq, Hkv):
    """Decode steps through attend() (the fused step gives way to the append
    and one decode per head group) and a causal chunk, with sinks."""
    B, P, L = 1, 900, 6
    T = P + L + 2
    k = synthetic.kv((B, Hkv, T, 128), 11 + Hq, kind="outliers", frac=0.02)
    v = synthetic.kv((B, Hkv, T, 128), 12 + Hq, kind="outliers", frac=0.02)
    sinks = torch.randn(Hq, device="cuda")
    cache = QuantizedKVCache(32, *bits)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    q = synthetic.query(B, Hq, L, 13, dtype=torch.bfloat16)
    out = attend(q, k[:, :, P:P + L], v[:, :, P:P + L], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    kq, vq = cache.keys_and_values()
    kh, vh = prefill_side(oracle_xhat(kq), kq, q.dtype), prefill_side(oracle_xhat(vq), vq, q.dtype)
    assert_close(f32(out), O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, q.dtype), "causal"), "chunk")
    for step in range(2):
        pos = P + L + step
        q1 = synthetic.query(B, Hq, 1, 20 + step, dtype=torch.bfloat16)
        out = attend(q1, k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], cache, SCALE, None, sinks,
                     out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert cache.offset == pos + 1
        kq, vq = cache.keys_and_values()
        assert_close(f32(out), O.attention(f32(q1), oracle_xhat(kq), oracle_xhat(vq), SCALE, f32(sinks)),
                     f"decode step {step}")


def test_large_gqa_per_head_mask(gpu):
    """A three-dimensional mask (G, L, T) is per query head of the group: each
    group of 8 heads takes its slice."""
    B, Hq, Hkv, T, L = 2, 24, 2, 300, 5
    G = Hq // Hkv
    k = synthetic.kv((B, Hkv, T, 128), 31, kind="outliers", frac=0.02)
    v = synthetic.kv((B, Hkv, T, 128), 32, kind="outliers", frac=0.02)
    cache = QuantizedKVCache(32, 8, 8)
    kq, vq = cache.update_and_fetch(k, v)
    q = synthetic.query(B, Hq, L, 33, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    keep = np.random.default_rng(34).random((G, L, T)) < 0.5
    keep[..., 0] = True
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, torch.from_numpy(keep).cuda(), sinks, 32, 8, 8,
                                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.attention(f32(q), oracle_xhat(kq), oracle_xhat(vq), SCALE, q_sinks(sinks, q.dtype), keep)
    assert_close(f32(out), ref, "per-head mask")


def test_large_gqa_bf16_caches(gpu):
    """FixedKVCache decode and chunk, and a sliding-ring chunk, at 16 query
    heads per KV head."""
    B, Hq, Hkv, P, L = 1, 64, 4, 600, 4
    T = P + L + 1
    k = synthetic.kv((B, Hkv, T, 128), 41, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 42, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    cache = FixedKVCache(KVStorage(1, 2048, Hkv, batch=B), 0)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    q = synthetic.query(B, Hq, L, 43, dtype=torch.bfloat16)
    out = attend(q, k[:, :, P:P + L], v[:, :, P:P + L], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(f32(out), O.attention(f32(q), f32(k[:, :, :P + L]), f32(v[:, :, :P + L]), SCALE,
                                       q_sinks(sinks, q.dtype), "causal"), "FixedKVCache chunk")
    q1 = synthetic.query(B, Hq, 1, 44, dtype=torch.bfloat16)
    out = attend(q1, k[:, :, P + L:], v[:, :, P + L:], cache, SCALE, None, sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(f32(out), O.attention(f32(q1), f32(k), f32(v), SCALE, q_sinks(sinks, q1.dtype)), "FixedKVCache step")

    W = 50
    ring = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W)
    ring.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:P + L], v[:, :, P:P + L], ring, SCALE, None, sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    lo = P - W
    qp = np.arange(P + L - lo - L, P + L - lo)[:, None]
    kp = np.arange(P + L - lo)[None]
    ref = O.attention(f32(q), f32(k[:, :, lo:P + L]), f32(v[:, :, lo:P + L]), SCALE, q_sinks(sinks, q.dtype),
                      (qp >= kp) & (qp < kp + W))
    assert_close(f32(out), ref, "ring chunk")

"""Sink logits in the dtype each reference branch hands them over in.

The quantized decode casts the per-head offsets to float32
(engine/src/rec_mlx/model.py:129); the prefill branch over the quantized
cache and the SDPA call over the bf16 caches pass them in the query dtype
(model.py:202, :211).  On rows that see few keys the sink carries a large share
of the weight, so the rounding moves outputs past the tolerance: every case
below first checks, on the CPU, that the float32-sink oracle would fail it.

Also here: the sliding ring's fused decode at 1, 8 and 513 held tokens with
batch 2, 32 / 4 heads and explicit split counts (the written slot in the
first, a middle and the last split), its ring contents against the unfused
ring after every step, and a windowed single query on a FixedKVCache taking
the same path fused or not.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import FixedKVCache, FixedSlidingKVCache, KVStorage, QuantizedKVCache, attend, synthetic
from tests.gpu_util import ATOL, RTOL, SCALE, assert_close, dequant, f32, oracle_quantize, q_sinks

pytestmark = pytest.mark.gpu


def bf16_np(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).float().cpu().numpy()


def odd_sinks(n, seed):
    """Sink logits near 3 (about the weight of 16-24 keys) that bf16 cannot
    hold: a bf16 value plus 0.3-0.45 of its last place."""
    g = torch.Generator().manual_seed(seed)
    base = (2.5 + torch.rand(n, generator=g)).to(torch.bfloat16).float()
    frac = 0.3 + 0.15 * torch.rand(n, generator=g)
    return (base + frac * 2.0**-6).cuda()


def fails_tolerance(got, ref):
    return bool(np.any(np.abs(np.asarray(got, np.float64) - ref) > ATOL + RTOL * np.abs(ref)))


def test_prefill_over_short_prefix_rounds_sinks(gpu):
    """A chunk of 8 bf16 queries over a 16-token int8 prefix: attend() (the
    prefill branch) uses bf16 sinks; quantized_attention_with_sinks keeps the
    function's float32 cast."""
    from rec_amd import quantized_attention_with_sinks

    B, Hq, Hkv, P, L = 1, 32, 4, 16, 8
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 501, kind="outliers", frac=0.05)
    v = synthetic.kv((B, Hkv, T, 128), 502, kind="outliers", frac=0.05)
    q = synthetic.query(B, Hq, L, 503, dtype=torch.bfloat16)
    sinks = odd_sinks(Hq, 504)
    cache = QuantizedKVCache(32, 8, 8)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
    kh, vh = dequant(8, *oracle_quantize(f32(k), 8)), dequant(8, *oracle_quantize(f32(v), 8))
    ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks), "causal", sink_dtype="bfloat16")
    ref32 = O.attention(f32(q), kh, vh, SCALE, f32(sinks), "causal")
    assert fails_tolerance(ref32, ref), "the case must tell the two sink dtypes apart"
    assert_close(f32(out), ref, "attend chunk, bf16 sinks")
    kq, vq = cache.keys_and_values()
    out32 = quantized_attention_with_sinks(q, kq, vq, SCALE, "causal", sinks, 32, 8, 8, out_dtype=torch.float32)
    assert_close(f32(out32), ref32, "quantized_attention_with_sinks, float32 sinks")


def test_quantized_decode_keeps_float32_sinks(gpu):
    """One decode token over a short quantized cache: float32 sinks
    (model.py:129), not the query dtype."""
    B, Hq, Hkv, T = 1, 32, 4, 12
    k = synthetic.kv((B, Hkv, T, 128), 511, kind="outliers", frac=0.05)
    v = synthetic.kv((B, Hkv, T, 128), 512, kind="outliers", frac=0.05)
    q = synthetic.query(B, Hq, 1, 513, dtype=torch.bfloat16)
    sinks = odd_sinks(Hq, 514)
    cache = QuantizedKVCache(32, 8, 8)
    cache.update_and_fetch(k[:, :, : T - 1], v[:, :, : T - 1])
    out = attend(q, k[:, :, T - 1 :], v[:, :, T - 1 :], cache, SCALE, None, sinks, out_dtype=torch.float32)
    kh, vh = dequant(8, *oracle_quantize(f32(k), 8)), dequant(8, *oracle_quantize(f32(v), 8))
    ref = O.attention(f32(q), kh, vh, SCALE, f32(sinks))
    assert fails_tolerance(O.attention(f32(q), kh, vh, SCALE, f32(sinks), sink_dtype="bfloat16"), ref)
    assert_close(f32(out), ref, "quantized decode, float32 sinks")


@pytest.mark.parametrize("qdt", [torch.bfloat16, torch.float16])
def test_fixed_kv_cache_decode_rounds_sinks(gpu, qdt):
    """FixedKVCache decode steps from an empty cache (1..6 tokens): sinks in the
    query dtype (model.py:211), fused and unfused alike."""
    B, Hq, Hkv, n = 1, 32, 4, 6
    k = synthetic.kv((B, Hkv, n, 128), 521, kind="outliers", frac=0.05, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, n, 128), 522, kind="outliers", frac=0.05, dtype=torch.bfloat16)
    sinks = odd_sinks(Hq, 523)
    caches = [FixedKVCache(KVStorage(1, 64, Hkv), 0) for _ in range(2)]
    told = False
    for t in range(n):
        q = synthetic.query(B, Hq, 1, 530 + t, dtype=qdt)
        ref = O.attention(f32(q), bf16_np(k[:, :, : t + 1]), bf16_np(v[:, :, : t + 1]), SCALE, q_sinks(sinks, qdt))
        told |= fails_tolerance(O.attention(f32(q), bf16_np(k[:, :, : t + 1]), bf16_np(v[:, :, : t + 1]), SCALE,
                                            f32(sinks)), ref)
        for fused, cache in zip((True, False), caches):
            out = attend(q, k[:, :, t : t + 1], v[:, :, t : t + 1], cache, SCALE, None, sinks,
                         out_dtype=torch.float32, fused=fused)
            assert_close(f32(out), ref, f"step {t} fused={fused}")
    if qdt == torch.bfloat16:
        assert told, "the case must tell the two sink dtypes apart"


@pytest.mark.parametrize("splits", [None, 1, 8])
def test_ring_decode_513(gpu, splits):
    """FixedSlidingKVCache(window 513), batch 2, 32 / 4 heads: decode steps at
    1-8 held tokens, then a 760-token chunk (the ring keeps the last 513 and
    the next slots sit mid-ring), then decode steps whose written slot falls
    in a middle split; each output against the oracle (bf16 sinks), the ring's
    window against an unfused ring after every step."""
    B, Hq, Hkv, W = 2, 32, 4, 513
    n = 8 + 760 + 6
    k = synthetic.kv((B, Hkv, n, 128), 541, kind="outliers", frac=0.02, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, n, 128), 542, kind="outliers", frac=0.02, dtype=torch.bfloat16)
    sinks = odd_sinks(Hq, 543)
    fused = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W, batch=B)
    plain = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W, batch=B)
    pos, told = 0, False
    for L in [1] * 8 + [760] + [1] * 6:
        q = synthetic.query(B, Hq, L, 550 + pos, dtype=torch.bfloat16)
        outs = [attend(q, k[:, :, pos : pos + L], v[:, :, pos : pos + L], c, SCALE, None if L == 1 else "causal",
                       sinks, out_dtype=torch.float32, splits=splits, fused=f)
                for c, f in ((fused, True), (plain, False))]
        end = pos + L
        torch.cuda.synchronize()
        if L == 1:
            lo = max(0, end - W)
            kk, vv = bf16_np(k[:, :, lo:end]), bf16_np(v[:, :, lo:end])
            ref = O.attention(f32(q), kk, vv, SCALE, q_sinks(sinks, q.dtype))
            told |= fails_tolerance(O.attention(f32(q), kk, vv, SCALE, f32(sinks)), ref)
            slot = pos % W
            for out, what in zip(outs, ("fused", "unfused")):
                assert_close(f32(out), ref, f"{what} step at {pos} (slot {slot}, {end - lo} held)")
        for a, b in zip(fused.window(), plain.window()):
            assert torch.equal(a, b), f"ring contents differ after the step at {pos}"
        np.testing.assert_array_equal(fused.window()[0].float().cpu().numpy(), bf16_np(k[:, :, max(0, end - W) : end]))
        pos = end
    assert told, "the small-window steps must tell the two sink dtypes apart"


def test_fixed_kv_cache_window_mask_fused_equals_unfused(gpu):
    """A windowed single query on a FixedKVCache: the fused branch takes the
    masked path too, so fused=True and fused=False agree and match the oracle
    over the last W keys."""
    B, Hq, Hkv, T, W = 1, 16, 2, 300, 100
    k = synthetic.kv((B, Hkv, T + 1, 128), 561, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T + 1, 128), 562, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, 1, 563, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    keep = np.zeros((1, T + 1), bool)
    keep[0, T + 1 - W :] = True
    outs = []
    for fused in (True, False):
        cache = FixedKVCache(KVStorage(1, 1024, Hkv), 0)
        cache.update_and_fetch(k[:, :, :T], v[:, :, :T])
        outs.append(attend(q, k[:, :, T:], v[:, :, T:], cache, SCALE, torch.from_numpy(keep).cuda(), sinks,
                           out_dtype=torch.float32, fused=fused))
        assert cache.offset == T + 1
    assert torch.equal(outs[0], outs[1])
    ref = O.attention(f32(q), bf16_np(k), bf16_np(v), SCALE, q_sinks(sinks, q.dtype), keep)
    assert_close(f32(outs[0]), ref, "windowed query over FixedKVCache")


def test_ring_decode_refuses_a_window_mask(gpu):
    """The ring applies its own window: a single decode token under a mask that
    drops held tokens is refused before anything is written."""
    cache = FixedSlidingKVCache(max_sequence_tokens=64, num_kv_heads=2, head_dim=128, window_size=32)
    k = synthetic.kv((1, 2, 20, 128), 571, dtype=torch.bfloat16)
    cache.update_and_fetch(k[:, :, :19], k[:, :, :19])
    q = synthetic.query(1, 8, 1, 572, dtype=torch.bfloat16)
    keep = np.zeros((1, 20), bool)
    keep[0, 10:] = True
    with pytest.raises(NotImplementedError):
        attend(q, k[:, :, 19:], k[:, :, 19:], cache, SCALE, torch.from_numpy(keep).cuda())
    assert cache.offset == 19
    out = attend(q, k[:, :, 19:], k[:, :, 19:], cache, SCALE, "causal", out_dtype=torch.float32)
    assert cache.offset == 20 and torch.isfinite(out).all()


def test_make_cache_mixed_layers(gpu):
    """make_cache over a mixed layer list (model.py:347-360): a 513-token bf16
    ring per sliding layer and the affine quantized cache per full-attention
    layer; a 600-token chunk and a decode step through attend() on each, the
    sliding layer's step equal to the oracle over the last 513 tokens and the
    full layer's to a cache built by hand."""
    from rec_amd import MixedQuantizedKVCache, make_cache

    kinds = ["sliding_attention", "full_attention", "sliding_attention"]
    caches = make_cache(kinds, max_tokens=2048)
    assert [type(c) for c in caches] == [FixedSlidingKVCache, MixedQuantizedKVCache, FixedSlidingKVCache]
    assert caches[0].window_size == 513 and caches[0].capacity == 513 and caches[0] is not caches[2]
    B, Hq, Hkv, P = 1, 32, 4, 600
    k = synthetic.kv((B, Hkv, P + 1, 128), 581, kind="outliers", frac=0.02, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, P + 1, 128), 582, kind="outliers", frac=0.02, dtype=torch.bfloat16)
    qc = synthetic.query(B, Hq, P, 583, dtype=torch.bfloat16)
    qd = synthetic.query(B, Hq, 1, 584, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    by_hand = MixedQuantizedKVCache(max_tokens=2048)
    outs = []
    for c in caches + [by_hand]:
        attend(qc, k[:, :, :P], v[:, :, :P], c, SCALE, "causal", sinks)
        outs.append(attend(qd, k[:, :, P:], v[:, :, P:], c, SCALE, None, sinks, out_dtype=torch.float32))
        assert c.offset == P + 1
    torch.cuda.synchronize()
    lo = P + 1 - 513
    ref = O.attention(f32(qd), bf16_np(k[:, :, lo:]), bf16_np(v[:, :, lo:]), SCALE, q_sinks(sinks, qd.dtype))
    assert_close(f32(outs[0]), ref, "sliding layer")
    assert torch.equal(outs[0], outs[2])
    assert torch.equal(outs[1], outs[3])

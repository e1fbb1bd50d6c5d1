"""Parity of the MLX-style affine group-64 cache (8-bit keys, 4-bit values;
the reference's MixedQuantizedKVCache format) with the CPU oracle.

Codes, scales and biases written by the append kernel must equal the oracle's
restatement of the affine quantizer bit for bit; attention outputs lie within
2e-3 absolute + 1e-3 relative of the float64 oracle over the dequantized cache
(x̂ = s·q + b with the stored scale and bias).  Scales and biases are
stored in the keys' dtype as the reference allocates them (model.py:57-58):
bf16, or fp16 for fp16 keys.  Byte parity with MLX itself is not pinned (MLX
cannot run here).
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import MixedQuantizedKVCache, attend, quantized_attention_with_sinks, synthetic, to_logical
from tests.gpu_util import SCALE, assert_close, f32, oracle_xhat, prefill_side, q_sinks

pytestmark = pytest.mark.gpu


def value_bits(a):
    """float32 bit patterns of stored 16-bit values (a tensor) or of oracle
    values held in float32 (an array): equal patterns, equal values and signs."""
    if isinstance(a, torch.Tensor):
        a = f32(a)
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def fill(cache, B, H, T, seed, dtype=torch.bfloat16, chunks=None, kind="outliers", frac=0.01):
    k = synthetic.kv((B, H, T, 128), seed, kind=kind, frac=frac, dtype=dtype)
    v = synthetic.kv((B, H, T, 128), seed + 1, kind=kind, frac=frac, dtype=dtype)
    pos = 0
    for L in chunks or [T]:
        cache.update_and_fetch(k[:, :, pos : pos + L], v[:, :, pos : pos + L])
        pos += L
    return f32(k), f32(v)


def check_cache(cache, k, v):
    kv_k, kv_v = cache.keys_and_values()
    for kv, x, bits in ((kv_k, k, 8), (kv_v, v, 4)):
        codes, sc, bi = to_logical(kv)
        meta = {torch.float16: "float16", torch.bfloat16: "bfloat16"}[sc.dtype]
        q, s, b = O.quantize_affine(x, bits, meta=meta)
        if bits == 4:
            q = q[..., 0::2] | (q[..., 1::2] << 4)
        np.testing.assert_array_equal(codes.cpu().numpy(), q, err_msg=f"{bits}-bit codes differ")
        np.testing.assert_array_equal(value_bits(sc), value_bits(s), err_msg=f"{bits}-bit scales differ")
        np.testing.assert_array_equal(value_bits(bi), value_bits(b), err_msg=f"{bits}-bit biases differ")


def dequantized(cache):
    kv_k, kv_v = cache.keys_and_values()
    kc, ks, kb = to_logical(kv_k)
    vc, vs, vb = to_logical(kv_v)
    vq = O.unpack_int4(vc.cpu().numpy())
    return (O.dequantize_affine(kc.cpu().numpy(), f32(ks), f32(kb)),
            O.dequantize_affine(vq, f32(vs), f32(vb)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_affine_append_bit_exact(gpu, dtype):
    cache = MixedQuantizedKVCache()
    assert cache.affine and cache.group_size == 64
    chunks = [5, 64, 1, 1, 70, 3, 200]
    k, v = fill(cache, 2, 3, sum(chunks), 41, dtype=dtype, chunks=chunks, kind="heavy", frac=0.05)
    # the keys' dtype (model.py:57-58); fp32 keys keep bf16 (16-bit scales only)
    want = torch.float16 if dtype == torch.float16 else torch.bfloat16
    assert cache.state[0][1].dtype == want and cache.state[1][1].dtype == want
    check_cache(cache, k, v)


def test_affine_append_special_rows(gpu):
    x = torch.randn(1, 2, 9, 128, device="cuda", dtype=torch.bfloat16)
    x[:, :, 0] = 0           # all-zero rows
    x[:, :, 1] = 1.5         # constant rows
    x[:, :, 2, 7] = 300.0    # one large element
    x[:, :, 3, :64] = -2.0   # a constant negative group
    x[:, :, 4] = x[:, :, 4].abs()  # all positive: the minimum is not 0
    cache = MixedQuantizedKVCache()
    cache.update_and_fetch(x, -x)
    check_cache(cache, f32(x), f32(-x))


CASES = [
    # B, Hq, Hkv, T, sinks, splits
    (1, 8, 1, 1024, False, None),
    (1, 32, 4, 4096, True, None),
    (1, 32, 4, 1000, False, 3),
    (2, 16, 2, 777, True, 256),
    (1, 4, 1, 1, True, None),
    (3, 24, 4, 65, True, 1),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_T{}_s{}_sp{}".format(*c))
def test_affine_decode_matches_oracle(gpu, case):
    B, Hq, Hkv, T, use_sinks, splits = case
    cache = MixedQuantizedKVCache()
    fill(cache, B, Hkv, T, 51 + T)
    q = synthetic.query(B, Hq, 1, 53, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda") if use_sinks else None
    kv_k, kv_v = cache.keys_and_values()
    out = quantized_attention_with_sinks(q, kv_k, kv_v, SCALE, None, sinks, 64, 8, 4,
                                         out_dtype=torch.float32, splits=splits)
    torch.cuda.synchronize()
    kh, vh = dequantized(cache)
    ref = O.attention(f32(q), kh, vh, SCALE, sinks=None if sinks is None else f32(sinks))
    assert_close(f32(out), ref, f"case {case}")


def test_affine_fused_decode_steps(gpu):
    """attend(): each step quantizes the new token inside the attention launch
    (odd and even positions, so both nibbles of a shared byte) and matches the
    oracle; the stored bytes stay bit-exact."""
    B, Hq, Hkv, P = 1, 32, 4, 301
    cache = MixedQuantizedKVCache()
    k = synthetic.kv((B, Hkv, P + 5, 128), 61, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, P + 5, 128), 62, dtype=torch.bfloat16)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    sinks = torch.randn(Hq, device="cuda")
    for step in range(5):
        T = P + step + 1
        q = synthetic.query(B, Hq, 1, 70 + step, dtype=torch.bfloat16)
        out = attend(q, k[:, :, T - 1 : T], v[:, :, T - 1 : T], cache, SCALE, None, sinks, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert cache.offset == T
        kh, vh = dequantized(cache)
        ref = O.attention(f32(q), kh, vh, SCALE, sinks=f32(sinks))
        assert_close(f32(out), ref, f"step {step}")
    check_cache(cache, f32(k), f32(v))


def test_affine_long_context(gpu):
    B, Hq, Hkv, T = 1, 32, 4, 32768
    cache = MixedQuantizedKVCache(max_tokens=T)
    fill(cache, B, Hkv, T, 81)
    q = synthetic.query(B, Hq, 1, 83, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    kv_k, kv_v = cache.keys_and_values()
    out = quantized_attention_with_sinks(q, kv_k, kv_v, SCALE, None, sinks, 64, 8, 4, out_dtype=torch.float32)
    torch.cuda.synchronize()
    kh, vh = dequantized(cache)
    ref = O.attention(f32(q), kh, vh, SCALE, sinks=f32(sinks))
    assert_close(f32(out), ref, "32K affine")


def test_affine_rejections(gpu):
    cache = MixedQuantizedKVCache()
    fill(cache, 1, 4, 64, 91)
    kv_k, kv_v = cache.keys_and_values()
    q = synthetic.query(1, 32, 1, 92, dtype=torch.bfloat16)
    with pytest.raises(ValueError):  # group size of the call disagrees with the cache
        quantized_attention_with_sinks(q, kv_k, kv_v, SCALE, None, None, 32, 8, 4)


F16_CASES = [
    # B, Hq, Hkv, P (cached first), L (queries, appended with them), splits
    (1, 32, 4, 3000, 1, None),
    (2, 16, 2, 777, 1, 3),
    (1, 32, 4, 2000, 4, None),   # a few queries: the streaming few-query kernel
    (1, 32, 4, 17000, 8, None),  # 64 rows per KV head over a long cache: the streaming kernel, four column tiles
    (1, 16, 2, 900, 3, 4),       # streaming, split
    (1, 8, 1, 500, 64, None),
    (2, 12, 4, 300, 100, 2),
]


@pytest.mark.parametrize("case", F16_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_sp{}".format(*c))
def test_affine_f16_scales_decode_and_prefill(gpu, case):
    """An fp16 model: fp16 keys, queries and scales.  The append writes fp16
    scale and bias bits equal to the oracle's; decode and prefill read them as
    fp16 and match the oracle (the prefill side rounded to the query dtype, its
    sinks in that dtype, model.py:194-202)."""
    B, Hq, Hkv, P, L, splits = case
    cache = MixedQuantizedKVCache()
    k = synthetic.kv((B, Hkv, P + L, 128), 900 + L, kind="heavy", frac=0.05, dtype=torch.float16)
    v = synthetic.kv((B, Hkv, P + L, 128), 901 + L, kind="heavy", frac=0.05, dtype=torch.float16)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    q = synthetic.query(B, Hq, L, 902 + L, dtype=torch.float16)
    sinks = torch.randn(Hq, device="cuda")
    mask = "causal" if L > 1 else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32, splits=splits)
    torch.cuda.synchronize()
    assert cache.keys[1].dtype == torch.float16 and cache.offset == P + L
    check_cache(cache, f32(k), f32(v))
    kq, vq = cache.keys_and_values()
    kh, vh = oracle_xhat(kq), oracle_xhat(vq)
    if L > 1:
        kh, vh = prefill_side(kh, kq, q.dtype), prefill_side(vh, vq, q.dtype)
    sk = q_sinks(sinks, q.dtype) if L > 1 else f32(sinks)
    ref = O.attention(f32(q), kh, vh, SCALE, sk, mask)
    assert_close(f32(out), ref, f"case {case}")


def test_affine_f16_scales_masked_and_fused_steps(gpu):
    """fp16 scales through the masked decode (a bool mask array) and through
    fused decode steps (the new token quantized inside the attention launch,
    both nibbles of a shared byte)."""
    B, Hq, Hkv, P = 1, 16, 2, 401
    cache = MixedQuantizedKVCache()
    k = synthetic.kv((B, Hkv, P + 4, 128), 911, dtype=torch.float16)
    v = synthetic.kv((B, Hkv, P + 4, 128), 912, dtype=torch.float16)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    sinks = torch.randn(Hq, device="cuda")
    for step in range(4):
        T = P + step + 1
        q = synthetic.query(B, Hq, 1, 913 + step, dtype=torch.float16)
        out = attend(q, k[:, :, T - 1 : T], v[:, :, T - 1 : T], cache, SCALE, None, sinks, out_dtype=torch.float32)
        torch.cuda.synchronize()
        kq, vq = cache.keys_and_values()
        ref = O.attention(f32(q), oracle_xhat(kq), oracle_xhat(vq), SCALE, f32(sinks))
        assert_close(f32(out), ref, f"fused step {step}")
    check_cache(cache, f32(k), f32(v))
    kq, vq = cache.keys_and_values()
    T = P + 4
    keep = np.random.default_rng(914).random((1, T)) < 0.3
    q = synthetic.query(B, Hq, 1, 915, dtype=torch.float16)
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, torch.from_numpy(keep).cuda(), sinks, 64, 8, 4,
                                         out_dtype=torch.float32)
    ref = O.attention(f32(q), oracle_xhat(kq), oracle_xhat(vq), SCALE, f32(sinks), keep)
    assert_close(f32(out), ref, "masked decode")

"""Prefill over the 4-bit, mixed and affine cache formats.

The reference's prefill branch dequantizes the cache to the query dtype
before its attention (engine/src/rec_mlx/model.py:191-203); ``rec_prefill_attn``
dequantizes each K/V tile into on-chip memory instead, 4-bit and affine values
rounded to the query dtype, int8 codes exactly.

* ``dequantize_kv`` (bf16 copies, ``rec_kv_dequant_bf16``, kept for callers)
  is bit-exact: bf16 round-to-nearest-even of the
  oracle's float32 x̂ (int8 q·s, uint4 (q - z)·s, affine q·s + b; every product
  is exact in float32, so one rounding in both);
* the attention output lies within 2e-3 absolute + 1e-3 relative of the
  float64 oracle over the values the kernel attends over.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import MixedQuantizedKVCache, QuantizedKVCache, attend, dequantize_kv, synthetic
from tests.gpu_util import SCALE, assert_close, f32, oracle_xhat, prefill_side, q_sinks

pytestmark = pytest.mark.gpu

FORMATS = {
    "i8_i8": lambda: QuantizedKVCache(32, 8, 8),
    "u4_u4": lambda: QuantizedKVCache(32, 4, 4),
    "i8_u4": lambda: QuantizedKVCache(32, 8, 4),
    "u4_i8": lambda: QuantizedKVCache(32, 4, 8),
    "affine": lambda: MixedQuantizedKVCache(),
}


def bits16(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16


@pytest.mark.parametrize("fmt", list(FORMATS))
@pytest.mark.parametrize("T", [1, 33, 777])
def test_dequant_bit_exact(gpu, fmt, T):
    B, H = 2, 3
    cache = FORMATS[fmt]()
    k = synthetic.kv((B, H, T, 128), 300 + T, kind="heavy", frac=0.05)
    v = synthetic.kv((B, H, T, 128), 301 + T, kind="heavy", frac=0.05)
    kv_k, kv_v = cache.update_and_fetch(k, v)
    kd, vd = dequantize_kv(kv_k, kv_v)
    torch.cuda.synchronize()
    assert kd.shape == (B, H, T, 128) and kd.dtype == torch.bfloat16
    for got, kv, name in ((kd, kv_k, "K"), (vd, kv_v, "V")):
        want = bits16(O.bf16_rn(oracle_xhat(kv)))
        np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), want,
                                      err_msg=f"{fmt} {name} T={T}")


CASES = [
    # format, B, Hq, Hkv, P, L, causal, sinks, dtype
    ("affine", 1, 8, 1, 192, 64, True, True, torch.bfloat16),
    ("affine", 1, 32, 4, 1000, 257, True, True, torch.bfloat16),
    ("affine", 2, 16, 2, 0, 100, False, False, torch.float16),
    ("u4_u4", 1, 32, 4, 300, 129, True, True, torch.bfloat16),
    ("i8_u4", 1, 8, 2, 33, 31, True, False, torch.float16),
    ("u4_i8", 2, 6, 3, 64, 96, False, True, torch.bfloat16),
    ("affine", 3, 4, 4, 40, 33, True, True, torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "{}_B{}_Hq{}_Hkv{}_P{}_L{}_c{}_s{}".format(*c[:8]))
def test_prefill_formats_match_oracle(gpu, case):
    fmt, B, Hq, Hkv, P, L, causal, with_sinks, dtype = case
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 21 + T, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 22 + T, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 23 + L, dtype=dtype)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = FORMATS[fmt]()
    if P:
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    mask = "causal" if causal else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    kv_k, kv_v = cache.keys_and_values()
    kh, vh = prefill_side(oracle_xhat(kv_k), kv_k, dtype), prefill_side(oracle_xhat(kv_v), kv_v, dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, q.dtype), mask)
    assert_close(f32(out), ref, f"case {case}")


def test_affine_chunked_prefill_then_decode(gpu):
    """The MixedQuantizedKVCache flow of Attention.__call__: chunked prefill,
    then fused decode steps over the same cache."""
    B, Hq, Hkv, T, steps = 1, 32, 4, 700, 3
    k = synthetic.kv((B, Hkv, T + steps, 128), 31, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T + steps, 128), 32, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, T + steps, 33, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    cache = MixedQuantizedKVCache()
    for a, b in ((0, 256), (256, 512), (512, T)):
        out = attend(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
        torch.cuda.synchronize()
        kv_k, kv_v = cache.keys_and_values()
        kh = prefill_side(oracle_xhat(kv_k), kv_k, torch.bfloat16)
        vh = prefill_side(oracle_xhat(kv_v), kv_v, torch.bfloat16)
        ref = O.attention(f32(q[:, :, a:b]), kh, vh, SCALE, q_sinks(sinks, q.dtype), "causal")
        assert_close(f32(out), ref, f"chunk [{a}, {b})")
    for t in range(T, T + steps):
        out = attend(q[:, :, t : t + 1], k[:, :, t : t + 1], v[:, :, t : t + 1], cache, SCALE, None, sinks,
                     out_dtype=torch.float32)
        torch.cuda.synchronize()
        kv_k, kv_v = cache.keys_and_values()
        ref = O.attention(f32(q[:, :, t : t + 1]), oracle_xhat(kv_k), oracle_xhat(kv_v), SCALE, f32(sinks))
        assert_close(f32(out), ref, f"decode step {t}")

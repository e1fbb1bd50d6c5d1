"""Parity of the few-query prefill path (prefill_few.hip) with the CPU oracle.

Chunks of at most 64 (query, head) rows per KV head over an int8 or affine
cache run on the streaming kernel instead of the tiled one (33-64 rows below
65,536 keys as two row groups); the outputs must lie within
2e-3 absolute + 1e-3 relative of the oracle, as the tiled kernel's do, for
causal and full masks, sinks, GQA ratios 1 to 8, bf16 and fp16 queries, key
splits (automatic, explicit, one) and ranges whose last chunk lies wholly past
some queries' causal limits.
"""

import pytest
import torch

import oracle as O
from rec_amd import MixedQuantizedKVCache, QuantizedKVCache, attend, synthetic
from tests.gpu_util import SCALE, assert_close, dequant, f32, oracle_quantize, oracle_xhat, prefill_side, q_sinks

pytestmark = pytest.mark.gpu

CASES = [
    # B, Hq, Hkv, P, L, causal, sinks, dtype, splits (0 = automatic)
    (1, 32, 4, 5000, 4, True, True, torch.bfloat16, 0),     # 32 rows: two column tiles
    (1, 32, 4, 65536, 2, True, True, torch.bfloat16, 0),    # a long cache, 64 splits
    (2, 8, 2, 300, 7, True, False, torch.float16, 0),       # 28 rows, two sequences
    (1, 4, 4, 1000, 16, True, True, torch.bfloat16, 0),     # one head per KV head, 16 queries
    (1, 8, 1, 33, 3, False, True, torch.bfloat16, 5),       # full attention, explicit splits
    (1, 16, 2, 31, 4, True, True, torch.float16, 0),        # the chunk at 32 lies past query 0's limit
    (1, 8, 1, 62, 3, True, True, torch.bfloat16, 1),        # unsplit, last chunk partly masked
    (3, 12, 4, 1500, 9, True, True, torch.bfloat16, 0),     # 27 rows, three sequences
    (1, 24, 8, 4096, 10, True, False, torch.float16, 7),    # 30 rows, G = 3
    (1, 8, 1, 130, 2, True, True, torch.float16, 3),        # splits past the causal end stay empty
    # three and four column tiles (over long caches)
    (1, 32, 4, 20000, 8, True, True, torch.bfloat16, 0),    # 64 rows
    (1, 16, 2, 16384, 6, True, False, torch.float16, 5),    # 48 rows, explicit splits
    (2, 24, 8, 17000, 14, True, True, torch.bfloat16, 0),   # 42 rows, G = 3, two sequences
    (1, 8, 1, 16400, 7, False, True, torch.bfloat16, 1),    # 56 rows, full attention, unsplit
    # 33-64 rows over short caches: two row groups
    (1, 32, 4, 4096, 8, True, True, torch.bfloat16, 0),     # 64 rows over 4K keys
    (1, 32, 4, 500, 5, True, True, torch.float16, 0),       # 40 rows, a 32-row and an 8-row group
    (2, 16, 2, 12000, 6, False, False, torch.bfloat16, 3),  # 48 rows, full attention, explicit splits
    (1, 8, 1, 40, 8, True, True, torch.bfloat16, 1),        # 64 rows, unsplit, chunk past early limits
]


@pytest.mark.parametrize("case", CASES,
                         ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_causal{}_s{}_{}_sp{}".format(*c[:7], str(c[7])[6:], c[8]))
def test_few_query_prefill_matches_oracle(gpu, case):
    B, Hq, Hkv, P, L, causal, with_sinks, dtype, splits = case
    assert L * (Hq // Hkv) <= 64
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 71 + T, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 72 + T, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 73 + L, dtype=dtype)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = QuantizedKVCache(32, 8, 8)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    mask = "causal" if causal else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32,
                 splits=splits or None)
    torch.cuda.synchronize()
    rk, rv = oracle_quantize(f32(k), 8), oracle_quantize(f32(v), 8)
    ref = O.attention(f32(q), dequant(8, *rk), dequant(8, *rv), SCALE, q_sinks(sinks, q.dtype), mask)
    assert_close(f32(out), ref, f"case {case}")


def test_few_query_prefill_large_v_scale(gpu):
    """V rows with |v| in the thousands (int8 scales of 2 or more): the
    probabilities stay at most 1 for those tokens, so P' = p·s stays finite."""
    B, Hq, Hkv, P, L = 1, 16, 2, 700, 4
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 81)
    v = synthetic.kv((B, Hkv, T, 128), 82) * 3000.0
    q = synthetic.query(B, Hq, L, 83, dtype=torch.bfloat16)
    cache = QuantizedKVCache(32, 8, 8)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rk, rv = oracle_quantize(f32(k), 8), oracle_quantize(f32(v), 8)
    ref = O.attention(f32(q), dequant(8, *rk), dequant(8, *rv), SCALE, None, "causal")
    assert_close(f32(out), ref, "large V")


AFFINE_CASES = [
    # B, Hq, Hkv, P, L, causal, sinks, dtype, splits (0 = automatic)
    (1, 32, 4, 5000, 4, True, True, torch.bfloat16, 0),     # 32 rows, exact P·V
    (1, 32, 4, 40000, 2, True, True, torch.bfloat16, 0),    # a long cache: P' in one fp16 part
    (2, 8, 2, 300, 7, True, False, torch.float16, 0),       # 28 rows, two sequences, fp16 queries
    (1, 8, 1, 33, 3, False, True, torch.bfloat16, 5),       # full attention, explicit splits
    (1, 16, 2, 31, 4, True, True, torch.float16, 0),        # the chunk at 32 lies past query 0's limit
    (1, 8, 1, 62, 2, True, True, torch.bfloat16, 1),        # 16 rows: one column tile, unsplit
    (1, 32, 4, 20000, 8, True, True, torch.bfloat16, 0),    # 64 rows: four column tiles
    (1, 24, 8, 16384, 14, True, False, torch.float16, 3),   # 42 rows, G = 3
    (1, 32, 4, 4096, 8, True, True, torch.bfloat16, 0),     # 64 rows over 4K keys: two row groups
    (1, 16, 2, 700, 3, True, False, torch.float16, 0),      # 48 rows over a short cache
]


@pytest.mark.parametrize("case", AFFINE_CASES,
                         ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_causal{}_s{}_{}_sp{}".format(*c[:7], str(c[7])[6:], c[8]))
def test_few_query_prefill_affine_matches_oracle(gpu, case):
    """The affine pair (8-bit K, 4-bit V, group 64): K and V values formed in
    registers as q·s + b rounded to the query dtype, as the reference
    dequantizes the cache before its attention."""
    B, Hq, Hkv, P, L, causal, with_sinks, dtype, splits = case
    assert L * (Hq // Hkv) <= 64
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 91 + T, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 92 + T, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 93 + L, dtype=dtype)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = MixedQuantizedKVCache()
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    mask = "causal" if causal else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32,
                 splits=splits or None)
    torch.cuda.synchronize()
    kv_k, kv_v = cache.keys_and_values()
    kh, vh = prefill_side(oracle_xhat(kv_k), kv_k, dtype), prefill_side(oracle_xhat(kv_v), kv_v, dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, q.dtype), mask)
    assert_close(f32(out), ref, f"affine case {case}")

"""Parity of the chunked prefill kernel with the CPU oracle.

The L queries are the newest L cached tokens (appended first, as
Attention.__call__ does, model.py:177-203); with the "causal" mask query i
sees tokens [0, T-L+i].  Outputs within 2e-3 absolute + 1e-3 relative.
"""

import os

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import QuantizedKVCache, attend, quantized_attention_with_sinks, synthetic, to_logical
from tests.gpu_util import SCALE, assert_close, dequant, f32, oracle_quantize, q_sinks

pytestmark = pytest.mark.gpu

CASES = [
    # B, Hq, Hkv, P, L, causal, sinks, dtype
    (1, 8, 1, 192, 64, True, True, torch.float16),
    (1, 8, 1, 0, 100, True, False, torch.bfloat16),
    (1, 32, 4, 1000, 257, True, True, torch.bfloat16),
    (2, 16, 2, 300, 64, False, True, torch.float16),
    (1, 8, 2, 33, 31, True, True, torch.bfloat16),
    (1, 6, 3, 64, 96, True, False, torch.float16),
    (3, 4, 4, 40, 33, True, True, torch.bfloat16),    # one query head per KV head, three sequences
    (1, 12, 4, 256, 96, True, True, torch.float16),   # three per KV head
    (2, 8, 1, 31, 1, True, True, torch.bfloat16),     # a one-token chunk (attend takes the decode path)
    (1, 20, 4, 300, 77, True, True, torch.bfloat16),  # five per KV head: 385 rows, the second block starts in query 51
    (2, 7, 1, 500, 100, False, True, torch.float16),  # seven per KV head, full attention
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_causal{}_s{}_{}".format(*c[:7], str(c[7])[6:]))
def test_prefill_matches_oracle(gpu, case):
    B, Hq, Hkv, P, L, causal, with_sinks, dtype = case
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 11 + T, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 12 + T, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 13 + L, dtype=dtype)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = QuantizedKVCache(32, 8, 8)
    if P:
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal" if causal else None, sinks,
                 out_dtype=torch.float32)
    rk, rv = oracle_quantize(f32(k), 8), oracle_quantize(f32(v), 8)
    # chunks hand the sinks over in the query dtype (model.py:202); one token decodes (float32, model.py:129)
    sk = q_sinks(sinks, q.dtype) if L > 1 else (None if sinks is None else f32(sinks))
    ref = O.attention(f32(q), dequant(8, *rk), dequant(8, *rv), SCALE, sk, "causal" if causal else None)
    assert_close(f32(out), ref, f"case {case}")


def test_prefill_golden(gpu):
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "prefill_causal.npz")
    with np.load(path, allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    P = int(g["prefix"])
    dev = torch.device("cuda")
    k, v = torch.from_numpy(g["k"]).to(dev), torch.from_numpy(g["v"]).to(dev)
    cache = QuantizedKVCache(32, 8, 8)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    q = torch.from_numpy(g["q"]).to(dev)
    sinks = torch.from_numpy(g["sinks"]).to(dev)
    # attend() is the prefill branch of Attention.__call__: sinks in the
    # query dtype (model.py:202); quantized_attention_with_sinks keeps the
    # function's float32 cast (model.py:129)
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
    kq_, vq_ = cache.keys_and_values()
    out32 = quantized_attention_with_sinks(q, kq_, vq_, SCALE, "causal", sinks, 32, 8, 8, out_dtype=torch.float32)
    assert_close(f32(out32), g["out_sinks"].astype(np.float64), "golden prefill, float32 sinks")
    kq, vq = cache.keys_and_values()
    for kv, p in ((kq, "k"), (vq, "v")):
        c, s, _ = (None if t is None else t.cpu().numpy() for t in to_logical(kv))
        np.testing.assert_array_equal(c, g[p + "_codes"])
        np.testing.assert_array_equal(s.view(np.uint16), g[p + "_scales"].view(np.uint16))
    assert_close(f32(out), g["out_sinks_qdtype"].astype(np.float64), "golden prefill")


def test_chunked_prefill_then_decode(gpu):
    """The QATSession loop (quantized.py:122-136): prefill in chunks, then decode."""
    B, Hq, Hkv, chunk = 1, 32, 4, 96
    T = 3 * chunk + 17
    k = synthetic.kv((B, Hkv, T + 3, 128), 40)
    v = synthetic.kv((B, Hkv, T + 3, 128), 41)
    q = synthetic.query(B, Hq, T + 3, 42, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    cache = QuantizedKVCache(32, 8, 8)
    rk, rv = oracle_quantize(f32(k), 8), oracle_quantize(f32(v), 8)
    kh, vh = dequant(8, *rk), dequant(8, *rv)
    for a in range(0, T, chunk):
        b = min(T, a + chunk)
        out = attend(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
        ref = O.attention(f32(q[:, :, a:b]), kh[:, :, :b], vh[:, :, :b], SCALE, q_sinks(sinks, q.dtype), "causal")
        assert_close(f32(out), ref, f"chunk {a}:{b}")
    for t in range(T, T + 3):
        out = attend(q[:, :, t : t + 1], k[:, :, t : t + 1], v[:, :, t : t + 1], cache, SCALE, None, sinks,
                     out_dtype=torch.float32)
        ref = O.attention(f32(q[:, :, t : t + 1]), kh[:, :, : t + 1], vh[:, :, : t + 1], SCALE, f32(sinks))
        assert_close(f32(out), ref, f"decode {t}")


@pytest.mark.parametrize("Hq,Hkv,P,L,rows", [
    (32, 4, 65536, 2048, [0, 1, 777, 1500, 2047]),
    # 3 query heads per KV head: 256-row blocks start inside queries (query 85
    # holds rows 255-257), the last block is partial
    (12, 4, 16384, 1000, [0, 85, 86, 170, 999]),
], ids=["Hq32_Hkv4_P65536_L2048", "Hq12_Hkv4_P16384_L1000"])
def test_prefill_full_size_rows(gpu, Hq, Hkv, P, L, rows):
    """Long causal chunks over a long prefix: sampled rows equal a decode over
    their prefix (a size-independent property), checked against the chunked
    CPU oracle."""
    B = 1
    T = P + L
    cache = QuantizedKVCache(32, 8, 8, max_tokens=T)
    k = synthetic.kv((B, Hkv, T, 128), 7, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 8, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 9, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
    kq, vq = cache.keys_and_values()
    kc, ksc, _ = (t.cpu().numpy() if t is not None else None for t in to_logical(kq))
    vc, vsc, _ = (t.cpu().numpy() if t is not None else None for t in to_logical(vq))
    del k, v
    qf, of, sf = f32(q), f32(out), q_sinks(sinks, q.dtype).astype(np.float32)
    for i in rows:
        Ti = P + i + 1
        cache_np = dict(k_bits=8, v_bits=8, kq=kc[:, :, :Ti], ks=ksc[:, :, :Ti], vq=vc[:, :, :Ti], vs=vsc[:, :, :Ti])
        ref = O.split_k_decode_quantized(qf[:, :, i], cache_np, Ti, SCALE, sf, chunk=8192)
        assert_close(of[:, :, i], ref.astype(np.float64), f"row {i}")


SPLIT_CASES = [
    # B, Hq, Hkv, P, L, causal, sinks, dtype, splits (0 = automatic)
    (1, 32, 4, 5000, 20, True, True, torch.bfloat16, 0),    # a short chat turn over a long cache
    (1, 8, 1, 3000, 40, True, False, torch.float16, 0),     # two query blocks
    (2, 16, 2, 2000, 5, False, True, torch.bfloat16, 7),
    (1, 8, 2, 700, 33, True, True, torch.bfloat16, 64),     # more splits asked than tiles
    (1, 8, 1, 130, 2, True, True, torch.float16, 3),        # splits past the causal end stay empty
    (3, 12, 4, 1500, 9, True, True, torch.bfloat16, 1),     # explicitly unsplit
    (1, 12, 4, 3000, 100, True, True, torch.bfloat16, 0),   # 300 rows: the second block starts inside query 85
    (1, 28, 4, 4000, 45, True, True, torch.float16, 0),     # seven per KV head: 315 rows over two blocks
    (4, 32, 4, 300, 256, True, True, torch.bfloat16, 0),    # half the chip's grid, short prefix: 128-row blocks
    (4, 32, 4, 1200, 256, True, False, torch.float16, 0),   # half the chip's grid, long prefix: two key splits
    (1, 32, 4, 1000, 128, True, True, torch.bfloat16, 0),   # splits capped at two tiles each: 64-row blocks too
]


@pytest.mark.parametrize("case", SPLIT_CASES,
                         ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_causal{}_s{}_{}_sp{}".format(*c[:7], str(c[7])[6:], c[8]))
def test_split_prefill_matches_oracle(gpu, case):
    """Key-split prefill (partials + merge) equals the oracle as the unsplit
    kernel does; the automatic plan splits a short chunk over a long cache."""
    B, Hq, Hkv, P, L, causal, with_sinks, dtype, splits = case
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 41 + T, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 42 + T, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 43 + L, dtype=dtype)
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


@pytest.mark.parametrize("splits", [0, 5, 64])
@pytest.mark.parametrize("window", [0, 300])
def test_split_prefill_bf16_window(gpu, splits, window):
    """The bf16-cache prefill with key splits, plain causal and under a
    sliding window (splits before the window start stay empty)."""
    from rec_amd import scaled_dot_product_attention

    B, Hq, Hkv, T, L = 1, 16, 2, 3000, 24
    k = synthetic.kv((B, Hkv, T, 128), 141, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 142, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, L, 143, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    out = scaled_dot_product_attention(q, k, v, SCALE, "causal", sinks, out_dtype=torch.float32,
                                       splits=splits or None, window=window or None)
    torch.cuda.synchronize()
    qi = np.arange(T - L, T)[:, None]
    ki = np.arange(T)[None]
    mask = (qi >= ki) & ((qi < ki + window) if window else True)
    kb = k.float().cpu().numpy()
    vb = v.float().cpu().numpy()
    ref = O.attention(f32(q), kb, vb, SCALE, sinks=f32(sinks), mask=mask)
    assert_close(f32(out), ref, f"splits={splits} window={window}")


U4_FEW_CASES = [
    # B, Hq, Hkv, P, L, causal, sinks, dtype, splits (0 = automatic)
    (1, 32, 4, 65536, 4, True, True, torch.bfloat16, 0),   # draft tokens over a long cache: 32 rows, split
    (1, 32, 4, 17000, 8, True, True, torch.float16, 0),    # 64 rows over >= 16,384 keys: four column tiles
    (2, 16, 2, 500, 3, True, False, torch.bfloat16, 1),    # unsplit, 24 rows
    (1, 4, 4, 700, 32, True, True, torch.float16, 3),      # one query head per KV head: 32 rows
    (1, 8, 1, 9000, 2, False, True, torch.bfloat16, 0),    # full attention, past the exact-P·V length
    (1, 32, 4, 4096, 8, True, True, torch.bfloat16, 0),    # 64 rows over 4K keys: two row groups
    (1, 16, 2, 900, 3, True, False, torch.float16, 2),     # 48 rows over a short cache, explicit splits
]


@pytest.mark.parametrize("bits", [(4, 4), (8, 4), (4, 8)], ids=["k4v4", "k8v4", "k4v8"])
@pytest.mark.parametrize("case", U4_FEW_CASES,
                         ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_causal{}_s{}_{}_sp{}".format(*c[:7], str(c[7])[6:], c[8]))
def test_4bit_few_query_prefill_matches_oracle(gpu, case, bits):
    """A short chunk over the uint4 cache, or a mixed int8 / uint4 pair,
    streams through the few-query kernel: uint4 K and V dequantized in
    registers ((q - z)·s rounded to the query dtype, as the reference
    dequantizes its cache to it, model.py:194-195), int8 ones as codes with
    their row scales, equal to the oracle over those values."""
    from tests.gpu_util import oracle_xhat, prefill_side

    B, Hq, Hkv, P, L, causal, with_sinks, dtype, splits = case
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 51 + L, kind="heavy", frac=0.05)
    v = synthetic.kv((B, Hkv, T, 128), 52 + L, kind="heavy", frac=0.05)
    q = synthetic.query(B, Hq, L, 53 + L, dtype=dtype)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = QuantizedKVCache(32, *bits)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    mask = "causal" if causal else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32,
                 splits=splits or None)
    torch.cuda.synchronize()
    kq, vq = cache.keys_and_values()
    kh, vh = prefill_side(oracle_xhat(kq), kq, dtype), prefill_side(oracle_xhat(vq), vq, dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, q.dtype), mask)
    assert_close(f32(out), ref, f"case {case}")


ROW_GROUP_CASES = [
    # B, Hq, Hkv, P, L, causal, sinks, dtype, splits (0 = automatic)
    (1, 32, 4, 16400, 20, True, True, torch.bfloat16, 0),   # 160 rows: four groups of three column tiles
    (1, 32, 4, 20000, 12, True, True, torch.float16, 0),    # 96 rows: two groups
    (1, 28, 4, 17000, 30, True, False, torch.bfloat16, 5),  # 210 rows in groups of 64: boundaries inside queries
                                                            # (a 4-bit V takes the tiled kernel here)
    (2, 16, 2, 16384, 10, False, True, torch.bfloat16, 1),  # unsplit, full attention: every group writes its rows
]
ROW_GROUP_FORMATS = {"k8v8": (8, 8), "k4v4": (4, 4), "k8v4": (8, 4), "k4v8": (4, 8), "affine": None}


@pytest.mark.parametrize("fmt", list(ROW_GROUP_FORMATS))
@pytest.mark.parametrize("case", ROW_GROUP_CASES,
                         ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_causal{}_s{}_{}_sp{}".format(*c[:7], str(c[7])[6:], c[8]))
def test_row_group_prefill_matches_oracle(gpu, case, fmt):
    """A chunk of 65-256 (query, head) rows per KV head over 16K-128K keys
    streams through the few-query kernel in row groups, one workgroup each
    (the groups of one split and KV head placed on one XCD); every format's
    output equals the oracle over the cache's stored values."""
    from rec_amd import MixedQuantizedKVCache
    from tests.gpu_util import oracle_xhat, prefill_side

    B, Hq, Hkv, P, L, causal, with_sinks, dtype, splits = case
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 61 + L, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 62 + L, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 63 + L, dtype=dtype)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    bits = ROW_GROUP_FORMATS[fmt]
    cache = MixedQuantizedKVCache(max_tokens=T) if bits is None else QuantizedKVCache(32, *bits, max_tokens=T)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    mask = "causal" if causal else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32,
                 splits=splits or None)
    torch.cuda.synchronize()
    kq, vq = cache.keys_and_values()
    kh, vh = prefill_side(oracle_xhat(kq), kq, dtype), prefill_side(oracle_xhat(vq), vq, dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, q.dtype), mask)
    assert_close(f32(out), ref, f"case {case} {fmt}")


GRAPH_CASES = [
    # name, B, Hq, Hkv, P, L, cache format (key bits, value bits) or "affine", mask
    ("tiled", 1, 32, 4, 2000, 300, (8, 8), "causal"),           # 256-row blocks, unsplit
    ("few_split_merge", 1, 32, 4, 20000, 4, (4, 4), "causal"),  # streaming kernel, key splits + merge
    ("row_groups", 1, 32, 4, 20000, 20, "affine", "causal"),    # row groups of the streaming kernel
    ("bias", 2, 16, 2, 700, 40, (8, 4), "bias"),                # a device mask array: the tiled kernel's bias
]


@pytest.mark.parametrize("case", GRAPH_CASES, ids=lambda c: c[0])
def test_prefill_in_hip_graph(gpu, case):
    """Chunked prefill (every kernel path: tiled, few-query with key splits
    and its merge, row groups, a mask array as a bias) captured in a HIP
    graph and replayed several times, with eager work between the replays,
    equals the eager call bit for bit every time (the launches record no
    memset and allocate nothing at replay)."""
    from rec_amd import MixedQuantizedKVCache

    name, B, Hq, Hkv, P, L, fmt, mask = case
    T = P + L
    k = synthetic.kv((B, Hkv, T, 128), 41 + L, kind="outliers", frac=0.01)
    v = synthetic.kv((B, Hkv, T, 128), 42 + L, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, L, 43 + L, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    cache = MixedQuantizedKVCache(max_tokens=T) if fmt == "affine" else QuantizedKVCache(32, *fmt, max_tokens=T)
    kq, vq = cache.update_and_fetch(k, v)
    group, bits = (64, (8, 4)) if fmt == "affine" else (32, fmt)
    m = "causal"
    if mask == "bias":
        keep = torch.rand((B, 1, L, T), device="cuda") < 0.7
        keep[..., 0] = True
        m = keep
    eager = quantized_attention_with_sinks(q, kq, vq, SCALE, m, sinks, group, *bits, out_dtype=torch.float32)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out.copy_(quantized_attention_with_sinks(q, kq, vq, SCALE, m, sinks, group, *bits, out_dtype=torch.float32))
    for rep in range(3):
        out.fill_(float("nan"))
        _ = quantized_attention_with_sinks(q[:, :, :1], kq, vq, SCALE, None, None, group, *bits)  # eager work between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, rtol=0, atol=0, msg=f"{name}: replay {rep}")

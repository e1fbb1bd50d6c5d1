"""A seeded sweep of chunked-prefill shapes over long caches against the oracle.

The prefill planner picks among the streaming few-query kernel (one
workgroup, or row groups of one to four column tiles), the tiled kernel with
or without key splits, and 256-, 128- or 64-row query blocks, from the row
count per KV head, the cache length, the grid size and the formats.  This
draw crosses those boundaries at random (cached prefixes up to 70,000
tokens, chunks of 2-300 queries, GQA 1-8, every cache format, bf16 / fp16 /
float32 queries, causal, full and sliding-window masks, automatic and
explicit splits) with the oracle's cost bounded; REC_PLAN_CASES=n draws n
(the first 40 run by default).  Outputs within 2e-3 abs + 1e-3 rel of the
float64 oracle over the cache read back from the GPU (4-bit and affine
values rounded to the query dtype for bf16 / fp16 chunks)."""

import os

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import FixedKVCache, KVStorage, MixedQuantizedKVCache, QuantizedKVCache, attend, synthetic
from tests.gpu_util import SCALE, assert_close, f32, oracle_xhat, prefill_side, q_sinks

pytestmark = pytest.mark.gpu

FORMATS = ["i8", "u4", "i8u4", "u4i8", "affine", "bf16"]
BUDGET = 5_000_000  # B * Hq * L * T: the float64 oracle takes about a second per 4M


def draw(n=int(os.environ.get("REC_PLAN_CASES", "40")), seed=77):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        i = len(cases)
        fmt = FORMATS[i % len(FORMATS)]
        G = int(rng.choice([1, 2, 4, 8]))
        Hkv = int(rng.choice([1, 2]))
        B = int(rng.choice([1, 1, 2]))
        P = int(rng.choice([0, 500, 4000, 16384, 20000, 33000, 70000]))
        L = int(rng.choice([2, 3, 4, 6, 8, 12, 20, 33, 100, 300]))
        dt = [torch.bfloat16, torch.float16, torch.float32][int(rng.choice([0, 0, 1, 2]))]
        mask = str(rng.choice(["causal", "causal", "none", "window"]))
        window = int(rng.choice([513, 4096])) if mask == "window" else 0
        splits = int(rng.choice([0, 0, 0, 2, 7]))
        sinks = bool(rng.integers(0, 2))
        data = 9000 + 11 * i
        if dt == torch.float32 and L > 12:
            L = 12  # a float32 chunk runs one decode per query
        if P + L == 0 or B * G * Hkv * L * (P + L) > BUDGET:
            continue
        cases.append((fmt, B, G * Hkv, Hkv, P, L, dt, mask, window, splits, sinks, data))
    return cases


def make_cache(fmt, B, Hkv, cap):
    if fmt == "bf16":
        return FixedKVCache(KVStorage(1, cap, Hkv, batch=B), 0)
    if fmt == "affine":
        return MixedQuantizedKVCache(max_tokens=cap)
    kb, vb = {"i8": (8, 8), "u4": (4, 4), "i8u4": (8, 4), "u4i8": (4, 8)}[fmt]
    return QuantizedKVCache(32, kb, vb, max_tokens=cap)


def keep_window(L, T, window):
    q = np.arange(T - L, T)[:, None]
    k = np.arange(T)[None]
    return (q >= k) & (q < k + window)


@pytest.mark.parametrize("case", draw(), ids=lambda c: "{}_B{}_Hq{}_Hkv{}_P{}_L{}_{}_{}{}_sp{}_s{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], str(c[6])[6:], c[7], c[8] or "", c[9], int(c[10])))
def test_plan_sweep(gpu, case):
    fmt, B, Hq, Hkv, P, L, dt, mask, window, splits, with_sinks, seed = case
    T = P + L
    # keys in bf16 or fp16 (an affine cache keeps its scales in the keys' dtype)
    kdt = torch.bfloat16 if fmt == "bf16" or seed % 2 else torch.float16
    k = synthetic.kv((B, Hkv, T, 128), seed, kind="outliers", frac=0.02, dtype=kdt)
    v = synthetic.kv((B, Hkv, T, 128), seed + 1, kind="outliers", frac=0.02, dtype=kdt)
    q = synthetic.query(B, Hq, L, seed + 2, dtype=dt)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = make_cache(fmt, B, Hkv, T + 64)
    if P:
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    m = {"causal": "causal", "none": None}.get(mask)
    if mask == "window":
        m = keep_window(L, T, window)  # a host array of the window pattern: the kernels' own window masking
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, m, sinks, out_dtype=torch.float32, splits=splits or None)
    torch.cuda.synchronize()
    if fmt == "bf16":
        kh, vh = f32(k), f32(v)
    else:
        kv_k, kv_v = cache.keys_and_values()
        kh, vh = prefill_side(oracle_xhat(kv_k), kv_k, dt), prefill_side(oracle_xhat(kv_v), kv_v, dt)
    ref = O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, dt), m)
    assert_close(f32(out), ref, f"case {case}")

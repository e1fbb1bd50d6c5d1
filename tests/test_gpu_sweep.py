"""A seeded sweep of shapes through every decode and prefill format against
the oracle: batch sizes, GQA ratios, ragged token counts, split counts, query
dtypes (float32 chunks included) and sinks drawn from a fixed generator (the
same 40 cases every run;
REC_SWEEP_CASES=n draws n, the first 40 being these; two cases of the
400-case draw always run as regressions).
Outputs within 2e-3 abs + 1e-3 rel of the float64 oracle over the cache read
back from the GPU and dequantized (for a prefill, 4-bit and affine values
rounded to the query dtype, as the kernel and the reference dequantize them)."""

import os

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import (FixedKVCache, KVStorage, MixedQuantizedKVCache, QuantizedKVCache, attend, synthetic,
                     to_logical)
from tests.gpu_util import SCALE, assert_close, dequant, f32, prefill_side, q_sinks

pytestmark = pytest.mark.gpu

FORMATS = ["i8", "u4", "i8u4", "u4i8", "affine", "bf16"]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def draw(n=int(os.environ.get("REC_SWEEP_CASES", "40")), seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        G = int(rng.choice([1, 2, 3, 4, 6, 8]))
        Hkv = int(rng.choice([1, 2, 4]))
        B = int(rng.integers(1, 4))
        T = int(rng.choice([1, 2, 31, 32, 33, 95, 256, 511, 1000, 2049]))
        L = int(rng.choice([1, 1, 1, 7, 40]))  # mostly decode
        L = min(L, T)
        fmt = FORMATS[i % len(FORMATS)]
        dt = DTYPES[int(rng.integers(0, 3))]  # float32 chunks run a decode per query
        splits = int(rng.choice([0, 0, 1, 3, 17, 64]))
        sinks = bool(rng.integers(0, 2))
        cases.append((fmt, B, G * Hkv, Hkv, T, L, dt, splits, sinks, 5000 + 7 * i))  # last: the data seed
    return cases


def make_cache(fmt, B, Hkv, cap):
    if fmt == "bf16":
        return FixedKVCache(KVStorage(1, cap, Hkv, batch=B), 0)
    if fmt == "affine":
        return MixedQuantizedKVCache(max_tokens=cap)
    kb, vb = {"i8": (8, 8), "u4": (4, 4), "i8u4": (8, 4), "u4i8": (4, 8)}[fmt]
    return QuantizedKVCache(32, kb, vb, max_tokens=cap)


def oracle_xhat(kv):
    codes, scales, extra = to_logical(kv)
    if kv.affine:
        c = codes.cpu().numpy()
        if kv.bits == 4:
            c = O.unpack_int4(c)
        return O.dequantize_affine(c, f32(scales), f32(extra))
    return dequant(kv.bits, codes.cpu().numpy(), scales.cpu().numpy(), None if extra is None else extra.cpu().numpy())


# Cases 182 and 204 of the 400-case draw once exceeded the tolerance (prefill
# rows that see 10 and 3 tokens, outlier channels near |v| = 25, when each
# probability entered the P·V product rounded once to fp16): always run.
REGRESSION = [draw(400)[182], draw(400)[204]]
CASES = draw() + [c for c in REGRESSION if c not in draw()]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "{}_B{}_Hq{}_Hkv{}_T{}_L{}_{}_sp{}_s{}_seed{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], str(c[6])[6:], c[7], c[8], c[9]))
def test_sweep(gpu, case):
    fmt, B, Hq, Hkv, T, L, dt, splits, with_sinks, seed = case
    kdt = torch.bfloat16 if fmt == "bf16" else torch.float16
    k = synthetic.kv((B, Hkv, T, 128), seed, kind="outliers", frac=0.02, dtype=kdt)
    v = synthetic.kv((B, Hkv, T, 128), seed + 1, kind="outliers", frac=0.02, dtype=kdt)
    q = synthetic.query(B, Hq, L, seed + 2, dtype=dt)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    cache = make_cache(fmt, B, Hkv, T + 32)
    P = T - L
    if P:
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", sinks, out_dtype=torch.float32,
                 splits=splits or None)
    torch.cuda.synchronize()
    if fmt == "bf16":
        kh, vh = f32(k), f32(v)
    else:
        kv_k, kv_v = cache.keys_and_values()
        kh, vh = oracle_xhat(kv_k), oracle_xhat(kv_v)
        if L > 1:  # the prefill rounds 4-bit and affine values to the query dtype
            kh, vh = prefill_side(kh, kv_k, dt), prefill_side(vh, kv_v, dt)
    # sinks in the query dtype for chunks and over the bf16 cache (model.py:202,211), float32 in the quantized decode
    sk = q_sinks(sinks, dt) if (L > 1 or fmt == "bf16") else (None if sinks is None else f32(sinks))
    ref = O.attention(f32(q), kh, vh, SCALE, sk, "causal")
    assert_close(f32(out), ref, f"case {case}")

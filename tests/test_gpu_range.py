"""Decode and prefill with large V scales and steeply rising scores, against
the float64 oracle.

The kernels take probabilities against a running maximum that moves only
when a score passes it by more than 2^8 (log2 units), so a probability can
reach 256 before the rescale; its product with the V scale feeds an fp16
matrix operand.  With int8 V scales near 470 (|v| up to 60,000) or 4-bit group
scales near 330 (group ranges near 5,000) those products would pass the fp16
range; the kernels must keep them finite and the outputs within 2e-3 abs +
1e-3 rel of the oracle, plus the fp32 rounding floor of such values (1e-6 of
the largest |v|).

Keys are built so that the scores climb along the sequence: key t is
lambda_t times the unit query direction plus noise, lambda_t rising from 0 to 12
score units, so every wave meets new maxima chunk after chunk.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import QuantizedKVCache, attend, synthetic
from tests.gpu_util import SCALE, assert_close, dequant, f32, oracle_quantize, prefill_side, q_sinks

pytestmark = pytest.mark.gpu


def rising_keys(B, H, T, q, seed, top=12.0):
    """Keys whose scores against the (single) query row rise along the
    sequence: k_t = lambda_t * u + 0.3 * noise, u = q / |q| per KV head's first
    query head, lambda_t = top * t / T / (|q| * SCALE) score units."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    noise = torch.randn((B, H, T, 128), generator=g, device="cuda")
    G = q.shape[1] // H
    u = q[:, ::G, 0].float()  # (B, H, 128): the first query head of each group
    norm = u.norm(dim=-1, keepdim=True)
    lam = torch.linspace(0, top, T, device="cuda") / (norm * SCALE)  # (B, H, T)
    k = lam[..., None] * (u / norm)[:, :, None, :] + 0.3 * noise
    return k.to(torch.float16)


def big_values(B, H, T, seed, sigma, clamp=65000.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    v = torch.randn((B, H, T, 128), generator=g, device="cuda") * sigma
    return v.clamp(-clamp, clamp).to(torch.float16)


CASES = [
    # k_bits, v_bits, V sigma, T, L (1 = decode), splits
    (8, 8, 16000.0, 3000, 1, None),  # int8 V scales near 470
    (8, 8, 16000.0, 3000, 1, 1),
    (8, 4, 1200.0, 3000, 1, None),  # 4-bit V group ranges near 5,000
    (4, 4, 1200.0, 5000, 1, 2),  # eight-wave uint4 workgroups
    (8, 8, 16000.0, 700, 40, None),  # int8 prefill
    (8, 4, 1200.0, 700, 40, None),  # prefill over a 4-bit V cache
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "k{}v{}_sigma{}_T{}_L{}_sp{}".format(*c))
def test_large_v_scales_rising_scores(gpu, case):
    kb, vb, sigma, T, L, splits = case
    B, Hq, Hkv = 1, 16, 2
    q = synthetic.query(B, Hq, L, seed=31)
    if L == 1:
        k = rising_keys(B, Hkv, T, q, seed=32)
    else:  # the prefill rows share the rising direction of their last query row
        k = rising_keys(B, Hkv, T, q[:, :, -1:], seed=32)
    v = big_values(B, Hkv, T, seed=33, sigma=sigma)
    sinks = torch.randn(Hq, device="cuda")
    cache = QuantizedKVCache(32, kb, vb)
    P = T - L
    if P:
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, "causal", sinks, out_dtype=torch.float32, splits=splits)
    torch.cuda.synchronize()
    rk, rv = oracle_quantize(f32(k), kb), oracle_quantize(f32(v), vb)
    kh, vh = dequant(kb, *rk), dequant(vb, *rv)
    if L > 1:  # the prefill rounds 4-bit values to the query dtype
        kq, vq = cache.keys_and_values()
        kh, vh = prefill_side(kh, kq, q.dtype), prefill_side(vh, vq, q.dtype)
    ref = O.attention(f32(q), kh, vh, SCALE, q_sinks(sinks, q.dtype), "causal")
    got = f32(out).astype(np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    # An output here is a weighted mean of values up to ~65,000, so fp32
    # arithmetic alone leaves errors near 2^-22 of the largest |v|: the
    # absolute tolerance grows with it (1e-6 * max|v|, about 16 fp32 ulps).
    # An overflowed or clamped product would be off by a sizeable fraction of
    # |v| instead.
    err = np.abs(got - ref)
    bound = 2e-3 + 1e-6 * np.abs(vh).max() + 1e-3 * np.abs(ref)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), f"case {case}: max |err| {err.max():.3e} at {worst} (bound {bound[worst]:.3e})"


def test_uint4_131k_heavy_tailed(gpu):
    """The 4-bit configuration at its full shape: 131,072 cached tokens, 32
    query heads over 4 KV heads, uint4 with an fp16 scale and zero-point per
    32 dims, Student-t(3) values in 5% of the channels; three fused append +
    attend steps, each against the oracle's split-K over the cache read back."""
    from rec_amd import to_logical

    B, Hq, Hkv, T0 = 1, 32, 4, 131072 - 3
    cache = QuantizedKVCache(32, 4, 4, max_tokens=131072)
    k = synthetic.kv((B, Hkv, T0, 128), 41, kind="heavy", frac=0.05)
    v = synthetic.kv((B, Hkv, T0, 128), 42, kind="heavy", frac=0.05)
    cache.update_and_fetch(k, v)
    del k, v
    sinks = torch.randn(Hq, device="cuda")
    for step in range(3):
        q = synthetic.query(B, Hq, 1, seed=43 + step)
        kn = synthetic.kv((B, Hkv, 1, 128), 50 + step, kind="heavy", frac=0.05)
        vn = synthetic.kv((B, Hkv, 1, 128), 60 + step, kind="heavy", frac=0.05)
        out = attend(q, kn, vn, cache, SCALE, None, sinks, out_dtype=torch.float32)
        torch.cuda.synchronize()
        T = cache.offset
        kq, vq = cache.keys_and_values()
        kc, ksc, kz = (t.cpu().numpy() for t in to_logical(kq))
        vc, vsc, vz = (t.cpu().numpy() for t in to_logical(vq))
        # the appended token's bytes are the oracle's quantization of it
        nk, nv = oracle_quantize(f32(kn), 4), oracle_quantize(f32(vn), 4)
        for got, want in ((kc, nk[0]), (ksc, nk[1]), (kz, nk[2]), (vc, nv[0]), (vsc, nv[1]), (vz, nv[2])):
            np.testing.assert_array_equal(got[:, :, T - 1 :].view(np.uint8), np.asarray(want).view(np.uint8))
        c = dict(k_bits=4, v_bits=4, kq=kc, ks=ksc, kz=kz, vq=vc, vs=vsc, vz=vz)
        ref = O.split_k_decode_quantized(f32(q)[:, :, 0], c, T, SCALE, f32(sinks), chunk=8192)
        assert_close(f32(out)[:, :, 0], ref.astype(np.float64), f"step {step}")

"""Pins the CPU oracle with checks that do not restate its formulas.

Quantizers: brute-force nearest-code search, closed forms and invariants.
Attention: torch's scaled_dot_product_attention in float64 (an independent
library routine), the T = 1 closed form, permutation / identical-key / GQA
invariants, and split-K merge over arbitrary partitions.
"""

import numpy as np
import pytest
import torch

import oracle as O


def _fp16_rows(rng, n, d, scale=1.0):
    return (rng.standard_normal((n, d)) * scale).astype(np.float16)


# ---------------------------------------------------------------- int8 ----


def _nearest_even(r):
    """Round-half-even in float64 without numpy.rint (brute force over k)."""
    fl = np.floor(r)
    cands = np.stack([fl - 1, fl, fl + 1, fl + 2], -1)
    dist = np.abs(cands - r[..., None])
    best = dist.min(-1, keepdims=True)
    ok = np.isclose(dist, best, rtol=0, atol=0)
    # among equidistant candidates prefer the even one
    even = (np.mod(cands, 2) == 0) & ok
    pick = np.where(even.any(-1, keepdims=True), even, ok)
    return (cands * pick).sum(-1) / pick.sum(-1)


def test_int8_codes_are_the_nearest_representable_code():
    rng = np.random.default_rng(1)
    x = _fp16_rows(rng, 64, 128, 3.0)
    codes, s16 = O.quantize_int8(x)
    s = s16.astype(np.float64)[:, None]
    # brute force: every code in [-127, 127], pick the closest q*s (ties -> even)
    ks = np.arange(-127, 128, dtype=np.float64)
    err = np.abs(x.astype(np.float64)[..., None] - ks * s[..., None])
    best = err.min(-1, keepdims=True)
    tie = err == best
    even_pref = np.where((tie & (np.mod(ks, 2) == 0)).any(-1, keepdims=True), tie & (np.mod(ks, 2) == 0), tie)
    brute = (ks * even_pref).sum(-1) / even_pref.sum(-1)
    np.testing.assert_array_equal(codes.astype(np.float64), brute)


def test_int8_scale_is_nearest_fp16_to_amax_over_127():
    rng = np.random.default_rng(2)
    x = _fp16_rows(rng, 256, 128, 2.0)
    _, s16 = O.quantize_int8(x)
    exact = np.abs(x.astype(np.float64)).max(-1) / 127.0
    # neighbours of s16 in fp16 are no closer to the exact ratio
    up = np.nextafter(s16, np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(s16, np.float16(-np.inf)).astype(np.float64)
    d0 = np.abs(s16.astype(np.float64) - exact)
    assert np.all(d0 <= np.abs(up - exact)) and np.all(d0 <= np.abs(dn - exact))


def test_int8_closed_forms_and_invariants():
    rng = np.random.default_rng(3)
    zero = np.zeros((3, 128), np.float16)
    c, s = O.quantize_int8(zero)
    assert not c.any() and not s.astype(np.float32).any()
    one = np.zeros((1, 128), np.float16)
    one[0, 17] = -5.5
    c, s = O.quantize_int8(one)
    assert c[0, 17] == -127 and np.count_nonzero(c) == 1
    assert s[0] == np.float16(5.5 / 127)
    x = _fp16_rows(rng, 128, 128, 4.0)
    c, s = O.quantize_int8(x)
    # the element of largest magnitude lands on +-127
    i = np.abs(x.astype(np.float32)).argmax(-1)
    np.testing.assert_array_equal(np.abs(c[np.arange(128), i]), 127)
    # symmetric: q(-x) = -q(x), same scale
    c2, s2 = O.quantize_int8(-x)
    np.testing.assert_array_equal(c2, -c)
    np.testing.assert_array_equal(s2, s)
    # reconstruction error within half a step (tiny slack for the clamp at 127)
    xh = O.dequantize_int8(c, s)
    sf = s.astype(np.float32)[:, None]
    assert np.all(np.abs(xh - x.astype(np.float32)) <= 0.5 * sf * 1.001 + 1e-12)
    assert np.abs(c.astype(np.int32)).max() <= 127


def test_int8_saturating_scale_for_huge_bf16_inputs():
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 1e30
    c, s = O.quantize_int8(x)
    assert s[0] == np.float16(65504) and c[0, 0] == 127


# ---------------------------------------------------------------- int4 ----


def test_int4_pack_order_low_nibble_even():
    q = np.array([[1, 2, 15, 0]], np.uint8)
    p = O.pack_int4(q)
    np.testing.assert_array_equal(p, np.array([[0x21, 0x0F]], np.uint8))
    np.testing.assert_array_equal(O.unpack_int4(p), q)


def test_int4_codes_nearest_given_scale_and_zero():
    rng = np.random.default_rng(4)
    x = _fp16_rows(rng, 64, 128, 1.5)
    x[:, 5] = (rng.standard_t(3, 64) * 2).astype(np.float16)
    p, s16, z16 = O.quantize_int4(x, 32)
    q = O.unpack_int4(p).astype(np.float64).reshape(64, 4, 32)
    s = s16.astype(np.float64)[..., None]
    z = z16.astype(np.float64)
    xg = x.astype(np.float64).reshape(64, 4, 32)
    # zero-point: nearest integer to -mn/s, inside [0, 15]
    mn = np.minimum(xg.min(-1), 0)
    np.testing.assert_array_equal(z, np.clip(_nearest_even(-mn / s[..., 0]), 0, 15))
    # codes: brute force over 0..15 of |x - (k - z) s|
    ks = np.arange(16, dtype=np.float64)
    err = np.abs(xg[..., None] - (ks - z[..., None, None]) * s[..., None])
    best = err.min(-1, keepdims=True)
    tie = err == best
    ev = tie & (np.mod(ks - z[..., None, None], 2) == 0)
    pick = np.where(ev.any(-1, keepdims=True), ev, tie)
    brute = (ks * pick).sum(-1) / pick.sum(-1)
    np.testing.assert_array_equal(q, brute)


def test_int4_closed_forms():
    # all-zero group -> zero scale, zero codes, exact zero
    z = np.zeros((2, 128), np.float16)
    p, s, zz = O.quantize_int4(z)
    assert not p.any() and not s.astype(np.float32).any() and not zz.astype(np.float32).any()
    # a constant positive group keeps its value (range contains 0)
    c = np.full((1, 128), 1.25, np.float16)
    p, s, zz = O.quantize_int4(c)
    xh = O.dequantize_int4(p, s, zz)
    assert np.all(zz.astype(np.float32) == 0)
    assert np.allclose(xh, 1.25, rtol=2e-3)
    # exact zeros stay exact zeros
    rng = np.random.default_rng(5)
    x = _fp16_rows(rng, 32, 128)
    x[:, ::7] = 0
    p, s, zz = O.quantize_int4(x)
    xh = O.dequantize_int4(p, s, zz)
    assert np.all(xh[:, ::7] == 0)
    sf = np.repeat(s.astype(np.float32), 32, axis=-1)
    assert np.all(np.abs(xh - x.astype(np.float32)) <= 0.5 * sf * 1.01 + 1e-12)


# ----------------------------------------------------------- attention ----


def _torch_reference(q, k, v, scale, sinks=None, mask=None):
    """Independent check: torch SDPA in float64; sinks become an extra zero key
    whose additive mask equals the sink logit."""
    q = torch.from_numpy(np.asarray(q, np.float64))
    k = torch.from_numpy(np.asarray(k, np.float64))
    v = torch.from_numpy(np.asarray(v, np.float64))
    B, Hq, L, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    k = k.repeat_interleave(Hq // Hkv, dim=1)
    v = v.repeat_interleave(Hq // Hkv, dim=1)
    bias = torch.zeros(B, Hq, L, T, dtype=torch.float64)
    if mask is not None:
        m = torch.from_numpy(np.asarray(O.causal_mask(L, T) if isinstance(mask, str) else mask))
        bias = bias.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else bias + m
    if sinks is not None:
        k = torch.cat([k, torch.zeros(B, Hq, 1, D, dtype=torch.float64)], 2)
        v = torch.cat([v, torch.zeros(B, Hq, 1, D, dtype=torch.float64)], 2)
        sb = torch.from_numpy(np.asarray(sinks, np.float64)).view(1, Hq, 1, 1).expand(B, Hq, L, 1)
        bias = torch.cat([bias, sb], -1)
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=bias, scale=scale)
    return out.numpy()


def _cache(rng, B, Hkv, T, D=128):
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float16)
    kc, ks = O.quantize_int8(k)
    vc, vs = O.quantize_int8(v)
    return O.dequantize_int8(kc, ks), O.dequantize_int8(vc, vs)


@pytest.mark.parametrize("with_sinks", [False, True])
def test_attention_matches_torch_sdpa(with_sinks):
    rng = np.random.default_rng(6)
    B, Hq, Hkv, T = 2, 8, 2, 200
    kh, vh = _cache(rng, B, Hkv, T)
    q = rng.standard_normal((B, Hq, 1, 128)).astype(np.float16)
    sinks = rng.standard_normal(Hq) if with_sinks else None
    scale = 1 / np.sqrt(128)
    ours = O.attention(q, kh, vh, scale, sinks)
    ref = _torch_reference(q, kh, vh, scale, sinks)
    np.testing.assert_allclose(ours, ref, rtol=1e-12, atol=1e-12)


def test_attention_causal_and_bool_mask_match_torch():
    rng = np.random.default_rng(7)
    B, Hq, Hkv, T, L = 1, 4, 1, 96, 16
    kh, vh = _cache(rng, B, Hkv, T)
    q = rng.standard_normal((B, Hq, L, 128))
    sinks = rng.standard_normal(Hq)
    scale = 0.0883883
    np.testing.assert_allclose(
        O.attention(q, kh, vh, scale, sinks, "causal"), _torch_reference(q, kh, vh, scale, sinks, "causal"), atol=1e-12
    )
    m = rng.random((L, T)) > 0.3
    np.testing.assert_allclose(O.attention(q, kh, vh, scale, sinks, m), _torch_reference(q, kh, vh, scale, sinks, m), atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(8)
    # T = 1: out = v0 * e^{s0} / (e^{s0} + e^{sink})
    k = rng.standard_normal((1, 1, 1, 128))
    v = rng.standard_normal((1, 1, 1, 128))
    q = rng.standard_normal((1, 2, 1, 128))
    sinks = np.array([0.3, -1.2])
    out = O.attention(q, k, v, 0.1, sinks)
    for h in range(2):
        s0 = 0.1 * float(q[0, h, 0] @ k[0, 0, 0])
        w = 1.0 / (1.0 + np.exp(sinks[h] - s0))
        np.testing.assert_allclose(out[0, h, 0], w * v[0, 0, 0], rtol=1e-13)
    # identical keys: uniform weights -> mean of values, scaled by the sink share
    T = 37
    k = np.repeat(rng.standard_normal((1, 1, 1, 128)), T, axis=2)
    v = rng.standard_normal((1, 1, T, 128))
    out = O.attention(q, k, v, 0.1, sinks)
    for h in range(2):
        s0 = 0.1 * float(q[0, h, 0] @ k[0, 0, 0])
        share = T / (T + np.exp(sinks[h] - s0))
        np.testing.assert_allclose(out[0, h, 0], share * v[0, 0].mean(0), rtol=1e-12)


def test_attention_invariants():
    rng = np.random.default_rng(9)
    kh, vh = _cache(rng, 1, 2, 120)
    q = rng.standard_normal((1, 16, 1, 128))
    q[:, 8:12] = q[:, 8:9]  # equal queries in one GQA group
    out = O.attention(q, kh, vh, 0.088, None)
    for h in range(9, 12):
        np.testing.assert_allclose(out[0, h], out[0, 8], rtol=1e-14)
    perm = rng.permutation(120)
    out2 = O.attention(q, kh[:, :, perm], vh[:, :, perm], 0.088, None)
    np.testing.assert_allclose(out, out2, rtol=1e-12, atol=1e-14)
    # all keys masked, no sink -> zeros (the merge's z == 0 branch)
    m = np.zeros((1, 120), bool)
    assert not O.attention(q, kh, vh, 0.088, None, m).any()


def test_prefill_rows_equal_decode_over_prefix():
    rng = np.random.default_rng(10)
    P, L = 50, 12
    kh, vh = _cache(rng, 1, 1, P + L)
    q = rng.standard_normal((1, 8, L, 128))
    sinks = rng.standard_normal(8)
    full = O.attention(q, kh, vh, 0.088, sinks, "causal")
    for i in range(L):
        row = O.attention(q[:, :, i : i + 1], kh[:, :, : P + i + 1], vh[:, :, : P + i + 1], 0.088, sinks)
        np.testing.assert_allclose(full[:, :, i : i + 1], row, rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("parts", [None, [0, 1, 7, 100, 101], [0, 64, 128, 192, 256, 300]])
def test_split_k_merge_equals_single_pass(parts):
    rng = np.random.default_rng(11)
    T = 333
    kh, vh = _cache(rng, 1, 4, T)
    q = rng.standard_normal((1, 32, 128)).astype(np.float32)
    sinks = rng.standard_normal(32)
    ref = O.attention(q[:, :, None], kh, vh, 0.088, sinks)[:, :, 0]
    got = O.split_k_decode(
        q, lambda a, b: kh[:, :, a:b], lambda a, b: vh[:, :, a:b], T, 0.088, sinks, parts=parts, chunk=64
    )
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_split_k_quantized_int4_and_mixed():
    rng = np.random.default_rng(12)
    T = 130
    k = rng.standard_normal((1, 2, T, 128)).astype(np.float16)
    v = rng.standard_normal((1, 2, T, 128)).astype(np.float16)
    kq, ks = O.quantize_int8(k)
    vq, vs, vz = O.quantize_int4(v)
    cache = dict(k_bits=8, v_bits=4, kq=kq, ks=ks, vq=vq, vs=vs, vz=vz)
    q = rng.standard_normal((1, 16, 128)).astype(np.float32)
    got = O.split_k_decode_quantized(q, cache, T, 0.088, None, chunk=48)
    ref = O.attention(q[:, :, None], O.dequantize_int8(kq, ks), O.dequantize_int4(vq, vs, vz), 0.088)[:, :, 0]
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_mutation_in_oracle_is_caught():
    """A planted mistake (dropped sink term) must fail the torch pin."""
    rng = np.random.default_rng(13)
    kh, vh = _cache(rng, 1, 1, 20)
    q = rng.standard_normal((1, 2, 1, 128))
    sinks = np.array([1.0, 2.0])
    wrong = O.attention(q, kh, vh, 0.088, None)  # sink dropped
    ref = _torch_reference(q, kh, vh, 0.088, sinks)
    assert not np.allclose(wrong, ref, rtol=1e-6, atol=1e-9)


def _sinks_bf16_unrepresentable(rng, n):
    """Sink logits with a 16-bit remainder under bf16: each is a bf16 value plus
    a quarter of its last place or more, so rounding moves it visibly."""
    base = torch.from_numpy(rng.uniform(-1.0, 3.0, n).astype(np.float32)).to(torch.bfloat16).float().numpy()
    ulp = np.abs(base) * 2.0**-7 + 2.0**-10
    return (base + rng.uniform(0.3, 0.45, n).astype(np.float32) * ulp).astype(np.float32)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_sink_logits_rounded_to_query_dtype_match_torch(dtype):
    """The SDPA call sites hand the sinks over in the query dtype
    (model.py:202,211).  On rows that see few keys, where the sink carries a
    large share of the weight, the oracle's rounding must equal torch's own
    cast of the sinks fed to torch SDPA, and the sinks taken as float32 (a
    planted mistake: no rounding) must not."""
    rng = np.random.default_rng(17)
    B, Hq, Hkv, P, L = 1, 8, 2, 2, 6
    kh, vh = _cache(rng, B, Hkv, P + L)
    vh = vh * 8.0
    q = rng.standard_normal((B, Hq, L, 128)).astype(np.float32)
    sinks = _sinks_bf16_unrepresentable(rng, Hq)
    tdt = getattr(torch, dtype)
    cast = torch.from_numpy(sinks).to(tdt).double().numpy()
    assert not np.array_equal(cast, sinks.astype(np.float64))
    np.testing.assert_array_equal(O.sink_logits(sinks, dtype), cast)
    ref = _torch_reference(q, kh, vh, 0.088, cast, "causal")
    ours = O.attention(q, kh, vh, 0.088, sinks, "causal", sink_dtype=dtype)
    np.testing.assert_allclose(ours, ref, rtol=1e-12, atol=1e-12)
    planted = O.attention(q, kh, vh, 0.088, sinks, "causal", sink_dtype="float32")
    # bf16 keeps 8 significant bits: the rounding moves outputs past the 2e-3
    # tolerance; fp16 keeps 11, its rounding is smaller but still seen
    assert np.abs(planted - ref).max() > (2e-3 if dtype == "bfloat16" else 1e-4)
    # float32 is the quantized decode's cast (model.py:129): values as given
    np.testing.assert_array_equal(O.sink_logits(sinks, "float32"), sinks.astype(np.float64))


# ---------------------------------------------------------------------------
# int4 group-64 GEMV


def _bf16_values(a):
    """float32 array rounded to bf16 values (kept as float32)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def _q4_problem(rng, M, N, K):
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = _bf16_values(rng.uniform(0.001, 0.05, size=(N, K // 64)))
    b = _bf16_values(rng.uniform(-0.3, 0.1, size=(N, K // 64)))
    x = _bf16_values(rng.standard_normal((M, K)))
    return x, w, s, b


def _dot16_form(x, w, s, b):
    """q4 / load16 / dot16 of engine/src/rec_mlx/kernels/megakernel.py:170-214
    taken literally: x divided by 1, 16, 256, 4096 by its place in each group
    of four, codes read with the masks 15, 240, 3840, 61440 from little-endian
    ushorts, s·a + sum·b per 16-element run (float64 here)."""
    M, K = x.shape
    N = w.shape[0]
    u16 = np.ascontiguousarray(w.astype("<u4")).view("<u2").reshape(N, K // 4).astype(np.int64)
    masks = np.array([15, 240, 3840, 61440], np.int64)
    div = np.tile(np.array([1.0, 16.0, 256.0, 4096.0]), 4)
    y = np.zeros((M, N))
    for run in range(K // 16):
        xs = x[:, 16 * run : 16 * run + 16].astype(np.float64)
        v = xs / div
        total = xs.sum(axis=1)
        a = np.zeros((M, N))
        for j in range(4):
            p = u16[:, 4 * run + j]
            for t in range(4):
                a += v[:, 4 * j + t][:, None] * (p & masks[t]).astype(np.float64)[None]
        gi = 16 * run // 64
        y += s[:, gi][None] * a + total[:, None] * b[:, gi][None]
    return y


def test_q4_unpack_order():
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    np.testing.assert_array_equal(O.q4_unpack(w)[0], np.arange(16))


def test_q4_gemv_matches_the_reference_dot16_form():
    rng = np.random.default_rng(21)
    x, w, s, b = _q4_problem(rng, 3, 40, 256)
    np.testing.assert_allclose(O.q4_gemv(x, w, s, b), _dot16_form(x, w, s, b), rtol=1e-12, atol=1e-12)


def test_q4_gemv_closed_forms():
    """One-hot x picks a column s·q + b; x = 1 gives Σ_g (s Σq + 64 b)."""
    rng = np.random.default_rng(22)
    _, w, s, b = _q4_problem(rng, 1, 24, 128)
    q = O.q4_unpack(w).astype(np.float64)
    for k in (0, 1, 63, 64, 127):
        x = np.zeros((1, 128))
        x[0, k] = 1.0
        np.testing.assert_array_equal(O.q4_gemv(x, w, s, b)[0], s[:, k // 64] * q[:, k] + b[:, k // 64])
    ones = O.q4_gemv(np.ones((1, 128)), w, s, b)[0]
    want = (s * q.reshape(24, 2, 64).sum(-1) + 64 * b).sum(-1)
    np.testing.assert_allclose(ones, want, rtol=1e-13)


def test_q4_planted_nibble_swap_is_caught():
    """A planted mistake (high/low nibble swapped) fails the dot16 pin."""
    rng = np.random.default_rng(23)
    x, w, s, b = _q4_problem(rng, 1, 16, 128)
    swapped = ((w & np.uint32(0x0F0F0F0F)) << np.uint32(4)) | ((w >> np.uint32(4)) & np.uint32(0x0F0F0F0F))
    assert not np.allclose(O.q4_gemv(x, swapped, s, b), _dot16_form(x, w, s, b), rtol=1e-6)


# ---------------------------------------------------------------------------
# MLX-style affine group-64 quantizer


def test_bf16_rn_and_round_half_away():
    x = np.random.default_rng(31).standard_normal(10000).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_rn(x), want)
    v = np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, -0.49999997, 3.0, -7.5], np.float32)
    np.testing.assert_array_equal(O.round_half_away(v), [1, -1, 2, 3, -3, 0, -0, 3, -8])


@pytest.mark.parametrize("bits", [8, 4])
def test_affine_closed_forms(bits):
    n = (1 << bits) - 1
    k = np.arange(64) % (n + 1) if bits == 4 else np.round(np.linspace(0, n, 64)).astype(np.int64)
    # levels 0 .. n of a step of 0.5, both ends present: codes n - k, scale -step, bias = max
    q, s, b = O.quantize_affine((0.5 * k).astype(np.float32)[None], bits)
    np.testing.assert_array_equal(q[0], n - k)
    assert s[0, 0] == -0.5 and b[0, 0] == 0.5 * n
    # the mirrored ramp: the negative edge wins, scale +step, bias = min
    q, s, b = O.quantize_affine((-0.5 * k).astype(np.float32)[None], bits)
    np.testing.assert_array_equal(q[0], n - k)
    assert s[0, 0] == 0.5 and b[0, 0] == -0.5 * n
    # constant and all-zero groups reconstruct to bf16 of the constant
    for c in (0.0, 3.3, -1.7):
        x = np.full((1, 64), c, np.float32)
        q, s, b = O.quantize_affine(x, bits)
        assert np.all(q == 0)
        np.testing.assert_array_equal(O.dequantize_affine(q, s, b), O.bf16_rn(x))


@pytest.mark.parametrize("bits", [8, 4])
def test_affine_error_bound_and_edges(bits):
    rng = np.random.default_rng(32 + bits)
    x = (rng.standard_normal((50, 128)) * rng.uniform(0.1, 10, (50, 1))).astype(np.float32)
    q, s, b = O.quantize_affine(x, bits)
    assert q.max() <= (1 << bits) - 1
    xh = O.dequantize_affine(q, s, b)
    g = x.reshape(50, 2, 64)
    # one step (the edge is made exact by stretching the step, so the far end
    # can be clamped by up to one code), plus the bf16 rounding of scale and bias
    slack = np.abs(s) * (1.0 + ((1 << bits) - 1) * 2.0**-8) + np.abs(b) * 2.0**-8
    err = np.abs(xh - x).reshape(50, 2, 64)
    assert np.all(err <= slack[..., None] * 1.001 + 1e-6)
    # the edge element (the larger-magnitude extreme, or the max when zero wins) is code 0
    w_min, w_max = g.min(-1), np.maximum(g.max(-1), 0)
    edge = np.where(np.abs(w_min) > np.abs(w_max), w_min, w_max)
    hit = (g == edge[..., None]) & (edge[..., None] != 0)
    assert np.all(q.reshape(50, 2, 64)[hit] == 0)
    # zero stays exact up to the bf16 rounding of scale and bias: the code of 0 is -q0
    q0 = O.round_half_away(edge / np.where(np.abs(w_min) > np.abs(w_max), 1, -1) / np.maximum((w_max - w_min) / ((1 << bits) - 1), 1e-7))
    assert np.all(np.abs(q0) <= (1 << bits) - 1)


@pytest.mark.parametrize("bits", [8, 4])
def test_affine_f16_metadata(bits):
    """fp16 scales and biases (the keys' dtype of an fp16 model, model.py:57-58):
    the codes are the bf16 variant's (the rounding comes after them), the values
    are fp16 numbers within half an ulp of fp16 and of bf16 of one float32
    source, and the reconstruction error has fp16's rounding slack."""
    n = (1 << bits) - 1
    rng = np.random.default_rng(61 + bits)
    x = (rng.standard_normal((40, 128)) * rng.uniform(0.1, 10, (40, 1))).astype(np.float32)
    q, s, b = O.quantize_affine(x, bits, meta="float16")
    qb, sb, bb = O.quantize_affine(x, bits)
    np.testing.assert_array_equal(q, qb)
    for v in (s, b):
        np.testing.assert_array_equal(v, v.astype(np.float16).astype(np.float32))
    assert not np.array_equal(s, sb)  # the two roundings differ somewhere
    assert np.all(np.abs(s - sb) <= np.abs(sb) * (2.0**-8 + 2.0**-11) * 1.0001)
    err = np.abs(O.dequantize_affine(q, s, b) - x).reshape(40, 2, 64)
    slack = np.abs(s) * (1.0 + n * 2.0**-11) + np.abs(b) * 2.0**-11
    assert np.all(err <= slack[..., None] * 1.001 + 1e-6)
    # the edge element (code 0, x̂ = bias) is the edge rounded once: to fp16
    # here, within 2^-11 of it, which bf16 metadata would miss
    g = x.reshape(40, 2, 64)
    w_min, w_max = g.min(-1), np.maximum(g.max(-1), 0)
    edge = np.where(np.abs(w_min) > np.abs(w_max), w_min, w_max)
    np.testing.assert_array_equal(b, edge.astype(np.float16).astype(np.float32))
    assert np.all(np.abs(b - edge) <= np.abs(edge) * 2.0**-11)
    assert np.any(np.abs(bb - edge) > np.abs(edge) * 2.0**-11)


def test_affine_planted_bias_sign_is_caught():
    x = (0.5 * (np.arange(64) % 16)).astype(np.float32)[None]
    q, s, b = O.quantize_affine(x, 4)
    assert not np.allclose(q * s.repeat(64, -1) - b.repeat(64, -1), x)  # wrong sign of the bias
    np.testing.assert_array_equal(O.dequantize_affine(q, s, b), x)


def _nearest_codes(x, s, b, n):
    """Brute force over every code 0..n: the code whose level b + k*s is
    nearest to x (float64), a tie going to the code farther from zero on the
    (x - b) / s axis (half away from zero; codes below 0 clamp to 0)."""
    k = np.arange(n + 1, dtype=np.float64)
    lv = b[..., None] + k * s[..., None]  # (..., n+1)
    d = np.abs(x[..., None].astype(np.float64) - lv)
    best = d.min(-1, keepdims=True)
    ties = d == best
    t = (x.astype(np.float64) - b) / s
    # among tied codes pick the largest when t >= 0, else the smallest
    idx = np.where(t >= 0, n - np.argmax(ties[..., ::-1], -1), np.argmax(ties, -1))
    return idx


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("sign", [1, -1])
def test_affine_codes_brute_force_exact_levels(bits, sign):
    """Groups whose scale and bias come out exactly (+-1 and the range end, so
    the stored bf16 values are the ones the codes were computed with) and
    whose elements sit on quarter steps, many on exact half-way points: every
    code is the nearest level, ties half away from zero (round-half-even
    would give the lower code at 12.5, 14.5, ...)."""
    n = (1 << bits) - 1
    rng = np.random.default_rng(77 + bits)
    groups = []
    for _ in range(20):
        quarters = rng.integers(0, 4 * n + 1, 62) / 4.0
        g = np.concatenate([[0.0, float(n)], quarters])
        groups.append(rng.permutation(g))
    x = (sign * np.array(groups)).astype(np.float32).reshape(10, 128)
    q, s, b = O.quantize_affine(x, bits)
    # the larger-magnitude end is n (sign +: scale -1, bias n) or -n (sign -: scale +1, bias -n)
    assert np.all(s == -sign) and np.all(b == sign * n)
    want = _nearest_codes(x.reshape(10, 2, 64), s[..., None].astype(np.float64), b[..., None].astype(np.float64), n)
    np.testing.assert_array_equal(q.reshape(10, 2, 64), want)
    halves = np.abs((x - sign * n) * 2 % 2) == 1
    assert halves.sum() > 100  # the draw exercises many exact ties


@pytest.mark.parametrize("bits", [8, 4])
def test_affine_codes_brute_force_random(bits):
    """Random groups (normal, heavy-tailed, one-signed, with an outlier): each
    code's level under the stored bf16 scale and bias is within the bf16
    rounding of those two of the best level any code gives (the codes were
    chosen under the float32 scale and bias, before that rounding)."""
    n = (1 << bits) - 1
    rng = np.random.default_rng(91 + bits)
    parts = [
        rng.standard_normal((40, 64)),
        rng.standard_t(3, (40, 64)),
        np.abs(rng.standard_normal((40, 64))) + 0.3,
        -np.abs(rng.standard_normal((40, 64))) - 0.3,
    ]
    x = np.concatenate(parts).astype(np.float32) * rng.uniform(0.01, 100, (160, 1)).astype(np.float32)
    x[::7, 5] *= 30.0
    x = x.reshape(80, 128)
    q, s, b = O.quantize_affine(x, bits)
    g = x.reshape(80, 2, 64).astype(np.float64)
    s64, b64 = s.astype(np.float64)[..., None], b.astype(np.float64)[..., None]
    mine = np.abs(g - (q.reshape(80, 2, 64) * s64 + b64))
    k = np.arange(n + 1, dtype=np.float64)
    best = np.abs(g[..., None] - (b64[..., None] + k * s64[..., None])).min(-1)
    # bf16 rounding moves each level k*s + b by up to 2^-8 (n|s| + |b|), so a
    # comparison of two levels by up to twice that
    slack = 2.0**-7 * (np.abs(s64) * n + np.abs(b64))
    assert np.all(mine <= best + slack)

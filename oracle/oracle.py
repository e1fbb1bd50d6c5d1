"""CPU restatement of rec's quantized-KV attention path — TEST INFRASTRUCTURE.

This module is the oracle the HIP kernels in ``rec_amd`` are checked against.
It is not part of the product: ``rec_amd`` never imports it, and only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg use it.  Everything is NumPy on logical layouts ``(B, H, T, D)``.

Reference semantics restated here (paths relative to the rec repository):

* quantize-on-append: ``engine/src/rec_mlx/model.py:45-82``
  (``MixedQuantizedKVCache.update_and_fetch``: quantize the new rows, write them
  at ``[prev:offset]``, attend over the cache *including* them).
* decode attention with sinks: ``engine/src/rec_mlx/model.py:108-139``
  (``quantized_attention_with_sinks``: scores = (q*scale)·k̂, optional mask,
  the per-head sink logit joins the softmax and is then dropped, out = P·v̂).
* sink logits per call site: the quantized decode casts the per-head offsets
  to float32 (``model.py:129``); the prefill branch over the quantized cache
  and the SDPA call over the bf16 caches hand them over in the query dtype
  (``sinks=self.softmax_offset.astype(q.dtype)``, ``model.py:202`` and
  ``:211``), as the fused decoder reads them as bf16
  (``kernels/megakernel.py:621,631``).  ``sink_logits`` / ``attention(...,
  sink_dtype=...)`` restate that rounding.
* masks: ``engine/src/rec_mlx/model.py:122-128`` ("causal" string →
  ``arange(kL-L, kL)[:, None] >= arange(kL)``; bool → where; float → add).
* split-K flash decode and merge: ``engine/src/rec_mlx/kernels/megakernel.py``
  ``:619-693`` (per-part (max, sum, acc) with the sink seeded once) and
  ``:276-318`` (merge: top = max m_p, z = Σ e^{m_p-top} l_p,
  out = Σ e^{m_p-top} acc_p / z, or acc when z == 0).
* chunked prefill over the quantized cache: ``engine/src/rec_mlx/model.py:191-203``.
* int4 group-64 GEMV of the decoder's projections:
  ``engine/src/rec_mlx/kernels/megakernel.py:161-232`` (``q4`` / ``dot16``:
  per run of 16 elements ``s·Σ q x + b·Σ x``, summed over the row) on MLX
  affine 4-bit matrices (``quantized.py:27-36``: group 64, bits 4).

KV formats.  The reference's own cache uses MLX affine group-64 quantization
(``model.py:77-78``); MLX is third-party (mlx==0.32.0) and cannot run here, so
byte parity with that layout is *not* claimed.  The formats below are this
project's specification, restated exactly so the GPU quantizer can be
compared bit-for-bit:

int8, symmetric, one fp16 scale per (token, head) row ``x[D]``::

    amax = max|x|                          (float32, exact)
    s16  = fp16_rn(amax / 127)             (IEEE float32 divide; overflow saturates to 65504)
    q    = clamp(rint(x / float(s16)), -127, 127)   (float32 divide, round-half-even)
    q    = 0 where s16 == 0
    x̂    = q * float(s16)

uint4, asymmetric, fp16 scale and integer-valued fp16 zero-point per group of
32 along D (two codes per byte, the low nibble holds the even element)::

    mn = min(0, min x), mx = max(0, max x)  (the range always contains 0)
    s16 = fp16_rn((mx - mn) / 15)          (saturating)
    z   = clamp(rint(-mn / float(s16)), 0, 15)   (stored as +0.0 when zero)
    q   = clamp(rint(x / float(s16)) + z, 0, 15)
    q = z = 0 where s16 == 0
    x̂   = (q - z) * float(s16)

MLX-style affine, group 64 (the reference's own KV format: ``mx.quantize``
with ``group_size=64``, 8-bit keys and 4-bit values, ``model.py:40-82``),
restated from MLX's published ``affine_quantize`` (mlx 0.32.0; MLX cannot run
here, so byte parity with MLX is not pinned) per group ``w[64]``::

    w_max = max(0, max w)      w_min = min w          (float32)
    scale = max((w_max - w_min) / n_bins, 1e-7)       n_bins = 2^bits - 1
    side  = |w_min| > |w_max|; scale = side ? scale : -scale
    edge  = side ? w_min : w_max
    q0    = round(edge / scale)                        (half away from zero)
    scale = q0 == 0 ? scale : edge / q0;  bias = q0 == 0 ? 0 : edge
    q     = min(round((w - bias) / scale), n_bins)     (codes 0 .. n_bins)
    scale, bias stored as bf16 (round to nearest even); x̂ = q · s_bf16 + b_bf16

Pinning (see ``tests/test_oracle.py``): the quantizers are checked against a
brute-force nearest-code search on small rows, closed forms (all-zero rows,
constant rows, the max element mapping to ±127) and invariants (symmetry,
|x̂ - x| ≤ s/2 inside the range); the attention functions against
``torch.nn.functional.scaled_dot_product_attention`` in float64 (sinks as an
extra zero key with an additive mask), the T = 1 closed form, identical-key and
permutation invariants, and split-merge over arbitrary partitions.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "FP16_MAX",
    "LOG2E",
    "fp16_rn_saturate",
    "quantize_int8",
    "dequantize_int8",
    "quantize_int4",
    "dequantize_int4",
    "pack_int4",
    "unpack_int4",
    "attention",
    "sink_logits",
    "split_k_decode",
    "split_k_decode_quantized",
    "causal_mask",
    "bf16_rn",
    "round_half_away",
    "quantize_affine",
    "dequantize_affine",
    "q4_unpack",
    "q4_dequantize",
    "q4_gemv",
]

FP16_MAX = np.float32(65504.0)
LOG2E = 1.4426950408889634


def fp16_rn_saturate(x):
    """Round float32 to fp16 (round-half-even); |overflow| saturates to 65504."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16)
    return np.where(np.isinf(h) & ~np.isinf(x), np.copysign(np.float16(65504), x).astype(np.float16), h)


def quantize_int8(x):
    """Symmetric int8 per row of the last axis.

    Restates the append-time quantization of ``model.py:77`` for this
    project's int8 format (module docstring).  Returns ``(codes int8 [..., D],
    scale fp16 [...])``.
    """
    xf = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(xf), axis=-1)
    s16 = fp16_rn_saturate(amax / np.float32(127.0))
    sf = s16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(xf / sf)
    q = np.clip(q, -127, 127)
    q = np.where(sf == 0, 0, q)
    return q.astype(np.int8), s16


def dequantize_int8(codes, scale):
    """x̂ = q · s in float32 (exact: 8-bit × 11-bit significands)."""
    return np.asarray(codes, np.float32) * np.asarray(scale, np.float16).astype(np.float32)[..., None]


def pack_int4(q):
    """Pack uint4 codes ``[..., D]`` two per byte; the low nibble is the even index."""
    q = np.asarray(q, dtype=np.uint8)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed):
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def quantize_int4(x, group=32):
    """Asymmetric uint4 with an fp16 scale and zero-point per ``group`` elements.

    Returns ``(codes uint8 [..., D/2], scale fp16 [..., D/group], zero fp16 [..., D/group])``.
    """
    xf = np.asarray(x, dtype=np.float32)
    D = xf.shape[-1]
    assert D % group == 0
    g = xf.reshape(xf.shape[:-1] + (D // group, group))
    mn = np.minimum(g.min(axis=-1), np.float32(0))
    mx = np.maximum(g.max(axis=-1), np.float32(0))
    s16 = fp16_rn_saturate((mx - mn) / np.float32(15.0))
    sf = s16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        z = np.clip(np.rint(-mn / sf), 0, 15) + np.float32(0.0)  # +0, never -0
        q = np.clip(np.rint(g / sf[..., None]) + z[..., None], 0, 15)
    z = np.where(sf == 0, 0, z)
    q = np.where(sf[..., None] == 0, 0, q)
    q = q.reshape(xf.shape).astype(np.uint8)
    return pack_int4(q), s16, z.astype(np.float16)


def dequantize_int4(packed, scale, zero, group=32):
    q = unpack_int4(packed).astype(np.float32)
    D = q.shape[-1]
    g = q.reshape(q.shape[:-1] + (D // group, group))
    s = np.asarray(scale, np.float16).astype(np.float32)[..., None]
    z = np.asarray(zero, np.float16).astype(np.float32)[..., None]
    return ((g - z) * s).reshape(q.shape)


def bf16_rn(x):
    """float32 -> nearest bf16 value (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)) << np.uint64(16)
    return r.astype(np.uint32).view(np.float32)


def round_half_away(x):
    """Round to the nearest integer, halves away from zero (exact in float32)."""
    x = np.asarray(x, dtype=np.float32)
    t = np.trunc(x)
    frac = x - t  # exact
    return (t + np.where(np.abs(frac) >= np.float32(0.5), np.sign(x), np.float32(0))).astype(np.float32)


def quantize_affine(x, bits, group=64, meta="bfloat16"):
    """MLX-style affine quantization of the last axis (module docstring).

    Returns ``(codes uint8 [..., D] (unpacked), scale [..., D/group],
    bias [..., D/group])``; scale and bias are ``meta`` values ("bfloat16" or
    "float16", the dtype the reference allocates them in: the keys' dtype,
    model.py:57-58) held in float32, rounded to nearest even once at the end.
    """
    xf = np.asarray(x, dtype=np.float32)
    D = xf.shape[-1]
    g = xf.reshape(xf.shape[:-1] + (D // group, group))
    n_bins = np.float32((1 << bits) - 1)
    w_max = np.maximum(g.max(axis=-1), np.float32(0))
    w_min = g.min(axis=-1)
    scale = np.maximum((w_max - w_min) / n_bins, np.float32(1e-7))
    side = np.abs(w_min) > np.abs(w_max)
    scale = np.where(side, scale, -scale)
    edge = np.where(side, w_min, w_max)
    q0 = round_half_away(edge / scale)
    at_zero = q0 == 0
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(at_zero, scale, edge / np.where(at_zero, np.float32(1), q0)).astype(np.float32)
    bias = np.where(at_zero, np.float32(0), edge).astype(np.float32)
    q = round_half_away((g - bias[..., None]) / scale[..., None])
    q = np.minimum(np.maximum(q, 0), n_bins)
    if meta == "float16":
        return (q.reshape(xf.shape).astype(np.uint8), scale.astype(np.float16).astype(np.float32),
                bias.astype(np.float16).astype(np.float32))
    return q.reshape(xf.shape).astype(np.uint8), bf16_rn(scale), bf16_rn(bias)


def dequantize_affine(codes, scale, bias, group=64):
    """x̂ = q · s + b per group, float32 (one rounding: the fma-free product then sum)."""
    q = np.asarray(codes, np.float32)
    D = q.shape[-1]
    s = np.repeat(np.asarray(scale, np.float32), group, axis=-1)
    b = np.repeat(np.asarray(bias, np.float32), group, axis=-1)
    return (q * s + b).reshape(q.shape[:-1] + (D,))


def causal_mask(L, T):
    """The "causal" string mask of ``model.py:124-125``: query i sits at T-L+i."""
    return np.arange(T - L, T)[:, None] >= np.arange(T)[None, :]


def _expand_mask(mask, L, T):
    if mask is None:
        return None
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask {mask!r}")
        return causal_mask(L, T)
    m = np.asarray(mask)
    if m.ndim > 3:  # (B, X, L, T) -> (B, X, 1, L, T), model.py:126-127
        m = np.expand_dims(m, -3)
    return m


def sink_logits(sinks, dtype="float32"):
    """The sink logits a softmax sees after the call site's cast, as float64.

    ``dtype`` is the type the call site casts the per-head offsets to:
    ``"float32"`` for the quantized decode (``model.py:129``:
    ``sinks.astype(mx.float32)``), the query dtype (``"bfloat16"`` or
    ``"float16"``) for the prefill branch over the quantized cache and for the
    SDPA call over the bf16 caches (``model.py:202,211``:
    ``softmax_offset.astype(q.dtype)``).  Rounding is to nearest even.
    """
    s = np.asarray(sinks, np.float32)
    if dtype == "float32":
        r = s
    elif dtype == "bfloat16":
        r = bf16_rn(s)
    elif dtype == "float16":
        r = s.astype(np.float16).astype(np.float32)
    else:
        raise ValueError(f"unknown sink dtype {dtype!r}")
    return np.asarray(r, np.float64)


def attention(q, k_hat, v_hat, scale, sinks=None, mask=None, sink_dtype=None):
    """Textbook GQA attention with sinks in float64.

    ``q`` is ``(B, Hq, L, D)``, ``k_hat``/``v_hat`` are dequantized
    ``(B, Hkv, T, D)``; q-head h reads kv-head ``h // (Hq // Hkv)``
    (``model.py:111-116``).  Returns ``(B, Hq, L, D)`` float64.  A row whose
    denominator is zero (every key masked and no sink) returns zeros, like the
    merge's ``z == 0`` branch (``megakernel.py:302-316``).  ``sink_dtype``,
    when given, first rounds the sinks as the call site does
    (:func:`sink_logits`); None takes them as given.
    """
    if sinks is not None and sink_dtype is not None:
        sinks = sink_logits(sinks, sink_dtype)
    q = np.asarray(q, np.float64)
    k = np.asarray(k_hat, np.float64)
    v = np.asarray(v_hat, np.float64)
    B, Hq, L, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qh = (q * scale).reshape(B, Hkv, G, L, D)
    s = np.einsum("bhgld,bhtd->bhglt", qh, k)
    m = _expand_mask(mask, L, T)
    if m is not None:
        s = np.where(m, s, -np.inf) if m.dtype == np.bool_ else s + m
    if sinks is None:
        sink = np.full((1, Hkv, G, 1, 1), -np.inf)
    else:
        sink = np.asarray(sinks, np.float64).reshape(1, Hkv, G, 1, 1)
    top = np.maximum(s.max(axis=-1, keepdims=True, initial=-np.inf), sink)
    top = np.where(np.isfinite(top), top, 0.0)
    p = np.exp(s - top)
    den = p.sum(axis=-1, keepdims=True) + np.exp(sink - top)
    num = np.einsum("bhglt,bhtd->bhgld", p, v)
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.where(den > 0, num / np.where(den > 0, den, 1.0), 0.0)
    return out.reshape(B, Hq, L, D)


def split_k_decode(q, k_hat_fn, v_hat_fn, T, scale, sinks=None, parts=None, chunk=4096, workers=None):
    """Split-K flash decode in float32 with a second merge pass.

    Follows ``megakernel.py:619-693`` (each part keeps a running max, a sum
    and an fp32 accumulator) and ``megakernel.py:276-318`` (the merge).  The
    sink enters the merge once, which equals seeding part 0 with
    ``hi = sink, z = 1`` as the reference kernel does.  ``k_hat_fn(a, b)`` and
    ``v_hat_fn(a, b)`` dequantize tokens ``[a, b)`` to float32
    ``(B, Hkv, b-a, D)``, so the whole cache is never materialised.
    Parts are contiguous token ranges of ``chunk`` tokens (the CPU analogue of
    the GPU's splits), computed on ``workers`` threads when given.  Returns
    ``(B, Hq, D)`` float32.
    """
    q = np.asarray(q, np.float32)
    B, Hq, D = q.shape
    kb = k_hat_fn(0, min(T, 1))
    Hkv = kb.shape[1]
    G = Hq // Hkv
    qh = (q * np.float32(scale)).reshape(B, Hkv, G, D)
    bounds = list(range(0, T, chunk)) if parts is None else list(parts)
    bounds = [b for b in bounds if b < T] + [T]

    def part(ab):
        a, b = ab
        k = k_hat_fn(a, b)
        v = v_hat_fn(a, b)
        s = np.matmul(qh, k.transpose(0, 1, 3, 2))  # (B, Hkv, G, n)
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        return m[..., 0], p.sum(axis=-1), np.matmul(p, v)  # acc (B, Hkv, G, D)

    ranges = list(zip(bounds[:-1], bounds[1:]))
    if workers and workers > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(workers) as ex:
            parts_out = list(ex.map(part, ranges))
    else:
        parts_out = [part(r) for r in ranges]
    m = np.stack([x[0] for x in parts_out], 0)
    l = np.stack([x[1] for x in parts_out], 0)
    acc = np.stack([x[2] for x in parts_out], 0)
    top = m.max(axis=0)
    if sinks is not None:
        sink = np.asarray(sinks, np.float32).reshape(1, Hkv, G)
        top = np.maximum(top, sink)
    w = np.exp(m - top[None])
    z = (w * l).sum(axis=0)
    if sinks is not None:
        z = z + np.exp(sink - top)
    num = (w[..., None] * acc).sum(axis=0)
    out = np.where(z[..., None] == 0, num, num / np.where(z == 0, 1, z)[..., None])
    return out.reshape(B, Hq, D).astype(np.float32)


def split_k_decode_quantized(q, cache, T, scale, sinks=None, chunk=4096, workers=None):
    """``split_k_decode`` over a logical quantized cache dict.

    ``cache`` holds ``k_bits``/``v_bits`` and logical arrays ``kq, ks[, kz]``
    and ``vq, vs[, vz]`` of shape ``(B, Hkv, T, ...)``; dequantization happens
    per chunk, as the CPU baseline does.
    """

    def deq(prefix, bits):
        def fn(a, b):
            if bits == 8:
                return dequantize_int8(cache[prefix + "q"][:, :, a:b], cache[prefix + "s"][:, :, a:b])
            return dequantize_int4(
                cache[prefix + "q"][:, :, a:b], cache[prefix + "s"][:, :, a:b], cache[prefix + "z"][:, :, a:b]
            )

        return fn

    return split_k_decode(
        q, deq("k", cache["k_bits"]), deq("v", cache["v_bits"]), T, scale, sinks, chunk=chunk, workers=workers
    )


# ---------------------------------------------------------------------------
# int4 group-64 GEMV (engine/src/rec_mlx/kernels/megakernel.py:161-232)


def q4_unpack(w):
    """MLX 4-bit words ``(N, K/8)`` uint32 -> codes ``(N, K)`` uint8.

    Code ``e`` of a word sits at bits ``4e``: ``dot16`` reads the same order
    through little-endian ushorts, element ``4j + t`` of a 16-element run at
    bits ``4t`` of ushort ``j`` (``megakernel.py:189-195``).
    """
    w = np.asarray(w).astype(np.uint32)
    shifts = np.arange(8, dtype=np.uint32) * np.uint32(4)
    return ((w[..., None] >> shifts) & np.uint32(15)).astype(np.uint8).reshape(w.shape[0], -1)


def q4_dequantize(w, scales, biases, group=64):
    """Element ``(r, k)`` of the matrix: ``s[r, k // 64] * q + b[r, k // 64]`` in float64."""
    q = q4_unpack(w).astype(np.float64)
    s = np.repeat(np.asarray(scales, np.float64), group, axis=1)
    b = np.repeat(np.asarray(biases, np.float64), group, axis=1)
    return s * q + b


def q4_gemv(x, w, scales, biases, group=64):
    """``y[m, r] = Σ_g s[r, g] Σ_{k∈g} q[r, k] x[m, k] + b[r, g] Σ_{k∈g} x[m, k]``.

    ``x`` is ``(M, K)`` (bf16 values), ``w`` ``(N, K/8)`` uint32, ``scales`` and
    ``biases`` ``(N, K/64)`` (bf16 values).  Float64; the reference sums the
    same terms in float32 and stores bfloat16 (``megakernel.py:198-214``).
    """
    x = np.asarray(x, np.float64)
    return x @ q4_dequantize(w, scales, biases, group).T

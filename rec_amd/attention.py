"""Attention over the quantized cache, with the reference's call surface.

* :func:`quantized_attention_with_sinks` keeps the signature of
  engine/src/rec_mlx/model.py:108-110 and runs the gfx950 split-K decode kernel
  (``rec_decode_attn``) for one query token, the chunked prefill kernel for
  several (model.py:191-203: ``rec_prefill_attn`` reads every cache format
  directly, dequantizing tiles on chip, and applies sliding-window masks, also
  for a single windowed query).
* :func:`attend` mirrors the cache/attention part of ``Attention.__call__``
  (model.py:177-203): append first, then attend, decode for ``L == 1`` and
  chunked prefill for ``L > 1``.  For a
  single decode token it issues ONE launch (``rec_decode_append_attn``) that
  quantizes the new token into the cache and attends over it.

There is no CPU path: without the built HIP library every call raises.
"""

from __future__ import annotations

import threading
import weakref
from typing import Optional

import torch

from . import _lib
from .cache import _DTYPES, HEAD_DIM, QuantizedKV, QuantizedKVCache
from .kvstorage import FixedKVCache, FixedSlidingKVCache

_ws_lock = threading.Lock()
_workspaces = {}


def workspace(device: torch.device, B: int, Hkv: int, splits: int, stream: int) -> torch.Tensor:
    """The decode workspace (split partials) for (device, stream), grown on
    demand.  One workspace per stream: launches on one stream are ordered, so
    one step's partials are merged before the next step overwrites them.
    """
    lib = _lib.load()
    need = lib.rec_decode_workspace_bytes(B, Hkv, splits)
    key = (device.index, stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.zeros(need, dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


def _rows_aligned(t: torch.Tensor) -> bool:
    """Rows the kernels read with vector loads: unit dim stride, 16-byte
    aligned start, other strides multiples of 4 elements."""
    return (
        t.stride(-1) == 1
        and t.data_ptr() % 16 == 0
        and all(s % 4 == 0 for s in t.stride()[:-1])
    )


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


_sink_lock = threading.Lock()
_sink_copies = {}  # id(sinks tensor) -> (weak reference to it, (version, dtype, device), rounded copy)


def _forget_sinks(i):
    def drop(_ref):
        with _sink_lock:
            _sink_copies.pop(i, None)
    return drop


def _sinks(sinks, Hq, device, dtype=None):
    """The per-head sink logits as a float32 device vector, first rounded to
    ``dtype`` when that is a 16-bit float type.

    The reference casts the offsets to float32 in the quantized decode
    (engine/src/rec_mlx/model.py:129) and to the query dtype where it calls
    the fused SDPA (model.py:202, :211); ``attend`` passes the query dtype for
    those paths.  A rounded copy is made once per tensor and in-place version
    (kept while the tensor lives), so decode steps launch no cast kernel; a
    copy first needed under HIP-graph capture is made inside the graph and not
    kept (its bytes exist only once the graph runs).
    """
    if sinks is None:
        return None
    if dtype not in (torch.bfloat16, torch.float16):
        s = torch.as_tensor(sinks, device=device).to(torch.float32).reshape(-1).contiguous()
    else:
        key = None
        if isinstance(sinks, torch.Tensor):
            key = (sinks._version, dtype, torch.device(device))
            with _sink_lock:
                hit = _sink_copies.get(id(sinks))
            if hit is not None and hit[0]() is sinks and hit[1] == key and hit[2].numel() == Hq:
                return hit[2]
        s = torch.as_tensor(sinks, device=device).to(dtype).to(torch.float32).reshape(-1).contiguous()
        if key is not None and not (s.is_cuda and torch.cuda.is_current_stream_capturing()):
            i = id(sinks)
            with _sink_lock:
                _sink_copies[i] = (weakref.ref(sinks, _forget_sinks(i)), key, s)
    if s.numel() != Hq:
        raise ValueError(f"sinks has {s.numel()} entries, expected {Hq}")
    return s


def _new_out(shape, out_dtype, queries):
    """The output tensor the kernels write: the requested dtype (default: the
    query dtype, as the reference returns) when it is one they store (fp32,
    bf16, fp16, rounded to nearest even in the kernel), else fp32 converted
    by the caller (:func:`_finish`)."""
    want = out_dtype or queries.dtype
    dt = want if want in _DTYPES else torch.float32
    return torch.empty(shape, dtype=dt, device=queries.device), want


def _finish(out, want):
    return out if out.dtype == want else out.to(want)


def _check_query(queries):
    if queries.dim() != 4:
        raise ValueError(f"queries must be (B, n_heads, L, head_dim), got {tuple(queries.shape)}")
    if queries.dtype not in _DTYPES:
        raise ValueError(f"queries dtype {queries.dtype} is not float16/bfloat16/float32")
    if not queries.is_cuda:
        raise ValueError("queries must be a GPU tensor")
    if queries.shape[-1] != HEAD_DIM:
        raise NotImplementedError(f"head_dim {queries.shape[-1]} is not supported (128 only)")


def _check_cache_shapes(queries, keys: QuantizedKV, values: QuantizedKV):
    """The kernels index the cache by (batch, KV head) from the query shape
    and cannot see tensor sizes: refuse a batch or head count the cache does
    not hold before anything is launched."""
    B, Hq = queries.shape[:2]
    kb, kh = keys.codes.shape[:2]
    if tuple(values.codes.shape[:2]) != (kb, kh) or values.length != keys.length:
        raise ValueError(f"keys (B={kb}, Hkv={kh}, T={keys.length}) and values (B={values.codes.shape[0]}, "
                         f"Hkv={values.codes.shape[1]}, T={values.length}) do not match")
    if B != kb:
        raise ValueError(f"queries have batch {B}, the cache holds {kb}")
    if Hq % kh != 0:
        raise ValueError(f"{Hq} query heads is not a multiple of the cache's {kh} KV heads")


def _decode_launch(queries, keys: QuantizedKV, values: QuantizedKV, scale, sinks, splits, out,
                   k_new=None, v_new=None, T=None, capacity=None, sink_dtype=None, bias=None):
    lib = _lib.load()
    B, Hq, L, D = queries.shape
    Hkv = keys.n_kv_heads
    T = keys.length if T is None else T
    capacity = keys.capacity if capacity is None else capacity
    q = queries[:, :, 0]
    if not _rows_aligned(q):
        q = q.contiguous()
    dev = queries.device
    stream = torch.cuda.current_stream(dev).cuda_stream
    if splits is None or splits <= 0:
        splits = lib.rec_decode_default_splits(B, Hkv, T)
    ws = workspace(dev, B, Hkv, splits, stream)
    sk = _sinks(sinks, Hq, dev, sink_dtype)
    shape_tail = (
        B, Hq, Hkv, D, int(T), int(capacity), int(splits),
        ws.data_ptr(), ws.numel(), _DTYPES[out.dtype], out.data_ptr(), stream,
    )
    common_tail = (_ptr(sk), float(scale), *shape_tail)
    if k_new is None:
        rc = lib.rec_decode_attn(
            q.data_ptr(), _DTYPES[q.dtype], q.stride(0), q.stride(1),
            keys.code, keys.codes.data_ptr(), keys.scales.data_ptr(), _ptr(keys.zeros),
            values.code, values.codes.data_ptr(), values.scales.data_ptr(), _ptr(values.zeros),
            _ptr(sk), float(scale), *_bias_args(bias, True), *shape_tail,
        )
        _lib.check(rc, "rec_decode_attn")
    else:
        rc = lib.rec_decode_append_attn(
            q.data_ptr(), _DTYPES[q.dtype], q.stride(0), q.stride(1),
            k_new.data_ptr(), v_new.data_ptr(), _DTYPES[k_new.dtype],
            k_new.stride(0), k_new.stride(1), v_new.stride(0), v_new.stride(1),
            keys.code, keys.codes.data_ptr(), keys.scales.data_ptr(), _ptr(keys.zeros),
            values.code, values.codes.data_ptr(), values.scales.data_ptr(), _ptr(values.zeros),
            *common_tail,
        )
        _lib.check(rc, "rec_decode_append_attn")


def prefill_workspace(device: torch.device, B: int, Hq: int, Hkv: int, L: int, splits: int,
                      stream: int) -> torch.Tensor:
    """The prefill workspace (key-split partials) for (device, stream), grown on
    demand; an empty tensor when the launch does not split.  Kept apart from the
    decode workspace: a chunk's prefill and the decode steps after it may
    interleave on one stream, but each launch pair (partials, merge) is ordered."""
    lib = _lib.load()
    need = lib.rec_prefill_workspace_bytes(B, Hq, Hkv, L, splits)
    key = ("prefill", device.index, stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


def _prefill_launch(queries, keys: QuantizedKV, values: QuantizedKV, scale, sinks, causal, out, splits=0, window=0,
                    sink_dtype=None, bias=None):
    lib = _lib.load()
    B, Hq, L, D = queries.shape
    q = queries if queries.stride(-1) == 1 else queries.contiguous()
    dev = queries.device
    sk = _sinks(sinks, Hq, dev, sink_dtype)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = prefill_workspace(dev, B, Hq, keys.n_kv_heads, L, splits, stream)
    rc = lib.rec_prefill_attn(
        q.data_ptr(), _DTYPES[q.dtype], q.stride(0), q.stride(1), q.stride(2),
        keys.code, keys.codes.data_ptr(), keys.scales.data_ptr(), _ptr(keys.zeros),
        values.code, values.codes.data_ptr(), values.scales.data_ptr(), _ptr(values.zeros),
        _ptr(sk), float(scale), int(causal), int(window), *_bias_args(bias, False),
        B, Hq, keys.n_kv_heads, D, L, int(keys.length),
        int(keys.capacity),
        int(splits), ws.data_ptr(), ws.numel(), _DTYPES[out.dtype], out.data_ptr(), stream,
    )
    _lib.check(rc, "rec_prefill_attn")


def dequantize_kv(keys: QuantizedKV, values: QuantizedKV):
    """bf16 ``(B, Hkv, T, 128)`` copies of the ``T = keys.length`` valid cache
    rows (x̂ in float32 from the stored codes, scales, zeros or biases, then
    rounded to bf16), as the reference's prefill branch dequantizes its cache
    before attention (engine/src/rec_mlx/model.py:194-195)."""
    lib = _lib.load()
    B, Hkv, T = keys.codes.shape[0], keys.n_kv_heads, int(keys.length)
    dev = keys.codes.device
    k = torch.empty((B, Hkv, T, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    rc = lib.rec_kv_dequant_bf16(
        keys.code, keys.codes.data_ptr(), keys.scales.data_ptr(), _ptr(keys.zeros),
        values.code, values.codes.data_ptr(), values.scales.data_ptr(), _ptr(values.zeros),
        B, Hkv, T, int(keys.capacity), k.data_ptr(), v.data_ptr(), torch.cuda.current_stream(dev).cuda_stream,
    )
    _lib.check(rc, "rec_kv_dequant_bf16")
    return k, v


MAX_GROUP = 8  # query heads per KV head that one launch holds (the MFMA columns)


def _head_groups(queries, sinks, mask, Hkv, call):
    """A GQA ratio G above MAX_GROUP: the G query heads of every KV head in
    groups of at most MAX_GROUP, one call each, outputs put back in head
    order.  ``call(q, sinks, mask)`` attends for one group (its queries
    ``(B, Hkv * g, L, D)``).  A mask broadcasts over the group's heads
    (model.py:126-127 gives a four-dimensional one a group axis); a
    three-dimensional one whose first extent is G is the per-head mask of the
    group and is sliced with it."""
    B, Hq, L, D = queries.shape
    G = Hq // Hkv
    qv = queries.reshape(B, Hkv, G, L, D)
    sv = None if sinks is None else torch.as_tensor(sinks, device=queries.device).reshape(Hkv, G)
    per_head = not isinstance(mask, str) and mask is not None and torch.as_tensor(mask).dim() == 3 \
        and torch.as_tensor(mask).shape[0] == G
    outs = []
    for g0 in range(0, G, MAX_GROUP):
        g1 = min(G, g0 + MAX_GROUP)
        q = qv[:, :, g0:g1].reshape(B, Hkv * (g1 - g0), L, D)
        sk = None if sv is None else sv[:, g0:g1].reshape(-1)
        m = mask[g0:g1] if per_head else mask
        outs.append(call(q, sk, m).reshape(B, Hkv, g1 - g0, L, D))
    return torch.cat(outs, dim=2).reshape(B, Hq, L, D)


def quantized_attention_with_sinks(
    queries, keys, values, scale, mask, sinks, group_size, key_bits, value_bits, *, out_dtype=None, splits=None,
    sink_dtype=None,
):
    """GQA attention of ``queries`` ``(B, n_q, L, 128)`` over a quantized cache.

    ``keys``/``values`` are what :meth:`QuantizedKVCache.update_and_fetch`
    returns; ``sinks`` (``n_q`` logits or None) join the softmax denominator;
    ``mask`` is None, "causal", or a boolean or additive float array with the
    reference's broadcasting against the scores (model.py:122-128: a
    four-dimensional mask is ``(B, n_kv, L, T)``): host arrays holding the
    causal or causal sliding-window pattern take those kernels' own masking
    (:func:`_mask_plan`), any other array is added to the scores as a bias
    inside the kernels (:func:`_mask_bias`; padding masks of a ragged batch,
    per-head masks, finite additive masks).  ``L == 1`` runs the split-K
    decode kernel (a window pattern as a bias over the keys); ``L > 1``
    (bf16/f16 queries, the newest ``L`` cached tokens) the chunked prefill
    kernel, which reads every cache format directly (4-bit and affine values
    rounded to the query dtype, as the reference dequantizes, int8 codes
    exactly) and applies a sliding-window pattern itself; float32 queries
    take one decode per query row (:func:`_rows_as_decodes`).  Returns ``(B, n_q, L, 128)`` in ``out_dtype``
    (default: the query dtype, as the reference returns, model.py:132-139).
    The sinks enter as float32 values at every ``L``, the cast this function
    makes in the reference (model.py:129); ``sink_dtype`` (bf16/f16) rounds
    them first, as the reference's prefill branch hands its SDPA the offsets
    in the query dtype (model.py:202) -- :func:`attend` passes it for chunks.
    """
    _check_query(queries)
    B, Hq, L, D = queries.shape
    if not isinstance(keys, QuantizedKV) or not isinstance(values, QuantizedKV):
        raise TypeError("keys/values must come from QuantizedKVCache.update_and_fetch")
    if (keys.bits, values.bits) != (key_bits, value_bits):
        raise ValueError(f"cache holds {keys.bits}/{values.bits}-bit K/V, call asked for {key_bits}/{value_bits}")
    if keys.affine != values.affine or keys.affine != (group_size == 64):
        raise ValueError(f"group_size={group_size} does not match the cache's format")
    if not keys.affine and 4 in (key_bits, value_bits) and group_size != 32:
        raise ValueError(f"4-bit caches use groups of 32, got group_size={group_size}")
    _check_cache_shapes(queries, keys, values)
    if L > keys.length:  # the L queries are the newest L cached tokens (model.py:122-125)
        raise ValueError(f"{L} queries but only {keys.length} cached tokens")
    Hkv = keys.n_kv_heads
    if Hq // Hkv > MAX_GROUP:
        return _head_groups(queries, sinks, mask, Hkv, lambda q, sk, m: quantized_attention_with_sinks(
            q, keys, values, scale, m, sk, group_size, key_bits, value_bits, out_dtype=out_dtype, splits=splits,
            sink_dtype=sink_dtype))
    T = int(keys.length)
    causal, win, bias = _resolve_mask(mask, B, Hkv, Hq // Hkv, L, T, queries.device)
    if L == 1 and win:
        # one query under a window: the decode kernel with the window as a
        # bias over the keys (-inf before the last `win`), the reference's
        # single-query arithmetic on the exact dequantized values (model.py:108-139)
        keep = torch.full((1, T), float("-inf"), dtype=torch.float32, device=queries.device)
        keep[:, T - win:] = 0.0
        bias, win = _mask_bias(keep, B, Hkv, Hq // Hkv, 1, T, queries.device), 0
    if L == 1:
        out, want = _new_out((B, Hq, D), out_dtype, queries)
        _decode_launch(queries, keys, values, scale, sinks, splits, out, sink_dtype=sink_dtype, bias=bias)
        out = out.view(B, Hq, 1, D)
    elif queries.dtype == torch.float32:
        return _rows_as_decodes(
            queries, T, Hkv, causal, win, bias, out_dtype,
            lambda q, t, o, b: _decode_launch(q, keys, values, scale, sinks, splits, o, T=t, sink_dtype=sink_dtype,
                                              bias=b))
    else:
        out, want = _new_out((B, Hq, L, D), out_dtype, queries)
        _prefill_launch(queries, keys, values, scale, sinks, causal, out, splits or 0, win, sink_dtype, bias)
    return _finish(out, want)


def _bf16_kv_ok(t: torch.Tensor) -> bool:
    return t.dtype == torch.bfloat16 and t.is_cuda and t.stride(-1) == 1 and t.stride(-2) == HEAD_DIM


def _bf16_decode_launch(queries, keys, values, scale, sinks, splits, out, k_new=None, v_new=None, T=None,
                        capacity=None, slot=None, sink_dtype=None, bias=None):
    lib = _lib.load()
    B, Hq, L, D = queries.shape
    Hkv = keys.shape[1]
    T = keys.shape[2] if T is None else T
    capacity = T if capacity is None else capacity
    q = queries[:, :, 0]
    if not _rows_aligned(q):
        q = q.contiguous()
    dev = queries.device
    stream = torch.cuda.current_stream(dev).cuda_stream
    # the library picks the plan when splits is 0 (a short cache runs one
    # workgroup per KV head and needs no partials); the workspace covers the
    # default split plan
    splits = 0 if splits is None or splits <= 0 else int(splits)
    ws = workspace(dev, B, Hkv, splits or lib.rec_decode_default_splits(B, Hkv, T), stream)
    sk = _sinks(sinks, Hq, dev, sink_dtype)
    if k_new is None:
        new = (None, None, _lib.REC_BF16, 0, 0, 0, 0)
    else:
        new = (k_new.data_ptr(), v_new.data_ptr(), _DTYPES[k_new.dtype], k_new.stride(0), k_new.stride(1),
               v_new.stride(0), v_new.stride(1))
    head = (q.data_ptr(), _DTYPES[q.dtype], q.stride(0), q.stride(1), *new,
            keys.data_ptr(), keys.stride(0), keys.stride(1), values.data_ptr(), values.stride(0), values.stride(1),
            _ptr(sk), float(scale))
    shape = (B, Hq, Hkv, D, int(T), int(capacity))
    tail = (int(splits), ws.data_ptr(), ws.numel(), _DTYPES[out.dtype], out.data_ptr(), stream)
    if slot is None:
        _lib.check(lib.rec_decode_bf16(*head, *_bias_args(bias, True), *shape, *tail), "rec_decode_bf16")
    else:  # a ring step: the new token goes to `slot`
        _lib.check(lib.rec_decode_bf16_ring(*head, *shape, int(slot), *tail), "rec_decode_bf16_ring")


def _bf16_prefill_launch(queries, keys, values, scale, sinks, causal, window, out, splits=0, sink_dtype=None,
                         bias=None):
    lib = _lib.load()
    B, Hq, L, D = queries.shape
    Hkv, T = keys.shape[1], keys.shape[2]
    if queries.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError("prefill queries must be bf16 or f16 (the matrix-core input type)")
    dev = queries.device
    sk = _sinks(sinks, Hq, dev, sink_dtype)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = prefill_workspace(dev, B, Hq, Hkv, L, splits, stream)
    rc = lib.rec_prefill_bf16(
        queries.data_ptr(), _DTYPES[queries.dtype], queries.stride(0), queries.stride(1), queries.stride(2),
        keys.data_ptr(), keys.stride(0), keys.stride(1), values.data_ptr(), values.stride(0), values.stride(1),
        _ptr(sk), float(scale), int(causal), int(window), *_bias_args(bias, False), B, Hq, Hkv, D, L, T,
        int(splits), ws.data_ptr(),
        ws.numel(), _DTYPES[out.dtype], out.data_ptr(), stream,
    )
    _lib.check(rc, "rec_prefill_bf16")


def _is_host(mask) -> bool:
    return not (isinstance(mask, torch.Tensor) and mask.device.type != "cpu")


def _mask_plan(mask, L, T):
    """The fast pattern of a host-resident ``mask`` for ``L`` queries at
    positions ``T - L .. T - 1`` over ``T`` keys: ``(causal, window)``, or
    None when the array holds another pattern (it then runs as a bias,
    :func:`_mask_bias`).

    The reference's rules (model.py:122-128): None keeps every key; "causal"
    keeps keys at or before each query's position; a boolean array keeps the
    keys where it is True; a float array is added to the scores (here a
    pattern only when it holds just 0 and -inf).  Three patterns have kernels
    of their own: every key ``(False, 0)``, causal ``(True, 0)``, and causal
    limited to the last ``window`` keys ``(True, window)``
    (engine/src/rec_mlx/cache.py:199-205).  Host arrays are checked here, on
    the host; device arrays are not inspected (that would wait for the GPU,
    and could not run under HIP-graph capture): they always run as a bias.
    """
    if mask is None:
        return False, 0
    if isinstance(mask, str):
        if mask != "causal":
            raise NotImplementedError(f"mask {mask!r} is not supported")
        return True, 0
    if not _is_host(mask):
        return None
    m = torch.as_tensor(mask)
    if m.dtype == torch.bool:
        keep = m
    elif m.is_floating_point():
        if not bool(((m == 0) | (m == float("-inf"))).all()):
            return None
        keep = m == 0
    else:
        raise NotImplementedError(f"mask dtype {m.dtype} is not supported (bool or float)")
    if keep.dim() > 4:
        raise NotImplementedError(f"masks of {keep.dim()} dimensions are not supported (at most 4)")
    if keep.dim() == 0 or keep.shape[-1] not in (1, T) or (keep.dim() >= 2 and keep.shape[-2] not in (1, L)):
        raise ValueError(f"mask of shape {tuple(m.shape)} does not broadcast to ({L}, {T})")
    while keep.dim() > 2:  # leading (head, batch) dims: a pattern only if every slice is alike
        if not bool((keep == keep[:1]).all()):
            return None
        keep = keep[0]
    if keep.dim() < 2:
        keep = keep.reshape(1, -1)
    keep = keep.expand(L, T)
    if bool(keep.all()):
        return False, 0
    q = torch.arange(T - L, T)[:, None]
    k = torch.arange(T)[None]
    causal = q >= k
    if torch.equal(keep, causal):
        return True, 0
    window = int(keep[-1].sum())
    if window > 0 and torch.equal(keep, causal & (q < k + window)):
        return True, window
    return None


def _mask_bias(mask, B, Hkv, G, L, T, device):
    """``mask`` as the additive score bias the kernels read: ``(tensor,
    (sb, skv, sg, sl, extent))``.

    As the reference (model.py:122-128): a boolean mask keeps the keys where
    it is True (bias 0, else -inf), a float mask is added to the scores; the
    mask broadcasts against the scores ``(B, Hkv, G, L, T)`` (G query heads
    per KV head) after a mask of four dimensions ``(B, Hkv, L, T)`` gains a
    group axis (``expand_dims(mask, -3)``).  The bias keeps the mask's own
    extents (strides 0 where it broadcasts), as float32 with the key axis
    padded to a multiple of 4 and 16-byte aligned rows: one copy on the
    device, no host synchronisation.
    """
    m = torch.as_tensor(mask, device=device)
    if m.dtype == torch.bool:
        m = torch.where(m, 0.0, float("-inf")).to(torch.float32)
    elif m.is_floating_point():
        m = m.to(torch.float32)
    else:
        raise NotImplementedError(f"mask dtype {m.dtype} is not supported (bool or float)")
    if m.dim() > 4:
        raise NotImplementedError(f"masks of {m.dim()} dimensions are not supported (at most 4)")
    if m.dim() == 4:
        m = m.unsqueeze(-3)
    while m.dim() < 5:
        m = m.unsqueeze(0)
    try:
        m.expand(B, Hkv, G, L, T)
    except RuntimeError:
        raise ValueError(f"mask of shape {tuple(mask.shape)} does not broadcast to the scores "
                         f"({B}, {Hkv}, {G}, {L}, {T})") from None
    lead = tuple(m.shape[:4])
    Tp = (T + 3) // 4 * 4
    buf = torch.empty(lead + (Tp,), dtype=torch.float32, device=device)
    buf[..., :T] = m.expand(lead + (T,))
    st = [buf.stride(i) if lead[i] > 1 else 0 for i in range(4)]
    if buf.numel() >= 1 << 29:
        raise NotImplementedError(f"a mask of {buf.numel()} elements is not supported (below 2^29)")
    return buf, (st[0], st[1], st[2], st[3], buf.numel())


def _resolve_mask(mask, B, Hkv, G, L, T, device):
    """``(causal, window, bias)`` for the kernels: a fast pattern
    (:func:`_mask_plan`) with ``bias`` None, or ``(False, 0, bias)`` with the
    bias of any other mask array (:func:`_mask_bias`)."""
    plan = _mask_plan(mask, L, T)
    if plan is not None:
        return plan[0], plan[1], None
    return False, 0, _mask_bias(mask, B, Hkv, G, L, T, device)


def _bias_args(bias, decode):
    """The bias arguments of a launch: pointer, strides (b, kv head, group
    member[, query]) and extent, or all zero."""
    if bias is None:
        return (None, 0, 0, 0, 0) if decode else (None, 0, 0, 0, 0, 0)
    t, (sb, skv, sg, sl, ext) = bias
    return (t.data_ptr(), sb, skv, sg, ext) if decode else (t.data_ptr(), sb, skv, sg, sl, ext)


def _rows_as_decodes(queries, T, Hkv, causal, window, bias, out_dtype, decode_one):
    """A chunk of float32 queries, each query row as one decode.

    The matrix-core prefill takes bf16 / fp16 operands; the reference's SDPA
    also takes float32 queries (model.py:196-203, 211), the cache then
    dequantized to float32.  The decode kernels attend with float32 queries
    over the exact dequantized values, so query ``i`` of the ``L`` runs as a
    decode over the keys it sees: the first ``T - L + i + 1`` under a causal
    mask, a sliding window or a mask array as that query's bias row.
    ``decode_one(q_i, T_i, out_i, bias_i)`` launches one of them; ``L``
    launch pairs instead of one launch, for float32 models, not for speed.
    """
    B, Hq, L, D = queries.shape
    dev = queries.device
    out, want = _new_out((L, B, Hq, D), out_dtype, queries)
    if window:
        # The causal window (always with the causal limit) as a bias, without
        # an (L, T) array: query i sees d = L - 1 - i keys fewer than the last
        # one and keeps key t iff t + d >= T - window, so its row is base[d:]
        # with base[j] = 0 from j = T - window on, else -inf.  Four copies of
        # base shifted by 0-3 keep every row start 16-byte aligned (row i is
        # copy d % 4 from element 4 (d // 4) on).
        Tp = (T + 3) // 4 * 4
        j = torch.arange(Tp, device=dev)[None] + torch.arange(4, device=dev)[:, None]
        flat = torch.where(j >= T - window, 0.0, float("-inf")).to(torch.float32).reshape(-1).contiguous()

        def row(i):
            d = L - 1 - i
            off = (d % 4) * Tp + d // 4 * 4
            return flat[off:], (0, 0, 0, 0, 4 * Tp - off)
    elif bias is not None:
        t, (sb, skv, sg, sl, ext) = bias
        flat = t.view(-1)

        def row(i):  # row i of the bias: 16-byte aligned (sl is a multiple of 4 elements)
            return flat[i * sl:], (sb, skv, sg, sl, ext - i * sl)
    else:
        def row(i):
            return None
    for i in range(L):
        decode_one(queries[:, :, i:i + 1], T - L + i + 1 if causal else T, out[i], row(i))
    return _finish(out.permute(1, 2, 0, 3).contiguous(), want)


def scaled_dot_product_attention(queries, keys, values, scale, mask=None, sinks=None, *, out_dtype=None,
                                 splits=None, window=None, sink_dtype=None):
    """Attention of ``queries`` ``(B, n_q, L, 128)`` over bf16 ``keys``/``values``
    ``(B, Hkv, T, 128)`` with token stride 128 (a :class:`FixedKVCache`'s views,
    or the keys a :class:`FixedSlidingKVCache` returns), the per-head ``sinks``
    in the softmax denominator: the call Attention.__call__ makes for those
    caches (model.py:204-211, the fused SDPA's sinks argument).  One query
    token decodes; ``L > 1`` queries are the newest ``L`` of the ``T`` keys,
    under ``mask`` None, "causal" or a boolean / additive array (the rules of
    :func:`quantized_attention_with_sinks`); ``window`` limits a causal mask
    to the last ``window`` keys.  The sinks
    are taken as given (as float32 values); ``sink_dtype`` (bf16/f16) rounds
    them first -- the reference's caller hands them over in the query dtype
    (model.py:211), and :func:`attend` passes it.
    """
    _check_query(queries)
    B, Hq, L, D = queries.shape
    if not (_bf16_kv_ok(keys) and _bf16_kv_ok(values)):
        raise ValueError("keys/values must be bf16 GPU tensors (B, Hkv, T, 128) with token stride 128")
    if keys.shape != values.shape or keys.shape[0] != B or keys.shape[-1] != D:
        raise ValueError(f"keys {tuple(keys.shape)} / values {tuple(values.shape)} do not match queries")
    T = keys.shape[2]
    if L > T:
        raise ValueError(f"{L} queries but only {T} keys")
    Hkv = keys.shape[1]
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads is not a multiple of {Hkv} KV heads")
    if Hq // Hkv > MAX_GROUP:
        return _head_groups(queries, sinks, mask, Hkv, lambda q, sk, m: scaled_dot_product_attention(
            q, keys, values, scale, m, sk, out_dtype=out_dtype, splits=splits, window=window, sink_dtype=sink_dtype))
    if window is not None:
        causal, win, bias = True, (0 if window >= T else int(window)), None
    else:
        causal, win, bias = _resolve_mask(mask, B, Hkv, Hq // Hkv, L, T, queries.device)
    if L == 1:
        if win:  # one query sees the last `win` keys: attend over that slice
            keys, values = keys[:, :, T - win:], values[:, :, T - win:]
        out, want = _new_out((B, Hq, D), out_dtype, queries)
        _bf16_decode_launch(queries, keys, values, scale, sinks, splits, out, sink_dtype=sink_dtype, bias=bias)
        out = out.view(B, Hq, 1, D)
    elif queries.dtype == torch.float32:
        return _rows_as_decodes(
            queries, T, Hkv, causal, win, bias, out_dtype,
            lambda q, t, o, b: _bf16_decode_launch(q, keys[:, :, :t], values[:, :, :t], scale, sinks, splits, o,
                                                   sink_dtype=sink_dtype, bias=b))
    else:
        out, want = _new_out((B, Hq, L, D), out_dtype, queries)
        _bf16_prefill_launch(queries, keys, values, scale, sinks, causal, win, out, splits or 0, sink_dtype, bias)
    return _finish(out, want)


def attend(queries, keys, values, cache, scale, mask=None, sinks=None, *, out_dtype=None,
           splits=None, fused=True):
    """The cache + attention part of ``Attention.__call__`` (model.py:177-211).

    New ``keys``/``values`` ``(B, Hkv, L, 128)`` go into ``cache`` first
    (quantized for a :class:`QuantizedKVCache`, stored as bf16 for a
    :class:`FixedKVCache`), then ``queries`` attend over the whole cache, the
    new tokens included.  A single decode token takes one fused launch.

    Sinks as the reference's branches see them: float32 in the quantized
    decode (model.py:129), rounded to the query dtype for chunks over the
    quantized cache (model.py:202) and on every call over the bf16 caches
    (model.py:211).  A :class:`FixedSlidingKVCache` applies its own window: a
    single decode token takes a mask that keeps every held token (None, as its
    ``make_mask`` returns, "causal", or such a host array), anything else
    raises NotImplementedError.  A decode step fuses its append with the
    attention when the mask keeps every key (None, "causal", a host array of
    that pattern); a mask array on the GPU (never inspected: :func:`_mask_plan`)
    takes the append, then the masked attention.
    """
    _check_query(queries)
    B, Hq, L, D = queries.shape
    qdt = queries.dtype
    ring = isinstance(cache, FixedSlidingKVCache)
    if keys.dim() == 4 and keys.shape[1] > 0 and Hq // keys.shape[1] > MAX_GROUP:
        fused = False  # the query heads of a KV head take several launches (_head_groups)
    # one query's host-checked pattern over the cache after the append (None:
    # a device array, or another pattern: a bias); for one query "causal"
    # keeps every key (window 0)
    plan1 = None
    if L == 1:
        plan1 = _mask_plan(mask, 1, min(cache.offset + 1, cache.capacity) if ring else cache.offset + 1)
    keeps_all = mask is None or (plan1 is not None and plan1[1] == 0)
    if ring:
        # a new token goes to its ring slot and decode attends over the valid
        # slots (order-free); a chunk attends over the ring in order plus
        # itself, causally within the window
        if L == 1 and not keeps_all:
            raise NotImplementedError("a decode step over the sliding ring sees every held token (mask None)")
        if L == 1 and fused:
            # one launch pair: the token written into its slot by the split
            # that reads it, attention over the occupied slots (order-free)
            if keys.shape != values.shape or keys.shape[2] != 1 or keys.dtype not in _DTYPES or values.dtype != keys.dtype:
                raise ValueError("a fused decode step takes one new K/V token of a float dtype")
            if tuple(keys.shape[:2]) != tuple(cache.keys.shape[:2]) or B != cache.keys.shape[0] \
                    or Hq % cache.keys.shape[1] != 0:
                raise ValueError(f"queries (B={B}, Hq={Hq}) / new keys {tuple(keys.shape[:2])} do not match the ring "
                                 f"{tuple(cache.keys.shape[:2])}")
            slot = cache.offset % cache.capacity
            n = min(cache.offset + 1, cache.capacity)
            kn = keys if _rows_aligned(keys) else keys.contiguous()
            vn = values if _rows_aligned(values) else values.contiguous()
            out, want = _new_out((B, Hq, D), out_dtype, queries)
            _bf16_decode_launch(queries, cache.keys, cache.values, scale, sinks, splits, out, kn, vn, T=n,
                                capacity=cache.capacity, slot=slot, sink_dtype=qdt)
            cache.offset += 1
            out = out.view(B, Hq, 1, D)
            return _finish(out, want)
        k, v = cache.update_and_fetch(keys, values)
        if L == 1:
            return scaled_dot_product_attention(queries, k, v, scale, None, sinks, out_dtype=out_dtype, splits=splits,
                                                sink_dtype=qdt)
        return scaled_dot_product_attention(queries, k, v, scale, "causal", sinks, out_dtype=out_dtype,
                                            window=cache.window_size, sink_dtype=qdt)
    if isinstance(cache, FixedKVCache):
        # the fused step attends over every token; any other single-query
        # mask (a window, a bias) takes the write, then the masked attention
        if fused and L == 1 and keeps_all:
            if keys.shape != values.shape or keys.shape[2] != 1 or keys.dtype not in _DTYPES or values.dtype != keys.dtype:
                raise ValueError("a fused decode step takes one new K/V token of a float dtype")
            st = cache.storage
            if tuple(keys.shape[:2]) != (st.batch, st.n_kv_heads) or B != st.batch or Hq % st.n_kv_heads != 0:
                raise ValueError(f"queries (B={B}, Hq={Hq}) / new keys (B={keys.shape[0]}, Hkv={keys.shape[1]}) "
                                 f"do not match the storage (B={st.batch}, Hkv={st.n_kv_heads})")
            T = cache.offset + 1
            cache._reserve(T)
            data = cache.storage.layer(cache.index)
            kn = keys if _rows_aligned(keys) else keys.contiguous()
            vn = values if _rows_aligned(values) else values.contiguous()
            out, want = _new_out((B, Hq, D), out_dtype, queries)
            _bf16_decode_launch(queries, data[:, 0], data[:, 1], scale, sinks, splits, out, kn, vn, T=T,
                                capacity=st.layer_capacity(cache.index), sink_dtype=qdt)
            cache.offset = T
            out = out.view(B, Hq, 1, D)
            return _finish(out, want)
        k, v = cache.update_and_fetch(keys, values)
        return scaled_dot_product_attention(queries, k, v, scale, mask, sinks, out_dtype=out_dtype, splits=splits,
                                            sink_dtype=qdt)
    # one query under a sliding window, or a mask array (a bias), takes the
    # append, then the masked attention
    if fused and L == 1 and keeps_all:
        cache._check_usable()
        if keys.shape != values.shape or keys.shape[2] != 1 or keys.dtype not in _DTYPES or values.dtype != keys.dtype:
            raise ValueError("a fused decode step takes one new K/V token of a float dtype")
        Bk, H = keys.shape[:2]
        if cache.keys is not None and tuple(cache.keys[0].shape[:2]) != (Bk, H):
            raise ValueError(f"new keys have (B, Hkv) = ({Bk}, {H}), the cache holds "
                             f"{tuple(cache.keys[0].shape[:2])}")
        if B != Bk:
            raise ValueError(f"queries have batch {B}, the new keys {Bk}")
        cache._reserve(Bk, H, cache.offset + 1, keys.device, keys.dtype)
        k_kv, v_kv = cache._view()
        _check_cache_shapes(queries, k_kv, v_kv)
        kn = keys if _rows_aligned(keys) else keys.contiguous()
        vn = values if _rows_aligned(values) else values.contiguous()
        out, want = _new_out((B, Hq, D), out_dtype, queries)
        try:
            _decode_launch(queries, k_kv, v_kv, scale, sinks, splits, out, kn, vn, T=cache.offset + 1,
                           capacity=cache.capacity)
        except _lib.RecError:
            cache._usable = False
            raise
        cache.offset += 1
        out = out.view(B, Hq, 1, D)
        return _finish(out, want)
    k, v = cache.update_and_fetch(keys, values)
    return quantized_attention_with_sinks(queries, k, v, scale, mask, sinks, cache.group_size, cache.key_bits,
                                          cache.value_bits, out_dtype=out_dtype, splits=splits,
                                          sink_dtype=qdt if L > 1 else None)

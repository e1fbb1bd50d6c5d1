"""Quantized KV cache with the reference's cache call surface.

Mirrors ``MixedQuantizedKVCache`` (engine/src/rec_mlx/model.py:40-105) and the
mlx-lm ``QuantizedKVCache`` methods it inherits (mlx-lm 0.31.3, third-party:
``step``, ``offset``, ``keys_and_values``, ``make_mask``, ``size``,
``empty``, ``is_trimmable``, ``trim``, ``meta_state``, ``nbytes``), with
torch tensors in HBM instead of MLX arrays and the quantize-on-append done by
the gfx950 kernel behind ``rec_kv_append``.

Formats (bits per K and V independently, ``group_size=32``):

* 8-bit: symmetric int8, one fp16 scale per (token, head).
* 4-bit: asymmetric uint4, fp16 scale and zero-point per 32 dims.

With ``group_size=64`` (the reference's default) the cache holds MLX-style
affine codes, 8-bit keys and 4-bit values with a scale and bias per 64 dims
(``mx.quantize``'s algorithm, restated by the kernel), stored in the keys'
dtype as the reference allocates them (model.py:57-58): fp16 for fp16 keys,
bf16 for bf16 keys (and for fp32 keys, whose fp32 scales the kernels do not
read: they are rounded to bf16).

Codes and scales are stored in 32-token blocks laid out for the matrix-core
operands of the decode kernel (table in ``rec_amd/csrc/common.h``), so the
capacity is a multiple of 32; :func:`to_logical` turns any cache tensor back
into the plain ``(B, Hkv, T, ...)`` layout.
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from . import _lib

BLOCK = 32
HEAD_DIM = 128
GROUP4 = 32
GROUP_AFFINE = 64

_DTYPES = {torch.float16: _lib.REC_F16, torch.bfloat16: _lib.REC_BF16, torch.float32: _lib.REC_F32}


class QuantizedKV(NamedTuple):
    """Quantized K or V of one layer: what ``update_and_fetch`` returns.

    ``codes``/``scales``/``zeros`` span the full capacity in 32-token blocks;
    ``length`` tokens are valid.  ``zeros`` is None for 8-bit.  ``blocked``
    marks the dim-major V layout (K blocks are token-major).
    """

    codes: torch.Tensor
    scales: torch.Tensor
    zeros: Optional[torch.Tensor]
    bits: int
    length: int
    blocked: bool
    affine: bool = False  # MLX-style affine group 64: ``scales`` holds [scale, bias], ``zeros`` is None

    @property
    def code(self) -> int:
        """Format code of the C ABI (8, 4, REC_AFFINE8 / REC_AFFINE4, or with
        fp16 scales REC_AFFINE8_F16 / REC_AFFINE4_F16)."""
        if self.affine:
            if self.scales.dtype == torch.float16:
                return _lib.REC_AFFINE8_F16 if self.bits == 8 else _lib.REC_AFFINE4_F16
            return _lib.REC_AFFINE8 if self.bits == 8 else _lib.REC_AFFINE4
        return self.bits

    @property
    def n_kv_heads(self) -> int:
        return self.codes.shape[1]

    @property
    def capacity(self) -> int:
        return self.codes.shape[2] * BLOCK


def affine_meta_dtype(dtype: torch.dtype) -> torch.dtype:
    """dtype of the affine scales and biases for keys of ``dtype``: the keys'
    own (model.py:57-58), fp32 keys excepted (bf16: the kernels read 16-bit
    scales)."""
    return torch.float16 if dtype == torch.float16 else torch.bfloat16


def _alloc(B, H, cap, bits, is_v, device, affine=False, meta_dtype=torch.bfloat16):
    """Zeroed codes/scales/zeros of one cache tensor (layout table in rec_amd/csrc/common.h)."""
    nb = cap // BLOCK
    if affine:  # [scale, bias] x 2 groups x 32 slots of bf16 (or fp16) per block
        codes = torch.zeros((B, H, nb, BLOCK * HEAD_DIM * bits // 8), dtype=torch.uint8, device=device)
        scales = torch.zeros((B, H, nb, 2, HEAD_DIM // GROUP_AFFINE, BLOCK), dtype=meta_dtype, device=device)
        return codes, scales, None
    if bits == 8:
        codes = torch.zeros((B, H, nb, BLOCK * HEAD_DIM), dtype=torch.int8, device=device)
        scales = torch.zeros((B, H, nb, BLOCK), dtype=torch.float16, device=device)
        zeros = None
    else:
        codes = torch.zeros((B, H, nb, BLOCK * HEAD_DIM // 2), dtype=torch.uint8, device=device)
        scales = torch.zeros((B, H, nb, HEAD_DIM // GROUP4, BLOCK), dtype=torch.float16, device=device)
        zeros = torch.zeros_like(scales)
    return codes, scales, zeros


def _grow_tensor(old, new):
    if old is None:
        return new
    idx = tuple(slice(0, s) for s in old.shape)
    new[idx] = old
    return new


def block_pos(t):
    """Position of token t (0..31) inside its 32-token cache block."""
    return ((t >> 2) & 3) * 8 + (t >> 4) * 4 + (t & 3)


_POS = [block_pos(t) for t in range(BLOCK)]


def s4_slot(p):
    """Slot of block position ``p`` in a 4-bit scale / zero-point row: each run
    of 8 positions is stored in the order 0,4,1,5,2,6,3,7."""
    return (p & ~7) | (2 * (p & 3)) | ((p >> 2) & 1)


_SLOT4 = [s4_slot(p) for p in _POS]


def _unpack_v4(kv, B, H, nb, pos):
    """4-bit V codes (blocked) -> (B, H, nb*32, 64) bytes, low nibble = even dim."""
    packed = kv.codes.view(B, H, nb, 2, 16, 4, 4, 4)  # (h, c, pg, n4, byte)
    packed = packed.permute(0, 1, 2, 3, 6, 4, 5, 7).reshape(B, H, nb, HEAD_DIM, BLOCK // 2)  # (n, c) -> dim
    q = torch.stack([packed & 0xF, packed >> 4], -1).reshape(B, H, nb, HEAD_DIM, BLOCK)[..., pos]
    q = q.permute(0, 1, 2, 4, 3).reshape(B, H, -1, HEAD_DIM)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).to(torch.uint8)


def to_logical(kv: QuantizedKV, length: Optional[int] = None):
    """Return ``(codes, scales, zeros)`` in the plain layout, first ``length`` tokens.

    8-bit: codes int8 ``(B, H, T, 128)``, scales fp16 ``(B, H, T)``.
    4-bit: codes uint8 ``(B, H, T, 64)`` (low nibble = even dim), scales and
    zeros fp16 ``(B, H, T, 4)``.
    Affine: codes uint8 ``(B, H, T, 128)`` (8-bit) or ``(B, H, T, 64)``
    (4-bit, low nibble = even dim); scales and biases bf16 ``(B, H, T, 2)``
    in place of scales and zeros.
    """
    T = kv.length if length is None else length
    B, H, nb = kv.codes.shape[:3]
    pos = torch.tensor(_POS, device=kv.codes.device)
    if not kv.blocked and kv.bits == 8:  # K: [nb][2 halves][32 tokens][64 bytes]
        w = HEAD_DIM // 2
        codes = kv.codes.view(B, H, nb, 2, BLOCK, w).permute(0, 1, 2, 4, 3, 5).reshape(B, H, nb * BLOCK, 2 * w)
    elif not kv.blocked:  # K: [nb][32 tokens][4 byte groups][2 halves][8 bytes]
        codes = kv.codes.view(B, H, nb, BLOCK, 4, 2, 8).permute(0, 1, 2, 3, 5, 4, 6).reshape(B, H, nb * BLOCK, 64)
    elif kv.bits == 8:  # V: [nb][n / 2][c][position group][n % 2][8 bytes], dim 16 n + c
        blocked = kv.codes.view(B, H, nb, 4, 16, 4, 2, 8)  # (h, c, pg, n2, e)
        blocked = blocked.permute(0, 1, 2, 3, 6, 4, 5, 7).reshape(B, H, nb, HEAD_DIM, BLOCK)  # (n, c) -> dim
        codes = blocked[..., pos].permute(0, 1, 2, 4, 3).reshape(B, H, -1, HEAD_DIM)
    else:  # V: [nb][n / 4][c][position group][n % 4][4 bytes], dim 16 n + c, position p in byte p // 2
        codes = _unpack_v4(kv, B, H, nb, pos)
    slot = torch.tensor(_SLOT4, device=kv.codes.device)
    if kv.affine:  # scales: [nb][scale, bias][2 groups][32 slots]
        sb = kv.scales[..., slot].permute(0, 1, 3, 2, 5, 4).reshape(B, H, 2, -1, HEAD_DIM // GROUP_AFFINE)
        sc, zp = sb[:, :, 0], sb[:, :, 1]
    elif kv.bits == 8:
        sc = kv.scales[..., pos].reshape(B, H, -1)
        zp = None
    else:
        sc = kv.scales[..., slot].permute(0, 1, 2, 4, 3).reshape(B, H, -1, HEAD_DIM // GROUP4)
        zp = kv.zeros[..., slot].permute(0, 1, 2, 4, 3).reshape(B, H, -1, HEAD_DIM // GROUP4)
    return (
        codes[:, :, :T].contiguous(),
        sc[:, :, :T].contiguous(),
        None if zp is None else zp[:, :, :T].contiguous(),
    )


def _stride3(x):
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x, x.stride(0), x.stride(1), x.stride(2)


class QuantizedKVCache:
    """Quantize-on-append KV cache of one attention layer (GPU resident).

    ``group_size`` is the 4-bit group (32); 8-bit uses one scale per row.
    ``max_tokens`` preallocates the whole context once (no growth copies);
    appending beyond it raises ``ValueError("Decode context limit
    exhausted")`` like the reference (engine/src/rec_mlx/kernels/megakernel.py:1330-1331).
    Without it the capacity grows in multiples of ``step``, preserving the
    contents, as ``update_and_fetch`` does in the reference (model.py:49-75).
    """

    step = 256

    def __init__(self, group_size: int = GROUP4, key_bits: int = 8, value_bits: int = 8, *, max_tokens=None):
        for name, bits in (("key_bits", key_bits), ("value_bits", value_bits)):
            if bits not in (4, 8):
                raise ValueError(f"{name} must be 4 or 8, got {bits}")
        if group_size == GROUP_AFFINE:
            if (key_bits, value_bits) != (8, 4):
                raise NotImplementedError("the group-64 affine format is built for 8-bit keys with 4-bit values")
        elif 4 in (key_bits, value_bits) and group_size != GROUP4:
            raise ValueError(f"4-bit caches use groups of {GROUP4} (or 64 for the affine format), got {group_size}")
        self.group_size = group_size
        self.affine = group_size == GROUP_AFFINE
        self.key_bits, self.value_bits = key_bits, value_bits
        self.bits = key_bits
        self.max_tokens = max_tokens
        self.keys = None  # (codes, scales, zeros)
        self.values = None
        self.offset = 0
        self.capacity = 0
        self._usable = True

    # ------------------------------------------------------------ helpers --
    def _check_usable(self):
        if not self._usable:
            raise RuntimeError("Quantized KV cache was invalidated by a failed GPU call")

    def _reserve(self, B, H, needed, device, dtype=torch.bfloat16):
        """Room for ``needed`` tokens; the first allocation fixes the affine
        scale dtype from the keys' ``dtype``, growth keeps it."""
        if self.max_tokens is not None and needed > self.max_tokens:
            raise ValueError("Decode context limit exhausted")
        if self.keys is not None and needed <= self.capacity:
            return
        if self.max_tokens is not None:
            cap = -(-self.max_tokens // BLOCK) * BLOCK
        else:
            cap = -(-needed // self.step) * self.step
        meta = self.keys[1].dtype if self.keys is not None else affine_meta_dtype(dtype)
        k = _alloc(B, H, cap, self.key_bits, False, device, self.affine, meta)
        v = _alloc(B, H, cap, self.value_bits, True, device, self.affine, meta)
        if self.keys is not None:
            k = tuple(_grow_tensor(o, n) if n is not None else None for o, n in zip(self.keys, k))
            v = tuple(_grow_tensor(o, n) if n is not None else None for o, n in zip(self.values, v))
        self.keys, self.values, self.capacity = k, v, cap

    def _view(self):
        k = QuantizedKV(*self.keys, self.key_bits, self.offset, False, self.affine)
        v = QuantizedKV(*self.values, self.value_bits, self.offset, True, self.affine)
        return k, v

    # ------------------------------------------------------ reference API --
    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Quantize ``keys``/``values`` ``(B, Hkv, L, 128)`` into positions
        ``[offset, offset+L)`` and return the quantized K and V covering
        ``[0, offset+L)`` (model.py:45-82)."""
        self._check_usable()
        B, H, L, D = keys.shape
        if values.shape != keys.shape:
            raise ValueError(f"keys {tuple(keys.shape)} and values {tuple(values.shape)} differ in shape")
        if D != HEAD_DIM:
            raise NotImplementedError(f"head_dim {D} is not supported (128 only)")
        if keys.dtype not in _DTYPES or values.dtype != keys.dtype:
            raise ValueError(f"keys/values must share a float16/bfloat16/float32 dtype, got {keys.dtype}/{values.dtype}")
        if not keys.is_cuda:
            raise ValueError("keys/values must be GPU tensors")
        if self.keys is not None and (self.keys[0].shape[0], self.keys[0].shape[1]) != (B, H):
            raise ValueError("batch/head shape differs from the cached one")
        prev = self.offset
        self._reserve(B, H, prev + L, keys.device, keys.dtype)
        k, ksb, ksh, kst = _stride3(keys)
        v, vsb, vsh, vst = _stride3(values)
        lib = _lib.load()
        stream = torch.cuda.current_stream(keys.device).cuda_stream
        kc, ks, kz = self.keys
        vc, vs, vz = self.values
        kv_k, kv_v = self._view()
        rc = lib.rec_kv_append(
            k.data_ptr(), v.data_ptr(), _DTYPES[keys.dtype], ksb, ksh, kst, vsb, vsh, vst,
            kv_k.code, kc.data_ptr(), ks.data_ptr(), kz.data_ptr() if kz is not None else None,
            kv_v.code, vc.data_ptr(), vs.data_ptr(), vz.data_ptr() if vz is not None else None,
            B, H, L, D, prev, self.capacity, stream,
        )
        if rc == _lib.REC_ELAUNCH:
            self._usable = False
        _lib.check(rc, "rec_kv_append")
        self.offset = prev + L
        return self.keys_and_values()

    def keys_and_values(self):
        return self._view()

    @property
    def state(self):
        return (self.keys, self.values, self.offset, self.group_size, self.key_bits, self.value_bits)

    @state.setter
    def state(self, v):
        (self.keys, self.values, self.offset, self.group_size, self.key_bits, self.value_bits) = v
        self.bits = self.key_bits
        self.affine = self.group_size == GROUP_AFFINE
        self.capacity = 0 if self.keys is None else QuantizedKV(*self.keys, self.key_bits, 0, False).capacity
        self._usable = True

    @property
    def meta_state(self):
        return tuple(map(str, (self.step, self.offset, self.group_size, self.key_bits, self.value_bits)))

    def size(self) -> int:
        return self.offset

    def empty(self) -> bool:
        return self.keys is None

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n

    def make_mask(self, n_tokens: int, window_size=None, return_array: bool = False):
        """None for a single decode token (engine/src/rec_mlx/cache.py:140-143),
        else "causal", or the boolean array when asked for one."""
        if window_size is not None:
            raise NotImplementedError("sliding-window masks are not supported by this cache")
        if n_tokens == 1 and not return_array:
            return None
        if not return_array:
            return "causal"
        T = self.offset + n_tokens
        q = torch.arange(T - n_tokens, T)
        return q[:, None] >= torch.arange(T)[None]

    @property
    def nbytes(self) -> int:
        if self.keys is None:
            return 0
        return sum(t.numel() * t.element_size() for t in (*self.keys, *self.values) if t is not None)


class MixedQuantizedKVCache(QuantizedKVCache):
    """8-bit keys and 4-bit values in the group-64 affine format by default,
    like the reference's ``MixedQuantizedKVCache(group_size=64, key_bits=8,
    value_bits=4)`` (model.py:40-43); ``group_size=32`` selects this library's
    int8 / uint4 formats."""

    def __init__(self, group_size: int = GROUP_AFFINE, key_bits: int = 8, value_bits: int = 4, **kw):
        super().__init__(group_size, key_bits, value_bits, **kw)

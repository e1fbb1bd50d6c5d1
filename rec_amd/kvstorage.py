"""bf16 KV cache with the reference's production cache surface.

Mirrors ``KVStorage`` / ``FixedKVCache`` (engine/src/rec_mlx/cache.py:48-150):
each layer owns a token-major bf16 region ``[2][Hkv][capacity][128]`` (K
then V, per batch row), written by ``rec_kv_write_bf16`` and read in place by
the bf16 decode kernel (``rec_decode_bf16``).  The reference grows its
storage in banks of 65,536 tokens up to four banks (cache.py:46-78); here a
layer's region is one allocation whose capacity grows in the same 65,536-token
steps to the same 262,144-token limit, the earlier contents copied over.
Sliding-window layers (``FixedSlidingKVCache``, cache.py:153-258) are not
covered.
"""

from __future__ import annotations

from typing import List, Optional

import torch

from . import _lib
from .cache import _DTYPES, HEAD_DIM

BLOCK_TOKENS = 65536
MAX_BLOCKS = 4


def _stride3(x):
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x, x.stride(0), x.stride(1), x.stride(2)


class KVStorage:
    """bf16 K/V regions of ``layers`` full-attention layers.

    ``layer(i, count)`` returns the ``(B, 2, Hkv, count, 128)`` view of layer
    ``i`` (the reference's ``(2, Hkv, count, 128)`` for ``B == 1``, cache.py:86-95);
    ``write(i, offset, keys, values)`` stores ``(B, Hkv, L, 128)`` rows at
    ``[offset, offset + L)`` (cache.py:97-119).
    """

    def __init__(self, layers: int, capacity: int, n_kv_heads: int = 4, *, batch: int = 1, device=None):
        if layers < 1 or n_kv_heads < 1 or batch < 1:
            raise ValueError("layers, n_kv_heads and batch must be positive")
        self.n_layers, self.n_kv_heads, self.batch = layers, n_kv_heads, batch
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.regions: List[Optional[torch.Tensor]] = [None] * layers
        self.capacity = 0
        self.grow(capacity)

    @property
    def nbytes(self) -> int:
        return sum(r.numel() * r.element_size() for r in self.regions if r is not None)

    def grow(self, capacity: int):
        if not 0 < capacity <= BLOCK_TOKENS * MAX_BLOCKS:
            raise ValueError("Decode context limit exhausted")
        cap = -(-capacity // BLOCK_TOKENS) * BLOCK_TOKENS
        if cap <= self.capacity:
            return
        for i, old in enumerate(self.regions):
            new = torch.zeros((self.batch, 2, self.n_kv_heads, cap, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
            if old is not None:
                new[:, :, :, : old.shape[3]] = old
            self.regions[i] = new
        self.capacity = cap

    def layer(self, index: int, count: Optional[int] = None) -> torch.Tensor:
        count = self.capacity if count is None else count
        return self.regions[index][:, :, :, :count]

    def write(self, index: int, offset: int, keys: torch.Tensor, values: torch.Tensor):
        B, H, L, D = keys.shape
        if values.shape != keys.shape:
            raise ValueError(f"keys {tuple(keys.shape)} and values {tuple(values.shape)} differ in shape")
        if (B, H) != (self.batch, self.n_kv_heads):
            raise ValueError(f"keys are (B={B}, Hkv={H}), storage holds (B={self.batch}, Hkv={self.n_kv_heads})")
        if D != HEAD_DIM:
            raise NotImplementedError(f"head_dim {D} is not supported (128 only)")
        if keys.dtype not in _DTYPES or values.dtype != keys.dtype:
            raise ValueError(f"keys/values must share a float16/bfloat16/float32 dtype, got {keys.dtype}/{values.dtype}")
        if offset < 0 or offset + L > self.capacity:
            raise ValueError("Decode context limit exhausted")
        region = self.regions[index]
        kr, vr = region[:, 0], region[:, 1]
        k, ksb, ksh, kst = _stride3(keys)
        v, vsb, vsh, vst = _stride3(values)
        rc = _lib.load().rec_kv_write_bf16(
            k.data_ptr(), v.data_ptr(), _DTYPES[keys.dtype], ksb, ksh, kst, vsb, vsh, vst,
            kr.data_ptr(), kr.stride(0), kr.stride(1), vr.data_ptr(), vr.stride(0), vr.stride(1),
            B, H, L, D, offset, self.capacity, torch.cuda.current_stream(self.device).cuda_stream,
        )
        _lib.check(rc, "rec_kv_write_bf16")


class FixedKVCache:
    """One layer's view of a :class:`KVStorage` (engine/src/rec_mlx/cache.py:121-150)."""

    def __init__(self, storage: KVStorage, index: int):
        self.storage, self.index = storage, index
        self.offset = 0

    @property
    def state(self):
        return self.storage.regions[self.index]

    def empty(self) -> bool:
        return self.offset == 0

    def size(self) -> int:
        return self.offset

    def is_trimmable(self) -> bool:
        return False

    def make_mask(self, n_tokens: int, window_size=None, return_array: bool = False):
        """None for a single decode token (cache.py:140-143), else "causal"
        or the boolean array when asked for one."""
        if window_size is not None:
            raise NotImplementedError("sliding-window masks are not supported by this cache")
        if n_tokens == 1 and not return_array:
            return None
        if not return_array:
            return "causal"
        T = self.offset + n_tokens
        q = torch.arange(T - n_tokens, T)
        return q[:, None] >= torch.arange(T)[None]

    def _reserve(self, needed: int):
        if needed > BLOCK_TOKENS * MAX_BLOCKS:
            raise ValueError("Decode context limit exhausted")
        if needed > self.storage.capacity:
            self.storage.grow(needed)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Store ``keys``/``values`` at ``[offset, offset + L)`` and return the
        ``(B, Hkv, offset + L, 128)`` K and V views (cache.py:145-150)."""
        stop = self.offset + keys.shape[-2]
        self._reserve(stop)
        self.storage.write(self.index, self.offset, keys, values)
        self.offset = stop
        data = self.storage.layer(self.index, stop)
        return data[:, 0], data[:, 1]

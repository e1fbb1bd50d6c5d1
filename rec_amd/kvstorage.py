"""bf16 KV cache with the reference's production cache surface.

Mirrors ``KVStorage`` / ``FixedKVCache`` (engine/src/rec_mlx/cache.py:48-150):
each layer owns a token-major bf16 region ``[2][Hkv][capacity][128]`` (K
then V, per batch row), written by ``rec_kv_write_bf16`` and read in place by
the bf16 decode kernel (``rec_decode_bf16``).  The reference grows its
storage in banks of 65,536 tokens up to four banks (cache.py:46-78); here a
layer's region is one allocation whose capacity grows in the same 65,536-token
steps to the same 262,144-token limit, the earlier contents copied over.
Sliding-window layers keep a ring of window slots, ``FixedSlidingKVCache``
(cache.py:153-258); decode attends over its valid slots with the same kernel.
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


class FixedSlidingKVCache:
    """Sliding-window bf16 cache (engine/src/rec_mlx/cache.py:153-258).

    Two slots of ``(B, Hkv, capacity, 128)`` bf16 buffers, ``capacity =
    min(window_size, max_sequence_tokens)``.  A single new token is written at
    the next free slot, then round the ring; a multi-token update returns the
    ring's tokens in order followed by the new ones (the keys a windowed
    prefill chunk attends to) and keeps the last ``capacity`` of them in the
    other slot.  Decode attention over the ring is order-free (softmax over a
    set of keys), so it reads the ``size()`` valid slots in place.
    """

    def __init__(self, *, max_sequence_tokens: int, num_kv_heads: int, head_dim: int, window_size: int,
                 dtype=torch.bfloat16, batch: int = 1, device=None):
        if head_dim != HEAD_DIM:
            raise NotImplementedError(f"head_dim {head_dim} is not supported (128 only)")
        if dtype != torch.bfloat16:
            raise NotImplementedError("the sliding cache holds bf16")
        self.window_size = window_size
        self.capacity = min(window_size, max_sequence_tokens)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        shape = (batch, num_kv_heads, self.capacity, head_dim)
        self.key_buffers = [torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(2)]
        self.value_buffers = [torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(2)]
        self.offset = 0
        self._valid = 0
        self._slot = 0
        self._ring_index = 0

    def grow(self, capacity: int):
        capacity = min(self.window_size, capacity)
        if capacity > self.capacity:
            pad = capacity - self.capacity
            grow = lambda t: torch.nn.functional.pad(t, (0, 0, 0, pad))  # noqa: E731
            self.key_buffers = [grow(t) for t in self.key_buffers]
            self.value_buffers = [grow(t) for t in self.value_buffers]
            self.capacity = capacity

    @property
    def state(self):
        return tuple(self.key_buffers), tuple(self.value_buffers)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (*self.key_buffers, *self.value_buffers))

    def empty(self) -> bool:
        return self.offset == 0

    def size(self) -> int:
        return self._valid

    def is_trimmable(self) -> bool:
        return False

    def make_mask(self, n_tokens: int, window_size=None, return_array: bool = False):
        """None for one decode token, "causal" for a first chunk within the
        window, else the windowed causal boolean array (cache.py:199-205)."""
        window = self.window_size if window_size is None else window_size
        if n_tokens == 1 and not return_array:
            return None
        if self._valid == 0 and n_tokens <= window and not return_array:
            return "causal"
        T = self._valid + n_tokens
        q = torch.arange(T - n_tokens, T)[:, None]
        k = torch.arange(T)[None]
        return (q >= k) & (q < k + window)

    def _next_index(self) -> int:
        """Slot the next single token goes to; advances the ring."""
        if self._valid < self.capacity:
            index = self._valid
            self._valid += 1
        else:
            index = self._ring_index
            self._ring_index = (self._ring_index + 1) % self.capacity
        return index

    def _write(self, index: int, keys: torch.Tensor, values: torch.Tensor):
        kb, vb = self.key_buffers[self._slot], self.value_buffers[self._slot]
        B, H, L, D = keys.shape
        k, ksb, ksh, kst = _stride3(keys)
        v, vsb, vsh, vst = _stride3(values)
        rc = _lib.load().rec_kv_write_bf16(
            k.data_ptr(), v.data_ptr(), _DTYPES[keys.dtype], ksb, ksh, kst, vsb, vsh, vst,
            kb.data_ptr(), kb.stride(0), kb.stride(1), vb.data_ptr(), vb.stride(0), vb.stride(1),
            B, H, L, D, index, self.capacity, torch.cuda.current_stream(self.device).cuda_stream,
        )
        _lib.check(rc, "rec_kv_write_bf16")

    def _prior(self):
        keys, values = self.key_buffers[self._slot], self.value_buffers[self._slot]
        if self._valid == self.capacity and self._ring_index:
            r = self._ring_index
            return (torch.cat((keys[:, :, r:], keys[:, :, :r]), dim=2),
                    torch.cat((values[:, :, r:], values[:, :, :r]), dim=2))
        return keys[:, :, : self._valid], values[:, :, : self._valid]

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        if keys.shape != values.shape or keys.dtype not in _DTYPES or values.dtype != keys.dtype:
            raise ValueError("keys/values must share a shape and a float dtype")
        if keys.shape[-2] == 1:
            self._write(self._next_index(), keys, values)
            self.offset += 1
            return (self.key_buffers[self._slot][:, :, : self._valid],
                    self.value_buffers[self._slot][:, :, : self._valid])
        prior_keys, prior_values = self._prior()
        attention_keys = torch.cat((prior_keys, keys.to(torch.bfloat16)), dim=2)
        attention_values = torch.cat((prior_values, values.to(torch.bfloat16)), dim=2)
        retained = min(self.capacity, attention_keys.shape[2])
        nxt = 1 - self._slot
        self.key_buffers[nxt][:, :, :retained] = attention_keys[:, :, -retained:]
        self.value_buffers[nxt][:, :, :retained] = attention_values[:, :, -retained:]
        self._slot = nxt
        self._valid = retained
        self._ring_index = 0
        self.offset += keys.shape[2]
        return attention_keys, attention_values

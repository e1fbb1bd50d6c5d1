"""bf16 KV cache with the reference's production cache surface.

Mirrors ``KVStorage`` / ``FixedKVCache`` (engine/src/rec_mlx/cache.py:48-150):
each layer owns a token-major bf16 region ``[B][2][Hkv][tokens][128]`` (K
then V, per batch row), written by ``rec_kv_write_bf16`` and read in place by
the bf16 decode and prefill kernels.  The reference grows its storage by
adding banks of 65,536 tokens, up to four, without copying, and its kernels
pick a bank per token (cache.py:46-84, megakernel.py:115-135).  Here each
layer reserves the address range of all four banks once (HIP virtual memory,
``rec_region_*``) and device memory is mapped into it a bank at a time:
growing copies nothing, mapped banks keep their addresses (views taken
before a growth stay valid), and the kernels see one strided tensor.
Sliding-window layers keep a ring of window slots, ``FixedSlidingKVCache``
(the surface of cache.py:153-258); decode attends over its occupied slots with
the same kernel.
"""

from __future__ import annotations

import ctypes
import warnings
from typing import List, NamedTuple, Optional

import numpy as np
import torch

from . import _lib
from .cache import _DTYPES, HEAD_DIM, MixedQuantizedKVCache

BLOCK_TOKENS = 65536
MAX_BLOCKS = 4
MAX_TOKENS = BLOCK_TOKENS * MAX_BLOCKS
LOCAL_TOKENS = 513  # a sliding-window layer's region in the metadata form (cache.py:60-63)
META_LAYERS = 49    # metadata rows that describe layers (cache.py:54-58)


def _stride3(x):
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x, x.stride(0), x.stride(1), x.stride(2)


# Regions dropped while a graph capture ran: their release needs a device
# synchronisation, which a capture forbids, so they wait here for the next
# region created or grown outside a capture.
_RETIRED: List[tuple] = []


def _release_retired():
    if not _RETIRED or torch.cuda.is_current_stream_capturing():
        return
    while _RETIRED:
        handle, device = _RETIRED.pop()
        torch.cuda.synchronize(device)
        _lib.load().rec_region_destroy(handle)


class _RegionMemory:
    """Exports a region's mapped range to torch; tensors made from it keep
    it, and so the region, alive."""

    def __init__(self, interface: dict, region: "_Region"):
        self.__cuda_array_interface__ = interface
        self.region = region


class _Region:
    """One layer's growable region: ``rows`` rows of MAX_TOKENS bf16 tokens
    reserved, banks of BLOCK_TOKENS mapped on demand (``rec_region_*``)."""

    def __init__(self, device: torch.device, batch: int, n_kv_heads: int):
        lib = _lib.load()
        _release_retired()
        self.device, self.shape = device, (batch, 2, n_kv_heads)
        rows = batch * 2 * n_kv_heads
        h, base = ctypes.c_void_p(), ctypes.c_void_p()
        with torch.cuda.device(device):
            rc = lib.rec_region_create(device.index, rows, MAX_TOKENS, HEAD_DIM * 2, BLOCK_TOKENS,
                                       ctypes.byref(h), ctypes.byref(base))
        _lib.check(rc, "rec_region_create")
        self.handle, self.base, self.capacity = h.value, base.value, 0

    def grow(self, tokens: int) -> torch.Tensor:
        """Back the first ``tokens`` tokens of every row, zero the new banks,
        and return the ``(B, 2, Hkv, capacity, 128)`` bf16 view."""
        _release_retired()
        cap = ctypes.c_int64()
        with torch.cuda.device(self.device):
            rc = _lib.load().rec_region_grow(self.handle, tokens, ctypes.byref(cap))
        _lib.check(rc, "rec_region_grow")
        old, self.capacity = self.capacity, cap.value
        view = self.view()
        if self.capacity > old:
            view[:, :, :, old:].zero_()  # the reference's banks start as zeros
        return view

    def view(self) -> torch.Tensor:
        B, two, H = self.shape
        row = MAX_TOKENS * HEAD_DIM  # elements between consecutive rows
        cai = {
            "shape": (B, two, H, self.capacity, HEAD_DIM),
            "strides": tuple(2 * x for x in (two * H * row, H * row, row, HEAD_DIM, 1)),
            "typestr": "<i2",
            "data": (self.base, False),
            "version": 3,
            "stream": None,
        }
        return torch.as_tensor(_RegionMemory(cai, self), device=self.device).view(torch.bfloat16)

    def __del__(self):
        handle, self.handle = getattr(self, "handle", None), None
        if not handle:
            return
        try:
            if torch.cuda.is_current_stream_capturing():
                _RETIRED.append((handle, self.device))  # no synchronisation inside a capture
                return
            torch.cuda.synchronize(self.device)  # no kernel may still read or write the banks
        except Exception as e:  # e.g. interpreter shutdown: the process exit releases the mappings
            try:
                warnings.warn(f"KV region not released ({e}); its memory stays mapped until the process exits")
            except Exception:
                pass
            return
        _lib.load().rec_region_destroy(handle)


def _metadata_rows(metadata):
    """The reference's layer table (cache.py:52-66): rows of uint32 columns,
    column 1 set for a full-attention layer; columns 61-62 receive the
    layer's (element offset, tokens per bank) in the reference's bank layout,
    full-attention layers first, then the 513-token sliding-window regions."""
    rows = [[int(x) for x in row] for row in metadata]
    if not rows or any(len(r) < 63 for r in rows[:META_LAYERS]):
        raise ValueError("metadata rows must have at least 63 columns")
    layers = rows[:META_LAYERS]
    n_global = sum(bool(r[1]) for r in layers)
    g = l = 0
    for r in layers:
        if r[1]:
            r[61:63] = [g * BLOCK_TOKENS * 1024, BLOCK_TOKENS]
            g += 1
        else:
            r[61:63] = [n_global * BLOCK_TOKENS * 1024 + l * LOCAL_TOKENS * 1024, LOCAL_TOKENS]
            l += 1
    return rows


class KVStorage:
    """bf16 K/V regions of the attention layers of one model.

    ``KVStorage(layers, capacity, n_kv_heads)``: ``layers`` full-attention
    layers.  ``KVStorage(metadata, capacity)``: the reference's constructor
    (cache.py:52-73) — the first 49 rows of the layer table, column 1 marking
    full-attention layers, four KV heads; the other (sliding-window) layers
    get fixed 513-token regions, as the reference places them beside the
    full-attention ones in its first bank; ``rows`` and ``metadata`` hold the
    table with the reference's columns 61-62 filled in.

    ``layer(i, count)`` returns the ``(B, 2, Hkv, count, 128)`` view of layer
    ``i`` (the reference's ``(2, Hkv, count, 128)`` for ``B == 1``, cache.py:86-95);
    ``write(i, offset, keys, values)`` stores ``(B, Hkv, L, 128)`` rows at
    ``[offset, offset + L)`` (cache.py:97-119).  ``grow`` maps further
    65,536-token banks (cache.py:63-70); the capacity never shrinks.
    """

    def __init__(self, layers, capacity: int, n_kv_heads: int = 4, *, batch: int = 1, device=None):
        self.rows = self.metadata = None
        if isinstance(layers, int):
            is_global = [True] * layers
        else:  # the reference's layer table
            self.rows = _metadata_rows(layers)
            self.metadata = np.array(self.rows, dtype=np.uint32)
            is_global = [bool(r[1]) for r in self.rows[:META_LAYERS]]
        if not is_global or n_kv_heads < 1 or batch < 1:
            raise ValueError("layers, n_kv_heads and batch must be positive")
        self.n_layers, self.n_kv_heads, self.batch = len(is_global), n_kv_heads, batch
        self.is_global = is_global
        dev = torch.device(device) if device is not None else torch.device("cuda")
        self.device = torch.device(dev.type, dev.index if dev.index is not None else torch.cuda.current_device())
        self._banks = {i: _Region(self.device, batch, n_kv_heads) for i, gl in enumerate(is_global) if gl}
        self._local = {i: torch.zeros((batch, 2, n_kv_heads, LOCAL_TOKENS, HEAD_DIM), dtype=torch.bfloat16,
                                      device=self.device)
                       for i, gl in enumerate(is_global) if not gl}
        self.regions: List[torch.Tensor] = [self._local.get(i) for i in range(self.n_layers)]
        self.capacity = 0
        self.grow(capacity)

    @property
    def nbytes(self) -> int:
        return sum(r.numel() * r.element_size() for r in self.regions)

    def grow(self, capacity: int):
        if not 0 < capacity <= MAX_TOKENS:
            raise ValueError("Decode context limit exhausted")
        if capacity <= self.capacity:
            return
        for i, r in self._banks.items():
            self.regions[i] = r.grow(capacity)
        mapped = [r.capacity for r in self._banks.values()]
        self.capacity = mapped[0] if mapped else -(-capacity // BLOCK_TOKENS) * BLOCK_TOKENS

    def layer_capacity(self, index: int) -> int:
        """Tokens layer ``index`` holds: the storage's capacity, or 513 for a
        sliding-window layer of the metadata form."""
        return self.capacity if self.is_global[index] else LOCAL_TOKENS

    def layer(self, index: int, count: Optional[int] = None) -> torch.Tensor:
        count = self.layer_capacity(index) if count is None else count
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
        cap = self.layer_capacity(index)
        if offset < 0 or offset + L > cap:
            raise ValueError("Decode context limit exhausted")
        region = self.regions[index]
        kr, vr = region[:, 0], region[:, 1]
        k, ksb, ksh, kst = _stride3(keys)
        v, vsb, vsh, vst = _stride3(values)
        rc = _lib.load().rec_kv_write_bf16(
            k.data_ptr(), v.data_ptr(), _DTYPES[keys.dtype], ksb, ksh, kst, vsb, vsh, vst,
            kr.data_ptr(), kr.stride(0), kr.stride(1), vr.data_ptr(), vr.stride(0), vr.stride(1),
            B, H, L, D, offset, cap, torch.cuda.current_stream(self.device).cuda_stream,
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
        if not self.storage.is_global[self.index]:  # a 513-token region of the metadata form
            if needed > LOCAL_TOKENS:
                raise ValueError("Decode context limit exhausted")
            return
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


class RingState(NamedTuple):
    """What a sliding ring holds at one point of the sequence: its tokens'
    K and V ``(B, Hkv, n, 128)`` oldest first (``n = min(offset,
    capacity)``), as private copies that nothing writes again, and the
    number of tokens the ring had taken."""

    keys: torch.Tensor
    values: torch.Tensor
    offset: int

    @property
    def nbytes(self) -> int:
        return self.keys.numel() * self.keys.element_size() + self.values.numel() * self.values.element_size()


class FixedSlidingKVCache:
    """Sliding-window bf16 cache with the surface of
    engine/src/rec_mlx/cache.py:153-258.

    One ring of ``capacity = min(window_size, max_sequence_tokens)`` token
    slots per (batch row, KV head): token ``p`` of the sequence lives in slot
    ``p % capacity``, so the ring always holds the last ``size() =
    min(offset, capacity)`` tokens.  A single new token overwrites the oldest
    slot and the decode attends over the occupied slots in place (softmax
    attention is order-free).  A chunk of several tokens attends over the
    window's tokens in sequence order followed by the chunk -- what
    ``update_and_fetch`` returns, as the reference does -- and the ring then
    keeps the last ``capacity`` of them.  :meth:`snapshot` and
    :meth:`restore` copy the window out and back (prompt-prefix rollback,
    ``rec_amd.prefix``).
    """

    def __init__(self, *, max_sequence_tokens: int, num_kv_heads: int, head_dim: int, window_size: int,
                 dtype=torch.bfloat16, batch: int = 1, device=None):
        if head_dim != HEAD_DIM:
            raise NotImplementedError(f"head_dim {head_dim} is not supported (128 only)")
        if dtype != torch.bfloat16:
            raise NotImplementedError("the sliding cache holds bf16")
        if window_size < 1 or max_sequence_tokens < 1:
            raise ValueError("window_size and max_sequence_tokens must be positive")
        self.window_size = window_size
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.offset = 0
        self._alloc(batch, num_kv_heads, min(window_size, max_sequence_tokens))

    def _alloc(self, batch, heads, capacity):
        self.capacity = capacity
        shape = (batch, heads, capacity, HEAD_DIM)
        self.keys = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)
        self.values = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)

    # ------------------------------------------------------------ window --
    def size(self) -> int:
        return min(self.offset, self.capacity)

    def empty(self) -> bool:
        return self.offset == 0

    def is_trimmable(self) -> bool:
        return False

    @property
    def state(self):
        return self.keys, self.values

    @property
    def nbytes(self) -> int:
        return self.keys.numel() * self.keys.element_size() + self.values.numel() * self.values.element_size()

    def window(self):
        """The held tokens' K and V in sequence order (oldest first): views
        while the ring has not wrapped, else the two arcs joined."""
        n = self.size()
        head = self.offset % self.capacity  # slot of the oldest token once the ring is full
        if self.offset <= self.capacity or head == 0:
            return self.keys[:, :, :n], self.values[:, :, :n]
        return (torch.cat((self.keys[:, :, head:], self.keys[:, :, :head]), dim=2),
                torch.cat((self.values[:, :, head:], self.values[:, :, :head]), dim=2))

    def make_mask(self, n_tokens: int, window_size=None, return_array: bool = False):
        """None for one decode token, "causal" for a first chunk within the
        window, else the windowed causal boolean array over the held tokens
        and the chunk (cache.py:199-205)."""
        window = self.window_size if window_size is None else window_size
        if n_tokens == 1 and not return_array:
            return None
        held = self.size()
        if held == 0 and n_tokens <= window and not return_array:
            return "causal"
        T = held + n_tokens
        q = torch.arange(T - n_tokens, T)[:, None]
        k = torch.arange(T)[None]
        return (q >= k) & (q < k + window)

    # ------------------------------------------------------------ writes --
    def _store(self, slot: int, keys: torch.Tensor, values: torch.Tensor):
        """Write rows ``(B, Hkv, L, 128)`` into slots ``[slot, slot + L)`` (no wrap)."""
        B, H, L, D = keys.shape
        k, ksb, ksh, kst = _stride3(keys)
        v, vsb, vsh, vst = _stride3(values)
        rc = _lib.load().rec_kv_write_bf16(
            k.data_ptr(), v.data_ptr(), _DTYPES[keys.dtype], ksb, ksh, kst, vsb, vsh, vst,
            self.keys.data_ptr(), self.keys.stride(0), self.keys.stride(1),
            self.values.data_ptr(), self.values.stride(0), self.values.stride(1),
            B, H, L, D, slot, self.capacity, torch.cuda.current_stream(self.device).cuda_stream,
        )
        _lib.check(rc, "rec_kv_write_bf16")

    def _place(self, keys: torch.Tensor, values: torch.Tensor, end: int):
        """Put the tokens ``[end - n, end)`` of the sequence (the rows of
        ``keys``/``values``, n <= capacity) into their slots, wrapping round."""
        n = keys.shape[2]
        if n == 0:
            return
        first = (end - n) % self.capacity
        run = min(n, self.capacity - first)
        self._store(first, keys[:, :, :run], values[:, :, :run])
        if run < n:
            self._store(0, keys[:, :, run:], values[:, :, run:])

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        if keys.shape != values.shape or keys.dtype not in _DTYPES or values.dtype != keys.dtype:
            raise ValueError("keys/values must share a shape and a float dtype")
        B, H, L, _ = keys.shape
        if (B, H) != tuple(self.keys.shape[:2]):
            raise ValueError(f"keys are (B={B}, Hkv={H}), the ring holds {tuple(self.keys.shape[:2])}")
        if L == 1:
            self._store(self.offset % self.capacity, keys, values)
            self.offset += 1
            n = self.size()
            return self.keys[:, :, :n], self.values[:, :, :n]
        # the held window in order, then the chunk, and the chunk's last
        # rows into their slots: one launch
        n = self.size()
        head = self.offset % self.capacity if self.offset > self.capacity else 0
        attend_k = torch.empty((B, H, n + L, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        attend_v = torch.empty_like(attend_k)
        k, ksb, ksh, kst = _stride3(keys)
        v, vsb, vsh, vst = _stride3(values)
        rc = _lib.load().rec_ring_join_bf16(
            self.keys.data_ptr(), self.values.data_ptr(), self.keys.stride(0), self.keys.stride(1),
            self.values.stride(0), self.values.stride(1), self.capacity, head, n, self.offset, 1,
            k.data_ptr(), v.data_ptr(), _DTYPES[keys.dtype], ksb, ksh, kst, vsb, vsh, vst,
            attend_k.data_ptr(), attend_v.data_ptr(), B, H, L, HEAD_DIM,
            torch.cuda.current_stream(self.device).cuda_stream,
        )
        _lib.check(rc, "rec_ring_join_bf16")  # the chunk's last rows are in their slots too
        self.offset += L
        return attend_k, attend_v

    def grow(self, capacity: int):
        """Widen the ring (up to the window); the held tokens move to their
        slots under the new modulus."""
        capacity = min(self.window_size, capacity)
        if capacity <= self.capacity:
            return
        held_k, held_v = (t.clone() for t in self.window())
        self._alloc(self.keys.shape[0], self.keys.shape[1], capacity)
        self._place(held_k, held_v, self.offset)

    # --------------------------------------------------- snapshot/restore --
    def snapshot(self) -> RingState:
        k, v = self.window()
        return RingState(k.clone(), v.clone(), self.offset)

    def restore(self, state: RingState):
        """Return the ring to ``state`` (the snapshot's tensors stay untouched)."""
        n = state.keys.shape[2]
        if n > self.capacity:
            self.grow(n)
        self.offset = state.offset
        self._place(state.keys, state.values, state.offset)

    def copy(self) -> "FixedSlidingKVCache":
        """An independent ring with the same window and contents."""
        other = object.__new__(FixedSlidingKVCache)
        other.window_size, other.device, other.offset, other.capacity = (
            self.window_size, self.device, self.offset, self.capacity)
        other.keys, other.values = self.keys.clone(), self.values.clone()
        return other


def make_cache(layer_types, *, kv_group_size: int = 64, kv_key_bits: int = 8, kv_value_bits: int = 4,
               sliding_window: int = LOCAL_TOKENS, num_kv_heads: int = 4, max_tokens: Optional[int] = None,
               batch: int = 1, device=None) -> list:
    """One cache per layer, as ``Model.make_cache`` builds them
    (engine/src/rec_mlx/model.py:347-360, defaults from its ModelArgs,
    model.py:30-37): a ``MixedQuantizedKVCache(kv_group_size, kv_key_bits,
    kv_value_bits)`` per ``"full_attention"`` layer (``max_tokens`` allocates
    its whole context at the first append), and per other layer a sliding
    window of ``sliding_window`` tokens -- the bf16 ring
    ``FixedSlidingKVCache`` (the engine's sliding cache, cache.py:153-258)
    where the reference's model takes mlx-lm's ``RotatingKVCache(max_size=
    sliding_window, keep=0)``; its ring is allocated here, on ``device``."""
    caches = []
    for kind in layer_types:
        if kind == "full_attention":
            caches.append(MixedQuantizedKVCache(kv_group_size, kv_key_bits, kv_value_bits, max_tokens=max_tokens))
        else:
            caches.append(FixedSlidingKVCache(max_sequence_tokens=max_tokens or sliding_window,
                                              num_kv_heads=num_kv_heads, head_dim=HEAD_DIM,
                                              window_size=sliding_window, batch=batch, device=device))
    return caches

"""Prompt-prefix reuse with rollback points.

Keeps the behaviour of engine/src/rec_mlx/prefix.py:14-118 (the names the
engine calls: ``PromptCache(tokens, layers, logits, storage)`` with
``fork``, ``advance``, ``checkpoint`` and ``checkpoint_bytes``,
``select_prefix`` and ``PrefillCancelled``) over this library's caches.

A prompt cache remembers the tokens whose K/V its layers hold.  A
full-attention layer keeps every token at its own position, so going back to
an earlier position only moves its ``offset``: the positions past it are
rewritten when the new suffix is prefilled.  A sliding ring overwrites its
oldest tokens, so going back needs what the ring held then.  A rollback point
is therefore the position, one :class:`~rec_amd.kvstorage.RingState` per
sliding layer and the logits at that position.  Points are immutable (a ring
is restored by copying a state in, never by adopting its tensors), so forks
share them and the point a rollback lands on stays usable.  At most two are
kept: the newest and the one before it.
"""

from __future__ import annotations

import copy
import logging
from typing import List, NamedTuple, Optional, Sequence, Tuple

import torch

from .kvstorage import FixedSlidingKVCache, RingState

log = logging.getLogger(__name__)


class PrefillCancelled(Exception):
    """A prefill stopped between chunks at the caller's request."""


class RollbackPoint(NamedTuple):
    position: int  # tokens covered
    rings: Tuple[Tuple[int, RingState], ...]  # (layer index, ring contents) for every sliding layer
    logits: Optional[torch.Tensor]

    @property
    def nbytes(self) -> int:
        n = sum(state.nbytes for _, state in self.rings)
        if self.logits is not None:
            n += self.logits.numel() * self.logits.element_size()
        return n


def _matching_length(a: Sequence[int], b: Sequence[int]) -> int:
    n = min(len(a), len(b))
    for i in range(n):
        if a[i] != b[i]:
            return i
    return n


class PromptCache:
    """Tokens already prefilled, the per-layer caches holding them, the logits
    after the last one, the storage the layers live in, and the rollback
    points (oldest first)."""

    KEEP = 2

    def __init__(self, tokens, layers, logits, storage, points: Optional[List[RollbackPoint]] = None):
        self.tokens: List[int] = list(tokens)
        self.layers = layers
        self.logits = logits
        self.storage = storage
        self.points: List[RollbackPoint] = list(points or [])

    def fork(self) -> "PromptCache":
        """A copy that can advance on its own: private rings, private offsets
        of the full-attention layers (over the shared storage), shared points."""
        layers = [layer.copy() if isinstance(layer, FixedSlidingKVCache) else copy.copy(layer)
                  for layer in self.layers]
        return PromptCache(self.tokens, layers, self.logits, self.storage, self.points)

    def advance(self, tokens, logits):
        """Record ``tokens`` as prefilled into the layers, ``logits`` after them."""
        self.tokens.extend(tokens)
        self.logits = logits

    def checkpoint(self):
        """Add a rollback point at the current position (nothing before the
        first token), keeping the newest ``KEEP``."""
        if not self.tokens:
            return
        rings = tuple((i, layer.snapshot()) for i, layer in enumerate(self.layers)
                      if isinstance(layer, FixedSlidingKVCache))
        self.points = (self.points + [RollbackPoint(len(self.tokens), rings, self.logits)])[-self.KEEP:]

    @property
    def checkpoint_bytes(self) -> int:
        return sum(p.nbytes for p in self.points)

    def rollback(self, point: RollbackPoint):
        """Return every layer to ``point``; later points no longer apply."""
        for layer in self.layers:
            if not isinstance(layer, FixedSlidingKVCache):
                layer.offset = point.position
        for i, state in point.rings:
            self.layers[i].restore(state)
        del self.tokens[point.position:]
        self.logits = point.logits
        self.points = [p for p in self.points if p.position <= point.position]


def select_prefix(prefix: Optional[PromptCache], tokens) -> Tuple[Optional[PromptCache], int]:
    """How much of ``prefix`` a prompt of ``tokens`` can reuse.

    Returns ``(cache, common)``: ``common`` is the length of the prompt's
    match with the cached tokens.  If every cached token matches, the cache
    is returned as it is.  Otherwise it is rolled back to its newest point at
    or before ``common`` and returned, or ``None`` when no such point exists
    (the prompt must be prefilled from scratch).
    """
    common = 0
    if prefix is not None:
        common = _matching_length(prefix.tokens, tokens)
        if common < len(prefix.tokens):
            usable = [p for p in prefix.points if p.position <= common]
            if usable:
                prefix.rollback(max(usable, key=lambda p: p.position))
            else:
                prefix = None
    reused = 0 if prefix is None else len(prefix.tokens)
    log.info("prompt of %d tokens: %d match the cached prefix, %d reused, %d to prefill", len(tokens), common, reused,
             len(tokens) - reused)
    return prefix, common

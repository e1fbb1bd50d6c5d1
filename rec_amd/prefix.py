"""Prompt-prefix checkpoints and rollback of sliding-window rings.

Restates engine/src/rec_mlx/prefix.py:14-118 over this library's caches: a
:class:`PromptCache` keeps the tokens already prefilled, the per-layer caches
and up to two checkpoints, each holding a copy of every
:class:`FixedSlidingKVCache` ring (the slot in use, its valid count and ring
index).  :func:`select_prefix` finds the longest common prefix with a new
prompt; when the prompt diverges inside the cached tokens it rolls every layer
back to the newest checkpoint at or before the divergence (full-attention
layers by offset, rings by restoring the copied slot), so only the suffix needs
prefilling again.  Host bookkeeping plus device copies; no kernels.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Any, List, Optional

import torch

from .kvstorage import FixedSlidingKVCache


class PrefillCancelled(Exception):
    pass


@dataclass
class Checkpoint:
    position: int
    sliding: list
    logits: Optional[torch.Tensor]


@dataclass
class PromptCache:
    tokens: List[int]
    layers: list
    logits: Optional[torch.Tensor]
    storage: Any
    checkpoints: List[Checkpoint] = field(default_factory=list)

    def fork(self) -> "PromptCache":
        """A copy whose rings are private (prefix.py:29-39)."""
        layers = [_shallow_copy(layer) for layer in self.layers]
        for layer in layers:
            if isinstance(layer, FixedSlidingKVCache):
                keys = layer.key_buffers[layer._slot].clone()
                values = layer.value_buffers[layer._slot].clone()
                layer.key_buffers = [keys, torch.zeros_like(keys)]
                layer.value_buffers = [values, torch.zeros_like(values)]
                layer._slot = 0
        return PromptCache(self.tokens[:], layers, self.logits, self.storage, self.checkpoints[:])

    def advance(self, tokens, logits):
        previous = len(self.tokens)
        self.tokens.extend(tokens)
        self.logits = logits
        if len(self.tokens) // 8192 != previous // 8192:
            logging.info("Prefill progress: %d tokens processed", len(self.tokens))

    def checkpoint(self):
        """Keep the newest checkpoint and add one at the current position
        (prefix.py:47-62)."""
        if not self.tokens:
            return
        self.checkpoints = self.checkpoints[-1:]
        sliding = []
        for layer in self.layers:
            if isinstance(layer, FixedSlidingKVCache):
                sliding.append((layer.key_buffers[layer._slot].clone(), layer.value_buffers[layer._slot].clone(),
                                layer._valid, layer._ring_index))
        self.checkpoints.append(Checkpoint(len(self.tokens), sliding, self.logits))

    @property
    def checkpoint_bytes(self) -> int:
        total = 0
        for cp in self.checkpoints:
            total += sum(k.numel() * k.element_size() + v.numel() * v.element_size() for k, v, _, _ in cp.sliding)
            if cp.logits is not None:
                total += cp.logits.numel() * cp.logits.element_size()
        return total


def _shallow_copy(layer):
    import copy

    return copy.copy(layer)


def select_prefix(prefix: Optional[PromptCache], tokens):
    """``(prefix or None, common)``: reuse ``prefix`` as far as it matches
    ``tokens``, rolling back to a checkpoint when they diverge inside it
    (prefix.py:74-118)."""
    common = 0
    if prefix is not None:
        for previous, current in zip(prefix.tokens, tokens):
            if previous != current:
                break
            common += 1
        if common != len(prefix.tokens):
            checkpoint = next((item for item in reversed(prefix.checkpoints) if item.position <= common), None)
            if checkpoint is None:
                prefix = None
            else:
                sliding = iter(checkpoint.sliding)
                for layer in prefix.layers:
                    layer.offset = checkpoint.position
                    if isinstance(layer, FixedSlidingKVCache):
                        keys, values, layer._valid, layer._ring_index = next(sliding)
                        layer.capacity = keys.shape[-2]
                        layer.key_buffers = [keys, torch.zeros_like(keys)]
                        layer.value_buffers = [values, torch.zeros_like(values)]
                        layer._slot = 0
                prefix.tokens = prefix.tokens[: checkpoint.position]
                prefix.logits = checkpoint.logits
                prefix.checkpoints = [item for item in prefix.checkpoints if item.position < checkpoint.position]
    cached = 0 if prefix is None else len(prefix.tokens)
    logging.info("Prefill: prompt=%d common_prefix=%d reused=%d new=%d", len(tokens), common, cached,
                 len(tokens) - cached)
    return prefix, common

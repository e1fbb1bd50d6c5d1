"""Prompt-prefix reuse and rollback (rec_amd.prefix) over a full-attention
bf16 layer and a 5-token sliding ring, on the GPU.

Scenarios (token sequences and the expected match lengths) follow the
reference's engine/tests/test_prefix_rollback.py; the checks are on this
library's layers: the ring's window in sequence order, the full-attention
layer's visible rows, the logits, and a decode step through ``attend`` after
a rollback against the same step on a cache prefilled from scratch.
"""

import pytest
import torch

from rec_amd import FixedKVCache, FixedSlidingKVCache, KVStorage, attend
from rec_amd.prefix import PromptCache, select_prefix

pytestmark = pytest.mark.gpu

WINDOW = 5


def rows(values):
    """K/V rows for token values: K repeats the value over the 128 dims, V is K + 0.5."""
    k = torch.tensor(values, dtype=torch.float32, device="cuda").reshape(1, 1, -1, 1).expand(1, 1, -1, 128)
    return k.to(torch.bfloat16), (k + 0.5).to(torch.bfloat16)


class Session:
    """A prompt cache over [full-attention layer, sliding ring]."""

    def __init__(self):
        full = FixedKVCache(KVStorage(1, 64, 1), 0)
        ring = FixedSlidingKVCache(max_sequence_tokens=WINDOW, num_kv_heads=1, head_dim=128, window_size=WINDOW)
        self.prompt = PromptCache([], [full, ring], None, full.storage)

    @property
    def full(self):
        return self.prompt.layers[0]

    @property
    def ring(self):
        return self.prompt.layers[1]

    def feed(self, values, prompt=None):
        prompt = prompt or self.prompt
        k, v = rows(values)
        for layer in prompt.layers:
            layer.update_and_fetch(k, v)
        prompt.advance(values, k[:, :, -1:, 0].float().clone())  # stand-in logits: the last token's value

    def state(self, prompt=None):
        """(visible full-attention K, V; the ring's window K, V) as clones."""
        prompt = prompt or self.prompt
        full, ring = prompt.layers
        data = full.storage.layer(full.index, full.offset)
        return [t.clone() for t in (data[:, 0], data[:, 1], *ring.window())]


def assert_same(a, b, what):
    for x, y in zip(a, b, strict=True):
        assert x.shape == y.shape and torch.equal(x, y), what


def decode_step(prompt, value=3.0, seed=5):
    """One decode token through attend() over each layer; returns both outputs."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((1, 8, 1, 128), generator=g, device="cuda", dtype=torch.bfloat16)
    k, v = rows([value])
    return [attend(q, k, v, layer, 0.0884, None, None, out_dtype=torch.float32) for layer in prompt.layers]


def test_divergence_rolls_back_to_newest_point_then_replays(gpu):
    s = Session()
    s.feed(list(range(7)))
    s.feed([7])
    at8 = s.state()
    s.prompt.checkpoint()
    s.feed([8, 9, 10])
    s.prompt.checkpoint()
    s.feed([11, 12])
    storage = s.prompt.storage
    # the prompt matches the first 9 cached tokens; the newest point at or
    # before 9 is at 8 (the one at 11 is past the divergence)
    prompt, common = select_prefix(s.prompt, list(range(9)) + [100, 101])
    assert prompt is s.prompt and prompt.storage is storage
    assert common == 9 and prompt.tokens == list(range(8))
    assert s.full.offset == 8 and s.ring.offset == 8
    assert_same(s.state(), at8, "rolled-back state differs from the state at the point")
    assert torch.equal(prompt.logits, torch.full((1, 1, 1), 7.0, device="cuda"))
    # replaying the new suffix gives what a prefill from scratch gives
    s.feed([8, 100, 101])
    fresh = Session()
    fresh.feed(list(range(9)) + [100, 101])
    assert prompt.tokens == fresh.prompt.tokens
    assert_same(s.state(), fresh.state(), "replayed state differs from a fresh prefill")
    for a, b in zip(decode_step(s.prompt), decode_step(fresh.prompt)):
        assert torch.equal(a, b)


def test_point_bound_exact_hit_shortening_and_early_edit(gpu):
    s = Session()
    for value in range(12):
        s.prompt.checkpoint()
        s.feed([value])
        assert len(s.prompt.points) <= PromptCache.KEEP
    assert [p.position for p in s.prompt.points] == [10, 11]
    assert s.prompt.checkpoint_bytes > 0
    # a longer prompt that extends the cached tokens reuses all of them
    prompt, common = select_prefix(s.prompt, list(range(13)))
    assert prompt is s.prompt and common == 12 and len(prompt.tokens) == 12
    # a shorter one rolls back to the point at its end
    prompt, common = select_prefix(prompt, list(range(10)))
    assert common == 10 and prompt.tokens == list(range(10))
    assert_same(s.state()[2:], [t[:, :, 5:10] for t in rows(list(range(12)))], "ring window after shortening")
    # an edit before every point leaves nothing to reuse
    assert select_prefix(prompt, [99]) == (None, 0)


def test_rollback_into_a_wrapped_ring(gpu):
    """Points taken after the ring has wrapped restore the window in sequence
    order whatever slot the oldest token sits in."""
    s = Session()
    s.feed(list(range(7)))  # a chunk: the ring keeps 2..6
    for value in range(7, 13):  # single tokens wrap the ring round
        if value == 10:
            s.prompt.checkpoint()
            at10 = s.state()
        s.feed([value])
    prompt, common = select_prefix(s.prompt, list(range(11)) + [50])
    assert common == 11 and prompt.tokens == list(range(10))
    assert_same(s.state(), at10, "window after rolling back into a wrapped ring")
    assert_same(s.state()[2:], [t[:, :, 5:10] for t in rows(list(range(12)))], "window holds tokens 5..9")
    s.feed([10, 50])
    fresh = Session()
    fresh.feed(list(range(11)) + [50])
    assert_same(s.state(), fresh.state(), "replay after a wrapped rollback")


def test_fork_has_private_rings_and_offsets(gpu):
    s = Session()
    s.feed(list(range(6)))
    s.prompt.checkpoint()
    before = s.state()
    fork = s.prompt.fork()
    s.feed([50], prompt=fork)
    assert fork.tokens == list(range(6)) + [50] and s.prompt.tokens == list(range(6))
    assert s.full.offset == 6 and fork.layers[0].offset == 7
    assert_same(s.state(), before, "the original changed when its fork advanced")
    assert not torch.equal(s.state(fork)[2], before[2])
    # points are immutable and shared
    assert len(fork.points) == 1 and all(a is b for a, b in zip(fork.points, s.prompt.points))

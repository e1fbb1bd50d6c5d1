"""Prompt-prefix checkpoints and ring rollback (engine/src/rec_mlx/prefix.py),
mirroring the reference's engine/tests/test_prefix_rollback.py:14-63 with
this library's sliding-window cache (head_dim 128: each token's value is
repeated over the 128 dims)."""

from types import SimpleNamespace

import pytest
import torch

from rec_amd import FixedSlidingKVCache
from rec_amd.prefix import PromptCache, select_prefix

pytestmark = pytest.mark.gpu


def make_prefix():
    ring = FixedSlidingKVCache(max_sequence_tokens=5, num_kv_heads=1, head_dim=128, window_size=5)
    return PromptCache([], [SimpleNamespace(offset=0), ring], None, object())


def append(prefix, values):
    data = torch.tensor(values, dtype=torch.bfloat16, device="cuda").reshape(1, 1, -1, 1).expand(1, 1, -1, 128)
    prefix.layers[1].update_and_fetch(data, -data)
    prefix.layers[0].offset += len(values)
    prefix.tokens.extend(values)
    prefix.logits = data[:, :, -1:]


def priors(prefix):
    return [x.clone() for x in prefix.layers[1]._prior()]


def test_mismatch_restores_physical_ring_then_replays_suffix(gpu):
    prefix = make_prefix()
    append(prefix, list(range(7)))
    append(prefix, [7])
    expected = priors(prefix)
    prefix.checkpoint()
    append(prefix, [8, 9, 10])
    prefix.checkpoint()
    append(prefix, [11, 12])
    storage = prefix.storage
    restored, common = select_prefix(prefix, list(range(9)) + [100, 101])
    assert restored is prefix and restored.storage is storage
    assert common == 9 and len(restored.tokens) == 8 and restored.layers[0].offset == 8
    for actual, wanted in zip(priors(restored), expected, strict=True):
        assert torch.equal(actual, wanted)
    append(restored, [8, 100, 101])
    fresh = make_prefix()
    append(fresh, list(range(9)) + [100, 101])
    for actual, wanted in zip(priors(restored), priors(fresh), strict=True):
        assert torch.equal(actual, wanted)


def test_shortening_exact_hit_early_edit_and_snapshot_bound(gpu):
    prefix = make_prefix()
    for value in range(12):
        prefix.checkpoint()
        append(prefix, [value])
        assert len(prefix.checkpoints) <= 2
    assert prefix.checkpoint_bytes > 0
    assert select_prefix(prefix, list(range(13)))[0] is prefix
    restored, common = select_prefix(prefix, list(range(10)))
    assert common == 10 and len(restored.tokens) == 10
    assert select_prefix(restored, [99])[0] is None


def test_fork_has_private_rings(gpu):
    prefix = make_prefix()
    append(prefix, list(range(6)))
    fork = prefix.fork()
    append(fork, [50])
    assert not torch.equal(priors(fork)[0], priors(prefix)[0])
    assert prefix.layers[1].key_buffers[prefix.layers[1]._slot].data_ptr() != fork.layers[1].key_buffers[0].data_ptr()

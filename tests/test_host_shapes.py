"""Host-side shape checks of the quantized attention path: a query batch or
head count the cache does not hold is refused before anything is launched
(the kernels index the cache from the query shape and cannot see tensor
sizes).  CPU tensors stand in for the cache; nothing reaches the GPU."""

import pytest
import torch

from rec_amd.attention import _check_cache_shapes
from rec_amd.cache import QuantizedKV


def kv(B, H, T, bits=8, blocked=False, cap=64):
    codes = torch.zeros((B, H, cap // 32, 32 * 128 * bits // 8), dtype=torch.int8 if bits == 8 else torch.uint8)
    scales = torch.zeros((B, H, cap // 32, 32), dtype=torch.float16)
    return QuantizedKV(codes, scales, None, bits, T, blocked)


def q(B, Hq):
    return torch.zeros((B, Hq, 1, 128))


def test_matching_shapes_pass():
    _check_cache_shapes(q(2, 16), kv(2, 4, 10), kv(2, 4, 10, blocked=True))


@pytest.mark.parametrize(
    "qs,ks,vs,msg",
    [
        ((3, 16), (2, 4, 10), (2, 4, 10), "batch 3"),
        ((1, 16), (2, 4, 10), (2, 4, 10), "batch 1"),
        ((2, 10), (2, 4, 10), (2, 4, 10), "not a multiple"),
        ((2, 16), (2, 4, 10), (2, 2, 10), "do not match"),
        ((2, 16), (2, 4, 10), (1, 4, 10), "do not match"),
        ((2, 16), (2, 4, 10), (2, 4, 11), "do not match"),
    ],
)
def test_mismatches_refused(qs, ks, vs, msg):
    with pytest.raises(ValueError, match=msg):
        _check_cache_shapes(q(*qs), kv(*ks), kv(*vs, blocked=True))

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


# ---- mask arrays (model.py:122-128) -> the kernels' (causal, window) ----
import numpy as np  # noqa: E402

from rec_amd.attention import _mask_bias, _mask_plan  # noqa: E402


def causal_keep(L, T, window=0):
    q = torch.arange(T - L, T)[:, None]
    k = torch.arange(T)[None]
    m = q >= k
    return m & (q < k + window) if window else m


def test_mask_plan_strings_and_none():
    assert _mask_plan(None, 5, 9) == (False, 0)
    assert _mask_plan("causal", 5, 9) == (True, 0)
    with pytest.raises(NotImplementedError):
        _mask_plan("sliding", 5, 9)


@pytest.mark.parametrize("L,T", [(1, 1), (1, 50), (7, 7), (7, 40), (64, 300)])
def test_mask_plan_boolean_and_additive(L, T):
    keep = causal_keep(L, T)
    want = (False, 0) if L == 1 else (True, 0)  # one query: causal keeps every key
    assert _mask_plan(keep, L, T) == want
    assert _mask_plan(keep[None, None], L, T) == want  # (1, 1, L, T)
    assert _mask_plan(keep.expand(2, 3, L, T), L, T) == want  # the same pattern for every sequence and head
    assert _mask_plan(keep.numpy(), L, T) == want
    additive = torch.zeros(L, T).masked_fill(~keep, float("-inf"))
    assert _mask_plan(additive, L, T) == want
    assert _mask_plan(torch.ones(L, T, dtype=torch.bool), L, T) == (False, 0)
    assert _mask_plan(torch.zeros(1, T), L, T) == (False, 0)  # a row broadcast over the queries
    if T > 3:
        w = T // 2
        assert _mask_plan(causal_keep(L, T, w), L, T) == (True, w)


def test_mask_plan_leaves_other_patterns_to_the_bias():
    """Host arrays of another pattern have no fast path (None: they run as a
    bias); shapes that do not broadcast and integer masks are refused."""
    L, T = 6, 20
    keep = causal_keep(L, T)
    odd = keep.clone()
    odd[2, 0] = False  # a hole in one row
    assert _mask_plan(odd, L, T) is None
    assert _mask_plan(torch.zeros(L, T).masked_fill(~keep, -1e4), L, T) is None  # finite additive
    per_head = torch.stack([keep, torch.ones_like(keep)])[None]
    assert _mask_plan(per_head, L, T) is None  # differs between heads
    with pytest.raises(ValueError, match="broadcast"):
        _mask_plan(keep[:, :-1], L, T)
    with pytest.raises(NotImplementedError):
        _mask_plan(np.zeros((L, T), np.int32), L, T)


def test_mask_plan_does_not_inspect_device_arrays():
    """A mask array on the GPU is never read on the host (no synchronisation,
    capturable): it always runs as a bias.  A stand-in object with a device
    other than the CPU shows the rule without a GPU."""

    class OnDevice(torch.Tensor):
        @property
        def device(self):
            return torch.device("cuda", 0)

    m = torch.ones(3, 9, dtype=torch.bool).as_subclass(OnDevice)
    assert _mask_plan(m, 3, 9) is None


def _scores_bias(mask, B, Hkv, G, L, T):
    """The bias the kernels would read, gathered back into (B, Hkv, G, L, T)
    from its strides (on the CPU)."""
    buf, (sb, skv, sg, sl, ext) = _mask_bias(mask, B, Hkv, G, L, T, "cpu")
    flat = buf.reshape(-1)
    assert flat.numel() == ext and buf.data_ptr() % 16 == 0
    assert all(x % 4 == 0 for x in (sb, skv, sg, sl))
    out = torch.empty(B, Hkv, G, L, T)
    for b in range(B):
        for h in range(Hkv):
            for g in range(G):
                for l in range(L):
                    o = b * sb + h * skv + g * sg + l * sl
                    out[b, h, g, l] = flat[o : o + T]
    return out


def test_mask_bias_follows_the_reference_broadcasting():
    """model.py:122-128: bool -> 0 / -inf, float as it is; a 4-D mask
    (B, Hkv, L, T) gains the group axis; 3-D (G, L, T) and 2-D (L, T) broadcast
    from the right.  Checked against explicit broadcasting of the same array."""
    B, Hkv, G, L, T = 2, 3, 4, 5, 11
    g = torch.Generator().manual_seed(3)
    cases = [
        torch.rand(L, T, generator=g) > 0.3,                  # (L, T)
        torch.rand(1, T, generator=g) > 0.3,                  # one row for every query
        torch.randn(G, L, T, generator=g),                    # per group member, additive
        torch.rand(B, 1, 1, T, generator=g) > 0.5,            # padding: per sequence
        torch.randn(B, Hkv, L, T, generator=g),               # per sequence and KV head
        torch.rand(1, Hkv, 1, T, generator=g) > 0.5,
        torch.rand(L, 1, generator=g) > 0.5,                  # broadcast over the keys
    ]
    for m in cases:
        got = _scores_bias(m, B, Hkv, G, L, T)
        ref = m.float() if m.is_floating_point() else torch.where(m, 0.0, float("-inf"))
        if ref.dim() == 4:
            ref = ref.unsqueeze(-3)
        assert torch.equal(got, ref.expand(B, Hkv, G, L, T)), tuple(m.shape)
    with pytest.raises(ValueError, match="broadcast"):
        _mask_bias(torch.ones(3, L, T, dtype=torch.bool), B, Hkv, G, L, T, "cpu")  # 3 is neither 1 nor G
    with pytest.raises(NotImplementedError):
        _mask_bias(torch.ones(1, 1, 1, L, T, dtype=torch.bool), B, Hkv, G, L, T, "cpu")


def test_sink_rounding_on_the_host():
    """The sinks the SDPA-style paths see: rounded to the query dtype once per
    tensor version (a kept copy, so decode steps launch no cast), float32 as
    given otherwise; an in-place change makes a new copy."""
    from rec_amd.attention import _sink_copies, _sinks

    s = torch.tensor([2.5 + 0.4 * 2.0**-6, -1.0, 3.0 + 2.0**-9, 0.1])
    f = _sinks(s, 4, "cpu")
    assert torch.equal(f, s)
    b = _sinks(s, 4, "cpu", torch.bfloat16)
    assert torch.equal(b, s.to(torch.bfloat16).float()) and not torch.equal(b, s)
    assert _sinks(s, 4, "cpu", torch.bfloat16) is b  # the kept copy
    h = _sinks(s, 4, "cpu", torch.float16)
    assert torch.equal(h, s.half().float()) and h is not b
    s.mul_(2.0)
    b2 = _sinks(s, 4, "cpu", torch.bfloat16)
    assert b2 is not b and torch.equal(b2, s.to(torch.bfloat16).float())
    n = len(_sink_copies)
    del s, f  # (f is s: float32 sinks pass through as they are)
    assert len(_sink_copies) == n - 1  # dropped with the tensor
    assert torch.equal(_sinks([0.3, 7.0], 2, "cpu", torch.bfloat16), torch.tensor([0.3, 7.0]).bfloat16().float())
    with pytest.raises(ValueError, match="expected 8"):
        _sinks(torch.zeros(4), 8, "cpu", torch.bfloat16)


def test_storage_metadata_rows_follow_the_reference():
    """Columns 61-62 of the reference's layer table (cache.py:54-63): a
    full-attention layer's element offset in its bank (layers in order,
    65,536 x 1,024 elements each) and 65,536 tokens; a sliding-window layer's
    offset past all of them (513 x 1,024 each) and 513 tokens."""
    from rec_amd.kvstorage import _metadata_rows

    rows = [[0] * 64 for _ in range(50)]
    for i, row in enumerate(rows[:49]):
        row[1] = int(i % 4 == 0)
    out = _metadata_rows(rows)
    n_global = 13
    assert out[0][61:63] == [0, 65536] and out[4][61:63] == [65536 * 1024, 65536]
    assert out[48][61:63] == [12 * 65536 * 1024, 65536]
    assert out[1][61:63] == [n_global * 65536 * 1024, 513]
    assert out[2][61:63] == [n_global * 65536 * 1024 + 513 * 1024, 513]
    assert out[47][61:63] == [n_global * 65536 * 1024 + 35 * 513 * 1024, 513]
    assert out[49] == rows[49] and rows[0][61] == 0  # row 50 untouched, the input not modified
    with pytest.raises(ValueError):
        _metadata_rows([[0] * 10])


def test_q4_routing_follows_the_measured_crossing(monkeypatch):
    """q4_gemv runs GEMV launches of 8 rows below gemm_min_rows(K) rows of x
    and one GEMM from there (the crossing measured on MI355X: between 32 and
    48 rows at K = 2048, between 48 and 64 at K = 4096).  The library is
    replaced by a recorder: no kernel runs."""
    from rec_amd import _lib, gemv

    assert [gemv.gemm_min_rows(K) for K in (512, 1024, 2048, 4096, 6144)] == [24, 32, 40, 56, 72]
    calls = []

    class Recorder:
        def rec_q4_gemm_workspace_bytes(self, M, K):
            return 16

        def rec_q4_gemm(self, *args):
            calls.append(("gemm", args[5]))
            return 0

        def rec_q4_gemv(self, *args):
            calls.append(("gemv", args[5]))
            return 0

    class Stream:
        cuda_stream = 0

    monkeypatch.setattr(_lib, "load", lambda: Recorder())
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: Stream())
    m = object.__new__(gemv.Q4Matrix)
    m.N, m.K, m.parts = 8, 2048, (8,)
    m.packed = torch.zeros(16, dtype=torch.uint8)
    for rows, want in ((1, [("gemv", 1)]), (39, [("gemv", 8)] * 4 + [("gemv", 7)]), (40, [("gemm", 40)])):
        calls.clear()
        y = gemv.q4_gemv(torch.zeros(rows, 2048, dtype=torch.bfloat16), m)
        assert y.shape == (rows, 8) and calls == want, (rows, calls)

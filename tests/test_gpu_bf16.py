"""Parity of the bf16 KV-cache path (KVStorage / FixedKVCache and its decode
kernel) with the CPU oracle.

Stored K/V must be the bf16 rounding of the inputs, bit for bit; attention
outputs within 2e-3 absolute + 1e-3 relative of the float64 oracle computed
on the stored bf16 values (the reference's cache holds bf16,
engine/src/rec_mlx/cache.py:30-45).
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import FixedKVCache, KVStorage, attend, scaled_dot_product_attention, synthetic
from tests.gpu_util import SCALE, assert_close, f32, q_sinks

pytestmark = pytest.mark.gpu


def bf16_np(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).float().cpu().numpy()


CASES = [
    # B, Hq, Hkv, T, q dtype, sinks, splits
    (1, 8, 1, 1024, torch.bfloat16, False, None),
    (1, 32, 4, 4096, torch.bfloat16, True, None),
    (1, 32, 4, 777, torch.float16, True, 5),
    (2, 16, 2, 300, torch.float32, False, 256),
    (1, 4, 1, 1, torch.bfloat16, True, None),
    (3, 24, 4, 65, torch.bfloat16, True, 1),
    (1, 8, 8, 2049, torch.float16, False, 3),
    # long splits (79 and 66 chunks)
    (1, 32, 4, 5000, torch.bfloat16, True, 2),
    (1, 8, 1, 2100, torch.float16, False, 1),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}_Hq{c[1]}_Hkv{c[2]}_T{c[3]}_{str(c[4])[6:]}_s{c[5]}_sp{c[6]}")
def test_bf16_decode_matches_oracle(gpu, case):
    B, Hq, Hkv, T, qdt, use_sinks, splits = case
    k = synthetic.kv((B, Hkv, T, 128), 21, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 22, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, 1, 23, dtype=qdt)
    sinks = torch.randn(Hq, device="cuda") if use_sinks else None
    out = scaled_dot_product_attention(q, k, v, SCALE, None, sinks, out_dtype=torch.float32, splits=splits)
    torch.cuda.synchronize()
    ref = O.attention(f32(q), f32(k), f32(v), SCALE, sinks=None if sinks is None else f32(sinks))
    assert_close(f32(out), ref, f"case {case}")


def test_fixed_kv_cache_prefill_then_fused_decode(gpu):
    """update_and_fetch stores bf16(x) bit for bit; fused decode steps (write the
    new token, then attend) match the oracle at every step."""
    B, Hq, Hkv, P = 1, 32, 4, 1000
    store = KVStorage(2, 2048, Hkv)
    cache = FixedKVCache(store, 1)
    assert cache.empty() and cache.make_mask(1) is None and cache.make_mask(5) == "causal"
    k = synthetic.kv((B, Hkv, P + 6, 128), 31, kind="outliers", frac=0.01, dtype=torch.float16)
    v = synthetic.kv((B, Hkv, P + 6, 128), 32, kind="outliers", frac=0.01, dtype=torch.float16)
    kk, vv = cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    assert kk.shape == (B, Hkv, P, 128) and cache.offset == P
    np.testing.assert_array_equal(kk.float().cpu().numpy(), bf16_np(k[:, :, :P]))
    np.testing.assert_array_equal(vv.float().cpu().numpy(), bf16_np(v[:, :, :P]))
    sinks = torch.randn(Hq, device="cuda")
    for step in range(6):
        T = P + step + 1
        q = synthetic.query(B, Hq, 1, 40 + step, dtype=torch.bfloat16)
        out = attend(q, k[:, :, T - 1 : T], v[:, :, T - 1 : T], cache, SCALE, None, sinks, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert cache.offset == T
        ref = O.attention(f32(q), bf16_np(k[:, :, :T]), bf16_np(v[:, :, :T]), SCALE, sinks=q_sinks(sinks, q.dtype))
        assert_close(f32(out), ref, f"step {step}")
    data = store.layer(1, cache.offset)
    np.testing.assert_array_equal(data[:, 0].float().cpu().numpy(), bf16_np(k))
    np.testing.assert_array_equal(data[:, 1].float().cpu().numpy(), bf16_np(v))
    assert torch.count_nonzero(store.layer(0)) == 0  # the other layer is untouched


@pytest.mark.parametrize("P,cap,splits", [(333, 1024, None), (2500, 4096, 1)])
def test_fused_equals_write_then_attend(gpu, P, cap, splits):
    """The fused write + attend launch equals a write then an attend: bit for
    bit where both partition the tokens alike; the second case (one split of
    78 chunks) partitions them differently, so it agrees to fp32 rounding."""
    B, Hq, Hkv = 2, 16, 2
    outs = []
    for fused in (True, False):
        store = KVStorage(1, cap, Hkv, batch=B)
        cache = FixedKVCache(store, 0)
        k = synthetic.kv((B, Hkv, P + 1, 128), 51, dtype=torch.bfloat16)
        v = synthetic.kv((B, Hkv, P + 1, 128), 52, dtype=torch.bfloat16)
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
        q = synthetic.query(B, Hq, 1, 53, dtype=torch.bfloat16)
        outs.append(attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, None, None, out_dtype=torch.float32,
                           fused=fused, splits=splits))
    torch.cuda.synchronize()
    tol = 0 if splits is None else 1e-5
    torch.testing.assert_close(outs[0], outs[1], rtol=tol, atol=tol)


@pytest.mark.parametrize("splits", [None, 8])
def test_long_context_bf16(gpu, splits):
    """32K tokens: the default split schedule over a long cache, and 8 splits
    of 4096 tokens."""
    B, Hq, Hkv, T = 1, 32, 4, 32768
    k = synthetic.kv((B, Hkv, T, 128), 61, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 62, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, 1, 63, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    out = scaled_dot_product_attention(q, k, v, SCALE, None, sinks, out_dtype=torch.float32, splits=splits)
    torch.cuda.synchronize()
    ref = O.attention(f32(q), f32(k), f32(v), SCALE, sinks=f32(sinks))
    assert_close(f32(out), ref, f"32K bf16, splits {splits}")


def test_fused_decode_in_hip_graph(gpu):
    """Fused bf16 decode steps captured in a HIP graph and replayed several
    times, with eager work between replays, match eager steps every time."""
    B, Hq, Hkv, P, steps = 1, 32, 4, 700, 4
    k = synthetic.kv((B, Hkv, P + steps, 128), 71, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, P + steps, 128), 72, dtype=torch.bfloat16)
    qs = [synthetic.query(B, Hq, 1, 80 + i, dtype=torch.bfloat16) for i in range(steps)]
    sinks = torch.randn(Hq, device="cuda")

    def run(cache, outs):
        for i in range(steps):
            T = P + i + 1
            outs[i].copy_(attend(qs[i], k[:, :, T - 1 : T], v[:, :, T - 1 : T], cache, SCALE, None, sinks,
                                 out_dtype=torch.float32))

    store = KVStorage(1, 1024, Hkv)
    cache = FixedKVCache(store, 0)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    eager = [torch.empty((B, Hq, 1, 128), device="cuda") for _ in range(steps)]
    run(cache, eager)
    torch.cuda.synchronize()

    cache.offset = P
    graph_out = [torch.empty_like(e) for e in eager]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(cache, graph_out)
    for rep in range(3):
        for o in graph_out:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i in range(steps):
            torch.testing.assert_close(graph_out[i], eager[i], rtol=0, atol=0, msg=f"replay {rep} step {i}")


def test_region_dropped_inside_a_capture_is_released_later(gpu):
    """A storage dropped while a graph is being captured cannot synchronise
    the device to release its region: the region waits and is released by
    the next region created outside the capture; the graph replays."""
    import gc

    from rec_amd import kvstorage

    kvstorage._release_retired()
    store = KVStorage(1, 256, 2)
    store.layer(0).fill_(1)
    x = torch.zeros(8, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        x.add_(1)
        del store
        gc.collect()
    assert len(kvstorage._RETIRED) == 1
    other = KVStorage(1, 256, 2)  # releases the retired region first
    assert not kvstorage._RETIRED
    assert other.layer(0).abs().sum().item() == 0  # a fresh region reads zeros
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    assert x.tolist() == [2.0] * 8


def test_bf16_rejects_bad_inputs(gpu):
    k = torch.zeros((1, 4, 64, 128), dtype=torch.float16, device="cuda")
    q = torch.zeros((1, 32, 1, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        scaled_dot_product_attention(q, k, k, SCALE)
    store = KVStorage(1, 100, 4)
    cache = FixedKVCache(store, 0)
    with pytest.raises(ValueError, match="Decode context limit exhausted"):
        cache.update_and_fetch(torch.zeros((1, 4, 262145, 128), dtype=torch.bfloat16, device="cuda"),
                               torch.zeros((1, 4, 262145, 128), dtype=torch.bfloat16, device="cuda"))


def test_storage_grows_by_banks_without_moving(gpu):
    """Growing past a 65,536-token bank maps the next bank behind the first
    (cache.py:63-84): earlier rows keep their addresses and bytes, views taken
    before the growth stay valid, new banks read zeros, and a decode step and a
    prefill chunk that straddle the bank boundary match the oracle."""
    B, Hq, Hkv, P, L = 1, 8, 1, 65530, 20
    store = KVStorage(2, 1000, Hkv)
    assert store.capacity == 65536 and store.nbytes == 2 * (2 * Hkv * 65536 * 128 * 2)
    base = [r.data_ptr() for r in store.regions]
    cache = FixedKVCache(store, 1)
    k = synthetic.kv((B, Hkv, P + L + 1, 128), 71, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, P + L + 1, 128), 72, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    early = store.layer(1, 64)  # a view taken before the growth
    # a chunk across the bank boundary: the storage grows to two banks
    q = synthetic.query(B, Hq, L, 73, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    out = attend(q, k[:, :, P : P + L], v[:, :, P : P + L], cache, SCALE, "causal", sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert store.capacity == 2 * 65536 and [r.data_ptr() for r in store.regions] == base
    assert store.nbytes == 2 * (2 * Hkv * 2 * 65536 * 128 * 2)
    T = P + L
    ref = O.attention(f32(q), f32(k[:, :, :T]), f32(v[:, :, :T]), SCALE, sinks=q_sinks(sinks, q.dtype), mask="causal")
    assert_close(f32(out), ref, "prefill chunk across the bank boundary")
    # one decode token after it
    q1 = synthetic.query(B, Hq, 1, 74, dtype=torch.bfloat16)
    out1 = attend(q1, k[:, :, T : T + 1], v[:, :, T : T + 1], cache, SCALE, None, sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref1 = O.attention(f32(q1), f32(k[:, :, : T + 1]), f32(v[:, :, : T + 1]), SCALE, sinks=q_sinks(sinks, q1.dtype))
    assert_close(f32(out1), ref1, "decode step after the bank boundary")
    data = store.layer(1, T + 1)
    assert torch.equal(data[:, 0], k) and torch.equal(data[:, 1], v)
    assert torch.equal(early[:, 0], k[:, :, :64]) and torch.equal(early[:, 1], v[:, :, :64])
    assert torch.count_nonzero(store.layer(1)[:, :, :, T + 1 :]) == 0
    assert torch.count_nonzero(store.layer(0)) == 0
    with pytest.raises(ValueError, match="Decode context limit exhausted"):
        store.grow(4 * 65536 + 1)
    store.grow(4 * 65536)  # the last two banks at once
    assert store.capacity == 4 * 65536 and [r.data_ptr() for r in store.regions] == base
    assert torch.equal(store.layer(1, T + 1)[:, 0], k)


def test_sliding_window_ring_decode(gpu):
    """A window-40 ring fed 1-token steps well past the window (and one
    multi-token chunk): every decode step attends exactly the last
    min(window, offset) tokens (cache.py:153-258)."""
    from rec_amd import FixedSlidingKVCache

    B, Hq, Hkv, W = 1, 16, 2, 40
    cache = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W)
    n = 130
    k = synthetic.kv((B, Hkv, n, 128), 91, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, n, 128), 92, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    pos = 0
    for step in range(n):
        if step == 60:  # one multi-token chunk: returns ring order + new tokens, keeps the last W
            kk, vv = cache.update_and_fetch(k[:, :, pos : pos + 7], v[:, :, pos : pos + 7])
            np.testing.assert_array_equal(kk.float().cpu().numpy(), bf16_np(k[:, :, max(0, pos + 7 - W - 7) : pos + 7])[:, :, -kk.shape[2]:])
            pos += 7
            assert cache.size() == W and cache.offset == pos
            continue
        if pos >= n:
            break
        q = synthetic.query(B, Hq, 1, 100 + step, dtype=torch.bfloat16)
        out = attend(q, k[:, :, pos : pos + 1], v[:, :, pos : pos + 1], cache, SCALE, None, sinks,
                     out_dtype=torch.float32)
        pos += 1
        lo = max(0, pos - W)
        torch.cuda.synchronize()
        assert cache.size() == pos - lo
        ref = O.attention(f32(q), bf16_np(k[:, :, lo:pos]), bf16_np(v[:, :, lo:pos]), SCALE, sinks=q_sinks(sinks, q.dtype))
        assert_close(f32(out), ref, f"step {step}")
    assert cache.make_mask(1) is None
    m = cache.make_mask(3, return_array=True)
    assert m.shape == (3, W + 3) and bool(m[0, 0]) is False and bool(m[2, -1]) is True


@pytest.mark.parametrize("P", [1000, 1276], ids=["slot487_wraps", "slot250_middle"])
@pytest.mark.parametrize("splits", [None, 1, 8], ids=["auto", "s1", "s8"])
def test_ring_decode_513_fused_vs_unfused(gpu, P, splits):
    """The 513-token window layer (B = 2, 32 query / 4 KV heads): fused steps
    (the new token written into its slot by the split that reads it) against
    a twin ring stepped unfused (update_and_fetch, then attention).  Each
    step's output matches the oracle over the last 513 tokens, and the two
    rings' slots are bit-equal after every step.  After 1,000 tokens the
    write slot starts at 487 and wraps past 512 within the steps; after
    1,276 it starts at 250, inside a middle split."""
    from rec_amd import FixedSlidingKVCache

    B, Hq, Hkv, W, steps = 2, 32, 4, 513, 30
    n = P + steps
    k = synthetic.kv((B, Hkv, n, 128), 201 + P, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, n, 128), 202 + P, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    fused = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W, batch=B)
    twin = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W, batch=B)
    assert fused.capacity == W
    fused.update_and_fetch(k[:, :, :P], v[:, :, :P])
    twin.update_and_fetch(k[:, :, :P], v[:, :, :P])
    for step in range(steps):
        pos = P + step
        q = synthetic.query(B, Hq, 1, 300 + step, dtype=torch.bfloat16)
        a = attend(q, k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], fused, SCALE, None, sinks,
                   out_dtype=torch.float32, splits=splits)
        b = attend(q, k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], twin, SCALE, None, sinks,
                   out_dtype=torch.float32, splits=splits, fused=False)
        torch.cuda.synchronize()
        assert fused.offset == twin.offset == pos + 1
        assert torch.equal(fused.keys, twin.keys) and torch.equal(fused.values, twin.values), f"ring slots, step {step}"
        ref = O.attention(f32(q), bf16_np(k[:, :, pos + 1 - W:pos + 1]), bf16_np(v[:, :, pos + 1 - W:pos + 1]), SCALE,
                          sinks=q_sinks(sinks, q.dtype))
        assert_close(f32(a), ref, f"fused step {step} (slot {pos % W})")
        assert_close(f32(b), ref, f"unfused step {step}")


# ---------------------------------------------------------------------------
# prefill over the bf16 cache (L > 1 queries, the newest L of the T cached tokens)


PREFILL_CASES = [
    # B, Hq, Hkv, P (prefix), L (new), q dtype, sinks, causal
    (1, 32, 4, 1000, 300, torch.bfloat16, True, True),
    (1, 8, 1, 0, 77, torch.bfloat16, False, True),
    (2, 16, 2, 130, 64, torch.float16, True, True),
    (1, 32, 4, 500, 129, torch.bfloat16, True, False),
    (3, 4, 4, 40, 33, torch.bfloat16, True, True),    # one query head per KV head
    (1, 12, 4, 256, 96, torch.float16, False, True),  # three per KV head
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_P{}_L{}_{}_s{}_c{}".format(
    c[0], c[1], c[2], c[3], c[4], str(c[5])[6:], c[6], c[7]))
def test_bf16_prefill_matches_oracle(gpu, case):
    """FixedKVCache: the prefix goes in, then a chunk of L tokens is appended
    and attends over everything (causal or full), as Attention.__call__ does."""
    B, Hq, Hkv, P, L, qdt, use_sinks, causal = case
    T = P + L
    store = KVStorage(1, T, Hkv, batch=B)
    cache = FixedKVCache(store, 0)
    k = synthetic.kv((B, Hkv, T, 128), 111, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 112, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    if P:
        cache.update_and_fetch(k[:, :, :P], v[:, :, :P])
    q = synthetic.query(B, Hq, L, 113, dtype=qdt)
    sinks = torch.randn(Hq, device="cuda") if use_sinks else None
    mask = "causal" if causal else None
    out = attend(q, k[:, :, P:], v[:, :, P:], cache, SCALE, mask, sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert cache.offset == T
    ref = O.attention(f32(q), bf16_np(k), bf16_np(v), SCALE, sinks=q_sinks(sinks, q.dtype), mask=mask)
    assert_close(f32(out), ref, f"case {case}")


WINDOW_CASES = [
    # Hq, Hkv, T, L, W
    (16, 2, 400, 150, 97),
    (12, 4, 700, 200, 40),  # 3 heads per KV head: a 256-row block spans 85 queries, more than the window
    (4, 4, 600, 300, 40),   # one head per KV head: 256 queries per block
]


@pytest.mark.parametrize("case", WINDOW_CASES, ids=lambda c: "Hq{}_Hkv{}_T{}_L{}_W{}".format(*c))
def test_bf16_prefill_window_mask_array(gpu, case):
    """A boolean sliding-window mask array (make_mask(..., return_array=True))
    is recognised and gives the same result as the oracle with that mask."""
    Hq, Hkv, T, L, W = case
    B = 1
    k = synthetic.kv((B, Hkv, T, 128), 121, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, T, 128), 122, dtype=torch.bfloat16)
    q = synthetic.query(B, Hq, L, 123, dtype=torch.bfloat16)
    qi = torch.arange(T - L, T)[:, None]
    ki = torch.arange(T)[None]
    mask = ((qi >= ki) & (qi < ki + W)).cuda()
    sinks = torch.randn(Hq, device="cuda")
    out = scaled_dot_product_attention(q, k, v, SCALE, mask, sinks, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.attention(f32(q), bf16_np(k), bf16_np(v), SCALE, sinks=f32(sinks), mask=mask.cpu().numpy())
    assert_close(f32(out), ref, "window mask array (a bias)")
    host = scaled_dot_product_attention(q, k, v, SCALE, mask.cpu(), sinks, out_dtype=torch.float32)  # the window kernel
    assert_close(f32(host), ref, "window mask array (host: the window kernel)")
    # the complement is no pattern of its own: a bias (a row may see no key at all)
    inv = ~mask
    out = scaled_dot_product_attention(q, k, v, SCALE, inv, sinks, out_dtype=torch.float32)
    ref = O.attention(f32(q), bf16_np(k), bf16_np(v), SCALE, sinks=f32(sinks), mask=inv.cpu().numpy())
    assert_close(f32(out), ref, "complement of the window")


def test_sliding_window_prefill_chunks(gpu):
    """FixedSlidingKVCache: chunks longer than the window, then decode steps;
    each chunk attends over the ring (in order) plus itself within the window
    (cache.py:153-258, the windowed prefill of m4_max_prefill.py:86-104)."""
    from rec_amd import FixedSlidingKVCache

    B, Hq, Hkv, W = 1, 32, 4, 100
    cache = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W)
    n = 400
    k = synthetic.kv((B, Hkv, n, 128), 131, dtype=torch.bfloat16)
    v = synthetic.kv((B, Hkv, n, 128), 132, dtype=torch.bfloat16)
    sinks = torch.randn(Hq, device="cuda")
    pos = 0
    for L in (150, 1, 1, 70, 130, 1):
        q = synthetic.query(B, Hq, L, 140 + pos, dtype=torch.bfloat16)
        lo = max(0, pos - W) if L == 1 else max(0, pos - cache.size())
        out = attend(q, k[:, :, pos : pos + L], v[:, :, pos : pos + L], cache, SCALE, "causal", sinks,
                     out_dtype=torch.float32)
        torch.cuda.synchronize()
        end = pos + L
        Tk = end - lo if L > 1 else min(end, W)
        kk, vv = bf16_np(k[:, :, end - Tk : end]), bf16_np(v[:, :, end - Tk : end])
        qi = np.arange(Tk - L, Tk)[:, None]
        ki = np.arange(Tk)[None]
        ref = O.attention(f32(q), kk, vv, SCALE, sinks=q_sinks(sinks, q.dtype), mask=(qi >= ki) & (qi < ki + W))
        assert_close(f32(out), ref, f"chunk at {pos} of {L}")
        pos = end


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_ring_join_bit_exact(gpu, dtype):
    """rec_ring_join_bf16 (FixedSlidingKVCache.update_and_fetch of a chunk):
    the held window in sequence order, then the chunk rounded to bf16, equal
    bit for bit to joining the same tokens of the full sequence, before and
    after the ring wraps and for chunks longer than the window; the ring
    then holds the last window of tokens (placed by the same launch)."""
    from rec_amd import FixedSlidingKVCache

    B, Hkv, W = 2, 3, 100
    n = 700
    k = synthetic.kv((B, Hkv, n, 128), 151, dtype=dtype)
    v = synthetic.kv((B, Hkv, n, 128), 152, dtype=dtype)
    cache = FixedSlidingKVCache(max_sequence_tokens=4096, num_kv_heads=Hkv, head_dim=128, window_size=W, batch=B)
    pos = 0
    for L in (40, 30, 1, 57, 150, 1, 1, 99, 203):
        held = min(pos, W)
        kk, vv = cache.update_and_fetch(k[:, :, pos:pos + L], v[:, :, pos:pos + L])
        torch.cuda.synchronize()
        end = pos + L
        if L > 1:
            assert kk.shape == (B, Hkv, held + L, 128) and kk.dtype == torch.bfloat16
            want_k = k[:, :, end - held - L:end].to(torch.bfloat16)
            want_v = v[:, :, end - held - L:end].to(torch.bfloat16)
            assert torch.equal(kk.view(torch.int16), want_k.contiguous().view(torch.int16)), f"K at {pos}+{L}"
            assert torch.equal(vv.view(torch.int16), want_v.contiguous().view(torch.int16)), f"V at {pos}+{L}"
        # the ring afterwards holds the last min(end, W) tokens
        wk, wv = cache.window()
        hold = min(end, W)
        assert torch.equal(wk.contiguous().view(torch.int16),
                           k[:, :, end - hold:end].to(torch.bfloat16).contiguous().view(torch.int16)), f"ring K at {end}"
        assert torch.equal(wv.contiguous().view(torch.int16),
                           v[:, :, end - hold:end].to(torch.bfloat16).contiguous().view(torch.int16)), f"ring V at {end}"
        pos = end


def shared_metadata():
    """The layer table of the reference's shared-storage test (50 rows of 64
    columns, every fourth of the first 49 layers full-attention)."""
    rows = [[0] * 64 for _ in range(50)]
    for i, row in enumerate(rows[:49]):
        row[1] = int(i % 4 == 0)
    return rows


def test_storage_from_the_reference_metadata(gpu):
    """KVStorage(metadata, capacity), the reference's constructor
    (cache.py:52-73), restating its shared-storage test: a full-attention
    layer's writes show in its views and survive a growth past one bank; a
    sliding-window layer holds 513 tokens beside them and keeps its bytes
    across the growth; a fused decode step on it attends over its region."""
    from rec_amd.kvstorage import BLOCK_TOKENS

    storage = KVStorage(shared_metadata(), 17)
    assert storage.n_layers == 49 and storage.capacity == BLOCK_TOKENS and storage.metadata.shape == (50, 64)
    cache = FixedKVCache(storage, 0)
    keys = torch.arange(4 * 9 * 128, device="cuda").reshape(1, 4, 9, 128).to(torch.bfloat16)
    k, v = cache.update_and_fetch(keys, -keys)
    assert torch.equal(k, keys) and torch.equal(storage.layer(0)[:, 1, :, :9], -keys)
    ring = torch.arange(4 * 513 * 128, device="cuda").reshape(1, 4, 513, 128).to(torch.bfloat16)
    storage.write(1, 0, ring, -ring)
    assert storage.layer(1).shape == (1, 2, 4, 513, 128)
    with pytest.raises(ValueError):
        storage.write(1, 1, ring[:, :, :1].expand(1, 4, 513, 128).contiguous(), -ring)
    storage.grow(BLOCK_TOKENS + 65)
    assert storage.capacity == 2 * BLOCK_TOKENS
    assert torch.equal(storage.layer(1)[:, 0], ring) and torch.equal(storage.layer(1)[:, 1], -ring)
    cache.offset = BLOCK_TOKENS - 2
    k, v = cache.update_and_fetch(keys, -keys)
    assert torch.equal(k[:, :, BLOCK_TOKENS - 2 :], keys) and torch.equal(v[:, :, BLOCK_TOKENS - 2 :], -keys)
    assert torch.equal(k[:, :, :9], keys)  # the first bank's tokens stay in place
    # a sliding-window layer through FixedKVCache: 512 tokens, then one fused step (513 = its region)
    local = FixedKVCache(storage, 2)
    kk = synthetic.kv((1, 4, 513, 128), 71, dtype=torch.bfloat16)
    vv = synthetic.kv((1, 4, 513, 128), 72, dtype=torch.bfloat16)
    local.update_and_fetch(kk[:, :, :512], vv[:, :, :512])
    q = synthetic.query(1, 32, 1, 73, dtype=torch.bfloat16)
    out = attend(q, kk[:, :, 512:], vv[:, :, 512:], local, SCALE, None, None, out_dtype=torch.float32)
    assert_close(f32(out), O.attention(f32(q), f32(kk), f32(vv), SCALE), "sliding-window layer of the storage")
    with pytest.raises(ValueError, match="exhausted"):
        attend(q, kk[:, :, :1], vv[:, :, :1], local, SCALE, None, None)

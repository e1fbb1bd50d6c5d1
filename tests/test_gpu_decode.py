"""Parity of the gfx950 append and decode kernels with the CPU oracle.

Cache bytes and scales must be bit-identical; attention outputs within
2e-3 absolute + 1e-3 relative of the float64 oracle.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import QuantizedKVCache, attend, quantized_attention_with_sinks, synthetic
from tests.gpu_util import SCALE, assert_cache_equal, assert_close, dequant, f32, oracle_quantize

pytestmark = pytest.mark.gpu

BITS = [(8, 8), (8, 4), (4, 8), (4, 4)]


def fill(cache, B, H, T, seed, kind="outliers", frac=0.01, dtype=torch.float16, chunks=None):
    """Append T tokens in chunks; return the float32 K/V that went in."""
    k = synthetic.kv((B, H, T, 128), seed, kind=kind, frac=frac, dtype=dtype)
    v = synthetic.kv((B, H, T, 128), seed + 1, kind=kind, frac=frac, dtype=dtype)
    pos = 0
    for L in chunks or [T]:
        cache.update_and_fetch(k[:, :, pos : pos + L], v[:, :, pos : pos + L])
        pos += L
    assert pos == T
    return f32(k), f32(v)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_append_bit_exact(gpu, bits, dtype):
    B, H = 2, 3
    cache = QuantizedKVCache(32, *bits)
    chunks = [5, 64, 1, 1, 70, 3, 200]
    k, v = fill(cache, B, H, sum(chunks), 11, kind="heavy", frac=0.05, dtype=dtype, chunks=chunks)
    kv_k, kv_v = cache.keys_and_values()
    assert cache.offset == sum(chunks) and cache.capacity % 64 == 0
    assert_cache_equal(kv_k, oracle_quantize(k, bits[0]))
    assert_cache_equal(kv_v, oracle_quantize(v, bits[1]))


@pytest.mark.parametrize("bits", BITS)
def test_append_strided_and_special_rows(gpu, bits):
    B, H, L = 1, 2, 9
    x = torch.randn(B, L, H, 128, device="cuda", dtype=torch.float16)
    x[:, 0] = 0  # all-zero rows
    x[:, 1] = 1.5  # constant rows
    x[:, 2, :, 7] = 300.0  # one large element
    k = x.transpose(1, 2)  # (B, H, L, D) view, non-contiguous
    v = (-x).transpose(1, 2)
    cache = QuantizedKVCache(32, *bits)
    cache.update_and_fetch(k, v)
    kv_k, kv_v = cache.keys_and_values()
    assert_cache_equal(kv_k, oracle_quantize(f32(k), bits[0]))
    assert_cache_equal(kv_v, oracle_quantize(f32(v), bits[1]))


DECODE_CASES = [
    # B, Hq, Hkv, T, k_bits, v_bits, sinks, splits
    (1, 8, 1, 1024, 8, 8, False, None),  # the tiny CPU-sized workload
    (1, 8, 1, 1024, 8, 8, True, None),
    (1, 32, 4, 4096, 8, 8, True, None),
    (1, 32, 4, 1000, 8, 8, False, 3),
    (2, 16, 2, 777, 8, 8, True, 256),
    (1, 4, 1, 1, 8, 8, True, None),
    (1, 4, 1, 1, 8, 8, False, None),
    (1, 8, 4, 130, 8, 8, False, 1),
    (1, 32, 4, 2048, 4, 4, True, None),
    (1, 32, 4, 2048, 8, 4, True, None),
    (1, 32, 4, 2048, 4, 8, False, 7),
    (1, 8, 8, 333, 4, 4, True, 2),
    (3, 24, 4, 65, 8, 4, True, None),
    # uint4 splits of >= 32 chunks run eight wavefronts per workgroup
    (1, 32, 4, 5000, 4, 4, True, 2),
    (2, 16, 2, 3000, 4, 4, False, 1),
    (1, 8, 1, 1100, 4, 4, True, 1),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_T{}_k{}v{}_s{}_sp{}".format(*c))
def test_decode_matches_oracle(gpu, case):
    B, Hq, Hkv, T, kb, vb, with_sinks, splits = case
    cache = QuantizedKVCache(32, kb, vb)
    k, v = fill(cache, B, Hkv, T, seed=100 + T, kind="outliers", frac=0.01)
    q = synthetic.query(B, Hq, 1, seed=7 + Hq)
    sinks = torch.randn(Hq, device="cuda") if with_sinks else None
    kq, vq = cache.keys_and_values()
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, None, sinks, 32, kb, vb, out_dtype=torch.float32,
                                         splits=splits)
    rk, rv = oracle_quantize(k, kb), oracle_quantize(v, vb)
    assert_cache_equal(kq, rk)
    assert_cache_equal(vq, rv)
    ref = O.attention(f32(q), dequant(kb, *rk), dequant(vb, *rv), SCALE, None if sinks is None else f32(sinks))
    assert_close(f32(out), ref, f"case {case}")


@pytest.mark.parametrize("bits,T0,splits", [(b, 511, None) for b in BITS] + [((4, 4), 2111, 2)],
                         ids=lambda x: str(x))
def test_fused_decode_steps(gpu, bits, T0, splits):
    """append-then-attend in one launch, several steps, vs the oracle (the
    last case: uint4 splits long enough for eight wavefronts)."""
    B, Hq, Hkv = 1, 32, 4
    cache = QuantizedKVCache(32, *bits)
    k0, v0 = fill(cache, B, Hkv, T0, seed=5)
    ks, vs = [k0], [v0]
    sinks = torch.randn(Hq, device="cuda")
    for step in range(4):  # crosses a 32-token block boundary and an odd/even pair
        q = synthetic.query(B, Hq, 1, seed=50 + step)
        kn = synthetic.kv((B, Hkv, 1, 128), 60 + step)
        vn = synthetic.kv((B, Hkv, 1, 128), 70 + step)
        out = attend(q, kn, vn, cache, SCALE, None, sinks, out_dtype=torch.float32, splits=splits)
        ks.append(f32(kn))
        vs.append(f32(vn))
        K, V = np.concatenate(ks, 2), np.concatenate(vs, 2)
        rk, rv = oracle_quantize(K, bits[0]), oracle_quantize(V, bits[1])
        ref = O.attention(f32(q), dequant(bits[0], *rk), dequant(bits[1], *rv), SCALE, f32(sinks))
        assert_close(f32(out), ref, f"step {step}")
    kq, vq = cache.keys_and_values()
    assert cache.offset == T0 + 4
    assert_cache_equal(kq, rk)
    assert_cache_equal(vq, rv)


def test_unfused_equals_fused(gpu):
    B, Hq, Hkv = 1, 32, 4
    c1, c2 = QuantizedKVCache(32, 8, 8), QuantizedKVCache(32, 8, 8)
    fill(c1, B, Hkv, 300, seed=9)
    fill(c2, B, Hkv, 300, seed=9)
    q = synthetic.query(B, Hq, 1, seed=1)
    kn, vn = synthetic.kv((B, Hkv, 1, 128), 2), synthetic.kv((B, Hkv, 1, 128), 3)
    a = attend(q, kn, vn, c1, SCALE, None, None, out_dtype=torch.float32, fused=True)
    b = attend(q, kn, vn, c2, SCALE, None, None, out_dtype=torch.float32, fused=False)
    torch.testing.assert_close(a, b, rtol=0, atol=0)


@pytest.mark.parametrize("T", [32768, 258048])
def test_long_context_int8(gpu, T):
    """Full-size 32K / 252K int8 decode against the chunked CPU oracle: the
    cache filled to T - 3, then three decode steps that each quantize one new
    token into the cache inside the attention launch (the benchmarked step),
    then the unfused attention over all T tokens."""
    from rec_amd import to_logical

    B, Hq, Hkv = 1, 32, 4
    cache = QuantizedKVCache(32, 8, 8, max_tokens=T)
    fill(cache, B, Hkv, T - 3, seed=3, kind="outliers", frac=0.01)
    sinks = torch.randn(Hq, device="cuda")
    for step in range(3):
        q = synthetic.query(B, Hq, 1, seed=4 + step)
        kn = synthetic.kv((B, Hkv, 1, 128), 30 + step, kind="outliers", frac=0.01)
        vn = synthetic.kv((B, Hkv, 1, 128), 40 + step, kind="outliers", frac=0.01)
        print(f"T={T} fused step {step}", flush=True)
        out = attend(q, kn, vn, cache, SCALE, None, sinks, out_dtype=torch.float32)
        Ti = T - 2 + step
        assert cache.offset == Ti
        kq, vq = cache.keys_and_values()
        kc, ksc, _ = (t.cpu().numpy() if t is not None else None for t in to_logical(kq))
        vc, vsc, _ = (t.cpu().numpy() if t is not None else None for t in to_logical(vq))
        for got, x in (((kc, ksc), kn), ((vc, vsc), vn)):  # the appended row, bit for bit
            c, sc = O.quantize_int8(f32(x))
            np.testing.assert_array_equal(got[0][:, :, Ti - 1 :], c)
            np.testing.assert_array_equal(got[1][:, :, Ti - 1 :].view(np.uint16), sc.view(np.uint16))
        cache_np = dict(k_bits=8, v_bits=8, kq=kc, ks=ksc, vq=vc, vs=vsc)
        ref = O.split_k_decode_quantized(f32(q)[:, :, 0], cache_np, Ti, SCALE, f32(sinks), chunk=8192)
        assert_close(f32(out)[:, :, 0], ref.astype(np.float64), f"T={Ti} fused step {step}")
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, None, sinks, 32, 8, 8, out_dtype=torch.float32)
    assert_close(f32(out)[:, :, 0], ref.astype(np.float64), f"T={T} unfused")


def test_repeated_launches_share_workspace(gpu):
    """Many launches on one workspace with changing split counts: the merge
    counters must re-arm and no stale partial may leak between launches."""
    B, Hq, Hkv = 1, 32, 4
    caches, refs = [], []
    for i, T in enumerate([700, 2048, 96]):
        c = QuantizedKVCache(32, 8, 8)
        k, v = fill(c, B, Hkv, T, seed=300 + i)
        caches.append(c)
        rk, rv = oracle_quantize(k, 8), oracle_quantize(v, 8)
        refs.append((dequant(8, *rk), dequant(8, *rv)))
    qs = [synthetic.query(B, Hq, 1, seed=400 + i) for i in range(4)]
    for it in range(24):
        i = it % 3
        q = qs[it % 4]
        kq, vq = caches[i].keys_and_values()
        splits = [2, 5, 8, 64, 200, 3][it % 6]
        out = quantized_attention_with_sinks(q, kq, vq, SCALE, None, None, 32, 8, 8, out_dtype=torch.float32,
                                             splits=splits)
        ref = O.attention(f32(q), *refs[i], SCALE)
        assert_close(f32(out), ref, f"iteration {it} cache {i} splits {splits}")


def test_partial_then_merge_equals_one_call(gpu):
    """rec_decode_partial + rec_decode_merge give the same bytes as rec_decode_append_attn."""
    import rec_amd
    from rec_amd import _lib
    from rec_amd.attention import workspace

    lib = rec_amd.library()
    B, Hq, Hkv, T0 = 1, 32, 4, 3000
    outs = []
    for phased in (False, True):
        c = QuantizedKVCache(32, 8, 8)
        fill(c, B, Hkv, T0, seed=21)
        c._reserve(B, Hkv, T0 + 1, "cuda")
        q = synthetic.query(B, Hq, 1, seed=22)[:, :, 0].contiguous()
        kn, vn = synthetic.kv((B, Hkv, 1, 128), 23), synthetic.kv((B, Hkv, 1, 128), 24)
        sinks = torch.randn(Hq, device="cuda", generator=torch.Generator("cuda").manual_seed(5))
        out = torch.empty((B, Hq, 128), dtype=torch.float32, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        ws = workspace(q.device, B, Hkv, 256, stream)
        (kc, ks, _), (vc, vs, _) = c.keys, c.values
        args = (q.data_ptr(), _lib.REC_F16, q.stride(0), q.stride(1), kn.data_ptr(), vn.data_ptr(), _lib.REC_F16,
                kn.stride(0), kn.stride(1), vn.stride(0), vn.stride(1), 8, kc.data_ptr(), ks.data_ptr(), None,
                8, vc.data_ptr(), vs.data_ptr(), None, sinks.data_ptr(), SCALE, B, Hq, Hkv, 128, T0 + 1,
                c.capacity, 0, ws.data_ptr(), ws.numel(), _lib.REC_F32, out.data_ptr(), stream)
        if phased:
            _lib.check(lib.rec_decode_partial(*args), "partial")
            _lib.check(lib.rec_decode_merge(sinks.data_ptr(), B, Hq, Hkv, T0 + 1, 0, 1, ws.data_ptr(), ws.numel(),
                                            _lib.REC_F32, out.data_ptr(), stream), "merge")
        else:
            _lib.check(lib.rec_decode_append_attn(*args), "append_attn")
        outs.append(out.clone())
    torch.testing.assert_close(outs[0], outs[1], rtol=0, atol=0)


@pytest.mark.parametrize("fmt", ["int8", "affine"])
def test_fused_decode_steps_in_hip_graph(gpu, fmt):
    """Four fused decode steps (append + attention + merge) captured in one HIP
    graph and replayed three times, with eager work between the replays: every
    replay's outputs and the cache bytes equal the eager run's, bit for bit."""
    from rec_amd import MixedQuantizedKVCache, to_logical

    B, Hq, Hkv, P, steps = 1, 32, 4, 700, 4

    def make():
        c = MixedQuantizedKVCache(max_tokens=1024) if fmt == "affine" else QuantizedKVCache(32, 8, 8, max_tokens=1024)
        fill(c, B, Hkv, P, seed=501)
        return c

    qs = [synthetic.query(B, Hq, 1, seed=510 + i) for i in range(steps)]
    kns = [synthetic.kv((B, Hkv, 1, 128), 520 + i) for i in range(steps)]
    vns = [synthetic.kv((B, Hkv, 1, 128), 530 + i) for i in range(steps)]
    sinks = torch.randn(Hq, device="cuda", generator=torch.Generator("cuda").manual_seed(7))

    eager_cache = make()
    eager = [attend(qs[i], kns[i], vns[i], eager_cache, SCALE, None, sinks, out_dtype=torch.float32)
             for i in range(steps)]
    torch.cuda.synchronize()
    want_k, want_v = (to_logical(kv) for kv in eager_cache.keys_and_values())

    cache = make()
    outs = [torch.empty_like(e) for e in eager]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            outs[i].copy_(attend(qs[i], kns[i], vns[i], cache, SCALE, None, sinks, out_dtype=torch.float32))
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        x = torch.randn(256, 256, device="cuda")
        (x @ x).sum().item()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for i in range(steps):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} step {i}"
        got_k, got_v = (to_logical(kv) for kv in cache.keys_and_values())
        for got, want in ((got_k, want_k), (got_v, want_v)):
            for a_, b_ in zip(got, want):
                assert (a_ is None and b_ is None) or torch.equal(a_, b_), f"replay {rep}: cache differs"

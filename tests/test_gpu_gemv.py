"""Parity of the int4 group-64 GEMV (rec_q4_pack + rec_q4_gemv) with the CPU oracle.

The products inside the kernel are exact and the sums run in fp32, so the fp32
output must lie within 1e-5 · (|x| · |W|ᵀ) + 1e-6 of the float64 oracle
(far inside the decode path's 2e-3 abs + 1e-3 rel); the bf16 output must be
the round-to-nearest-even of the fp32 output, bit for bit.
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import Q4Matrix, q4_gemv, q4_gemv_parts, quantized_matmul

pytestmark = pytest.mark.gpu


def problem(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-(2**31), 2**31, (N, K // 8), dtype=torch.int64, generator=g).to(torch.int32)
    s = (torch.rand((N, K // 64), generator=g) * 0.049 + 0.001).to(torch.bfloat16)
    b = (torch.rand((N, K // 64), generator=g) * 0.4 - 0.3).to(torch.bfloat16)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    return x.cuda(), w.cuda(), s.cuda(), b.cuda()


def oracle_rows(x, w, s, b, rows=None):
    wn = w.cpu().numpy().view(np.uint32)
    sn, bn = s.float().cpu().numpy(), b.float().cpu().numpy()
    if rows is not None:
        wn, sn, bn = wn[rows], sn[rows], bn[rows]
    xn = x.float().cpu().numpy()
    ref = O.q4_gemv(xn, wn, sn, bn)
    mag = np.abs(xn.astype(np.float64)) @ np.abs(O.q4_dequantize(wn, sn, bn)).T
    return ref, mag


def check(got, ref, mag, what):
    got = got.double().cpu().numpy()
    err = np.abs(got - ref)
    bound = 1e-5 * mag + 1e-6
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert np.all(err <= bound), f"{what}: max err {err.max():.3e}, max err/bound {(err / bound).max():.2f}"


CASES = [
    # M, N, K
    (1, 4096, 2048),   # q_proj
    (1, 512, 2048),    # k_proj / v_proj
    (1, 2048, 4096),   # o_proj: 128 row tiles, 8 waves per tile
    (1, 2048, 6144),   # dense MLP down: 16 waves per tile
    (4, 300, 8192),    # 19 row tiles of 64 spans: 16 waves per tile, four vectors
    (2, 200, 3072),    # 24 spans: 8 waves per tile, a ragged last tile
    (1, 6144, 2048),   # dense MLP gate / up
    (3, 1000, 512),    # ragged rows, expert down (K = 512)
    (8, 100, 2048),
    (5, 16, 128),
    (1, 1, 128),
    (2, 33, 384),
    (1, 24000, 256),   # 1500 row tiles: two waves per tile
    (2, 40000, 128),   # 2500 row tiles: one wave per tile
    (39, 512, 2048),   # one row short of gemm_min_rows(2048): five GEMV launches
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"M{c[0]}_N{c[1]}_K{c[2]}")
def test_q4_gemv_matches_oracle(gpu, case):
    M, N, K = case
    x, w, s, b = problem(M, N, K, seed=N + K + M)
    m = Q4Matrix(w, s, b)
    y32 = q4_gemv(x, m, out_dtype=torch.float32)
    y16 = q4_gemv(x, m)
    torch.cuda.synchronize()
    ref, mag = oracle_rows(x, w, s, b)
    check(y32, ref, mag, f"case {case}")
    assert y16.dtype == torch.bfloat16 and y16.shape == (M, N)
    assert torch.equal(y16.view(torch.int16), y32.to(torch.bfloat16).view(torch.int16)), "bf16 output is not RNE(fp32)"


def test_lm_head_size(gpu):
    """The lm head (150,144 x 2048): sampled rows against the oracle, every row
    against a float32 torch reference of the dequantized matrix."""
    N, K = 150144, 2048
    x, w, s, b = problem(1, N, K, seed=5)
    y = q4_gemv(x, Q4Matrix(w, s, b), out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(5).choice(N, 384, replace=False))
    rows = np.concatenate([rows, [0, N - 1]])
    ref, mag = oracle_rows(x, w, s, b, rows)
    check(y[:, rows], ref, mag, "lm head sampled rows")
    # full-size torch reference, dequantized on the GPU in float32
    shifts = torch.arange(0, 32, 4, device="cuda", dtype=torch.int32)
    q = ((w.unsqueeze(-1) >> shifts) & 15).reshape(N, K).float()
    deq = q * s.float().repeat_interleave(64, 1) + b.float().repeat_interleave(64, 1)
    full = (x.float() @ deq.T).double()
    mag_full = (x.float().abs() @ deq.abs().T).double()
    err = (y.double() - full).abs()
    assert bool((err <= 2e-5 * mag_full + 1e-5).all()), f"max err {err.max().item():.3e}"


def test_strided_rows_and_many_vectors(gpu):
    """x with a row stride larger than K and more than 8 vectors (two launches),
    leading dims kept; quantized_matmul has mx.quantized_matmul's call shape."""
    N, K = 300, 1024
    _, w, s, b = problem(1, N, K, seed=9)
    big = torch.randn((11, K + 64), device="cuda").to(torch.bfloat16)
    x = big[:, :K]
    m = Q4Matrix(w, s, b)
    y = q4_gemv(x.reshape(11, 1, K), m, out_dtype=torch.float32)
    assert y.shape == (11, 1, N)
    ref, mag = oracle_rows(x, w, s, b)
    check(y.reshape(11, N), ref, mag, "strided")
    y2 = quantized_matmul(x, w, s, b, transpose=True, group_size=64, bits=4)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.reshape(11, N).to(torch.bfloat16).view(torch.int16))
    with pytest.raises(NotImplementedError):
        quantized_matmul(x, w, s, b, transpose=False)
    with pytest.raises(ValueError):
        q4_gemv(x.float(), m)


@pytest.mark.parametrize("M", [2, 100], ids=["gemv", "gemm"])
def test_q4_gemv_in_hip_graph(gpu, M):
    """Captured launches (the GEMV, or the group sums and GEMM for a prefill
    chunk's rows) replayed several times, with eager work between the replays, match
    the eager result every time."""
    N, K = 2048, 4096
    x, w, s, b = problem(M, N, K, seed=13)
    m = Q4Matrix(w, s, b)
    eager = q4_gemv(x, m, out_dtype=torch.float32)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out.copy_(q4_gemv(x, m, out_dtype=torch.float32))
    for rep in range(3):
        out.fill_(float("nan"))
        _ = q4_gemv(x[:1], m)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, rtol=0, atol=0, msg=f"replay {rep}")


@pytest.mark.parametrize("parts,M", [((4096, 512, 512), 1), ((100, 33, 1000), 3)], ids=["qkv", "ragged"])
def test_stacked_matrices_one_launch(gpu, parts, M):
    """Q4Matrix.stack packs several matrices of one K as one (a layer's q, k
    and v projections, megakernel.py:871-886): q4_gemv_parts returns each
    part's output from one launch, equal to the oracle for that part, also
    where the parts share 16-row tiles (ragged row counts)."""
    K = 2048
    probs = [problem(M, N, K, seed=31 + i) for i, N in enumerate(parts)]
    x = probs[0][0]
    m = Q4Matrix.stack([(w, s, b) for _, w, s, b in probs])
    assert m.shape == (sum(parts), K) and m.parts == parts
    ys = q4_gemv_parts(x, m, out_dtype=torch.float32)
    y16 = q4_gemv_parts(x, m)
    torch.cuda.synchronize()
    assert [y.shape for y in ys] == [(M, N) for N in parts]
    for i, (_, w, s, b) in enumerate(probs):
        ref, mag = oracle_rows(x, w, s, b)
        check(ys[i], ref, mag, f"part {i}")
        assert torch.equal(y16[i].view(torch.int16), ys[i].to(torch.bfloat16).view(torch.int16))
    with pytest.raises(ValueError):  # parts of different K
        Q4Matrix.stack([probs[0][1:], problem(1, 16, 1024, seed=3)[1:]])


GEMM_CASES = [
    # M, N, K: from gemm_min_rows(K) vectors on, rec_q4_gemm (x's group sums, then a GEMM in 64-vector tiles)
    (28, 300, 512),
    (64, 1000, 1024),      # one full 64-vector tile, a ragged last row tile
    (130, 257, 384),       # three vector tiles, the last of 2
    (200, 48, 2048),
    (40, 512, 2048),       # exactly gemm_min_rows(2048)
    (77, 4096, 128),       # one span
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: f"M{c[0]}_N{c[1]}_K{c[2]}")
def test_q4_gemm_matches_oracle(gpu, case):
    """Prefill-sized x (from gemm_min_rows(K) rows on): fp32 output within 1e-5·(|x|·|W|ᵀ)
    of the float64 oracle, bf16 output the RNE of the fp32 one."""
    M, N, K = case
    x, w, s, b = problem(M, N, K, seed=7 * M + N + K)
    m = Q4Matrix(w, s, b)
    y32 = q4_gemv(x, m, out_dtype=torch.float32)
    y16 = q4_gemv(x, m)
    torch.cuda.synchronize()
    ref, mag = oracle_rows(x, w, s, b)
    check(y32, ref, mag, f"gemm {case}")
    assert torch.equal(y16.view(torch.int16), y32.to(torch.bfloat16).view(torch.int16)), "bf16 output is not RNE(fp32)"


def test_q4_gemm_c_abi_small_m_and_strides(gpu):
    """rec_q4_gemm through the C ABI at M = 3 and M = 1 (a partial vector
    tile), x rows with a stride longer than K, out rows with a stride longer
    than N; equal to the GEMV within the bound; a short workspace refused."""
    import ctypes

    from rec_amd import _lib

    lib = _lib.load()
    N, K = 200, 1024
    _, w, s, b = problem(1, N, K, seed=21)
    m = Q4Matrix(w, s, b)
    big = torch.randn((3, K + 64), device="cuda").to(torch.bfloat16)
    x = big[:, :K]
    for M in (3, 1):
        out = torch.full((M, N + 8), float("nan"), device="cuda")
        ws = torch.empty(lib.rec_q4_gemm_workspace_bytes(M, K), dtype=torch.uint8, device="cuda")
        rc = lib.rec_q4_gemm(m.packed.data_ptr(), N, K, x.data_ptr(), K + 64, M, out.data_ptr(), _lib.REC_F32,
                             N + 8, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "rec_q4_gemm")
        torch.cuda.synchronize()
        ref, mag = oracle_rows(x[:M], w, s, b)
        check(out[:, :N], ref, mag, f"c-abi M={M}")
        assert bool(torch.isnan(out[:, N:]).all()), "wrote past N"
        gv = q4_gemv(x[:M], m, out_dtype=torch.float32)
        torch.testing.assert_close(out[:, :N], gv, rtol=1e-5, atol=1e-4)
    rc = lib.rec_q4_gemm(m.packed.data_ptr(), N, K, x.data_ptr(), K + 64, 3, out.data_ptr(), _lib.REC_F32, N + 8,
                         ws.data_ptr(), 4, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.REC_EWORKSPACE


def test_q4_gemm_prefill_projection_size(gpu):
    """A 2,048-token chunk through the q projection (4096 x 2048): every
    output against a float32 torch reference of the dequantized matrix."""
    M, N, K = 2048, 4096, 2048
    x, w, s, b = problem(M, N, K, seed=23)
    y = q4_gemv(x, Q4Matrix(w, s, b), out_dtype=torch.float32)
    shifts = torch.arange(0, 32, 4, device="cuda", dtype=torch.int32)
    q = ((w.unsqueeze(-1) >> shifts) & 15).reshape(N, K).float()
    deq = q * s.float().repeat_interleave(64, 1) + b.float().repeat_interleave(64, 1)
    full = (x.float() @ deq.T).double()
    mag = (x.float().abs() @ deq.abs().T).double()
    err = (y.double() - full).abs()
    assert bool((err <= 2e-5 * mag + 1e-5).all()), f"max err {err.max().item():.3e}"

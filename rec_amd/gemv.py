"""int4 group-64 GEMV of the decoder's projections (MLX affine 4-bit weights).

The reference decodes with 4-bit affine weights (group 64, bf16 scales and
biases: engine/src/rec_mlx/quantized.py:27-36) and multiplies them by the
bf16 activations with ``q4`` / ``dot16`` (engine/src/rec_mlx/kernels/
megakernel.py:161-232) after packing its weight banks once
(megakernel.py:1017-1040).  Here a :class:`Q4Matrix` packs an MLX-layout
matrix once (``rec_q4_pack``) and :func:`q4_gemv` runs ``rec_q4_gemv``;
:meth:`Q4Matrix.stack` packs several matrices of one K (a layer's q, k and v
projections) as one, so a single launch computes them all.
:func:`quantized_matmul` keeps the call shape of ``mx.quantized_matmul`` for
the one configuration the reference uses (``transpose=True``, group 64, 4 bits).
"""

from __future__ import annotations

import torch

from . import _lib

GROUP = 64
MAX_VECTORS = 8  # rows of x per GEMV launch


def gemm_min_rows(K: int) -> int:
    """Rows of x from which one ``rec_q4_gemm`` beats GEMV launches of 8 rows:
    the GEMM takes ≈27.5 µs per 2,048 of K at any M up to a few hundred (it
    waits on one 128-element span's loads per step), a GEMV launch ≈6-7 µs.
    Measured crossings: between 32 (24.7 against 28.2 µs) and 48 rows (36.8
    against 28.6 µs) at K = 2048, between 48 and 64 rows at K = 4096."""
    return 24 + 8 * (K // 1024)


def _words(w: torch.Tensor) -> torch.Tensor:
    if w.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"packed weights must be 32-bit words (int32/uint32), got {w.dtype}")
    return w.contiguous()


class Q4Matrix:
    """An ``(N, K)`` MLX affine 4-bit matrix repacked for ``rec_q4_gemv``.

    ``w`` is ``(N, K/8)`` 32-bit words (code ``e`` of a word at bits ``4e``),
    ``scales`` and ``biases`` ``(N, K/64)`` bfloat16, all on the GPU.
    """

    def __init__(self, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor):
        if w.dim() != 2 or scales.dim() != 2 or biases.dim() != 2:
            raise ValueError("w, scales and biases must be 2-D")
        N, K = w.shape[0], w.shape[1] * 8
        if scales.shape != (N, K // GROUP) or biases.shape != scales.shape:
            raise ValueError(
                f"scales/biases {tuple(scales.shape)}/{tuple(biases.shape)} do not match w {tuple(w.shape)} "
                f"at group {GROUP}"
            )
        if scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
            raise ValueError("scales and biases must be bfloat16")
        lib = _lib.load()
        nbytes = lib.rec_q4_packed_bytes(N, K)
        if nbytes == 0:
            raise NotImplementedError(f"K={K} is not a positive multiple of 128")
        self.N, self.K = N, K
        self.device = w.device
        w = _words(w)
        scales, biases = scales.contiguous(), biases.contiguous()
        self.packed = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
        rc = lib.rec_q4_pack(
            w.data_ptr(), scales.data_ptr(), biases.data_ptr(), N, K, self.packed.data_ptr(), nbytes,
            torch.cuda.current_stream(w.device).cuda_stream,
        )
        _lib.check(rc, "rec_q4_pack")
        self.parts = (N,)

    @classmethod
    def stack(cls, mats) -> "Q4Matrix":
        """One matrix of the rows of several ``(w, scales, biases)`` triples of
        one K, in order: a single launch of :func:`q4_gemv` then computes all
        of their outputs from the same x, as the reference's decoder computes
        the 32 query, 4 key and 4 value heads of a layer in one pass over its
        normalised input (engine/src/rec_mlx/kernels/megakernel.py:871-886).
        :func:`q4_gemv_parts` splits the result back into the parts."""
        mats = list(mats)
        if not mats:
            raise ValueError("stack() needs at least one matrix")
        ws, ss, bs = zip(*mats)
        if len({int(w.shape[-1]) for w in ws}) != 1:
            raise ValueError(f"stacked matrices need one K, got {[int(w.shape[-1]) * 8 for w in ws]}")
        m = cls(torch.cat([_words(w) for w in ws]), torch.cat(ss), torch.cat(bs))
        m.parts = tuple(int(w.shape[0]) for w in ws)
        return m

    @property
    def shape(self):
        return (self.N, self.K)

    @property
    def nbytes(self) -> int:
        return self.packed.numel()


def q4_gemv(x: torch.Tensor, m: Q4Matrix, out_dtype=None) -> torch.Tensor:
    """``x @ Wᵀ`` for bf16 ``x`` of shape ``(..., K)``; returns ``(..., N)``
    in bfloat16 (rounded to nearest even, as the reference stores it) or in
    ``out_dtype=torch.float32``.  A few rows of x run the GEMV
    (``rec_q4_gemv``, 8 per launch), from :func:`gemm_min_rows` on (a prefill
    chunk's tokens) one GEMM on matrix cores with the same arithmetic
    (``rec_q4_gemm``)."""
    if x.shape[-1] != m.K:
        raise ValueError(f"x has {x.shape[-1]} features, the matrix {m.K}")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"x must be bfloat16, got {x.dtype}")
    out_dtype = torch.bfloat16 if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out_dtype must be bfloat16 or float32, got {out_dtype}")
    lead = x.shape[:-1]
    xs = x.reshape(-1, m.K)
    if xs.stride(-1) != 1 or xs.data_ptr() % 16 or (xs.shape[0] > 1 and xs.stride(0) % 8):
        xs = xs.contiguous()
    rows = xs.shape[0]
    out = torch.empty((rows, m.N), dtype=out_dtype, device=x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    code = _lib.REC_F32 if out_dtype == torch.float32 else _lib.REC_BF16
    if rows >= gemm_min_rows(m.K):
        # a prefill chunk's rows: one GEMM over the packed matrix (x's group
        # sums in a workspace first); fewer rows take GEMV launches of 8
        ws = torch.empty(lib.rec_q4_gemm_workspace_bytes(rows, m.K), dtype=torch.uint8, device=x.device)
        rc = lib.rec_q4_gemm(
            m.packed.data_ptr(), m.N, m.K, xs.data_ptr(), xs.stride(0), rows, out.data_ptr(), code, out.stride(0),
            ws.data_ptr(), ws.numel(), stream,
        )
        _lib.check(rc, "rec_q4_gemm")
        return out.reshape(*lead, m.N)
    for r0 in range(0, rows, MAX_VECTORS):
        M = min(MAX_VECTORS, rows - r0)
        xr, orow = xs[r0 : r0 + M], out[r0 : r0 + M]
        rc = lib.rec_q4_gemv(
            m.packed.data_ptr(), m.N, m.K, xr.data_ptr(), xs.stride(0), M, orow.data_ptr(), code, out.stride(0),
            stream,
        )
        _lib.check(rc, "rec_q4_gemv")
    return out.reshape(*lead, m.N)


def q4_gemv_parts(x: torch.Tensor, m: Q4Matrix, out_dtype=None):
    """:func:`q4_gemv` over a :meth:`Q4Matrix.stack` matrix, returned as one
    ``(..., N_i)`` view per stacked part (one launch for all of them)."""
    y = q4_gemv(x, m, out_dtype)
    return tuple(torch.split(y, list(m.parts), dim=-1))


def quantized_matmul(x, w, scales, biases, transpose=True, group_size=GROUP, bits=4, mode="affine"):
    """``mx.quantized_matmul`` for 4-bit affine group-64 weights with
    ``transpose=True`` (``x @ Wᵀ``), the configuration of the reference's
    projections.  Packs ``w`` on every call; keep a :class:`Q4Matrix` to pack once."""
    if not transpose or group_size != GROUP or bits != 4 or mode != "affine":
        raise NotImplementedError("only transpose=True, group_size=64, bits=4, mode='affine' is implemented")
    return q4_gemv(x, Q4Matrix(w, scales, biases))

"""Helpers shared by the GPU parity tests (oracle on the CPU, kernels on the GPU)."""

import numpy as np
import torch

import oracle as O
from rec_amd import to_logical

SCALE = 1.0 / np.sqrt(128.0)
ATOL, RTOL = 2e-3, 1e-3  # output tolerance of the decode path (fp32 accumulation)


def f32(x: torch.Tensor) -> np.ndarray:
    return x.detach().float().cpu().numpy()


def oracle_quantize(x: np.ndarray, bits: int):
    """Logical (codes, scales, zeros) of the oracle quantizer; zeros None for 8-bit."""
    if bits == 8:
        c, s = O.quantize_int8(x)
        return c, s, None
    return O.quantize_int4(x, 32)


def dequant(bits, codes, scales, zeros):
    if bits == 8:
        return O.dequantize_int8(codes, scales)
    return O.dequantize_int4(codes, scales, zeros, 32)


def gpu_logical(kv):
    c, s, z = to_logical(kv)
    return (c.cpu().numpy(), s.cpu().numpy(), None if z is None else z.cpu().numpy())


def assert_cache_equal(kv, ref):
    got = gpu_logical(kv)
    np.testing.assert_array_equal(got[0], ref[0], err_msg="codes differ")
    np.testing.assert_array_equal(got[1].view(np.uint16), np.asarray(ref[1]).view(np.uint16), err_msg="scales differ")
    if ref[2] is not None:
        np.testing.assert_array_equal(got[2].view(np.uint16), np.asarray(ref[2]).view(np.uint16), err_msg="zeros differ")


def assert_close(got: np.ndarray, ref: np.ndarray, what=""):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref)
    bound = ATOL + RTOL * np.abs(ref)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert np.all(err <= bound), (
        f"{what}: max |err| {err.max():.3e} (at {worst}: got {got[worst]:.6f} ref {ref[worst]:.6f})"
    )


def round_to(x: np.ndarray, dtype) -> np.ndarray:
    """float32 values rounded to nearest even in a 16-bit torch dtype."""
    if dtype == torch.bfloat16:
        return O.bf16_rn(x)
    if dtype == torch.float16:
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, np.float32)


def prefill_side(xhat: np.ndarray, quantized_kv, qdtype) -> np.ndarray:
    """One side (K or V) of a quantized cache as the prefill kernel attends
    over it: int8 codes exactly (x̂ as dequantized), 4-bit and affine values
    rounded to the query dtype, as the reference dequantizes the cache to it
    before its attention (model.py:194-195)."""
    if quantized_kv.bits == 8 and not quantized_kv.affine:
        return xhat
    return round_to(xhat, qdtype)


def oracle_xhat(kv) -> np.ndarray:
    """float32 x̂ of the valid rows of one quantized cache tensor, from its
    stored bytes (int8 q·s, uint4 (q - z)·s, affine q·s + b)."""
    codes, scales, extra = to_logical(kv)
    if kv.affine:
        c = codes.cpu().numpy()
        if kv.bits == 4:
            c = O.unpack_int4(c)
        return O.dequantize_affine(c, f32(scales), f32(extra))
    z = None if extra is None else extra.cpu().numpy()
    return dequant(kv.bits, codes.cpu().numpy(), scales.cpu().numpy(), z)


_DT_NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def q_sinks(sinks, qdtype):
    """The sink logits of a path that hands them over in the query dtype (the
    prefill branch over the quantized cache and every call over the bf16
    caches, model.py:202,211), as float64 NumPy; None stays None."""
    if sinks is None:
        return None
    return O.sink_logits(f32(sinks), _DT_NAMES[qdtype])

"""ctypes binding of ``librec_amd.so`` (declared in ``include/rec_amd.h``).

torch is imported before the library is loaded: torch ships the HIP runtime
(``libamdhip64.so``, soname ``libamdhip64.so.7``) and the library's dependency
on that soname then binds to torch's copy, so device pointers and streams are
shared.  :func:`library` checks that only one HIP runtime is mapped.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librec_amd.so")

REC_OK = 0
REC_EINVAL = -1
REC_EALIGN = -2
REC_ECAPACITY = -3
REC_EWORKSPACE = -4
REC_ELAUNCH = -5
REC_EUNSUPPORTED = -6

REC_F16, REC_BF16, REC_F32 = 0, 1, 2
REC_AFFINE8, REC_AFFINE4 = 0x108, 0x104  # MLX-style affine group 64: 8-bit keys, 4-bit values
REC_AFFINE8_F16, REC_AFFINE4_F16 = 0x208, 0x204  # the same with fp16 scales and biases

# Every symbol include/rec_amd.h declares, with (restype, argtypes).
_i, _i64, _f, _p, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
SIGNATURES = {
    "rec_version": (ctypes.c_char_p, []),
    "rec_last_error": (ctypes.c_char_p, []),
    "rec_kv_append": (
        _i,
        [_p, _p, _i, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _p],
    ),
    "rec_decode_default_splits": (_i, [_i, _i, _i64]),
    "rec_stream_read": (_i, [_p, _i64, _i, _p, _p]),
    "rec_region_create": (_i, [_i, _i64, _i64, _i64, _i64, ctypes.POINTER(_p), ctypes.POINTER(_p)]),
    "rec_region_grow": (_i, [_p, _i64, ctypes.POINTER(_i64)]),
    "rec_region_destroy": (_i, [_p]),
    "rec_decode_workspace_bytes": (_sz, [_i, _i, _i]),
    "rec_workspace_init": (_i, [_p, _sz, _p]),
    "rec_decode_attn": (
        _i,
        [_p, _i, _i64, _i64, _i, _p, _p, _p, _i, _p, _p, _p, _p, _f,
         _p, _i64, _i64, _i64, _i64,  # bias, strides (b, kv head, group member), extent
         _i, _i, _i, _i, _i64, _i64, _i, _p, _sz, _i, _p, _p],
    ),
    "rec_decode_append_attn": (
        _i,
        [
            _p, _i, _i64, _i64,  # q
            _p, _p, _i, _i64, _i64, _i64, _i64,  # new k/v
            _i, _p, _p, _p, _i, _p, _p, _p,  # cache
            _p, _f, _i, _i, _i, _i, _i64, _i64, _i, _p, _sz, _i, _p, _p,  # ... workspace, out_dtype, out, stream
        ],
    ),
}
SIGNATURES["rec_decode_partial"] = SIGNATURES["rec_decode_append_attn"]
SIGNATURES["rec_decode_append_attn_noalloc"] = (
    _i, SIGNATURES["rec_decode_append_attn"][1][:-5] + [_i, _p, _p]  # no workspace, workspace_bytes
)
SIGNATURES["rec_decode_scratch_bytes"] = (_sz, [])
SIGNATURES["rec_decode_merge"] = (_i, [_p, _i, _i, _i, _i64, _i, _i, _p, _sz, _i, _p, _p])
SIGNATURES["rec_prefill_attn"] = (
    _i,
    [_p, _i, _i64, _i64, _i64, _i, _p, _p, _p, _i, _p, _p, _p, _p, _f, _i, _i,
     _p, _i64, _i64, _i64, _i64, _i64,  # bias, strides (b, kv head, group member, query), extent
     _i, _i, _i, _i, _i, _i64, _i64, _i, _p, _sz, _i, _p, _p],
)
SIGNATURES["rec_prefill_workspace_bytes"] = (_sz, [_i, _i, _i, _i, _i])

SIGNATURES["rec_kv_write_bf16"] = (
    _i,
    [_p, _p, _i, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i, _i, _i, _i, _i64, _i64, _p],
)
SIGNATURES["rec_ring_join_bf16"] = (
    _i,
    [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i,  # ring
     _p, _p, _i, _i64, _i64, _i64, _i64, _i64, _i64,  # new rows
     _p, _p, _i, _i, _i, _i, _p],
)
SIGNATURES["rec_decode_bf16"] = (
    _i,
    [
        _p, _i, _i64, _i64,  # q
        _p, _p, _i, _i64, _i64, _i64, _i64,  # new k/v
        _p, _i64, _i64, _p, _i64, _i64,  # bf16 K, V
        _p, _f, _p, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _i64, _i64, _i, _p, _sz, _i, _p, _p,
    ],
)
SIGNATURES["rec_decode_bf16_ring"] = (
    _i,
    [
        _p, _i, _i64, _i64,  # q
        _p, _p, _i, _i64, _i64, _i64, _i64,  # new k/v
        _p, _i64, _i64, _p, _i64, _i64,  # the ring's K, V
        _p, _f, _i, _i, _i, _i, _i64, _i64, _i64, _i, _p, _sz, _i, _p, _p,  # ... T, capacity, slot, splits ...
    ],
)

SIGNATURES["rec_kv_dequant_bf16"] = (_i, [_i, _p, _p, _p, _i, _p, _p, _p, _i, _i, _i64, _i64, _p, _p, _p])
SIGNATURES["rec_prefill_bf16"] = (
    _i,
    [_p, _i, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _f, _i, _i,
     _p, _i64, _i64, _i64, _i64, _i64,  # bias
     _i, _i, _i, _i, _i, _i64, _i, _p, _sz, _i, _p, _p],
)
SIGNATURES["rec_q4_packed_bytes"] = (_sz, [_i64, _i64])
SIGNATURES["rec_q4_pack"] = (_i, [_p, _p, _p, _i64, _i64, _p, _sz, _p])
SIGNATURES["rec_q4_gemv"] = (_i, [_p, _i64, _i64, _p, _i64, _i, _p, _i, _i64, _p])
SIGNATURES["rec_q4_gemm_workspace_bytes"] = (_sz, [_i, _i64])
SIGNATURES["rec_q4_gemm"] = (_i, [_p, _i64, _i64, _p, _i64, _i, _p, _i, _i64, _p, _sz, _p])

_lock = threading.Lock()
_lib = None


class RecError(RuntimeError):
    """A failed library call that maps to no more specific Python error."""


def _hip_runtimes_mapped():
    try:
        with open("/proc/self/maps") as f:
            return sorted({line.split()[-1] for line in f if "libamdhip64" in line})
    except OSError:
        return []


def load(path: str = LIB_PATH):
    """Load the shared library and declare its signatures (no GPU work)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (binds the HIP runtime first)

        if not os.path.exists(path):
            raise RuntimeError(
                f"rec_amd HIP library not built ({path} missing); run `python -m rec_amd.build` first"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise RuntimeError(f"more than one HIP runtime is mapped into this process: {runtimes}")
        _lib = lib
        return lib


def last_error() -> str:
    return (load().rec_last_error() or b"").decode()


def check(code: int, what: str) -> None:
    """Raise the Python exception matching a library return code."""
    if code == REC_OK:
        return
    msg = f"{what}: {last_error()}"
    if code in (REC_EINVAL, REC_EALIGN):
        raise ValueError(msg)
    if code == REC_ECAPACITY:
        raise ValueError(msg)
    if code == REC_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RecError(msg)

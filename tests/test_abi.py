"""The C-ABI library loads and exports every symbol include/rec_amd.h declares.

No kernel is launched: argument validation runs on the host before any HIP
call, so these tests run without a GPU.
"""

import os
import re

import pytest

import rec_amd
from rec_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rec_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rec_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("librec_amd.so is not built (run python -m rec_amd.build)")
    return rec_amd.library()


def test_header_symbols_exported(lib):
    syms = declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in rec_amd.h but not exported"
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_version_and_sizes(lib):
    assert lib.rec_version().startswith(b"rec_amd")
    assert lib.rec_decode_default_splits(1, 4, 32768) >= 64
    assert lib.rec_decode_default_splits(1, 1, 10) == 1
    assert lib.rec_decode_default_splits(1, 4, 258048) <= 256
    small = lib.rec_decode_workspace_bytes(1, 4, 16)
    big = lib.rec_decode_workspace_bytes(1, 4, 256)
    assert 0 < small < big
    # counters + stats + acc for 4 heads x 256 splits x 8 rows x 128 floats
    assert big >= 4 * 256 * 8 * 128 * 4


def _append(lib, **kw):
    a = dict(k=None, v=None, dt=0, kb=8, vb=8, B=1, H=1, L=1, D=128, off=0, cap=64)
    a.update(kw)
    return lib.rec_kv_append(
        a["k"], a["v"], a["dt"], 0, 0, 0, 0, 0, 0, a["kb"], 16, 16, 16, a["vb"], 16, 16, 16,
        a["B"], a["H"], a["L"], a["D"], a["off"], a["cap"], None,
    )


def test_append_validation(lib):
    assert _append(lib, kb=5) == _lib.REC_EINVAL
    assert "k_bits" in _lib.last_error()
    assert _append(lib, D=64) == _lib.REC_EUNSUPPORTED
    assert _append(lib, cap=100) == _lib.REC_EINVAL
    assert _append(lib, off=64, L=1, cap=64) == _lib.REC_ECAPACITY
    assert "capacity" in _lib.last_error()
    assert _append(lib, L=0) == _lib.REC_OK  # nothing to do, nothing launched
    assert _append(lib, dt=7) == _lib.REC_EINVAL


def _decode(lib, **kw):
    a = dict(q=16, dt=0, kb=8, vb=8, B=1, Hq=8, Hkv=1, D=128, T=10, cap=64, splits=0, ws=16, wsb=1 << 30, out=16,
             odt=_lib.REC_F32, bias=(None, 0, 0, 0, 0))
    a.update(kw)
    return lib.rec_decode_attn(
        a["q"], a["dt"], 0, 0, a["kb"], 16, 16, 16, a["vb"], 16, 16, 16, None, 0.088, *a["bias"],
        a["B"], a["Hq"], a["Hkv"], a["D"], a["T"], a["cap"], a["splits"], a["ws"], a["wsb"], a["odt"], a["out"], None,
    )


def test_decode_validation(lib):
    assert _decode(lib, Hq=12, Hkv=8) == _lib.REC_EINVAL
    assert _decode(lib, Hq=16, Hkv=1) == _lib.REC_EUNSUPPORTED
    assert "GQA" in _lib.last_error()
    assert _decode(lib, T=0) == _lib.REC_EINVAL
    assert _decode(lib, T=65) == _lib.REC_ECAPACITY
    assert _decode(lib, wsb=16) == _lib.REC_EWORKSPACE
    assert _decode(lib, ws=8) == _lib.REC_EALIGN
    assert _decode(lib, out=4) == _lib.REC_EALIGN
    assert _decode(lib, D=96) == _lib.REC_EUNSUPPORTED
    assert _decode(lib, odt=5) == _lib.REC_EINVAL  # output dtype: REC_F32, REC_BF16 or REC_F16
    assert "output" in _lib.last_error()
    # a score bias (mask array): 16-byte aligned, strides multiples of 4, extent below 2^29
    assert _decode(lib, bias=(8, 0, 0, 0, 64)) == _lib.REC_EALIGN
    assert _decode(lib, bias=(16, 6, 0, 0, 64)) == _lib.REC_EALIGN
    assert "multiples of 4" in _lib.last_error()
    assert _decode(lib, bias=(16, 0, 0, 0, 1 << 29)) == _lib.REC_EUNSUPPORTED
    assert _decode(lib, bias=(16, 0, 0, 0, 0)) == _lib.REC_EUNSUPPORTED
    # the affine format comes as REC_AFFINE8 keys with REC_AFFINE4 values only
    assert _decode(lib, kb=_lib.REC_AFFINE8, vb=8) == _lib.REC_EUNSUPPORTED
    assert _decode(lib, kb=_lib.REC_AFFINE4, vb=_lib.REC_AFFINE8) == _lib.REC_EUNSUPPORTED
    assert "affine" in _lib.last_error()
    assert _append(lib, kb=_lib.REC_AFFINE8, vb=4) == _lib.REC_EUNSUPPORTED
    assert _append(lib, kb=_lib.REC_AFFINE8, vb=_lib.REC_AFFINE4, L=0) == _lib.REC_OK


def test_error_mapping():
    with pytest.raises(ValueError):
        _lib.check(_lib.REC_ECAPACITY, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.REC_EUNSUPPORTED, "x")
    with pytest.raises(_lib.RecError):
        _lib.check(_lib.REC_ELAUNCH, "x")
    _lib.check(_lib.REC_OK, "x")


def _decode_bf16(lib, **kw):
    a = dict(q=16, dt=1, kn=None, vn=None, k=16, sb=0, sh=0, v=16, B=1, Hq=8, Hkv=1, D=128, T=10, cap=64,
             splits=0, ws=16, wsb=1 << 30, out=16, odt=_lib.REC_F32, bias=(None, 0, 0, 0, 0))
    a.update(kw)
    return lib.rec_decode_bf16(
        a["q"], a["dt"], 0, 0, a["kn"], a["vn"], 1, 0, 0, 0, 0, a["k"], a["sb"], a["sh"], a["v"], a["sb"], a["sh"],
        None, 0.088, *a["bias"], a["B"], a["Hq"], a["Hkv"], a["D"], a["T"], a["cap"], a["splits"], a["ws"], a["wsb"],
        a["odt"], a["out"], None,
    )


def test_decode_bf16_validation(lib):
    assert _decode_bf16(lib, T=65) == _lib.REC_ECAPACITY
    assert _decode_bf16(lib, T=0) == _lib.REC_EINVAL
    assert _decode_bf16(lib, k=8) == _lib.REC_EALIGN
    assert _decode_bf16(lib, sh=4) == _lib.REC_EALIGN
    assert "multiples of 8" in _lib.last_error()
    assert _decode_bf16(lib, Hq=16, Hkv=1) == _lib.REC_EUNSUPPORTED
    # split plans need the workspace; the automatic plan over a short cache
    # (one workgroup per KV head writing the output) needs none
    assert _decode_bf16(lib, T=100, cap=128, wsb=16, splits=3) == _lib.REC_EWORKSPACE
    assert _decode_bf16(lib, T=1025, cap=2048, wsb=16) == _lib.REC_EWORKSPACE
    assert _decode_bf16(lib, odt=3) == _lib.REC_EINVAL
    assert _decode_bf16(lib, bias=(16, 0, 2, 0, 64)) == _lib.REC_EALIGN
    assert _decode_bf16(lib, kn=16) == _lib.REC_EINVAL  # new keys without new values
    assert _decode_bf16(lib, D=64) == _lib.REC_EUNSUPPORTED
    assert _decode_bf16(lib, q=8) == _lib.REC_EALIGN


def _write_bf16(lib, **kw):
    a = dict(k=16, v=16, dt=1, s=16, B=1, H=4, L=1, D=128, off=0, cap=64)
    a.update(kw)
    return lib.rec_kv_write_bf16(
        16, 16, a["dt"], 0, 0, 0, 0, 0, 0, a["k"], 0, a["s"], a["v"], 0, a["s"],
        a["B"], a["H"], a["L"], a["D"], a["off"], a["cap"], None,
    )


def test_write_bf16_validation(lib):
    assert _write_bf16(lib, off=64) == _lib.REC_ECAPACITY
    assert _write_bf16(lib, L=0) == _lib.REC_OK
    assert _write_bf16(lib, D=64) == _lib.REC_EUNSUPPORTED
    assert _write_bf16(lib, k=8) == _lib.REC_EALIGN
    assert _write_bf16(lib, s=12) == _lib.REC_EALIGN
    assert _write_bf16(lib, dt=9) == _lib.REC_EINVAL


def _q4_gemv(lib, **kw):
    a = dict(p=16, N=64, K=256, x=16, xs=256, M=1, o=16, dt=1, os=64)
    a.update(kw)
    return lib.rec_q4_gemv(a["p"], a["N"], a["K"], a["x"], a["xs"], a["M"], a["o"], a["dt"], a["os"], None)


def test_q4_validation(lib):
    assert lib.rec_q4_packed_bytes(16, 256) == 2 * 1152
    assert lib.rec_q4_packed_bytes(17, 256) == 2 * 2 * 1152
    assert lib.rec_q4_packed_bytes(16, 192) == 0
    assert lib.rec_q4_packed_bytes(0, 256) == 0
    assert lib.rec_q4_pack(16, 16, 16, 16, 256, 16, 2303, None) == _lib.REC_EWORKSPACE
    assert lib.rec_q4_pack(16, 16, 16, 16, 200, 16, 9999, None) == _lib.REC_EINVAL
    assert lib.rec_q4_pack(8, 16, 16, 16, 256, 16, 2304, None) == _lib.REC_EALIGN
    assert _q4_gemv(lib, K=192) == _lib.REC_EINVAL
    assert _q4_gemv(lib, M=0) == _lib.REC_EINVAL
    assert _q4_gemv(lib, M=9) == _lib.REC_EINVAL
    assert _q4_gemv(lib, dt=0) == _lib.REC_EINVAL
    assert _q4_gemv(lib, x=8) == _lib.REC_EALIGN
    assert _q4_gemv(lib, M=2, xs=260) == _lib.REC_EALIGN
    assert _q4_gemv(lib, M=2, xs=128) == _lib.REC_EINVAL
    assert _q4_gemv(lib, M=8, K=12288, xs=12288) == _lib.REC_EUNSUPPORTED


def _dequant(lib, **kw):
    a = dict(kb=8, vb=8, B=1, H=2, T=10, cap=64, ko=16, vo=16)
    a.update(kw)
    return lib.rec_kv_dequant_bf16(a["kb"], 16, 16, 16, a["vb"], 16, 16, 16, a["B"], a["H"], a["T"], a["cap"],
                                   a["ko"], a["vo"], None)


def test_dequant_validation(lib):
    assert _dequant(lib, kb=5) == _lib.REC_EINVAL
    assert _dequant(lib, kb=_lib.REC_AFFINE8, vb=4) == _lib.REC_EUNSUPPORTED
    assert _dequant(lib, cap=100) == _lib.REC_EINVAL
    assert _dequant(lib, T=65) == _lib.REC_ECAPACITY
    assert _dequant(lib, T=-1) == _lib.REC_EINVAL
    assert _dequant(lib, H=0) == _lib.REC_EINVAL
    assert _dequant(lib, ko=None) == _lib.REC_EINVAL
    assert _dequant(lib, vo=8) == _lib.REC_EALIGN
    assert _dequant(lib, T=0) == _lib.REC_OK  # nothing to do, nothing launched
    assert _dequant(lib, kb=_lib.REC_AFFINE8, vb=_lib.REC_AFFINE4, T=0) == _lib.REC_OK


def test_capacity_bound(lib):
    """2^24 tokens per KV head is the largest cache the decode accepts."""
    assert _decode(lib, cap=(1 << 24) + 32, T=100) == _lib.REC_EUNSUPPORTED
    assert "16M" in _lib.last_error()


def _prefill(lib, **kw):
    a = dict(L=4, T=1000, cap=1024, splits=0, ws=16, wsb=1 << 30, window=0, causal=1, bias=(None, 0, 0, 0, 0, 0))
    a.update(kw)
    return lib.rec_prefill_attn(
        16, _lib.REC_BF16, 0, 0, 0, 8, 16, 16, None, 8, 16, 16, None, None, 0.088, a["causal"], a["window"],
        *a["bias"], 1, 8, 1, 128, a["L"], a["T"], a["cap"], a["splits"], a["ws"], a["wsb"], _lib.REC_F32, 16, None,
    )


def test_prefill_split_validation(lib):
    """Explicit key splits need a workspace; too many splits are refused."""
    assert _prefill(lib, splits=65) == _lib.REC_EINVAL
    assert _prefill(lib, splits=3, ws=None, wsb=0) == _lib.REC_EWORKSPACE
    assert _prefill(lib, splits=3, wsb=1024) == _lib.REC_EWORKSPACE
    assert _prefill(lib, splits=3, ws=8) == _lib.REC_EALIGN
    assert _prefill(lib, window=-1) == _lib.REC_EINVAL
    assert "window" in _lib.last_error()
    # a bias carries the whole mask: no causal flag or window beside it
    assert _prefill(lib, bias=(16, 0, 0, 0, 1000, 4000)) == _lib.REC_EINVAL
    assert "bias" in _lib.last_error()
    assert _prefill(lib, causal=0, bias=(16, 0, 0, 0, 1001, 4004)) == _lib.REC_EALIGN


def test_prefill_workspace_bytes(lib):
    row = 256 * (128 + 2) * 4  # one block of 256 (query, head) rows of one KV head, one split
    # 20 queries x 8 heads = 160 rows: one block per KV head, 4 workgroups;
    # the automatic plan allows 64 splits
    assert lib.rec_prefill_workspace_bytes(1, 32, 4, 20, 0) == 4 * 64 * row
    # 64 blocks x 4 KV heads fill the chip: no split, no workspace
    assert lib.rec_prefill_workspace_bytes(1, 32, 4, 2048, 0) == 0
    # one query head per KV head: 2048 rows = 8 blocks x 4 KV heads, 8 splits
    assert lib.rec_prefill_workspace_bytes(1, 4, 4, 2048, 0) == 4 * 8 * 8 * row
    assert lib.rec_prefill_workspace_bytes(2, 16, 2, 40, 7) == 2 * 2 * 7 * 2 * row
    assert lib.rec_prefill_workspace_bytes(1, 32, 4, 20, 1) == 0
    assert lib.rec_prefill_workspace_bytes(1, 30, 4, 20, 0) == 0  # Hq not a multiple of Hkv


def _append_attn(lib, **kw):
    a = dict(B=1, Hq=8, Hkv=1, T=100, cap=128, splits=0, ws=8, wsb=1 << 30)
    a.update(kw)
    return lib.rec_decode_append_attn(
        16, 0, 0, 0, 16, 16, 0, 0, 0, 0, 0, 8, 16, 16, None, 8, 16, 16, None, None, 0.088,
        a["B"], a["Hq"], a["Hkv"], 128, a["T"], a["cap"], a["splits"], a["ws"], a["wsb"], _lib.REC_F32, 16, None,
    )


@pytest.mark.parametrize("B,Hkv,splits", [(64, 4, 0), (1, 1, 1), (1, 4, 1), (2, 4, 2), (1, 4, 0)])
def test_fused_decode_workspace_size(lib, B, Hkv, splits):
    """A fused decode (append + attend) adds the newest token's split to the
    regular ones, so a request for one split launches two.  The size the
    library reports for a request must cover that plan: called with exactly
    that many bytes, the size check passes and the (deliberately misaligned)
    workspace pointer is what is refused -- nothing is launched either way."""
    req = splits if splits > 0 else lib.rec_decode_default_splits(B, Hkv, 4000)
    need = lib.rec_decode_workspace_bytes(B, Hkv, req)
    rc = _append_attn(lib, B=B, Hq=8 * Hkv, Hkv=Hkv, T=4000, cap=4096, splits=splits, ws=8, wsb=need)
    assert rc == _lib.REC_EALIGN, _lib.last_error()
    assert "workspace must be 16-byte aligned" in _lib.last_error()
    # one byte short of a two-split plan is refused for a one-split request
    if req == 1:
        short = lib.rec_decode_workspace_bytes(B, Hkv, 2) - 1
        assert _append_attn(lib, B=B, Hq=8 * Hkv, Hkv=Hkv, T=4000, cap=4096, splits=1, ws=16, wsb=short) == (
            _lib.REC_EWORKSPACE)


def test_region_validation(lib):
    import ctypes

    h, base = ctypes.c_void_p(), ctypes.c_void_p()
    # rows, token bytes and bank size must be positive, max_tokens a multiple of the bank
    assert lib.rec_region_create(0, 0, 262144, 256, 65536, ctypes.byref(h), ctypes.byref(base)) == _lib.REC_EINVAL
    assert lib.rec_region_create(0, 8, 100000, 256, 65536, ctypes.byref(h), ctypes.byref(base)) == _lib.REC_EINVAL
    assert "bank_tokens" in _lib.last_error()
    assert lib.rec_region_create(0, 8, 262144, 256, 65536, None, None) == _lib.REC_EINVAL
    assert lib.rec_region_grow(None, 1, None) == _lib.REC_EINVAL
    assert lib.rec_region_destroy(None) == _lib.REC_OK


def test_stream_read_validation(lib):
    assert lib.rec_stream_read(None, 1024, 256, 16, None) == _lib.REC_EINVAL
    assert lib.rec_stream_read(16, 1000, 256, 16, None) == _lib.REC_EINVAL  # not a multiple of 16
    assert "multiple of 16" in _lib.last_error()
    assert lib.rec_stream_read(8, 1024, 256, 16, None) == _lib.REC_EALIGN
    assert lib.rec_stream_read(16, 1024, 0, 16, None) == _lib.REC_EINVAL


def test_decode_bf16_ring_validation(lib):
    """rec_decode_bf16_ring: the new token is required and its slot must be
    one of the T occupied slots (checked before anything is launched)."""
    def call(kn, slot, T=10):
        return lib.rec_decode_bf16_ring(
            16, 1, 0, 0, kn, kn, 1, 0, 0, 0, 0, 16, 0, 0, 16, 0, 0, None, 0.088, 1, 8, 1, 128, T, 64, slot, 0, 16,
            1 << 30, _lib.REC_F32, 16, None,
        )
    assert call(None, 3) == _lib.REC_EINVAL
    assert "required" in _lib.last_error()
    assert call(16, 10) == _lib.REC_EINVAL
    assert call(16, -1) == _lib.REC_EINVAL
    assert "slot" in _lib.last_error()

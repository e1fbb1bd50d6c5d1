"""rec_decode_append_attn_noalloc (split partials in the library's static
device scratch, no workspace argument, no allocation) against
rec_decode_append_attn on identical caches: outputs and cache bytes equal bit
for bit, on two calls in a row, the second one smaller; an over-size plan is
refused before anything is launched."""

import numpy as np
import pytest
import torch

import rec_amd
from rec_amd import MixedQuantizedKVCache, QuantizedKVCache, _lib, synthetic, to_logical
from rec_amd.attention import workspace
from tests.gpu_util import SCALE

pytestmark = pytest.mark.gpu

HQ, HKV = 32, 4


def make(fmt, B, T0, seed):
    if fmt == "affine":
        c = MixedQuantizedKVCache(max_tokens=T0 + 64)
    else:
        c = QuantizedKVCache(32, fmt, fmt, max_tokens=T0 + 64)
    k = synthetic.kv((B, HKV, T0, 128), seed, kind="outliers", frac=0.02)
    v = synthetic.kv((B, HKV, T0, 128), seed + 1, kind="outliers", frac=0.02)
    c.update_and_fetch(k, v)
    c._reserve(B, HKV, T0 + 1, "cuda")
    return c


def call(lib, noalloc, c, q, kn, vn, sinks, out, splits):
    (kc, ks, kz), (vc, vs, vz) = c.keys, c.values
    kcode, vcode = c._view()[0].code, c._view()[1].code
    B = q.shape[0]
    stream = torch.cuda.current_stream().cuda_stream
    head = (q.data_ptr(), _lib.REC_F16, q.stride(0), q.stride(1), kn.data_ptr(), vn.data_ptr(), _lib.REC_F16,
            kn.stride(0), kn.stride(1), vn.stride(0), vn.stride(1),
            kcode, kc.data_ptr(), ks.data_ptr(), None if kz is None else kz.data_ptr(),
            vcode, vc.data_ptr(), vs.data_ptr(), None if vz is None else vz.data_ptr(),
            sinks.data_ptr(), SCALE, B, HQ, HKV, 128, c.offset + 1, c.capacity, splits)
    if noalloc:
        return lib.rec_decode_append_attn_noalloc(*head, _lib.REC_F32, out.data_ptr(), stream)
    ws = workspace(q.device, B, HKV, splits if splits > 0 else lib.rec_decode_default_splits(B, HKV, c.offset + 1),
                   stream)
    return lib.rec_decode_append_attn(*head, ws.data_ptr(), ws.numel(), _lib.REC_F32, out.data_ptr(), stream)


@pytest.mark.parametrize("fmt", [8, 4, "affine"])
def test_noalloc_equals_workspace_entry_point(gpu, fmt):
    lib = rec_amd.library()
    assert lib.rec_decode_scratch_bytes() == 8 << 20
    sinks = torch.randn(HQ, device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    # two calls in a row, the second with a smaller input (fewer tokens, one sequence fewer, one split)
    for i, (B, T0, splits) in enumerate([(2, 20000, 0), (1, 700, 1)]):
        a, b = make(fmt, B, T0, 100 + i), make(fmt, B, T0, 100 + i)
        q = synthetic.query(B, HQ, 1, 110 + i)[:, :, 0].contiguous()
        kn, vn = synthetic.kv((B, HKV, 1, 128), 120 + i), synthetic.kv((B, HKV, 1, 128), 130 + i)
        outs = []
        for c, noalloc in ((a, False), (b, True)):
            out = torch.full((B, HQ, 128), float("nan"), device="cuda")
            rc = call(lib, noalloc, c, q, kn, vn, sinks, out, splits)
            assert rc == 0, _lib.last_error()
            c.offset += 1
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.isfinite(outs[1]).all()
        assert torch.equal(outs[0], outs[1]), f"call {i}: outputs differ"
        for x, y in zip(a.keys_and_values(), b.keys_and_values()):
            for u, w in zip(to_logical(x), to_logical(y)):
                assert (u is None and w is None) or torch.equal(u, w), f"call {i}: cache bytes differ"


def test_noalloc_refuses_oversize_plan(gpu):
    lib = rec_amd.library()
    B, T0 = 64, 4000
    c = QuantizedKVCache(32, 8, 8, max_tokens=T0 + 64)
    c._reserve(B, HKV, T0 + 1, "cuda")
    c.offset = T0
    q = torch.zeros((B, HQ, 128), dtype=torch.float16, device="cuda")
    kn = torch.zeros((B, HKV, 1, 128), dtype=torch.float16, device="cuda")
    out = torch.full((B, HQ, 128), float("nan"), device="cuda")
    sinks = torch.zeros(HQ, device="cuda")
    rc = call(lib, True, c, q, kn, kn, sinks, out, 64)  # 64 x 4 heads x 64 splits of partials: 17 MB
    assert rc == _lib.REC_EWORKSPACE
    assert "static scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(out).all()  # nothing was launched
    assert np.all(to_logical(c.keys_and_values()[0])[0].cpu().numpy() == 0)

"""Decode at the largest cache the kernels accept: 2^24 tokens per KV head.

A full oracle pass over 16M tokens is out of reach on the CPU, so the inputs
are chosen to make the answer cheap to compute: every key is the same row, so
every score is equal and the softmax weights are uniform, and the values of
each 2^20-token chunk i repeat a P-token pattern plus a chunk constant c_i.
The attention output is then the mean over chunks of the mean of the
dequantized pattern rows (the oracle quantizes and dequantizes the 16 x P
rows; per-row quantization keeps v̂ periodic inside a chunk), within 2e-3 abs
+ 1e-3 rel; a chunk read from the wrong place or skipped moves the mean by
about 1/16 of its constant.  This covers the 32-bit buffer offsets of a 2 GiB code
slice, splits of 65,536 tokens and the top of the ABI's capacity range (2^24
accepted; 2^24 + 32 is refused, tests/test_abi.py).
"""

import numpy as np
import pytest
import torch

import oracle as O
from rec_amd import MixedQuantizedKVCache, QuantizedKVCache, quantized_attention_with_sinks, synthetic
from tests.gpu_util import SCALE, assert_close, dequant, f32, oracle_quantize

pytestmark = pytest.mark.gpu

T_MAX = 1 << 24
PERIOD = 4096
CHUNK = 1 << 20


def v_hat_rows(v_pat, vb, affine):
    """Dequantized pattern rows as the oracle forms them (float64)."""
    x = f32(v_pat)
    if affine:
        q, s, b = O.quantize_affine(x, vb)
        return O.dequantize_affine(q, s, b).astype(np.float64)
    return dequant(vb, *oracle_quantize(x, vb)).astype(np.float64)


@pytest.mark.parametrize("fmt", [(8, 8, False), (4, 4, False), (8, 4, True)], ids=["k8v8", "k4v4", "affine"])
def test_decode_at_max_capacity(gpu, fmt):
    kb, vb, affine = fmt
    Hq, Hkv = 8, 1
    cache = (MixedQuantizedKVCache(max_tokens=T_MAX) if affine
             else QuantizedKVCache(32, kb, vb, max_tokens=T_MAX))
    k_row = synthetic.kv((1, Hkv, 1, 128), 901)
    v_pat = synthetic.kv((1, Hkv, PERIOD, 128), 902, kind="outliers", frac=0.01)
    k_chunk = k_row.expand(1, Hkv, CHUNK, 128).contiguous()
    consts = [0.25 * i - 1.5 for i in range(T_MAX // CHUNK)]
    for c in consts:
        cache.update_and_fetch(k_chunk, (v_pat + c).repeat(1, 1, CHUNK // PERIOD, 1))
    del k_chunk
    assert cache.offset == T_MAX and cache.capacity == T_MAX
    q = synthetic.query(1, Hq, 1, 903, dtype=torch.bfloat16)
    kq, vq = cache.keys_and_values()
    out = quantized_attention_with_sinks(q, kq, vq, SCALE, None, None, 64 if affine else 32, kb, vb,
                                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    mean = np.mean([v_hat_rows(v_pat + c, vb, affine).mean(axis=2) for c in consts], axis=0)  # (1, 1, 128)
    ref = np.broadcast_to(mean[:, :, None, :], (1, Hq, 1, 128))
    assert_close(f32(out), ref, f"{kb}/{vb}-bit at {T_MAX} tokens")
    with pytest.raises(ValueError, match="Decode context limit exhausted"):
        cache.update_and_fetch(k_row, v_pat[:, :, :1])
    del cache
    torch.cuda.empty_cache()



def test_row_kernels_stride_past_their_grid(gpu):
    """An append of 4.8M rows (600K tokens x 8 KV heads) needs more than the
    2^20 workgroups the row kernels launch, so they stride; the rows written
    last (and their bf16 dequantization) equal the oracle's, bit for bit."""
    from rec_amd import dequantize_kv, to_logical

    B, Hkv, L, tail = 1, 8, 600_000, 256
    cache = QuantizedKVCache(32, 8, 8, max_tokens=L)
    g = torch.Generator(device="cuda").manual_seed(77)
    k = torch.randn((B, Hkv, L, 128), generator=g, device="cuda").to(torch.float16)
    v = torch.randn((B, Hkv, L, 128), generator=g, device="cuda").to(torch.float16)
    kq, vq = cache.update_and_fetch(k, v)
    kd, vd = dequantize_kv(kq, vq)
    torch.cuda.synchronize()
    for kv, x, xd, name in ((kq, k, kd, "K"), (vq, v, vd, "V")):
        codes, scales, _ = to_logical(kv)
        want_c, want_s = O.quantize_int8(f32(x[:, :, L - tail :]))
        np.testing.assert_array_equal(codes[:, :, L - tail : L].cpu().numpy(), want_c, err_msg=f"{name} codes")
        np.testing.assert_array_equal(scales[:, :, L - tail : L].cpu().numpy().view(np.uint16),
                                      np.asarray(want_s, np.float16).view(np.uint16), err_msg=f"{name} scales")
        want_d = O.bf16_rn(O.dequantize_int8(want_c, want_s))
        got_d = xd[:, :, L - tail :].float().cpu().numpy()
        np.testing.assert_array_equal(got_d, want_d, err_msg=f"{name} dequantized")
    del cache, k, v, kd, vd
    torch.cuda.empty_cache()

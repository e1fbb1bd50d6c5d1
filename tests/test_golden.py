"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

On the CPU: the oracle reproduces every fixture bit for bit (a regression pin
on the oracle), and the fixture outputs agree with torch's scaled dot-product
attention in float64 over the dequantized cache (an independent pin).
On the GPU: the kernels reproduce the fixture cache bytes exactly and the
outputs within 2e-3 absolute + 1e-3 relative.
"""

import os

import numpy as np
import pytest
import torch

import oracle as O
from tests.gpu_util import SCALE, assert_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DECODE = ["cfg1_int8", "int4_heavy", "mixed_k8v4"]


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _deq(f, p, bits):
    if bits == 8:
        return O.dequantize_int8(f[p + "_codes"], f[p + "_scales"])
    return O.dequantize_int4(f[p + "_codes"], f[p + "_scales"], f[p + "_zeros"])


@pytest.mark.parametrize("name", DECODE)
def test_oracle_reproduces_fixture(name):
    f = load(name)
    kb, vb = int(f["k_bits"]), int(f["v_bits"])
    for p, bits, x in (("k", kb, f["k"]), ("v", vb, f["v"])):
        got = O.quantize_int8(x) if bits == 8 else O.quantize_int4(x)
        np.testing.assert_array_equal(got[0], f[p + "_codes"])
        np.testing.assert_array_equal(got[1].view(np.uint16), f[p + "_scales"].view(np.uint16))
        if bits == 4:
            np.testing.assert_array_equal(got[2].view(np.uint16), f[p + "_zeros"].view(np.uint16))
    kh, vh = _deq(f, "k", kb), _deq(f, "v", vb)
    np.testing.assert_array_equal(O.attention(f["q"], kh, vh, SCALE).astype(np.float32), f["out"])
    np.testing.assert_array_equal(O.attention(f["q"], kh, vh, SCALE, f["sinks"]).astype(np.float32), f["out_sinks"])


@pytest.mark.parametrize("name", DECODE)
def test_fixture_matches_torch_sdpa(name):
    f = load(name)
    kh, vh = _deq(f, "k", int(f["k_bits"])), _deq(f, "v", int(f["v_bits"]))
    q = torch.from_numpy(f["q"].astype(np.float64))
    G = q.shape[1] // kh.shape[1]
    k = torch.from_numpy(kh.astype(np.float64)).repeat_interleave(G, 1)
    v = torch.from_numpy(vh.astype(np.float64)).repeat_interleave(G, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=SCALE).numpy()
    np.testing.assert_allclose(f["out"], ref, rtol=1e-6, atol=1e-7)


def test_prefill_fixture():
    f = load("prefill_causal")
    P = int(f["prefix"])
    kh, vh = O.dequantize_int8(f["k_codes"], f["k_scales"]), O.dequantize_int8(f["v_codes"], f["v_scales"])
    out = O.attention(f["q"], kh, vh, SCALE, f["sinks"], "causal").astype(np.float32)
    np.testing.assert_array_equal(out, f["out_sinks"])
    out_q = O.attention(f["q"], kh, vh, SCALE, f["sinks"], "causal", sink_dtype="float16").astype(np.float32)
    np.testing.assert_array_equal(out_q, f["out_sinks_qdtype"])
    # the fp16-rounded sinks are torch's own cast of the stored float32 ones
    s16 = torch.from_numpy(f["sinks"]).half().double().numpy()
    np.testing.assert_array_equal(
        O.attention(f["q"], kh, vh, SCALE, s16, "causal").astype(np.float32), f["out_sinks_qdtype"])
    # the last query row sees every key: equal to a plain decode over the whole cache
    last = O.attention(f["q"][:, :, -1:], kh, vh, SCALE, f["sinks"]).astype(np.float32)
    np.testing.assert_allclose(out[:, :, -1:], last, rtol=1e-6, atol=1e-7)
    assert out.shape[2] == f["q"].shape[2] and kh.shape[2] == P + f["q"].shape[2]


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
def test_gpu_reproduces_fixture(gpu, name):
    import rec_amd

    f = load(name)
    kb, vb = int(f["k_bits"]), int(f["v_bits"])
    dev = torch.device("cuda")
    cache = rec_amd.QuantizedKVCache(32, kb, vb)
    kq, vq = cache.update_and_fetch(torch.from_numpy(f["k"]).to(dev), torch.from_numpy(f["v"]).to(dev))
    for p, kv in (("k", kq), ("v", vq)):
        c, s, z = (None if t is None else t.cpu().numpy() for t in rec_amd.to_logical(kv))
        np.testing.assert_array_equal(c, f[p + "_codes"])
        np.testing.assert_array_equal(s.view(np.uint16), f[p + "_scales"].view(np.uint16))
        if z is not None:
            np.testing.assert_array_equal(z.view(np.uint16), f[p + "_zeros"].view(np.uint16))
    q = torch.from_numpy(f["q"]).to(dev)
    for sinks, key in ((None, "out"), (torch.from_numpy(f["sinks"]).to(dev), "out_sinks")):
        out = rec_amd.quantized_attention_with_sinks(q, kq, vq, SCALE, None, sinks, 32, kb, vb, out_dtype=torch.float32)
        assert_close(out.cpu().numpy(), f[key].astype(np.float64), f"{name} {key}")

"""Write the golden fixtures of the quantized-KV decode path.

Inputs are seeded NumPy draws (stored in the files, so the fixtures do not
depend on the generator's stream); expected cache bytes and outputs come from
the oracle.  Run from the repository root:

    python tests/golden/make_golden.py

Fixtures:
* cfg1_int8.npz — the tiny CPU-sized workload: batch 1, 8 query heads over 1 KV
  head, head_dim 128, 1024 tokens, Q/K/V ~ N(0,1) fp16, int8 KV; outputs
  without and with sink logits.
* int4_heavy.npz — 32 query / 4 KV heads, 128 tokens, uint4 KV (group 32),
  N(0,1) with 5% of channels Student-t(3).
* mixed_k8v4.npz — 8 query / 2 KV heads, 96 tokens, int8 K and uint4 V, 1%
  outlier channels x8.
* prefill_causal.npz — 8 query / 1 KV head, 192 cached + 64 new causal queries,
  int8 KV; outputs with the sinks as float32 values (``out_sinks``, the
  function of model.py:108-139) and rounded to the fp16 query dtype
  (``out_sinks_qdtype``, the prefill branch of model.py:202).
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402

SCALE = 1.0 / np.sqrt(128.0)


def _kv(rng, shape, kind=None, frac=0.0):
    x = rng.standard_normal(shape)
    if kind is not None:
        B, H, T, D = shape
        n = max(1, int(round(frac * D)))
        for h in range(H):
            idx = rng.choice(D, n, replace=False)
            if kind == "outliers":
                x[:, h, :, idx] *= 8.0
            else:
                x[:, h, :, idx] = rng.standard_t(3, (B, T, n)).transpose(2, 0, 1)
    return x.astype(np.float16)


def _quant(x, bits):
    if bits == 8:
        c, s = O.quantize_int8(x)
        return dict(codes=c, scales=s), O.dequantize_int8(c, s)
    c, s, z = O.quantize_int4(x)
    return dict(codes=c, scales=s, zeros=z), O.dequantize_int4(c, s, z)


def decode_fixture(path, seed, B, Hq, Hkv, T, k_bits, v_bits, kind=None, frac=0.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, 1, 128)).astype(np.float16)
    k = _kv(rng, (B, Hkv, T, 128), kind, frac)
    v = _kv(rng, (B, Hkv, T, 128), kind, frac)
    sinks = rng.standard_normal(Hq).astype(np.float32)
    kq, kh = _quant(k, k_bits)
    vq, vh = _quant(v, v_bits)
    out = O.attention(q, kh, vh, SCALE).astype(np.float32)
    out_sinks = O.attention(q, kh, vh, SCALE, sinks).astype(np.float32)
    arrays = dict(q=q, k=k, v=v, sinks=sinks, out=out, out_sinks=out_sinks, k_bits=k_bits, v_bits=v_bits)
    arrays.update({f"k_{n}": a for n, a in kq.items()})
    arrays.update({f"v_{n}": a for n, a in vq.items()})
    np.savez_compressed(path, **arrays)


def prefill_fixture(path, seed, Hq, Hkv, P, L):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((1, Hq, L, 128)).astype(np.float16)
    k = _kv(rng, (1, Hkv, P + L, 128))
    v = _kv(rng, (1, Hkv, P + L, 128))
    sinks = rng.standard_normal(Hq).astype(np.float32)
    kq, kh = _quant(k, 8)
    vq, vh = _quant(v, 8)
    out = O.attention(q, kh, vh, SCALE, sinks, "causal").astype(np.float32)
    # the prefill branch of Attention.__call__ hands the sinks over in the
    # query dtype (model.py:202)
    out_q = O.attention(q, kh, vh, SCALE, sinks, "causal", sink_dtype="float16").astype(np.float32)
    np.savez_compressed(path, q=q, k=k, v=v, sinks=sinks, out_sinks=out, out_sinks_qdtype=out_q, prefix=P,
                        **{f"k_{n}": a for n, a in kq.items()}, **{f"v_{n}": a for n, a in vq.items()})


def main():
    decode_fixture(os.path.join(HERE, "cfg1_int8.npz"), 20261201, 1, 8, 1, 1024, 8, 8)
    decode_fixture(os.path.join(HERE, "int4_heavy.npz"), 20261202, 1, 32, 4, 128, 4, 4, "heavy", 0.05)
    decode_fixture(os.path.join(HERE, "mixed_k8v4.npz"), 20261203, 1, 8, 2, 96, 8, 4, "outliers", 0.01)
    prefill_fixture(os.path.join(HERE, "prefill_causal.npz"), 20261204, 8, 1, 192, 64)


if __name__ == "__main__":
    if sys.argv[1:] == ["prefill"]:
        prefill_fixture(os.path.join(HERE, "prefill_causal.npz"), 20261204, 8, 1, 192, 64)
    else:
        main()

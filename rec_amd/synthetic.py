"""Seeded synthetic Q/K/V for the decode-attention workloads.

* ``normal``: N(0, 1).
* ``outliers``: N(0, 1) with a fraction of channels (the same channel indices
  for every token, chosen per head) scaled by 8.
* ``heavy``: N(0, 1) with a fraction of channels per head drawn from a
  Student-t distribution with 3 degrees of freedom.

Generated in float32 with a seeded ``torch.Generator`` on the target device,
then cast to the requested dtype.
"""

from __future__ import annotations

import torch


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def kv(shape, seed, *, kind="normal", frac=0.0, dtype=torch.float16, device="cuda"):
    """Tensor ``(B, H, T, D)`` of the given kind."""
    B, H, T, D = shape
    dev = torch.device(device)
    g = _gen(dev, seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
    if kind == "normal" or frac == 0.0:
        return x.to(dtype)
    n = max(1, int(round(frac * D)))
    gc = _gen("cpu", seed + 7919)
    for h in range(H):
        idx = torch.randperm(D, generator=gc)[:n].to(dev)
        if kind == "outliers":
            x[:, h, :, idx] *= 8.0
        elif kind == "heavy":
            z = torch.randn((B, T, n), generator=g, device=dev)
            chi2 = torch.randn((B, T, n, 3), generator=g, device=dev).square().sum(-1)
            x[:, h, :, idx] = z / torch.sqrt(chi2 / 3.0)
        else:
            raise ValueError(f"unknown kind {kind!r}")
    return x.to(dtype)


def query(B, Hq, L, seed, *, dtype=torch.float16, device="cuda", D=128):
    g = _gen(torch.device(device), seed)
    return torch.randn((B, Hq, L, D), generator=g, device=device, dtype=torch.float32).to(dtype)

"""Shared helpers for the GPU parity tests: seeded input generation (the draw order the
benchmark configs use) and oracle evaluation on the exact values the GPU consumed."""
from __future__ import annotations

import torch

from oracle.formula import rel_err, tda_chunked, tda_grads  # noqa: F401

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def make_inputs(shape, seed, count, dtype, device="cuda"):
    """`count` i.i.d. N(0,1) tensors drawn in argument order from one CPU generator seeded
    with `seed`, rounded to `dtype` and moved to `device`."""
    g = torch.Generator("cpu").manual_seed(seed)
    xs = [torch.randn(shape, generator=g, dtype=torch.float32) for _ in range(count)]
    return [x.to(dtype).to(device) for x in xs]


def host(x, dtype=torch.float64):
    return None if x is None else x.detach().to("cpu", dtype)


def oracle_out(q1, q2, k1, k2, v, beta, lam, p, normalize, branches, heads=None, dtype=torch.float64):
    """The CPU oracle on the values the GPU saw (bf16 inputs are upcast exactly)."""
    return tda_chunked(host(q1, dtype), host(q2, dtype), host(k1, dtype), host(k2, dtype), host(v, dtype),
                       float(beta), float(lam), p, normalize, branches=branches, heads=heads, dtype=dtype)


def heads_of(x, heads):
    return torch.stack([x[b, h] for (b, h) in heads])

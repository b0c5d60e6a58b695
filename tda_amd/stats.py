"""Sparsity statistics of threshold attention, from the kernels' own tile bookkeeping.

The reference describes the weights as ultra-sparse (README.md:10) but exposes nothing about
it; the forward kernels here already decide, for every 32x32 (query tile, key tile) block of
every branch, whether it holds a non-zero weight (the tile-occupancy bitmask that drives the
sparse A.V pass and the backward), and count what they visit.  `tile_sparsity` runs one
forward pass and returns that map and those counts next to the output.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .api import _offset, _power, _scalar

TILE = 32  # rows and columns of one occupancy tile


@dataclass
class TileStats:
    """occupancy: bool (branches, B, H, T, TK), T = ceil(Nq / 32), TK = ceil(Nk / 32): True
    where the 32x32 weight tile (query tile, key tile) of that branch holds a non-zero weight
    (always False past a query tile's last position).
    tiles_causal: (branch, head, query tile, key tile) blocks holding a causal pair.
    tiles_nonzero: those holding a non-zero weight (the A.V work actually done).
    tiles_screened: those the int8 screen passed on to the exact pass (a superset of the
    non-zero ones), for normalised bf16 and for normalised float32 with more than 32 query rows;
    None otherwise (no screen: the single pass tests every causal tile exactly)."""
    occupancy: torch.Tensor
    tiles_causal: int
    tiles_nonzero: int
    tiles_screened: int | None

    @property
    def skipped_fraction(self) -> float:
        """Fraction of causal tiles whose A.V work was skipped."""
        return 1.0 - self.tiles_nonzero / max(self.tiles_causal, 1)

    @property
    def density(self) -> torch.Tensor:
        """Per branch: non-zero tiles / causal tiles (float64, shape (branches,))."""
        causal = self.tiles_causal / self.occupancy.shape[0]
        return self.occupancy.flatten(1).sum(1, dtype=torch.float64) / max(causal, 1)


def _unpack(words: torch.Tensor, branches: int, b: int, h: int, t: int, tk: int | None = None) -> torch.Tensor:
    w = words.view(branches, b, h, t, -1).to(torch.int64) & 0xFFFFFFFF
    bits = (w.unsqueeze(-1) >> torch.arange(32, device=w.device)) & 1
    return bits.flatten(-2)[..., :(t if tk is None else tk)].bool()


def tile_sparsity(q, k, v, beta, relu_power=2.0, normalize=False, *, q2=None, k2=None, lambda_param=None,
                  q_offset=None):
    """One forward pass of TRA (q2 = k2 = None) or TDA (q2, k2, lambda_param given) with the
    tile statistics.  Arguments as threshold_rela_triton / differential_threshold_rela_triton
    (float32 or bfloat16 inputs).  Returns (out, TileStats); no gradient is recorded."""
    branches = 2 if q2 is not None else 1
    if branches == 2 and (k2 is None or lambda_param is None):
        raise ValueError("the differential form needs q2, k2 and lambda_param")
    tensors = (q, k, v) if branches == 1 else (q, q2, k, k2, v)
    ops._check_inputs(tensors, ("q", "k", "v") if branches == 1 else ("q", "q2", "k", "k2", "v"),
                      kv_from=1 if branches == 1 else 2)
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"tile_sparsity takes float32 or bfloat16 inputs, got {q.dtype}")
    if q.shape[-1] not in (64, 128, 256):
        raise ValueError(f"head_dim must be 64, 128 or 256, got {q.shape[-1]}")
    b, h, n, _ = q.shape
    nk = k.shape[2]
    if n == 0 or nk == 0:
        raise ValueError("tile_sparsity needs seq_len >= 1 and seq_len_kv >= 1")
    off = _offset(q_offset, n, nk)
    p = _power(relu_power)
    dev = q.device
    beta_t = _scalar(beta, dev, "beta").detach()
    lam_t = _scalar(lambda_param, dev, "lambda_param").detach() if branches == 2 else None
    norms, occ = ops.side_buffers(q.shape, branches, normalize, dev, nk)
    stats = torch.zeros(3, dtype=torch.int64, device=dev)
    with torch.no_grad():
        out = ops.forward(q, k, q2, k2, v, beta_t, lam_t, p, bool(normalize), branches,
                          norms=norms, occupancy=occ, stats=stats, q_offset=off)
    causal, nonzero, screened = (int(x) for x in stats.tolist())
    t, tk = (n + TILE - 1) // TILE, (nk + TILE - 1) // TILE
    occupancy = _unpack(occ, branches, b, h, t, tk)
    return out, TileStats(occupancy=occupancy, tiles_causal=causal, tiles_nonzero=nonzero,
                          tiles_screened=screened if q.shape[-1] <= 128 and normalize and
                          (q.dtype == torch.bfloat16 or n > TILE) else None)


__all__ = ["TileStats", "tile_sparsity", "TILE"]

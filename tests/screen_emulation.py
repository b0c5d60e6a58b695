"""Host emulation of the normalised bf16 screen's threshold test, and an adversarial input
built with it.

The screen (tda_amd/csrc/tda_fwd_sparse.hip, fwd_screen with normalisation) keeps key j for a
query tile when  fl(sh_ij * rk_j) > tlo  for some row i of the tile, where
  qh_i  = bf16(fl32(q_i * rq_i))           the pre-scaled query row, rounded once,
  sh_ij = qh_i . k_j                       (fp32 MFMA accumulation of exact bf16 products),
  rq_i, rk_j = 1 / max(|x|, 1e-12)         fp32 inverse row norms,
  tlo   = min_i tau_i - |min_i tau_i| 2^-19 - margin.
The reference keeps every weight with ReLU(cos(q_i, k_j) - tau_i) > 0 (TTA:86-101, with the
normalisation of TTA:505-509).  A margin is sound when no key with a positive weight fails the
test.  `margin_row_bound` is the kernel's per-tile bound (the largest |qh_i - fl(q_i rq_i)| of
the tile, times 1 + 2^-14, plus 2^-14); `MARGIN_FIXED_OLD` is the constant the kernel used
before, which assumed a bf16 unit roundoff of 2^-9 (it is 2^-8).

Used by tests/test_screen_margin.py (CPU) and tests/test_gpu_screen_margin.py (GPU input).
"""
from __future__ import annotations

import numpy as np
import torch

MARGIN_FIXED_OLD = 2.0 ** -9 + 2.0 ** -13


def bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest even), returned as float32."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def inv_norm(x: np.ndarray) -> np.float32:
    ss = np.float32(np.sum(x.astype(np.float32) ** 2, dtype=np.float32))
    return np.float32(1.0) / np.maximum(np.sqrt(ss, dtype=np.float32), np.float32(1e-12))


def prescale(q: np.ndarray):
    """(qh, rq, |r|): the screen's pre-scaled bf16 row, the inverse norm and the norm of the
    bf16 rounding residual r = qh - fl32(q rq)."""
    rq = inv_norm(q)
    a = (q.astype(np.float32) * rq).astype(np.float32)
    qh = bf16(a)
    r = float(np.sqrt(np.sum((qh.astype(np.float64) - a.astype(np.float64)) ** 2)))
    return qh, rq, r


def margin_row_bound(r_max: float) -> float:
    return r_max * (1.0 + 2.0 ** -14) + 2.0 ** -14


def screen_value(q: np.ndarray, k: np.ndarray) -> float:
    """fl(sh * rk) for one (query row, key row) pair (the sum in fp64, rounded to fp32: the
    fp32 MFMA accumulation differs by far less than the margins tested here)."""
    qh, _, _ = prescale(q)
    sh = np.float32(np.dot(qh.astype(np.float64), k.astype(np.float64)))
    return float(np.float32(sh * inv_norm(k)))


def exact_cos(q: np.ndarray, k: np.ndarray) -> float:
    q64, k64 = q.astype(np.float64), k.astype(np.float64)
    return float(q64 @ k64 / (np.linalg.norm(q64) * np.linalg.norm(k64)))


def tlo(tmin: float, margin: float) -> float:
    return tmin - abs(tmin) * 2.0 ** -19 - margin


def adversarial_row(d: int, seed: int, steps: int = 4000) -> np.ndarray:
    """A bf16 row whose pre-scaled copy carries a large rounding residual |r| / |qh| (random
    start, then greedy single-element moves over nearby bf16 values)."""
    rng = np.random.default_rng(seed)
    q = bf16(rng.standard_normal(d).astype(np.float32))
    best = prescale(q)[2]
    for it in range(steps):
        i = int(rng.integers(d))
        cand = q.copy()
        if it % 2:  # about one bf16 step up or down
            f = 1.0 + (2.0 ** -7 if rng.integers(2) else -2.0 ** -7)
        else:
            f = 1.0 + rng.uniform(-0.3, 0.3)
        cand[i:i + 1] = bf16(cand[i:i + 1] * np.float32(f))
        r = prescale(cand)[2]
        if r > best:
            q, best = cand, r
    return q


def adversarial_key(q: np.ndarray, tau: float, lo: float = 2e-5, hi: float = 1.5e-4, seed: int = 0):
    """A bf16 key row k with exact cosine(q, k) - tau in [lo, hi] (a non-zero weight, well clear
    of fp32 rounding) whose screen value fl(sh rk) is as low as the search finds: k leans against
    the part of q's rounding residual orthogonal to q.  Returns (k, cos, screen value)."""
    qh, rq, _ = prescale(q)
    u = q.astype(np.float64) / np.linalg.norm(q.astype(np.float64))
    r = qh.astype(np.float64) - (q.astype(np.float64) * float(rq))
    rp = r - (r @ u) * u
    rp /= np.linalg.norm(rp)
    rng = np.random.default_rng(seed)
    best = None
    for _ in range(6000):
        c = tau + rng.uniform(lo - 3e-4, hi + 3e-4)
        c = min(max(c, -0.999), 0.999)
        k = c * u - np.sqrt(1.0 - c * c) * rp
        k = bf16((k * rng.uniform(1.0, 8.0)).astype(np.float32))
        cs = exact_cos(q, k)
        if not (tau + lo <= cs <= tau + hi):
            continue
        sv = screen_value(q, k)
        if best is None or sv < best[2]:
            best = (k, cs, sv)
    if best is None:
        raise RuntimeError("no key found in the cosine window")
    return best

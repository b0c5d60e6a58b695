"""Host emulation of the normalised int8 screen's threshold test, and adversarial inputs built
with it.

The screen (tda_amd/csrc/tda_fwd_sparse.hip: key_prep and fwd_screen_i8) keeps key j for a
query tile when, for some row i of the tile,
    fl(fl(float(A_ij) * fl(sq * s_j))) > thr_j,
with
    kh_j = fl(k_j rk_j),  s_j = max|kh_j| / 127,  b_j = rint(kh_j * fl(127 / max|kh_j|))   (key_prep)
    qh_i = fl(q_i rq_i),  sq = m / 127 with m = max_i rq_i max|q_i| over the tile's rows,
    a_i = rint(qh_i * fl(127 / m)),
both rints of the exact product (one fma against 1.5 * 2^23),
    A_ij = a_i . b_j (exact int32)
(rint ties to even)
    ek_j, eq >= the norms of the residuals kh_j - s_j b_j and qh_i - sq a_i (eq: the tile's
    largest), times 1 + 2^-12,
    thr_j = tmin - |tmin| 2^-19 - 2^-14 - eq (1 + 2^-10) - ek_j (1 + 2^-10 + 4 eq),
and rq, rk = 1 / max(|x|, 1e-12) in fp32.  The reference keeps every weight with
cos(q_i, k_j) > tau_i (TTA:86-101 on the normalised rows of TTA:505-509); the bound is sound
when no such key fails the test.  `thr` takes the terms to include, so that a test can show
each term is needed: an adversarial key whose weight is non-zero fails the test without it.

Used by tests/test_screen_margin.py (CPU) and tests/test_gpu_edge.py (GPU input).
"""
from __future__ import annotations

import numpy as np
import torch

F32 = np.float32


def bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest even), returned as float32."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def inv_norm(x: np.ndarray) -> np.float32:
    ss = F32(np.sum(x.astype(np.float32) ** 2, dtype=np.float32))
    return F32(1.0) / np.maximum(np.sqrt(ss, dtype=np.float32), F32(1e-12))


def _fma32(a, b, c):
    """fp32 fma: a * b + c rounded once (the fp64 product of two fp32 values is exact)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def rint_prod(x: np.ndarray, inv) -> np.ndarray:
    """rint(x * inv) of the exact product of fp32 values (exact in fp64), ties to even: the
    kernels' fma(x, inv, 1.5 * 2^23)."""
    return np.rint(np.asarray(x, np.float64) * np.float64(inv))


def res_bound(r: np.ndarray) -> float:
    """The kernels' bound on a residual's norm: fp32 sum of squares (fma chain), square root,
    times 1 + 2^-12."""
    e2 = F32(0.0)
    for x in r.astype(np.float32):
        e2 = _fma32(x, x, e2)
    return float(F32(np.sqrt(e2, dtype=np.float32) * F32(1.0 + 2.0 ** -12)))


def quant_key(k: np.ndarray):
    """key_prep of one bf16 key row: (b int, s_j, ek_j, rk_j, kh)."""
    rk = inv_norm(k)
    kh = (k.astype(np.float32) * rk).astype(np.float32)
    m = F32(np.max(np.abs(kh)))
    s = F32(m * F32(1.0 / 127.0))
    inv = F32(127.0) / m if m > 0 else F32(0.0)
    b = rint_prod(kh, inv)
    assert np.all(np.abs(b) <= 127)
    r = _fma32(-s, b.astype(np.float32), kh)
    return b.astype(np.int64), float(s), res_bound(r), rk, kh


def quant_tile(qs: np.ndarray):
    """fwd_screen_i8's quantisation of a query tile (rows x d bf16 values): (a int, sq, eq, qh)."""
    rq = np.array([inv_norm(q) for q in qs], dtype=np.float32)
    mq = np.max(np.abs(qs.astype(np.float32)), axis=1).astype(np.float32)
    m = F32(np.max((mq * rq).astype(np.float32)))
    sq = F32(m * F32(1.0 / 127.0))
    inv = F32(127.0) / m if m > 0 else F32(0.0)
    qh = (qs.astype(np.float32) * rq[:, None]).astype(np.float32)
    a = rint_prod(qh, inv)
    assert np.all(np.abs(a) <= 127)
    r = _fma32(-sq, a.astype(np.float32), qh)
    eq = max(res_bound(x) for x in r)
    return a.astype(np.int64), float(sq), eq, qh


def screen_value(a_i: np.ndarray, sq: float, b_j: np.ndarray, s_j: float) -> float:
    """fl(fl(float(A_ij)) * fl(sq s_j)) for one (query row, key row) pair."""
    A = int(np.dot(a_i, b_j))
    return float(F32(F32(A) * F32(F32(sq) * F32(s_j))))


def thr(tmin: float, eq: float, ek: float, terms=("tau", "const", "eq", "ek", "cross")) -> float:
    """The screen's threshold for one key, with only the listed terms of the bound."""
    t = F32(tmin)
    if "tau" in terms:
        t = F32(t - F32(abs(t) * F32(2.0 ** -19)))
    if "const" in terms:
        t = F32(t - F32(2.0 ** -14))
    if "eq" in terms:
        t = F32(t - F32(F32(eq) * F32(1.0 + 2.0 ** -10)))
    c = F32(1.0 + 2.0 ** -10) if "ek" in terms else F32(0.0)
    if "cross" in terms:
        c = F32(c + F32(4.0) * F32(eq))
    return float(_fma32(-F32(ek), c, t))


def exact_cos(q: np.ndarray, k: np.ndarray) -> float:
    q64, k64 = q.astype(np.float64), k.astype(np.float64)
    return float(q64 @ k64 / (np.linalg.norm(q64) * np.linalg.norm(k64)))


def tile_with(q: np.ndarray, seed: int, rows: int = 32) -> np.ndarray:
    """A query tile whose row 0 is q and the rest N(0, 1) bf16 rows."""
    rng = np.random.default_rng(seed)
    t = bf16(rng.standard_normal((rows, q.shape[0])).astype(np.float32))
    t[0] = q
    return t


def adversarial_key(q: np.ndarray, tile: np.ndarray, tau: float, lo: float = 2e-5, hi: float = 1.5e-4,
                    seed: int = 0, tries: int = 6000, score=None, climb: int = 0):
    """A bf16 key row k with exact cos(q, k) - tau in [lo, hi] (a non-zero weight, well clear of
    fp32 rounding) that makes `score(k)` (default: the screen value minus its threshold with every
    term) as low as the search finds: k leans towards the part of q's quantisation residual
    orthogonal to q (the int8 score of q is its normalised row minus that residual), and the
    search over small perturbations, then `climb` greedy element moves, let k's own quantisation
    push further.  Returns (k, cos, screen value, s_j, ek_j) for row 0 of `tile`."""
    a, sq, eq, qh = quant_tile(tile)
    u = q.astype(np.float64) / np.linalg.norm(q.astype(np.float64))
    r = qh[0].astype(np.float64) - sq * a[0].astype(np.float64)  # the row's residual
    rp = r - (r @ u) * u
    rp /= max(np.linalg.norm(rp), 1e-30)
    rng = np.random.default_rng(seed)
    best = None
    for _ in range(tries):
        c = tau + rng.uniform(lo - 3e-4, hi + 3e-4)
        c = min(max(c, -0.999), 0.999)
        w = rng.standard_normal(q.shape[0])
        w -= (w @ u) * u + (w @ rp) * rp
        w /= np.linalg.norm(w)
        mix = rng.uniform(0.0, 0.3)
        side = np.sqrt(1.0 - c * c)
        k = c * u + side * (np.sqrt(1.0 - mix * mix) * rp + mix * w)
        k = bf16((k * rng.uniform(1.0, 8.0)).astype(np.float32))
        cs = exact_cos(q, k)
        if not (tau + lo <= cs <= tau + hi):
            continue
        b, s, ek, _, _ = quant_key(k)
        sv = screen_value(a[0], sq, b, s)
        val = score(sv, eq, ek) if score else sv - thr(tau, eq, ek)
        if best is None or val < best[0]:
            best = (val, k, cs, sv, s, ek)
    if best is None:
        raise RuntimeError("no key found in the cosine window")
    # then greedy single-element moves (about one bf16 step) that lower the score and keep the
    # cosine in its window: they steer k's own rounding residual
    val, k = best[0], best[1]
    for it in range(climb):
        cand = k.copy()
        i = int(rng.integers(q.shape[0]))
        cand[i:i + 1] = bf16(cand[i:i + 1] * np.float32(1.0 + (2.0 ** -7 if it % 2 else -2.0 ** -7)))
        cs = exact_cos(q, cand)
        if not (tau + lo <= cs <= tau + hi):
            continue
        b, s, ek, _, _ = quant_key(cand)
        sv = screen_value(a[0], sq, b, s)
        v2 = score(sv, eq, ek) if score else sv - thr(tau, eq, ek)
        if v2 < val:
            val, k, best = v2, cand, (v2, cand, cs, sv, s, ek)
    return best[1:]

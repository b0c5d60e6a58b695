"""Brute-force restatement of threshold attention with explicit Python loops.

TEST INFRASTRUCTURE ONLY (see oracle/formula.py).  Independent of torch
matmul/normalize: every sum is an explicit float64 loop, for tiny shapes only.
Used to pin oracle/formula.py.

Follows /root/reference/triton_threshold_attention.py:
  tau_i = beta * sqrt(2 ln(i+1) / d)                       TTA:59-63
  S_ij  = q_i . k_j, causal j <= i                         TTA:75-80
  P_ij  = (S_ij - tau_i)^p if S_ij - tau_i > 0 else 0      TTA:86-101
  out_i = sum_j P_ij v_j                                   TTA:103-109
  TDA   = out(n(q1), n(k1)) - clamp(lam, 0, 1) out(n(q2), n(k2))  TTA:505-517
"""
from __future__ import annotations

import math


def _norm(row):
    s = 0.0
    for x in row:
        s += x * x
    n = max(math.sqrt(s), 1e-12)
    return [x / n for x in row]


def tra_rows(q, k, v, beta, p, normalize=False, q_offset=0):
    """q: list of Nq rows, k, v: lists of Nk rows (lists of d floats); query row i sits at
    position q_offset + i (0 and Nq = Nk in the reference).  Returns Nq rows."""
    n, d = len(q), len(q[0])
    if normalize:
        q = [_norm(r) for r in q]
        k = [_norm(r) for r in k]
    out = []
    for i in range(n):
        pos = q_offset + i
        t = beta * math.sqrt(2.0 * math.log(pos + 1.0) / d)
        acc = [0.0] * d
        for j in range(min(len(k), pos + 1)):
            s = 0.0
            for c in range(d):
                s += q[i][c] * k[j][c]
            x = s - t
            if x > 0.0:
                w = x ** p
                for c in range(d):
                    acc[c] += w * v[j][c]
        out.append(acc)
    return out


def tda_rows(q1, q2, k1, k2, v, beta, lam, p, normalize=True, q_offset=0):
    o1 = tra_rows(q1, k1, v, beta, p, normalize, q_offset)
    o2 = tra_rows(q2, k2, v, beta, p, normalize, q_offset)
    lc = min(max(lam, 0.0), 1.0)
    return [[a - lc * b for a, b in zip(r1, r2)] for r1, r2 in zip(o1, o2)]

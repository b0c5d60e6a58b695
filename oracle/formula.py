"""CPU oracle: a PyTorch restatement of the reference's threshold-attention formula.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (`tda_amd`) imports,
calls or links this module.  Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker (or as the
timed CPU baseline), never as the thing measured on the GPU.

What it restates (reference = /root/reference/triton_threshold_attention.py,
cited as TTA:<line>):

* tau(i) = beta * sqrt(2 * ln(i + 1) / d), 0-based absolute query index i
  (TTA:59-63, :164-166, :276-278).
* scores S = Q K^T, no 1/sqrt(d) scaling and no softmax (TTA:75, :186, :282).
* causal: key j contributes to query i only when j <= i (TTA:77-80).  The
  reference zeroes masked scores *before* thresholding (TTA:80); for beta >= 0
  that is identical to excluding them because ReLU(0 - tau_i) = 0.  The default
  here is true exclusion; ``mask="zero"`` restates the reference literally.
* strict ReLU of S - tau, then the power p (TTA:86-101): p = 2 -> x^2,
  p = 1 -> x, otherwise x^p for x > 0.  The reference's general-p path adds a
  1e-10 bias inside the log (TTA:99); the oracle uses the exact power.
* out = P @ V with float accumulation (TTA:103-109).
* differential form: optional F.normalize(p=2, dim=-1, eps=1e-12) of q1, k1,
  q2, k2 (TTA:505-509), two branches sharing v (TTA:512-513), then
  out1 - clamp(lambda, 0, 1) * out2 (TTA:516-517).

Position offset (a superset of the reference, whose query index is always the
absolute position, TTA:62): queries may be a block of q_offset.. q_offset+Nq-1
against Nk keys (KV-cache decode, chunked prefill); query row i then uses
tau(q_offset + i) and sees keys j <= q_offset + i.  q_offset = 0 with Nq = Nk
is the reference's case.

Gradients for q, k, v, beta and lambda come from torch autograd of these
expressions (the reference returns None for beta, TTA:469; the build adds it).

Pinned by tests/test_oracle.py: a brute-force loop restatement
(oracle/brute.py), closed forms (N = 1, huge beta, beta = 0 linear case,
lambda identities), invariants (causality, prefix invariance, linearity in v,
(b, h) equivariance) and fp64 gradcheck.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

NORM_EPS = 1e-12  # torch.nn.functional.normalize default eps (TTA:506-509)


def tau(n: int, d: int, beta, dtype=torch.float64, device="cpu", offset: int = 0) -> torch.Tensor:
    """Per-row threshold tau_i = beta * sqrt(2 ln(i+1) / d) for the absolute positions
    i = offset .. offset+n-1 (TTA:59-63).

    ``beta`` may be a float or a 0-dim tensor (kept differentiable)."""
    i = torch.arange(offset, offset + n, dtype=dtype, device=device)
    c = torch.sqrt(2.0 * torch.log(i + 1.0) / d)
    return beta * c


def tau_coeff(n: int, d: int, dtype=torch.float64) -> torch.Tensor:
    """c_i = sqrt(2 ln(i+1) / d), so that tau_i = beta * c_i."""
    i = torch.arange(n, dtype=dtype)
    return torch.sqrt(2.0 * torch.log(i + 1.0) / d)


def relu_pow(x: torch.Tensor, p: float) -> torch.Tensor:
    """ReLU(x)^p with a strict x > 0 test (TTA:86-101), written so that autograd
    gives p * x^(p-1) on x > 0 and exactly 0 elsewhere (no 0^(p-1) NaNs)."""
    pos = x > 0
    xs = torch.where(pos, x, torch.ones_like(x))
    if p == 2.0:
        y = xs * xs
    elif p == 1.0:
        y = xs
    else:
        y = torch.pow(xs, p)
    return torch.where(pos, y, torch.zeros_like(x))


def _normalize(x: torch.Tensor) -> torch.Tensor:
    return F.normalize(x, p=2.0, dim=-1, eps=NORM_EPS)


def causal_mask(nq: int, nk: int, q_offset: int = 0, device="cpu") -> torch.Tensor:
    """(nq, nk) bool: key j is visible to query row i when j <= q_offset + i (TTA:77-80)."""
    i = torch.arange(nq, device=device).unsqueeze(1) + q_offset
    return torch.arange(nk, device=device).unsqueeze(0) <= i


def tra(q, k, v, beta, relu_power: float = 2.0, normalize: bool = False,
        mask: str = "exclude", q_offset: int = 0) -> torch.Tensor:
    """Threshold rectified attention, out = ReLU(mask(Q K^T) - tau)^p V.

    Follows TTA:19-115 (forward kernel) and TTA:472-486 (public wrapper); the
    ``normalize`` flag applies TTA:505-509 to q and k.  Computes in the dtype
    of the inputs (callers upcast bf16 inputs to float32/float64 first).
    Shapes q (B, H, Nq, d), k and v (B, H, Nk, d) (Nq = Nk and q_offset = 0 in the
    reference).  ``mask`` is "exclude" (j > i contributes nothing) or "zero" (the
    reference's literal rule: S_ij := 0 for j > i, TTA:80)."""
    if normalize:
        q = _normalize(q)
        k = _normalize(k)
    n, d = q.shape[-2], q.shape[-1]
    s = torch.matmul(q, k.transpose(-1, -2))
    causal = causal_mask(n, k.shape[-2], q_offset, device=q.device)
    t = tau(n, d, beta, dtype=q.dtype, device=q.device, offset=q_offset).unsqueeze(-1)
    if mask == "zero":
        s = torch.where(causal, s, torch.zeros_like(s))
        p = relu_pow(s - t, relu_power)
    elif mask == "exclude":
        p = relu_pow(s - t, relu_power)
        p = torch.where(causal, p, torch.zeros_like(p))
    else:
        raise ValueError(mask)
    return torch.matmul(p, v)


def tda(q1, q2, k1, k2, v, beta, lambda_param, relu_power: float = 2.0,
        normalize: bool = True, mask: str = "exclude", q_offset: int = 0) -> torch.Tensor:
    """Threshold differential attention (TTA:489-519):
    TRA(n(q1), n(k1), v) - clamp(lambda, 0, 1) * TRA(n(q2), n(k2), v)."""
    out1 = tra(q1, k1, v, beta, relu_power, normalize, mask, q_offset)
    out2 = tra(q2, k2, v, beta, relu_power, normalize, mask, q_offset)
    if not isinstance(lambda_param, torch.Tensor):
        lambda_param = torch.tensor(float(lambda_param), dtype=out1.dtype)
    lam = torch.clamp(lambda_param, min=0.0, max=1.0)
    return out1 - lam * out2


# ----------------------------------------------------------------------------
# Chunked, no-grad evaluation for large shapes (bench CPU baseline, full-size
# head samples in the GPU parity tests).  Same formula, evaluated one (b, h)
# head and one block of query rows at a time so the N x N temporaries stay
# bounded.
# ----------------------------------------------------------------------------

@torch.no_grad()
def tra_head_rows(q, k, v, beta: float, relu_power: float, r0: int, r1: int,
                  q_offset: int = 0) -> torch.Tensor:
    """Query rows r0..r1-1 of TRA for one head; q is (Nq, d), k and v (Nk, d), already
    normalised if required.  Keys after position q_offset + r1 - 1 are causally excluded."""
    d = q.shape[-1]
    kn = min(k.shape[0], q_offset + r1)
    kk = k[:kn]
    s = q[r0:r1] @ kk.T                                     # (r1-r0, kn)
    i = torch.arange(q_offset + r0, q_offset + r1, dtype=q.dtype)
    t = (beta * torch.sqrt(2.0 * torch.log(i + 1.0) / d)).unsqueeze(-1)
    x = s - t
    j = torch.arange(kn)
    causal = j.unsqueeze(0) <= torch.arange(q_offset + r0, q_offset + r1).unsqueeze(1)
    x = torch.where(causal, x, torch.full_like(x, -1.0))
    pos = x > 0
    npos = int(pos.sum())
    if npos * 20 < pos.numel():
        # Few non-zero weights (the usual case: TDA is ultra-sparse): the same sum
        # out_i = sum_j ReLU(x_ij)^p v_j over the non-zero terms only, which skips the dense
        # power and the dense product (tests/test_oracle.py pins it against the dense form).
        out = torch.zeros(r1 - r0, v.shape[-1], dtype=v.dtype)
        if npos:
            ii, jj = pos.nonzero(as_tuple=True)
            w = relu_pow(x[ii, jj], relu_power)
            out.index_add_(0, ii, w.unsqueeze(-1) * v[jj])
        return out
    p = relu_pow(x, relu_power)
    return p @ v[:kn]


@torch.no_grad()
def tda_chunked(q1, q2, k1, k2, v, beta: float, lambda_param: float, relu_power: float,
                normalize: bool, branches: int = 2, block: int = 1024,
                heads=None, dtype=torch.float32, q_offset: int = 0) -> torch.Tensor:
    """No-grad evaluation of TRA (branches=1: q1, k1, v) or TDA (branches=2) on
    CPU, head by head and ``block`` query rows at a time.  Returns (B, H, N, d)
    in ``dtype`` (only the selected ``heads`` [(b, h), ...] are filled when
    given; the others stay zero)."""
    b_, h_, n, d = q1.shape
    out = torch.zeros(b_, h_, n, d, dtype=dtype)
    lam = min(max(float(lambda_param), 0.0), 1.0)
    sel = heads if heads is not None else [(b, h) for b in range(b_) for h in range(h_)]
    for (b, h) in sel:
        def prep(x):
            x = x[b, h].to(dtype)
            return _normalize(x) if normalize else x
        qa, ka = prep(q1), prep(k1)
        vv = v[b, h].to(dtype)
        if branches == 2:
            qb, kb = prep(q2), prep(k2)
        for r0 in range(0, n, block):
            r1 = min(n, r0 + block)
            o = tra_head_rows(qa, ka, vv, beta, relu_power, r0, r1, q_offset)
            if branches == 2:
                o = o - lam * tra_head_rows(qb, kb, vv, beta, relu_power, r0, r1, q_offset)
            out[b, h, r0:r1] = o
    return out


def tda_grads(q1, q2, k1, k2, v, dout, beta: float, lambda_param: float,
              relu_power: float, normalize: bool, branches: int = 2,
              dtype=torch.float64, q_offset: int = 0):
    """Autograd gradients of sum(out * dout) for TRA (branches=1) or TDA.

    Returns a dict with out, dq1, dk1, dv, dbeta and (branches=2) dq2, dk2,
    dlambda, all in ``dtype`` on CPU."""
    def leaf(x):
        return x.detach().to("cpu", dtype).clone().requires_grad_(True)
    tq1, tk1, tv = leaf(q1), leaf(k1), leaf(v)
    tb = torch.tensor(float(beta), dtype=dtype, requires_grad=True)
    go = dout.detach().to("cpu", dtype)
    res = {}
    if branches == 2:
        tq2, tk2 = leaf(q2), leaf(k2)
        tl = torch.tensor(float(lambda_param), dtype=dtype, requires_grad=True)
        out = tda(tq1, tq2, tk1, tk2, tv, tb, tl, relu_power, normalize, q_offset=q_offset)
        out.backward(go)
        res.update(dq2=tq2.grad, dk2=tk2.grad, dlambda=tl.grad)
    else:
        out = tra(tq1, tk1, tv, tb, relu_power, normalize, q_offset=q_offset)
        out.backward(go)
    res.update(out=out.detach(), dq1=tq1.grad, dk1=tk1.grad, dv=tv.grad, dbeta=tb.grad)
    return res


def causal_dense_flops(batch: int, heads: int, n: int, d: int, units: float) -> float:
    """FlashAttention-convention causal FLOPs: one 'unit' is one N x N x d
    contraction over the causal half, 2 * (N^2 / 2) * d per head."""
    return units * batch * heads * float(n) * n * d


def rel_err(y: torch.Tensor, y_ref: torch.Tensor) -> float:
    """Normwise max relative error max|y - y_ref| / max|y_ref| (outputs are
    ultra-sparse, so element-wise relative error is ill-defined)."""
    y = y.detach().to("cpu", torch.float64)
    y_ref = y_ref.detach().to("cpu", torch.float64)
    den = y_ref.abs().max().item() if y_ref.numel() else 0.0
    num = (y - y_ref).abs().max().item() if y_ref.numel() else 0.0
    if den == 0.0:
        return 0.0 if num == 0.0 else math.inf
    return num / den

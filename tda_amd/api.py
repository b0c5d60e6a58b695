"""Public entry points, drop-in for snap-research/TDA's triton_threshold_attention module.

Same names, argument order, defaults and meaning as the reference
(triton_threshold_attention.py, TTA:472-519, README.md:54-60):

  threshold_rela_triton(q, k, v, beta, relu_power=2.0, normalize=False)
  differential_threshold_rela_triton(q1, q2, k1, k2, v, beta, lambda_param,
                                     relu_power=2.0, normalize=True)

Superset behaviour (all results identical where the reference is defined):
  * `normalize` also exists on the single-branch function (default False, which is what the
    reference computes: it never normalises there, TTA:472-486);
  * beta and lambda_param may be Python floats or tensors; when they require grad they
    receive a gradient (the reference returns None for beta, TTA:469);
  * all four (B, H, N, d) strides are honoured (the reference ignores the batch stride,
    TTA:49);
  * errors raise ValueError with a message instead of an assert (TTA:348);
  * keys and values may be longer or shorter than the queries (Nk != Nq), and the keyword
    q_offset places query row i at absolute position q_offset + i: tau uses that position
    and the row sees keys j <= q_offset + i (KV-cache decode, chunked prefill).  The default
    q_offset is max(Nk - Nq, 0): the queries are the last Nq positions of the keys, and 0
    when Nq = Nk, which is the reference's case.
Only the causal form exists, as in the reference.  Supported head_dim: 16, 32, 64, 128, 256
(the reference takes any power of two >= 16, TTA:348, :366-368).  The kernels run d = 64, 128
and 256 (256: column-split kernels, each wave owning half of the output columns);
d = 16 and 32 are computed at d = 64 with the rows zero-padded (dot products and norms
unchanged) and beta scaled by sqrt(64 / d), so that tau = beta sqrt(2 ln(P+1) / d) is the same
threshold; the padding's gradients are dropped and beta's gradient flows through the scaling.
Other head_dims raise ValueError.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import ops

_KERNEL_DIMS = (64, 128, 256)
_PADDED_DIMS = (16, 32)  # computed at d = 64


def _head_dim(d: int) -> int:
    """The kernel head_dim for a caller head_dim d (ValueError when unsupported)."""
    if d in _KERNEL_DIMS:
        return d
    if d in _PADDED_DIMS:
        return 64
    raise ValueError(f"head_dim must be 16, 32, 64, 128 or 256, got {d}")


def _pad(t: torch.Tensor, dk: int) -> torch.Tensor:
    return t if t.shape[-1] == dk else F.pad(t, (0, dk - t.shape[-1]))

_COMPUTE = {torch.float32: torch.float32, torch.bfloat16: torch.bfloat16,
            torch.float16: torch.float32, torch.float64: torch.float32}


def _scalar(x, device, name):
    """0-dim float32 device tensor for beta / lambda, differentiable when x is a tensor."""
    if isinstance(x, torch.Tensor):
        if x.numel() != 1:
            raise ValueError(f"{name} must be a scalar, got shape {tuple(x.shape)}")
        x = x.to(device=device, dtype=torch.float32)
        return x if x.dim() == 0 else x.reshape(())
    return torch.full((), float(x), dtype=torch.float32, device=device)


def _power(relu_power) -> float:
    p = float(relu_power.item() if isinstance(relu_power, torch.Tensor) else relu_power)
    if not (p >= 0.0 and p < float("inf")):
        raise ValueError(f"relu_power must be finite and >= 0, got {p}")
    return p


def _offset(q_offset, nq: int, nk: int) -> int:
    if q_offset is None:
        return max(nk - nq, 0)
    off = int(q_offset)
    if off < 0:
        raise ValueError(f"q_offset must be >= 0, got {off}")
    return off


def _run(tensors, names, beta, lam, relu_power, normalize, branches, q_offset=None):
    kv_from = 1 if branches == 1 else 2
    ops._check_inputs(tensors, names, kv_from=kv_from)
    ref = tensors[0]
    off = _offset(q_offset, ref.shape[2], tensors[kv_from].shape[2])
    d = ref.shape[-1]
    dk = _head_dim(d)
    p = _power(relu_power)
    dev = ref.device
    cdt = _COMPUTE.get(ref.dtype)
    if cdt is None:
        raise ValueError(f"unsupported dtype {ref.dtype}")
    beta_t = _scalar(beta, dev, "beta")
    lam_t = _scalar(lam, dev, "lambda_param") if branches == 2 else None
    if any(t.numel() == 0 for t in tensors):  # no query rows, or no keys: the output is 0
        zero = sum(t.sum() for t in tensors) * 0.0 + beta_t * 0.0
        if lam_t is not None:
            zero = zero + lam_t * 0.0
        return torch.zeros_like(ref) + zero
    xs = [_pad(t if t.dtype == cdt else t.to(cdt), dk) for t in tensors]
    if dk != d:  # same tau at the padded width
        beta_t = beta_t * math.sqrt(dk / d)
    if branches == 2:
        q1, q2, k1, k2, v = xs
    else:
        (q1, k1, v), q2, k2 = xs, None, None
    out = ops.TDAFunction.apply(q1, k1, q2, k2, v, beta_t, lam_t, p, bool(normalize), branches, off)
    if dk != d:
        out = out[..., :d]
    return out if out.dtype == ref.dtype else out.to(ref.dtype)


def threshold_rela_triton(q, k, v, beta, relu_power=2.0, normalize=False, *, q_offset=None):
    """Threshold Rectified Attention: out = ReLU(Q K^T - tau)^p V, causal,
    tau_i = beta * sqrt(2 ln(i+1) / d)  (TTA:472-486).

    q: (batch, heads, seq_len, head_dim), k, v: (batch, heads, seq_len_kv, head_dim) on the
    GPU, float32 or bfloat16 (float16 and float64 are computed in float32).  beta: float or
    scalar tensor.  relu_power: float (p == 1 and p == 2 take integer fast paths).
    normalize: cosine scores.  q_offset: position of query row 0 (default
    max(seq_len_kv - seq_len, 0))."""
    return _run((q, k, v), ("q", "k", "v"), beta, None, relu_power, normalize, 1, q_offset)


def differential_threshold_rela_triton(q1, q2, k1, k2, v, beta, lambda_param, relu_power=2.0,
                                       normalize=True, *, q_offset=None):
    """Threshold Differential Attention (TTA:489-519):
    TRA(n(q1), n(k1), v) - clamp(lambda_param, 0, 1) * TRA(n(q2), n(k2), v),
    computed by one fused kernel; n() is the L2 row normalisation when normalize=True.
    q1, q2: (batch, heads, seq_len, head_dim); k1, k2, v: (..., seq_len_kv, head_dim);
    q_offset as for threshold_rela_triton."""
    return _run((q1, q2, k1, k2, v), ("q1", "q2", "k1", "k2", "v"), beta, lambda_param,
                relu_power, normalize, 2, q_offset)


class ThresholdRelaFunction(torch.autograd.Function):
    """The reference's autograd Function (TTA:327-469) with its interface:
    forward(ctx, q, k, v, beta, relu_power) -> out and backward(ctx, dout) -> (dq, dk, dv,
    None, None), single branch, no normalisation, causal.  Like the reference it gives beta and
    relu_power no gradient (TTA:469); threshold_rela_triton above gives beta one.  Runs the same
    kernels as TDAFunction (ops.py) through the C ABI."""

    @staticmethod
    def forward(ctx, q, k, v, beta, relu_power):
        ops._check_inputs((q, k, v), ("q", "k", "v"), kv_from=1)
        d = q.shape[-1]
        dk = _head_dim(d)
        p = _power(relu_power)
        cdt = _COMPUTE.get(q.dtype)
        if cdt is None:
            raise ValueError(f"unsupported dtype {q.dtype}")
        off = _offset(None, q.shape[2], k.shape[2])
        beta_t = _scalar(beta, q.device, "beta").detach()
        if dk != d:  # same tau at the padded width
            beta_t = beta_t * math.sqrt(dk / d)
        qc, kc, vc = (_pad(t if t.dtype == cdt else t.to(cdt), dk) for t in (q, k, v))
        ctx.dtype = q.dtype
        ctx.d = d
        ctx.cfg = (p, off)
        if any(t.numel() == 0 for t in (q, k, v)):  # no query rows or no keys: the output is 0
            ctx.empty = True
            return torch.zeros_like(q)
        ctx.empty = False
        need = any(ctx.needs_input_grad[:3])
        occ = pairs = gbuf = None
        grads = [None] * 5
        if need:
            _, occ = ops.side_buffers(qc.shape, 1, False, qc.device, kc.shape[2])
            if cdt == torch.bfloat16:
                pairs = ops.pair_buffer(qc.shape, 1, qc.device)
                if all(ctx.needs_input_grad[:3]) and ops.grad_prealloc_enabled():
                    gbuf, grads = ops.grad_buffers(qc, kc, None, None, vc, 1)
        out = ops.forward(qc, kc, None, None, vc, beta_t, None, p, False, 1, None, occ, q_offset=off,
                          pairs=pairs, zero=gbuf)
        ctx.save_for_backward(qc, kc, vc, beta_t, occ, pairs, *grads)
        ctx.zeroed = gbuf is not None
        out = out[..., :d] if dk != d else out
        return out if out.dtype == q.dtype else out.to(q.dtype)

    @staticmethod
    def backward(ctx, dout):
        if ctx.empty:
            return None, None, None, None, None
        qc, kc, vc, beta_t, occ, pairs, *grads = ctx.saved_tensors
        p, off = ctx.cfg
        d = ctx.d
        dout = _pad(dout.to(qc.dtype), qc.shape[-1])
        zeroed, ctx.zeroed = ctx.zeroed, False  # the cleared buffers serve the first backward only
        dq, dk, _, _, dv, _, _ = ops.backward(qc, kc, None, None, vc, dout, beta_t, None, p, False, 1,
                                              None, occ, q_offset=off, pairs=pairs,
                                              grads=grads if zeroed else None)
        dq, dk, dv = (g[..., :d] if g.shape[-1] != d else g for g in (dq, dk, dv))
        dq, dk, dv = (g if g.dtype == ctx.dtype else g.to(ctx.dtype) for g in (dq, dk, dv))
        ng = ctx.needs_input_grad
        return dq if ng[0] else None, dk if ng[1] else None, dv if ng[2] else None, None, None

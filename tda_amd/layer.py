"""Multi-head threshold differential attention as an nn.Module.

The reference ships only the functional operator (snap-research/TDA
triton_threshold_attention.py, TTA:472-519); the layer of the paper it accompanies (README.md:10)
wraps it between projections and learns beta and lambda.  This module is that wrapper:

    x (B, N, E) --fused projection--> q1, q2, k1, k2, v (B, N, H, d each)
      --> differential_threshold_rela_triton(q1, q2, k1, k2, v, beta, lambda, p, normalize)
      --> (B, N, H*d) --output projection--> (B, N, E)

The five projected tensors are strided (B, H, N, d) views of one (B, N, 5, H, d) projection
output, and the attention output is written in (B, N, H, d) order: no transposing copies on
either side (the kernels honour all four strides).  beta and lambda are learnable scalars by
default; lambda is clamped to [0, 1] inside the operator, with the inclusive gate of
torch.clamp on its gradient (TTA:516).
"""
from __future__ import annotations

import torch
from torch import nn

from .api import differential_threshold_rela_triton, threshold_rela_triton


class ThresholdDifferentialAttention(nn.Module):
    """Causal multi-head threshold differential attention (two-branch, TDA) or, with
    differential=False, threshold rectified attention (one branch, TRA).

    Args:
        embed_dim: model width E of the input and output.
        num_heads: H.
        head_dim: d, 16, 32, 64, 128 or 256 (default E // H).
        relu_power: p of ReLU(.)^p.
        normalize: cosine scores (L2-normalised q and k rows).
        beta_init, lambda_init: initial threshold scale and branch weight.
        learn_beta, learn_lambda: register them as parameters (else as buffers).
        differential: two branches (TDA) or one (TRA).
        bias: biases on the projections.
    """

    def __init__(self, embed_dim: int, num_heads: int, head_dim: int | None = None, *,
                 relu_power: float = 2.0, normalize: bool = True, beta_init: float = 1.0,
                 lambda_init: float = 0.5, learn_beta: bool = True, learn_lambda: bool = True,
                 differential: bool = True, bias: bool = False, device=None, dtype=None):
        super().__init__()
        head_dim = head_dim if head_dim is not None else embed_dim // num_heads
        if head_dim not in (16, 32, 64, 128, 256):
            raise ValueError(f"head_dim must be 16, 32, 64, 128 or 256, got {head_dim}")
        self.embed_dim, self.num_heads, self.head_dim = embed_dim, num_heads, head_dim
        self.relu_power, self.normalize, self.differential = float(relu_power), bool(normalize), differential
        self.n_proj = 5 if differential else 3  # q1, q2, k1, k2, v  |  q, k, v
        fk = {"device": device, "dtype": dtype}
        self.in_proj = nn.Linear(embed_dim, self.n_proj * num_heads * head_dim, bias=bias, **fk)
        self.out_proj = nn.Linear(num_heads * head_dim, embed_dim, bias=bias, **fk)
        beta = torch.tensor(float(beta_init), dtype=torch.float32, device=device)
        lam = torch.tensor(float(lambda_init), dtype=torch.float32, device=device)
        if learn_beta:
            self.beta = nn.Parameter(beta)
        else:
            self.register_buffer("beta", beta)
        if differential:
            if learn_lambda:
                self.lambda_param = nn.Parameter(lam)
            else:
                self.register_buffer("lambda_param", lam)
        else:
            self.lambda_param = None

    def project(self, x: torch.Tensor):
        """The (B, H, N, d) views of the projected q1, q2, k1, k2, v (q, k, v for TRA)."""
        b, n, _ = x.shape
        y = self.in_proj(x).view(b, n, self.n_proj, self.num_heads, self.head_dim)
        return [y[:, :, i].transpose(1, 2) for i in range(self.n_proj)]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: (batch, seq_len, embed_dim), causal over seq_len."""
        if x.dim() != 3 or x.shape[-1] != self.embed_dim:
            raise ValueError(f"x must have shape (batch, seq_len, {self.embed_dim}), got {tuple(x.shape)}")
        b, n, _ = x.shape
        parts = self.project(x)
        if self.differential:
            q1, q2, k1, k2, v = parts
            o = differential_threshold_rela_triton(q1, q2, k1, k2, v, self.beta, self.lambda_param,
                                                   self.relu_power, self.normalize)
        else:
            q, k, v = parts
            o = threshold_rela_triton(q, k, v, self.beta, self.relu_power, self.normalize)
        # o is (B, H, N, d) in (B, N, H, d) memory order when the inputs are such views
        return self.out_proj(o.transpose(1, 2).reshape(b, n, self.num_heads * self.head_dim))

    def extra_repr(self) -> str:
        return (f"embed_dim={self.embed_dim}, num_heads={self.num_heads}, head_dim={self.head_dim}, "
                f"relu_power={self.relu_power}, normalize={self.normalize}, differential={self.differential}")

"""CPU oracle for the threshold-attention hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the tda_amd package.
"""
from .formula import (  # noqa: F401
    NORM_EPS, causal_dense_flops, rel_err, relu_pow, tau, tau_coeff, tda, tda_chunked,
    tda_grads, tra, tra_head_rows,
)

"""tda_amd -- MI355X-native fused threshold attention (TRA / differential TDA).

Drop-in for snap-research/TDA's triton_threshold_attention module on one GPU; the compute
runs in hand-written gfx950 HIP kernels in libtda_hip.so (build: python -m tda_amd.build).
"""
from .api import (  # noqa: F401
    ThresholdRelaFunction,
    differential_threshold_rela_triton,
    threshold_rela_triton,
)
from .layer import ThresholdDifferentialAttention  # noqa: F401
from .ops import grad_prealloc, grad_prealloc_enabled, set_grad_prealloc  # noqa: F401
from .stats import TileStats, tile_sparsity  # noqa: F401

__all__ = ["threshold_rela_triton", "differential_threshold_rela_triton", "ThresholdRelaFunction",
           "ThresholdDifferentialAttention", "tile_sparsity", "TileStats", "set_grad_prealloc",
           "grad_prealloc", "grad_prealloc_enabled"]

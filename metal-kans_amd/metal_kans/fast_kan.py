"""FastKAN: Gaussian-RBF KAN layer on the fused gfx950 kernel.

Drop-in for the reference ``metal_kans/fast_kan.py`` forward surface:
constructor (fast_kan.py:25-54: ``grid = linspace(lo, hi, K)``,
``inv_denominator = 1 / (2 h^2)``, then the Kaiming-uniform draws in the
reference order), ``half``/``float`` (:60-78; ``half`` also casts the grid),
``forward`` (:99-147).  phi_k(x) = exp(-(x - grid[k])^2 * inv_denominator)
for arbitrary centres in ``grid``.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

from ._layer import KANLayerBase


class FastKAN(KANLayerBase):
    """Fused Gaussian-RBF KAN layer.

    Parameters:
        in_features: Number of input features.
        out_features: Number of output features.
        num_centers: Number of Gaussian RBF centres (default 8).
        grid_range: (min, max) range of the centres (default (-1, 1)).
        bias: Whether to add a trainable additive bias (default True).
        use_base: Whether to include the residual SiLU base branch (default True).
    """
    _basis = "rbf"
    _weight_attr = "w_rbf"

    def __init__(self, in_features: int, out_features: int, num_centers: int = 8,
                 grid_range: Tuple[float, float] = (-1.0, 1.0), bias: bool = True, use_base: bool = True):
        self.in_features = in_features
        self.out_features = out_features
        self.num_centers = num_centers
        self.has_base = 1 if use_base else 0
        self.has_bias = 1 if bias else 0
        self.grid = np.linspace(grid_range[0], grid_range[1], num_centers, dtype=np.float32)
        h = (grid_range[1] - grid_range[0]) / (num_centers - 1)
        self.inv_denominator = float(1.0 / (2.0 * (h ** 2)))
        bound = 1.0 / math.sqrt(in_features)
        self.w_rbf = np.random.uniform(-bound, bound, (out_features, in_features * num_centers)).astype(np.float32)
        self.w_base = (np.random.uniform(-bound, bound, (out_features, in_features)).astype(np.float32)
                       if use_base else np.zeros((1,), dtype=np.float32))
        self.bias = (np.zeros((out_features,), dtype=np.float32) if bias else np.zeros((1,), dtype=np.float32))
        self._saved_x: Optional[np.ndarray] = None
        self._compute = "float32"

    def _num_basis(self) -> int:
        return self.num_centers

    def _basis_params(self) -> tuple:
        g = np.asarray(self.grid).astype(np.float32)
        return (tuple(float(v) for v in g.ravel()), float(self.inv_denominator))

    def half(self) -> "FastKAN":
        """Converts layer parameters (and the grid) to FP16 half precision."""
        self._cast_params(np.float16)
        self.grid = self.grid.astype(np.float16)
        self._compute = "float16"
        return self

    def _benchmark_args(self) -> tuple:
        return "benchmark_metal_fastkan", self.w_rbf, (self.grid,), (int(self.num_centers), float(self.inv_denominator))

    def float(self) -> "FastKAN":
        """Converts layer parameters (and the grid) to FP32 single precision."""
        self._cast_params(np.float32)
        self.grid = self.grid.astype(np.float32)
        self._compute = "float32"
        self.__dict__.pop("_quantized_from", None)
        return self

"""BSplineKAN (KAN): clamped uniform cubic B-spline KAN layer on the fused kernel.

Drop-in for the reference ``metal_kans/bspline_kan.py`` forward surface:
constructor (bspline_kan.py:26-61: ``num_bases = grid_size + 3``,
``grid_params = [grid_min, inv_h]`` in fp32, Kaiming-uniform draws in the
reference order), ``half``/``float`` (:67-83; the grid stays fp32),
``forward`` (:104-152).  ``spline_order`` is stored and ignored: the basis is
always the closed-form uniform cubic with span = clamp(floor(pos), 0, G-1) and
u = clamp(pos - span, 0, 1) (fused_kan.metal:254-275), i.e. it saturates
outside the grid.  ``KAN`` is an alias (bspline_kan.py:342).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np

from ._layer import KANLayerBase


class BSplineKAN(KANLayerBase):
    """Fused cubic B-spline KAN layer.

    Parameters:
        in_features: Number of input features.
        out_features: Number of output features.
        grid_size: Number of grid intervals G (default 5).
        spline_order: Accepted for compatibility; the basis is always cubic.
        grid_range: (min, max) of the knot grid (default (-1, 1)).
        bias: Whether to add a trainable additive bias (default True).
        use_base: Whether to include the residual SiLU base branch (default True).
    """
    _basis = "bspline"
    _weight_attr = "w_spline"

    def __init__(self, in_features: int, out_features: int, grid_size: int = 5, spline_order: int = 3,
                 grid_range: Sequence[float] = (-1.0, 1.0), bias: bool = True, use_base: bool = True):
        self.in_features = in_features
        self.out_features = out_features
        self.grid_size = grid_size
        self.spline_order = spline_order
        self.num_bases = grid_size + 3
        self.has_base = 1 if use_base else 0
        self.has_bias = 1 if bias else 0
        self.grid_min = float(grid_range[0])
        self.grid_max = float(grid_range[1])
        self.inv_h = float(grid_size) / (self.grid_max - self.grid_min)
        self.grid_params = np.array([self.grid_min, self.inv_h], dtype=np.float32)
        self.grid = self.grid_params
        bound = 1.0 / math.sqrt(in_features)
        self.w_spline = np.random.uniform(-bound, bound,
                                          (out_features, in_features * self.num_bases)).astype(np.float32)
        self.w_base = (np.random.uniform(-bound, bound, (out_features, in_features)).astype(np.float32)
                       if use_base else np.zeros((1,), dtype=np.float32))
        self.bias = (np.zeros((out_features,), dtype=np.float32) if bias else np.zeros((1,), dtype=np.float32))
        self._saved_x: Optional[np.ndarray] = None
        self._compute = "float32"

    def _num_basis(self) -> int:
        return self.num_bases

    def _basis_params(self) -> tuple:
        g = np.asarray(self.grid, dtype=np.float32)
        return (int(self.grid_size), float(g[0]), float(g[1]))

    def half(self) -> "BSplineKAN":
        """Converts layer parameters to FP16 half precision (grid stays fp32)."""
        self._cast_params(np.float16)
        self._compute = "float16"
        return self

    def _benchmark_args(self) -> tuple:
        return "benchmark_metal_bspline", self.w_spline, (self.grid,), (int(self.grid_size), int(self.spline_order))

    def float(self) -> "BSplineKAN":
        """Converts layer parameters to FP32 single precision."""
        self._cast_params(np.float32)
        self._compute = "float32"
        self.__dict__.pop("_quantized_from", None)
        return self


KAN = BSplineKAN

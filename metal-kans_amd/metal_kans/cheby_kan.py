"""ChebyKAN: Chebyshev-polynomial KAN layer on the fused gfx950 kernel.

Drop-in for the reference ``metal_kans/cheby_kan.py`` forward surface:
constructor (cheby_kan.py:24-49, same Kaiming-uniform draws in the same order,
so ``np.random.seed`` reproduces the reference weights), ``half``/``float``
(:55-71), ``forward`` (:92-141).  ``degree`` is the number of Chebyshev
coefficients K (T_0..T_{K-1}); inputs are clamped to [-1, 1]
(fused_kan.metal:216); the SiLU base branch sees the raw input.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

from ._layer import KANLayerBase


class ChebyKAN(KANLayerBase):
    """Fused Chebyshev KAN layer.

    Parameters:
        in_features: Number of input features.
        out_features: Number of output features.
        degree: Number of Chebyshev coefficients K (default 4).
        bias: Whether to add a trainable additive bias (default True).
        use_base: Whether to include the residual SiLU base branch (default True).
    """
    _basis = "cheby"
    _weight_attr = "w_cheby"

    def __init__(self, in_features: int, out_features: int, degree: int = 4, bias: bool = True,
                 use_base: bool = True):
        self.in_features = in_features
        self.out_features = out_features
        self.degree = degree
        self.has_base = 1 if use_base else 0
        self.has_bias = 1 if bias else 0
        bound = 1.0 / math.sqrt(in_features)
        self.w_cheby = np.random.uniform(-bound, bound, (out_features, in_features * degree)).astype(np.float32)
        self.w_base = (np.random.uniform(-bound, bound, (out_features, in_features)).astype(np.float32)
                       if use_base else np.zeros((1,), dtype=np.float32))
        self.bias = (np.zeros((out_features,), dtype=np.float32) if bias else np.zeros((1,), dtype=np.float32))
        self._saved_x: Optional[np.ndarray] = None
        self._compute = "float32"

    def _num_basis(self) -> int:
        return self.degree

    def half(self) -> "ChebyKAN":
        """Converts layer parameters to FP16 half precision."""
        self._cast_params(np.float16)
        self._compute = "float16"
        return self

    def float(self) -> "ChebyKAN":
        """Converts layer parameters to FP32 single precision."""
        self._cast_params(np.float32)
        self._compute = "float32"
        self.__dict__.pop("_quantized_from", None)
        return self

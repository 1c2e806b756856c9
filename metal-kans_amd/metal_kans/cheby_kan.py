"""ChebyKAN: Chebyshev-polynomial KAN layer on the fused gfx950 kernel.

Drop-in for the reference ``metal_kans/cheby_kan.py`` forward surface:
constructor (cheby_kan.py:24-49, same Kaiming-uniform draws in the same order,
so ``np.random.seed`` reproduces the reference weights), ``half``/``float``
(:55-71), ``forward`` (:92-141), ``backward`` / ``zero_grad`` (:145-231).  ``degree`` is the number of Chebyshev
coefficients K (T_0..T_{K-1}); inputs are clamped to [-1, 1]
(fused_kan.metal:216); the SiLU base branch sees the raw input.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

from . import device
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
        # gradient arrays exist from construction, as in the reference (cheby_kan.py:44-46), so an
        # optimizer can pair them with the parameters before the first backward
        self.grad_w_cheby = np.zeros_like(self.w_cheby)
        self.grad_w_base = np.zeros_like(self.w_base) if use_base else None
        self.grad_bias = np.zeros_like(self.bias) if bias else None
        self._saved_x: Optional[np.ndarray] = None
        self._compute = "float32"

    def _num_basis(self) -> int:
        return self.degree

    def half(self) -> "ChebyKAN":
        """Converts layer parameters to FP16 half precision."""
        self._cast_params(np.float16)
        self._compute = "float16"
        return self

    def _benchmark_args(self) -> tuple:
        return "benchmark_metal_cheby", self.w_cheby, (), (int(self.degree),)

    def float(self) -> "ChebyKAN":
        """Converts layer parameters to FP32 single precision."""
        self._cast_params(np.float32)
        self._compute = "float32"
        self.__dict__.pop("_quantized_from", None)
        return self

    # ---- backward (cheby_kan.py:145-231) ------------------------------------
    grad_w_cheby: Optional[np.ndarray] = None
    grad_w_base: Optional[np.ndarray] = None
    grad_bias: Optional[np.ndarray] = None

    def backward(self, dY: np.ndarray, fused: bool = True) -> np.ndarray:
        """GPU backward of the last ``forward``: fills ``grad_w_cheby`` / ``grad_w_base`` /
        ``grad_bias`` and returns dX (reshaped like the forward input).

        Same contract as the reference (cheby_kan.py:145-222): dY is read as fp32 with the forward's
        output shape; without a base / bias branch the matching gradient is a zero array of shape
        (1,).  ``fused`` selects ``metal_kan_cheby_backward_fused`` or ``metal_kan_cheby_backward``
        (the same gradients; neither materialises Phi here).  A 16-bit layer is differentiated in
        fp32 on its 16-bit weights and the saved input.
        """
        if self._saved_x is None:
            raise RuntimeError("Cannot run backward before forward() has been called.")
        x = np.ascontiguousarray(self._saved_x, dtype=np.float32)
        B, D_in = x.shape
        dY = np.asarray(dY, dtype=np.float32)
        if dY.ndim > 2 or dY.shape != (B, self.out_features):
            dY = dY.reshape(B, self.out_features)
        dY = np.ascontiguousarray(dY)

        def grad_like(name, shape, live):
            g = getattr(self, name)
            if not live:
                g = np.zeros((1,), dtype=np.float32)
            elif g is None or g.shape != shape or g.dtype != np.float32:
                g = np.zeros(shape, dtype=np.float32)
            else:
                g.fill(0)
            setattr(self, name, g)
            return g

        gw = grad_like("grad_w_cheby", self.w_cheby.shape, True)
        gwb = grad_like("grad_w_base", (self.out_features, self.in_features), self.has_base)
        gb = grad_like("grad_bias", (self.out_features,), self.has_bias)
        W = np.ascontiguousarray(self.w_cheby, dtype=np.float32)
        Wb = np.ascontiguousarray(self.w_base, dtype=np.float32) if self.has_base else None
        dX = np.empty((B, D_in), dtype=np.float32)
        lib = device.get_metal_bridge()
        fn = lib.metal_kan_cheby_backward_fused if fused else lib.metal_kan_cheby_backward
        device.check(fn(dY.ctypes.data, x.ctypes.data, W.ctypes.data, Wb.ctypes.data if Wb is not None else None,
                        gw.ctypes.data, gwb.ctypes.data if self.has_base else None,
                        gb.ctypes.data if self.has_bias else None, dX.ctypes.data, B, D_in, self.out_features,
                        self.degree, int(self.has_base), int(self.has_bias)),
                     "metal_kan_cheby_backward" + ("_fused" if fused else ""))
        shape = getattr(self, "_saved_shape", None)
        if shape is not None and len(shape) > 2:
            return dX.reshape(shape)
        return dX

    def zero_grad(self) -> None:
        """Zeros stored parameter gradients."""
        for name in ("grad_w_cheby", "grad_w_base", "grad_bias"):
            g = getattr(self, name)
            if g is not None:
                g.fill(0)

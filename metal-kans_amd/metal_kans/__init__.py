"""metal_kans (MI355X build): fused KAN layer forward on hand-written gfx950 HIP kernels.

Drop-in for the hot-path surface of Shuril/metal-kans (metal_kans/__init__.py:6-40):
Chebyshev / Gaussian-RBF / cubic B-spline layers, the multi-layer container, the
GatedKAN block, INT8 / INT4 / ternary weight quantization, the Chebyshev layer
backward and the torch modules.  Optimizers, pruning, symbolic export and the
other KAN families are outside this build's scope.
"""
from .device import get_metal_bridge, is_gpu_available, is_metal_available, set_async, sync
from .cheby_kan import ChebyKAN
from .fast_kan import FastKAN
from .bspline_kan import BSplineKAN, KAN
from .metal_kan import MetalKAN
from .gated_kan import GatedKAN
from .quantization import (QuantizedWeight, TernaryQuantizedWeight, quantize, to_int4, to_int8, to_ternary)

__version__ = "0.6.0+mi355x"


def __getattr__(name):
    # TorchMetalKANLinear / TorchMetalKAN (torch_module.py), imported on first use so that
    # `import metal_kans` does not import torch; None without torch, as in the reference
    # (metal_kans/__init__.py:34-38).
    if name in ("TorchMetalKANLinear", "TorchMetalKAN"):
        try:
            from . import torch_module
        except ImportError:
            return None
        return getattr(torch_module, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")

__all__ = [
    "set_async", "sync", "get_metal_bridge", "is_metal_available", "is_gpu_available",
    "ChebyKAN", "FastKAN", "BSplineKAN", "KAN", "MetalKAN", "GatedKAN",
    "QuantizedWeight", "TernaryQuantizedWeight", "quantize", "to_int8", "to_int4", "to_ternary",
    "TorchMetalKANLinear", "TorchMetalKAN",
]

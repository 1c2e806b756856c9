"""MetalKAN: sequential multi-layer KAN network, run as one device-resident chain.

Drop-in for the reference ``metal_kans/metal_kan.py`` forward surface
(constructor :41-85, ``half``/``float`` :91-103, ``async_stream`` :105-119,
``forward`` :121-135).  The basis families on this build's hot path are
``cheby``/``chebyshev``, ``fastkan``/``rbf`` (``degree`` = number of centres)
and ``bspline``/``spline``/``kan`` (``degree`` = grid size); the reference's
other families raise ``ValueError``.

Where the reference chains layers on the GPU only for fp32 Chebyshev with
``pipeline=True`` and K = 4 (metal_kan.py:130, metal_kan_bridge.mm:1210), every
multi-layer network here runs as one chain: activations stay in HBM between
layers (ping-pong buffers) and the whole host call -- H2D, all layers, D2H --
replays one captured HIP graph.  ``pipeline`` is accepted for compatibility.
Activations between layers stay fp32 in HBM for every dtype, and an fp32
input to a 16-bit network is used unrounded (see ``_layer.py``).
"""
from __future__ import annotations

import ctypes
from typing import List, Sequence

import numpy as np

from . import device
from ._engine import DT_BF16, DT_F16, DT_F32, from_bf16_bits
from ._layer import device_layer_handle
from .bspline_kan import BSplineKAN
from .cheby_kan import ChebyKAN
from .fast_kan import FastKAN

MetalChebyKAN = ChebyKAN
MetalFastKAN = FastKAN

_OUT_OF_SCOPE = {"relukan", "relu", "tent", "wav", "wavkan", "wavelet", "fourier", "fourierkan", "jacobi",
                 "jacobikan", "rational", "rationalkan", "mult", "multkan", "lowrank", "lowrankkan"}


class MetalKAN:
    """Multi-layer KAN network on the MI355X fused kernels.

    Parameters:
        layers_hidden: layer widths, e.g. [4, 16, 8, 2].
        basis_type: 'cheby', 'fastkan' / 'rbf', or 'bspline' / 'spline' / 'kan'.
        degree: coefficients (cheby), centres (fastkan) or grid intervals (bspline); default 4.
        bias: include the bias term (default True).
        use_base: include the residual SiLU base branch (default True).
        pipeline: accepted for compatibility; multi-layer networks always run as one chain.
    """

    def __init__(self, layers_hidden: Sequence[int], basis_type: str = "cheby", degree: int = 4, bias: bool = True,
                 use_base: bool = True, pipeline: bool = False):
        self.layers_hidden = list(layers_hidden)
        self.basis_type = basis_type.lower()
        self.degree = degree
        self.bias = bias
        self.use_base = use_base
        self.pipeline = pipeline and (self.basis_type in ("cheby", "chebyshev"))
        self.layers: List = []
        for i in range(len(layers_hidden) - 1):
            in_f, out_f = layers_hidden[i], layers_hidden[i + 1]
            if self.basis_type in ("cheby", "chebyshev"):
                layer = ChebyKAN(in_f, out_f, degree=degree, bias=bias, use_base=use_base)
            elif self.basis_type in ("fastkan", "rbf"):
                layer = FastKAN(in_f, out_f, num_centers=degree, bias=bias, use_base=use_base)
            elif self.basis_type in ("bspline", "spline", "kan"):
                layer = BSplineKAN(in_f, out_f, grid_size=degree, bias=bias, use_base=use_base)
            elif self.basis_type in _OUT_OF_SCOPE:
                raise ValueError(f"basis_type {basis_type!r} is outside this build's fused-forward scope "
                                 "(cheby, fastkan/rbf, bspline)")
            else:
                raise ValueError(f"Unknown basis_type: {basis_type}")
            self.layers.append(layer)
        self._chain = None
        self._chain_key = None

    def __del__(self):
        self._drop_chain()

    def _drop_chain(self):
        try:
            if self._chain:
                device.load_library().kans_chain_destroy(self._chain)
        except Exception:
            pass
        self._chain = None
        self._chain_key = None

    @property
    def dtype(self) -> np.dtype:
        return getattr(self.layers[0], "dtype", np.dtype(np.float32)) if self.layers else np.dtype(np.float32)

    def half(self) -> "MetalKAN":
        """Converts all layers to FP16."""
        for layer in self.layers:
            layer.half()
        return self

    def float(self) -> "MetalKAN":
        """Converts all layers to FP32."""
        for layer in self.layers:
            layer.float()
        return self

    def bfloat16(self) -> "MetalKAN":
        """Converts all layers to bfloat16 (see the layer classes)."""
        for layer in self.layers:
            layer.bfloat16()
        return self

    def async_stream(self, batches: Sequence[np.ndarray]) -> List[np.ndarray]:
        """Runs a sequence of batches with one synchronisation at the end (metal_kan.py:105-119)."""
        from .device import set_async, sync
        results = []
        set_async(True)
        try:
            for b in batches:
                results.append(self.forward(b))
        finally:
            sync()
            set_async(False)
        return results

    def _compute(self) -> str:
        kinds = {layer._resolve_compute() for layer in self.layers}
        if len(kinds) != 1:
            raise ValueError(f"layers disagree on compute dtype: {sorted(kinds)}")
        return kinds.pop()

    def forward(self, x: np.ndarray) -> np.ndarray:
        """Runs all layers on the device; one graph replay per call for multi-layer networks."""
        if len(self.layers) == 1:
            return self.layers[0](x)
        compute = self._compute()
        io = np.float16 if compute == "float16" else np.float32   # weight / output element type
        x = np.asarray(x)
        x_in = np.float16 if (compute == "float16" and x.dtype == np.float16) else np.float32
        if x.dtype != x_in:
            x = x.astype(x_in)
        orig_shape = x.shape
        x2 = np.ascontiguousarray(x.reshape(-1, self.layers_hidden[0]))
        B = x2.shape[0]
        handles = [device_layer_handle(layer, compute) for layer in self.layers]
        lib = device.get_metal_bridge()
        # handle serial numbers, not addresses: a re-created handle can reuse a destroyed one's address
        key = (tuple(layer._engine().serial for layer in self.layers), compute)
        if self._chain_key != key:
            self._drop_chain()
            arr = (ctypes.c_void_p * len(handles))(*handles)
            h = ctypes.c_void_p()
            device.check(lib.kans_chain_create(arr, len(handles), ctypes.byref(h)), "kans_chain_create")
            self._chain = h
            self._chain_key = key
        out_dim = self.layers_hidden[-1]
        x_dt = DT_F16 if x2.dtype == np.float16 else DT_F32
        if compute == "bfloat16":
            yb = np.empty((B, out_dim), dtype=np.uint16)
            device.check(lib.kans_chain_forward_host_ex(self._chain, x2.ctypes.data, x_dt, yb.ctypes.data, B),
                         "kans_chain_forward_host_ex")
            y = from_bf16_bits(yb).reshape(B, out_dim)
        else:
            y = np.empty((B, out_dim), dtype=io)
            device.check(lib.kans_chain_forward_host_ex(self._chain, x2.ctypes.data, x_dt, y.ctypes.data, B),
                         "kans_chain_forward_host_ex")
        if len(orig_shape) > 2:
            return y.reshape(*orig_shape[:-1], out_dim)
        return y

    def __call__(self, x: np.ndarray) -> np.ndarray:
        return self.forward(x)

"""INT8 / INT4 block-affine and 1.58-bit ternary weight quantization.

Drop-in for the reference ``metal_kans/quantization.py`` (QuantizedWeight
:13-148, quantize/to_int8/to_int4 :152-188, TernaryQuantizedWeight :191-286,
to_ternary :396-421): same classes, attributes (``qweight``, ``scales``,
``biases``, ``padded_in_features``, ``w_packed``), packed formats and in-place
model semantics (``_<attr>_quantized`` / ``_<attr>_ternary`` holds the packed
weight, ``<attr>`` becomes the fp32 dequantized array).

The quantizers run natively on the host (``metal_kan_quantize_*`` in
libkans_hip.so) with the rounding of the reference's NumPy fallback (the path
the reference takes off-macOS); the dequantizers run on the GPU and are
bit-identical to the reference's.  There is no NumPy fallback.

Each packed object remembers (``_deq_snapshot``) the dequantized array it put
in place, so a fused kernel that reads the packed weights directly can check
that they still are the layer's weights (``_qengine.packed_format``).  The
dequantized arrays stay writeable, as in the reference (its optimizers update
them in place, optim.py; torch_module.py:101 assigns into them): an in-place
edit or a new array retires the packed path for that layer, which then runs on
the edited fp32 weights.  The check compares contents (a copy up to 4 MB, a
hash above), so ``layer.freeze_weights()`` (``GatedKAN.freeze_weights()``)
skips it for large arrays in inference loops.

One addition: a layer that computed in fp16/bf16 before quantization keeps
that compute dtype (``_quantized_from``), so a quantized ``GatedKAN(dtype=
float16)`` still runs fp16 activations; fp32 layers behave exactly as in the
reference (fp32 forward on the dequantized weights).
"""
from __future__ import annotations

from typing import Any

import numpy as np

from . import device
from ._engine import _Snapshot

WEIGHT_ATTRS = ["w_cheby", "w_rbf", "w_relu", "w_wav", "w_fourier", "w_jacobi", "w_p", "w_q", "w_spline", "w_up",
                "w_base"]


class QuantizedWeight:
    """Affine block-quantized weight matrix: INT8 (1 byte/weight) or INT4 (2 weights/byte)."""

    def __init__(self, weight: np.ndarray, bits: int = 8, group_size: int = 64):
        if bits not in (8, 4):
            raise ValueError(f"Unsupported bits: {bits}. Choose 8 or 4.")
        self.bits = bits
        self.group_size = group_size
        self.shape = weight.shape
        out_features, in_features = weight.shape
        pad_in = (group_size - (in_features % group_size)) % group_size
        if pad_in > 0:
            padded = np.pad(weight, ((0, 0), (0, pad_in)), mode="constant", constant_values=0.0)
        else:
            padded = weight
        padded = np.ascontiguousarray(padded, dtype=np.float32)
        self.padded_in_features = padded.shape[1]
        num_groups = padded.size // group_size
        self.scales = np.empty((num_groups, 1), dtype=np.float32)
        self.biases = np.empty((num_groups, 1), dtype=np.float32)
        lib = device.load_library()
        if bits == 8:
            self.qweight = np.empty((num_groups, group_size), dtype=np.uint8)
            fn = lib.metal_kan_quantize_int8
        else:
            self.qweight = np.empty((num_groups, group_size // 2), dtype=np.uint8)
            fn = lib.metal_kan_quantize_int4
        device.check(fn(padded.ctypes.data, self.qweight.ctypes.data, self.scales.ctypes.data,
                        self.biases.ctypes.data, num_groups, group_size), f"metal_kan_quantize_int{bits}")

    def dequantize(self) -> np.ndarray:
        """Dequantizes on the GPU back into an fp32 array of the original shape."""
        lib = device.get_metal_bridge()
        num_groups = self.scales.shape[0]
        out = np.empty(num_groups * self.group_size, dtype=np.float32)
        q = np.ascontiguousarray(self.qweight)
        s = np.ascontiguousarray(self.scales, dtype=np.float32)
        b = np.ascontiguousarray(self.biases, dtype=np.float32)
        fn = lib.metal_kan_dequantize_int8 if self.bits == 8 else lib.metal_kan_dequantize_int4
        device.check(fn(q.ctypes.data, s.ctypes.data, b.ctypes.data, out.ctypes.data, num_groups, self.group_size),
                     f"metal_kan_dequantize_int{self.bits}")
        return out.reshape(-1, self.padded_in_features)[: self.shape[0], : self.shape[1]]


class TernaryQuantizedWeight:
    """1.58-bit ternary weights ({-1, 0, +1} x per-(row, group) absmean scale), 16 per uint32."""

    def __init__(self, weight: np.ndarray, group_size: int = 32):
        self.group_size = group_size
        self.shape = weight.shape
        D_out, K_dim = weight.shape
        w = np.ascontiguousarray(weight, dtype=np.float32)
        words_per_row = (K_dim + 15) // 16
        groups_per_row = (K_dim + group_size - 1) // group_size
        self.w_packed = np.zeros((D_out, words_per_row), dtype=np.uint32)
        self.scales = np.zeros((D_out, groups_per_row), dtype=np.float32)
        lib = device.load_library()
        device.check(lib.metal_kan_quantize_ternary(w.ctypes.data, self.w_packed.ctypes.data,
                                                    self.scales.ctypes.data, D_out, K_dim, group_size),
                     "metal_kan_quantize_ternary")

    def dequantize(self) -> np.ndarray:
        D_out, K_dim = self.shape
        lib = device.get_metal_bridge()
        out = np.empty((D_out, K_dim), dtype=np.float32)
        p = np.ascontiguousarray(self.w_packed)
        s = np.ascontiguousarray(self.scales)
        device.check(lib.metal_kan_dequantize_ternary(p.ctypes.data, s.ctypes.data, out.ctypes.data, D_out, K_dim,
                                                      self.group_size), "metal_kan_dequantize_ternary")
        return out


def _remember_compute(model: Any) -> None:
    cd = getattr(model, "_compute", None)
    if cd in ("float16", "bfloat16") and not hasattr(model, "_quantized_from"):
        model._quantized_from = cd


def quantize(model: Any, bits: int = 8, group_size: int = 64) -> Any:
    """Quantizes all weight matrices of a layer or network in place (quantization.py:152-178)."""
    if hasattr(model, "layers"):
        for layer in model.layers:
            quantize(layer, bits=bits, group_size=group_size)
        return model
    _remember_compute(model)
    for attr in WEIGHT_ATTRS:
        if hasattr(model, attr):
            w = getattr(model, attr)
            if w is not None and isinstance(w, np.ndarray) and w.ndim == 2:
                qw = QuantizedWeight(w, bits=bits, group_size=group_size)
                setattr(model, f"_{attr}_quantized", qw)
                setattr(model, attr, qw.dequantize())
                qw._deq_snapshot = _Snapshot(getattr(model, attr))
    if hasattr(model, "sub_layer"):
        quantize(model.sub_layer, bits=bits, group_size=group_size)
    if hasattr(model, "down_layer"):
        quantize(model.down_layer, bits=bits, group_size=group_size)
    return model


def to_int8(model: Any, group_size: int = 64) -> Any:
    """Quantizes all weights to INT8."""
    return quantize(model, bits=8, group_size=group_size)


def to_int4(model: Any, group_size: int = 64) -> Any:
    """Quantizes all weights to INT4."""
    return quantize(model, bits=4, group_size=group_size)


def to_ternary(model: Any, group_size: int = 32) -> Any:
    """Quantizes all weight matrices to 1.58-bit ternary in place (quantization.py:396-421)."""
    if hasattr(model, "layers"):
        for layer in model.layers:
            to_ternary(layer, group_size=group_size)
        return model
    _remember_compute(model)
    for attr in WEIGHT_ATTRS:
        if hasattr(model, attr):
            w = getattr(model, attr)
            if w is not None and isinstance(w, np.ndarray) and w.ndim == 2:
                qw = TernaryQuantizedWeight(w, group_size=group_size)
                setattr(model, f"_{attr}_ternary", qw)
                setattr(model, attr, qw.dequantize())
                qw._deq_snapshot = _Snapshot(getattr(model, attr))
    if hasattr(model, "sub_layer"):
        to_ternary(model.sub_layer, group_size=group_size)
    if hasattr(model, "down_layer"):
        to_ternary(model.down_layer, group_size=group_size)
    return model

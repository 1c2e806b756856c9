"""Device-resident quantized KAN layers (Chebyshev, Gaussian RBF, B-spline) and GatedKAN blocks.

A layer quantized with ``to_int8`` / ``to_int4`` (group 64) or ``to_ternary``
(group 32) keeps its packed weights in ``_<attr>_quantized`` /
``_<attr>_ternary`` for its basis weight ``<attr>`` (``w_cheby``, ``w_rbf``,
``w_spline``) and ``w_base``, in the reference's formats (quantization.py:13-99,
191-246).  ``QLayerEngine`` uploads those packed arrays once and runs the fused
kernels on them, which move the packed bytes instead of dequantized fp32
weights: the decode GEMVs for batches of at most ``MAX_DECODE_B`` rows (every
basis and K) and the fused prefill kernel for larger batches where it is built
(``kans_qlayer_fused``).  The engine is rebuilt when the packed objects or the
basis parameters change (a new ``to_int8`` / ``to_int4`` / ``to_ternary``, a new
grid).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import device
from ._engine import DT_BF16, DT_F16, DT_F32, from_bf16_bits

MAX_DECODE_B = 32
# Chebyshev degrees (coefficients per feature) the fused prefill kernel is built for (the GatedKAN block;
# INT8 with the base branch is not built at K = 7)
PREFILL_K = (1, 2, 3, 4, 5, 6, 7, 8, 9)
KANS_ERR_UNSUPPORTED = -5


def fused_batch_ok(fmt: str, K: int, B: int) -> bool:
    """Whether a batch of B rows of a Chebyshev GatedKAN block in packed format ``fmt`` with K coefficients
    runs on the fused quantized kernels (else the caller uses the dequantized weights).  Single layers ask
    their engine (``QLayerEngine.fused``)."""
    if B <= 0:
        return False
    if B <= MAX_DECODE_B:
        return True
    return K in PREFILL_K and not (fmt == "int8" and K == 7)


def packed_format(layer) -> Optional[str]:
    """'int8' / 'int4' / 'ternary' when every weight matrix of a KAN layer (its basis weight and W_base) is
    packed in a format the fused kernels read (INT8 / INT4 with group 64, ternary with group 32), else None."""
    from .quantization import QuantizedWeight, TernaryQuantizedWeight

    def fmt(attr):
        # the packed object counts only while the layer still holds the array it dequantized to
        # (a later quantization, assignment or in-place edit makes it stale)
        cur = getattr(layer, attr, None)

        def live(obj):
            snap = getattr(obj, "_deq_snapshot", None)
            return snap is not None and snap.same(cur, verify=not getattr(layer, "_frozen", False))
        q = getattr(layer, f"_{attr}_quantized", None)
        if isinstance(q, QuantizedWeight) and q.group_size == 64 and live(q):
            return "int4" if q.bits == 4 else "int8"
        t = getattr(layer, f"_{attr}_ternary", None)
        if isinstance(t, TernaryQuantizedWeight) and t.group_size == 32 and live(t):
            return "ternary"
        return None

    f = fmt(getattr(layer, "_weight_attr", "w_cheby"))
    if f is None:
        return None
    if getattr(layer, "has_base", False) and fmt("w_base") != f:
        return None
    return f


def _key(layer, fmt):
    suffix = "_ternary" if fmt == "ternary" else "_quantized"
    attr = "_" + getattr(layer, "_weight_attr", "w_cheby")
    objs = [getattr(layer, attr + suffix, None), getattr(layer, "_w_base" + suffix, None),
            getattr(layer, "bias", None) if layer.has_bias else None]
    return tuple(id(o) for o in objs) + (layer._basis_params(),)


class QLayerEngine:
    """Owns a ``kans_qlayer`` handle built from a quantized KAN layer (ChebyKAN, FastKAN, BSplineKAN)."""

    def __init__(self, layer, fmt: str):
        self.fmt = fmt
        self.key = _key(layer, fmt)
        self.d_in, self.d_out = int(layer.in_features), int(layer.out_features)
        lib = device.get_metal_bridge()
        self.handle = ctypes.c_void_p()
        has_base, has_bias = int(bool(layer.has_base)), int(bool(layer.has_bias))
        K = int(layer._num_basis())
        attr = "_" + layer._weight_attr
        bias = None
        if has_bias:
            bias = np.ascontiguousarray(layer.bias, dtype=np.float32)
        bias_ptr = bias.ctypes.data if bias is not None else None
        self.K = K
        if fmt in ("int4", "int8"):
            w = getattr(layer, attr + "_quantized")
            wb = layer._w_base_quantized if has_base else None
            arrs = [np.ascontiguousarray(w.qweight), np.ascontiguousarray(w.scales, dtype=np.float32),
                    np.ascontiguousarray(w.biases, dtype=np.float32)]
            barrs = ([np.ascontiguousarray(wb.qweight), np.ascontiguousarray(wb.scales, dtype=np.float32),
                      np.ascontiguousarray(wb.biases, dtype=np.float32)] if wb is not None else [None, None, None])
            ptr = [a.ctypes.data if a is not None else None for a in arrs + barrs]
            name = f"kans_qlayer_create_{fmt}"
            device.check(getattr(lib, name)(self.d_in, self.d_out, K, has_base, has_bias, 64, *ptr, bias_ptr, DT_F32,
                                            ctypes.byref(self.handle)), name)
        else:
            w = getattr(layer, attr + "_ternary")
            wb = layer._w_base_ternary if has_base else None
            arrs = [np.ascontiguousarray(w.w_packed), np.ascontiguousarray(w.scales, dtype=np.float32)]
            barrs = ([np.ascontiguousarray(wb.w_packed), np.ascontiguousarray(wb.scales, dtype=np.float32)]
                     if wb is not None else [None, None])
            ptr = [a.ctypes.data if a is not None else None for a in arrs + barrs]
            device.check(lib.kans_qlayer_create_ternary(self.d_in, self.d_out, K, has_base, has_bias, 32, *ptr,
                                                        bias_ptr, DT_F32, ctypes.byref(self.handle)),
                         "kans_qlayer_create_ternary")
        # the layer's basis (the same parameters its dense forward uses, _basis_params)
        params = layer._basis_params()
        if layer._basis == "rbf":
            centers = np.ascontiguousarray(params[0], dtype=np.float32)
            device.check(lib.kans_qlayer_set_rbf(self.handle, centers.ctypes.data, float(params[1])),
                         "kans_qlayer_set_rbf")
        elif layer._basis == "bspline":
            device.check(lib.kans_qlayer_set_bspline(self.handle, int(params[0]), float(params[1]),
                                                     float(params[2])), "kans_qlayer_set_bspline")

    def __del__(self):
        try:
            if self.handle:
                device.load_library().kans_qlayer_destroy(self.handle)
        except Exception:
            pass

    def current(self, layer) -> bool:
        return packed_format(layer) == self.fmt and _key(layer, self.fmt) == self.key

    def fused(self, B: int) -> bool:
        """Whether a forward of B rows runs on the fused packed-weight kernels (kans_qlayer_fused)."""
        return B > 0 and device.get_metal_bridge().kans_qlayer_fused(self.handle, int(B)) == 1

    def forward_host(self, x: np.ndarray, out_dtype) -> np.ndarray:
        """y = layer(x) on the packed weights; out_dtype np.float16, np.float32 or "bfloat16" (the
        result rounded to bf16, returned as float32 values)."""
        x = np.ascontiguousarray(x)
        B = x.shape[0]
        xdt = DT_F16 if x.dtype == np.float16 else DT_F32
        if xdt == DT_F32 and x.dtype != np.float32:
            x = x.astype(np.float32)
        bf16 = isinstance(out_dtype, str) and out_dtype == "bfloat16"
        y = np.empty((B, self.d_out), dtype=np.uint16 if bf16 else out_dtype)
        ydt = DT_BF16 if bf16 else DT_F16 if out_dtype == np.float16 else DT_F32
        device.check(device.get_metal_bridge().kans_qlayer_forward_host(self.handle, x.ctypes.data, xdt, y.ctypes.data,
                                                                          ydt, B), "kans_qlayer_forward_host")
        return from_bf16_bits(y).reshape(B, self.d_out) if bf16 else y


def layer_engine(layer) -> Optional["QLayerEngine"]:
    """The fused quantized engine of a KAN layer (Chebyshev, RBF, B-spline) that computes in fp16 or bf16
    after ``to_int8`` / ``to_int4`` / ``to_ternary`` (cached on the layer, rebuilt when its packed weights or
    basis parameters change), else None.  A bf16 layer runs the same kernels: fp16 basis values and decoded
    weights (each at least as precise as its bf16 rounding in the value ranges these take), fp32
    accumulation, the result rounded to bf16."""
    q = getattr(layer, "_quantized_from", None)
    if getattr(layer, "_basis", "") not in ("cheby", "rbf", "bspline") \
            or q not in ("float16", "bfloat16") or layer._resolve_compute() != q:
        return None
    fmt = packed_format(layer)
    if fmt is None:
        return None
    eng = layer.__dict__.get("_qlayer_engine")
    if eng is None or not eng.current(layer):
        eng = QLayerEngine(layer, fmt)
        layer._qlayer_engine = eng
    return eng


class GatedEngine:
    """Owns the three ``kans_qlayer`` handles and the ``kans_gated`` block of a quantized GatedKAN."""

    def __init__(self, block, fmt: str):
        self.fmt = fmt
        self.K = int(block.degree)
        self.layers = [QLayerEngine(k, fmt) for k in (block.gate_kan, block.up_kan, block.down_kan)]
        self.handle = ctypes.c_void_p()
        device.check(device.get_metal_bridge().kans_gated_create(self.layers[0].handle, self.layers[1].handle,
                                                                 self.layers[2].handle, ctypes.byref(self.handle)),
                     "kans_gated_create")
        self.d_model = self.layers[0].d_in

    def __del__(self):
        try:
            if self.handle:
                device.load_library().kans_gated_destroy(self.handle)
        except Exception:
            pass

    def current(self, block) -> bool:
        return all(e.current(k) for e, k in zip(self.layers, (block.gate_kan, block.up_kan, block.down_kan)))

    def forward_host(self, x: np.ndarray, out_dtype, round16: int) -> np.ndarray:
        """The block on the packed weights; out_dtype np.float16, np.float32 or "bfloat16" (returned as
        float32 values); round16 1 / 2 rounds gate, up and hidden to fp16 / bf16."""
        x = np.ascontiguousarray(x)
        B = x.shape[0]
        xdt = DT_F16 if x.dtype == np.float16 else DT_F32
        if xdt == DT_F32 and x.dtype != np.float32:
            x = x.astype(np.float32)
        bf16 = isinstance(out_dtype, str) and out_dtype == "bfloat16"
        y = np.empty((B, self.d_model), dtype=np.uint16 if bf16 else out_dtype)
        ydt = DT_BF16 if bf16 else DT_F16 if out_dtype == np.float16 else DT_F32
        device.check(device.get_metal_bridge().kans_gated_forward_host(self.handle, x.ctypes.data, xdt, y.ctypes.data,
                                                                         ydt, B, round16), "kans_gated_forward_host")
        return from_bf16_bits(y).reshape(B, self.d_model) if bf16 else y

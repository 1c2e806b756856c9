"""Shared forward plumbing of the ChebyKAN / FastKAN / BSplineKAN layers.

The forward mirrors the reference layers (cheby_kan.py:92-141,
fast_kan.py:99-147, bspline_kan.py:104-152): cast x to the compute dtype,
flatten leading dims, make it C-contiguous, keep it in ``_saved_x``, check
``in_features``, allocate ``y`` and call the device.  The device call is the
fused HIP kernel through a device-resident layer (weights uploaded and re-tiled
once, see ``_engine.py``).

Compute dtypes: ``float32`` and ``float16`` as in the reference (``.float()``,
``.half()``); ``bfloat16`` is new (``.bfloat16()``).  NumPy has no bf16, so a
bf16 layer keeps float32 attribute arrays holding bf16-rounded values and
returns float32 arrays holding bf16 values.

Inputs of 16-bit layers: an fp16 input to an fp16 layer is used as given (the
reference casts x to the weight dtype, cheby_kan.py:97-101); a float32 input
is NOT rounded to 16 bits first -- the kernel reads it in fp32 and evaluates the
basis in fp32 ("FP32-internal"), only the weights and the MFMA operands are
16-bit.  Rounding x first costs accuracy for large K: T_k'(+-1) = k^2.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from ._engine import DT_BF16, DT_F16, DT_F32, LayerEngine, _Snapshot, from_bf16_bits, to_bf16_bits
from . import device


class KANLayerBase:
    _basis: str = ""
    _weight_attr: str = ""

    # subclasses set: in_features, out_features, has_base, has_bias, w_base, bias
    _compute: str = "float32"
    _engine_obj: Optional[LayerEngine] = None

    # ---- to be provided by subclasses ------------------------------------
    def _num_basis(self) -> int:
        raise NotImplementedError

    def _basis_params(self) -> tuple:
        return ()

    # ---- dtype handling --------------------------------------------------
    @property
    def dtype(self) -> np.dtype:
        """dtype of the basis weight array, as in the reference."""
        return getattr(self, self._weight_attr).dtype

    @property
    def compute_dtype(self) -> str:
        """'float32' | 'float16' | 'bfloat16': the arithmetic the forward runs in."""
        return self._compute

    def _cast_params(self, dtype) -> None:
        setattr(self, self._weight_attr, getattr(self, self._weight_attr).astype(dtype))
        if self.has_base:
            self.w_base = self.w_base.astype(dtype)
        if self.has_bias:
            self.bias = self.bias.astype(dtype)

    def bfloat16(self):
        """Converts layer parameters to bfloat16 (stored as bf16-rounded float32 arrays)."""
        def rnd(a):
            return from_bf16_bits(to_bf16_bits(a)).reshape(a.shape)
        setattr(self, self._weight_attr, rnd(getattr(self, self._weight_attr)))
        if self.has_base:
            self.w_base = rnd(self.w_base)
        if self.has_bias:
            self.bias = rnd(self.bias)
        self._compute = "bfloat16"
        return self

    def invalidate(self) -> None:
        """Force the next forward to re-upload the weights (in-place edits are detected without it)."""
        if self._engine_obj is not None:
            self._engine_obj.invalidate()

    _frozen: bool = False

    def freeze_weights(self, frozen: bool = True):
        """Declare that the weight arrays will not be edited in place (opt-in, for inference loops): the
        forward then compares arrays larger than 4 MB by identity only instead of hashing their bytes on
        every call.  Assigning a new array is still detected; an in-place edit of a frozen layer's large
        array must be followed by ``invalidate()``."""
        self._frozen = bool(frozen)
        return self

    def set_tiling(self, wm: int, nb: int, splits: int = 0, wave_groups: int = 0) -> None:
        """Force the fused kernel's tile shape (tuning/testing); (0, 0) restores the heuristic.
        ``wave_groups`` (1, 2, 4; 0 = automatic) splits a 16-bit Chebyshev tile's feature blocks over
        wave groups of one workgroup where the tile is instantiated with them."""
        self._engine().set_tiling(wm, nb, splits, wave_groups)

    def _engine(self) -> LayerEngine:
        if self._engine_obj is None:
            self._engine_obj = LayerEngine(self._basis, self.in_features, self.out_features, self._num_basis(),
                                           self.has_base, self.has_bias)
        return self._engine_obj

    def _resolve_compute(self) -> str:
        wd = self.dtype
        if self._compute == "bfloat16":
            return "bfloat16"
        if self._compute == "float16" and getattr(self, "_quantized_from", None) == "float16":
            return "float16"  # quantized layer keeps its fp16 activations
        return "float16" if wd == np.float16 else "float32"

    # ---- forward ----------------------------------------------------------
    def forward(self, x: np.ndarray) -> np.ndarray:
        compute = self._resolve_compute()
        x = x if isinstance(x, np.ndarray) else np.asarray(x)
        if compute == "float32":
            io_dtype = np.float32
        elif compute == "float16" and x.dtype == np.float16:
            io_dtype = np.float16          # fp16 input used as given (reference semantics)
        else:
            io_dtype = np.float32          # fp32 input to a 16-bit layer is not rounded first
        if x.dtype != io_dtype:
            x = x.astype(io_dtype)
        orig_shape = x.shape
        if x.ndim > 2:
            x = x.reshape(-1, self.in_features)
        if not x.flags["C_CONTIGUOUS"]:
            x = np.ascontiguousarray(x)
        self._saved_x = x
        self._saved_shape = orig_shape
        B, D_in = x.shape
        if D_in != self.in_features:
            raise ValueError(f"Expected in_features={self.in_features}, got {D_in}")

        # a layer quantized from fp16 / bf16 runs on its packed weights (fused quantized kernels)
        from ._qengine import layer_engine
        qeng = layer_engine(self) if B > 0 else None
        if qeng is not None and qeng.fused(B):
            y = qeng.forward_host(x, np.float16 if compute == "float16" else "bfloat16")
            if len(orig_shape) > 2:
                return y.reshape(*orig_shape[:-1], self.out_features)
            return y

        W = getattr(self, self._weight_attr)
        Wb = self.w_base if self.has_base else None
        bias = self.bias if self.has_bias else None
        eng = self._engine()
        if compute == "bfloat16":
            eng.prepare_f32(DT_BF16, np.ascontiguousarray(W, dtype=np.float32),
                            None if Wb is None else np.ascontiguousarray(Wb, dtype=np.float32),
                            None if bias is None else np.ascontiguousarray(bias, dtype=np.float32),
                            self._basis_params(), verify=not self._frozen)
            yb = np.empty((B, self.out_features), dtype=np.uint16)
            eng.forward_host(x, yb)
            y = from_bf16_bits(yb).reshape(B, self.out_features)
        else:
            np_dt = np.float16 if compute == "float16" else np.float32
            dt = DT_F16 if compute == "float16" else DT_F32

            def conv(a):
                if a is None:
                    return None
                return a if (a.dtype == np_dt and a.flags["C_CONTIGUOUS"]) else self._converted(a, np_dt)
            eng.prepare(dt, conv(W), conv(Wb), conv(bias), self._basis_params(), verify=not self._frozen)
            y = np.empty((B, self.out_features), dtype=np_dt)
            eng.forward_host(x, y)
        if len(orig_shape) > 2:
            return y.reshape(*orig_shape[:-1], self.out_features)
        return y

    __call__ = forward

    def _converted(self, a: np.ndarray, np_dt) -> np.ndarray:
        """Cached dtype conversion of a parameter array, redone when the source array changes (identity
        or content, as the device upload checks it)."""
        cache = self.__dict__.setdefault("_conv_cache", {})
        key = (id(a), np.dtype(np_dt).str)
        hit = cache.get(key)
        if hit is not None and hit[0].same(a, not self._frozen):
            return hit[1]
        conv = np.ascontiguousarray(a, dtype=np_dt)
        if len(cache) >= 8:  # entries hold their source arrays: keep only recent ones
            cache.clear()
        cache[key] = (_Snapshot(a), conv)
        return conv

    def backward(self, *args, **kwargs):
        raise NotImplementedError("training (backward) is outside this build's forward-only scope")

    # ---- benchmark (cheby_kan.py:233-257, fast_kan.py:223-247, bspline_kan.py:227-251) ----------
    def _benchmark_args(self) -> tuple:
        """(entry-point name, basis weight array, arrays passed between W_base and bias, integer / float
        arguments between D_out and has_base) of the reference-named benchmark_metal_* call."""
        raise NotImplementedError

    def benchmark(self, x: np.ndarray, warmup: int = 10, iters: int = 50) -> float:
        """Mean wall-clock ms per full host call of the fp32 reference-named forward on x (the reference's
        benchmark: host arrays in, host array out, synchronous).  The weights are passed as float32 (a
        16-bit layer's arrays are converted first; the reference would hand their raw bytes on)."""
        x = np.asarray(x, dtype=np.float32)
        x_flat = np.ascontiguousarray(x.reshape(-1, self.in_features))
        B = x_flat.shape[0]
        y = np.empty((B, self.out_features), dtype=np.float32)
        name, W, mid, tail = self._benchmark_args()
        f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
        W, Wb, bias = f32(W), f32(self.w_base), f32(self.bias)
        mid = [f32(a) for a in mid]
        ms = getattr(device.get_metal_bridge(), name)(x_flat.ctypes.data, W.ctypes.data, Wb.ctypes.data,
                                                      *[a.ctypes.data for a in mid],
                                                      bias.ctypes.data, y.ctypes.data, B, self.in_features,
                                                      self.out_features, *tail, self.has_base, self.has_bias,
                                                      int(warmup), int(iters))
        if ms < 0:
            raise RuntimeError(f"{name} failed: {device.last_error()}")
        return float(ms)


def device_layer_handle(layer: KANLayerBase, compute: str) -> int:
    """Make the layer's device weights current for compute dtype ``compute`` and return its ``kans_layer``
    handle (used by the multi-layer chain and the GatedKAN block, which launch the layers themselves).
    Key anything that keeps the handle on ``layer._engine().serial`` with it (see ``_engine``)."""
    dt = {"float32": DT_F32, "float16": DT_F16, "bfloat16": DT_BF16}[compute]
    eng = layer._engine()
    W = getattr(layer, layer._weight_attr)
    Wb = layer.w_base if layer.has_base else None
    bias = layer.bias if layer.has_bias else None
    if compute == "bfloat16":
        f32 = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
        eng.prepare_f32(dt, f32(W), f32(Wb), f32(bias), layer._basis_params(), verify=not layer._frozen)
    else:
        io = np.float16 if compute == "float16" else np.float32
        conv = lambda a: None if a is None else (  # noqa: E731
            a if (a.dtype == io and a.flags["C_CONTIGUOUS"]) else layer._converted(a, io))
        eng.prepare(dt, conv(W), conv(Wb), conv(bias), layer._basis_params(), verify=not layer._frozen)
    return eng.handle.value

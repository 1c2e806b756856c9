"""GatedKAN: SwiGLU-style block of three Chebyshev KAN layers.

Drop-in for the reference ``metal_kans/gated_kan.py`` forward surface:
constructor (gated_kan.py:36-84: gate, up, down ChebyKAN built in that order,
``.half()`` when dtype is float16), ``forward`` (:86-138: gate = Gate(x),
up = Up(x), hidden = SiLU(gate) * up with the +-20 clip, out = Down(hidden),
(B, S, d) inputs flattened), ``to_int8`` / ``to_int4`` / ``to_ternary``
(:239-258), ``parameter_count``.  SwiGLU runs on the GPU for every dtype.

Unquantized blocks (and fp32 quantized ones, which run on their dequantized
weights as in the reference) keep gate, up, SwiGLU and down on the device: one
HIP graph per batch size with one host-to-device and one device-to-host copy
(``kans_gated_dense_*``).

Quantized path: a float16 block quantized with ``to_int8()`` / ``to_int4()``
(group 64) or ``to_ternary()`` (group 32) runs through the fused quantized block
(``_qengine.GatedEngine``): the packed weights are read from HBM once per
forward instead of being dequantized, and gate/up, SwiGLU and down run back to
back on the device (decode GEMVs up to 32 rows, the fused prefill kernels -- one
launch for gate|up with the SwiGLU epilogue, one for down -- above).  A block
whose three layers were bf16 when quantized takes the same kernels with gate,
up, hidden and the result rounded to bf16.  Other cases use the three layers.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import device
from ._engine import DT_F16, DT_F32, from_bf16_bits
from ._layer import device_layer_handle
from .cheby_kan import ChebyKAN
from .quantization import to_int4, to_int8, to_ternary
from ._qengine import GatedEngine, fused_batch_ok, packed_format


class GatedKAN:
    """out = Down(SiLU(Gate(x)) * Up(x)) with Chebyshev KAN projections."""

    def __init__(self, d_model: int, d_ffn: Optional[int] = None, degree: int = 4, has_base: bool = True,
                 has_bias: bool = False, dtype: np.dtype = np.float32):
        self.d_model = int(d_model)
        self.d_ffn = int(d_ffn if d_ffn is not None else 2 * d_model)
        self.degree = int(degree)
        self.has_base = bool(has_base)
        self.has_bias = bool(has_bias)
        self.dtype = np.dtype(dtype)
        self.gate_kan = ChebyKAN(self.d_model, self.d_ffn, degree=self.degree, bias=self.has_bias,
                                 use_base=self.has_base)
        self.up_kan = ChebyKAN(self.d_model, self.d_ffn, degree=self.degree, bias=self.has_bias,
                               use_base=self.has_base)
        self.down_kan = ChebyKAN(self.d_ffn, self.d_model, degree=self.degree, bias=self.has_bias,
                                 use_base=self.has_base)
        if self.dtype == np.float16:
            self.gate_kan.half()
            self.up_kan.half()
            self.down_kan.half()
        self._saved_x = None
        self._saved_gate = None
        self._saved_up = None
        self._saved_hidden = None

    def _packed_compute(self) -> Optional[str]:
        """"float16" for a float16 block, "bfloat16" when its three layers were bf16 when quantized and
        still compute in bf16, else None (no packed-weight path)."""
        if self.dtype == np.float16:
            return "float16"
        layers = (self.gate_kan, self.up_kan, self.down_kan)
        if all(getattr(k, "_quantized_from", None) == "bfloat16" and k._resolve_compute() == "bfloat16"
               for k in layers):
            return "bfloat16"
        return None

    def _decode_engine(self) -> Optional[GatedEngine]:
        """The fused quantized block, when this block's weights allow it (see module docstring)."""
        if self._packed_compute() is None:
            return None
        fmt = packed_format(self.gate_kan)
        if fmt is None or packed_format(self.up_kan) != fmt or packed_format(self.down_kan) != fmt:
            return None
        eng = self.__dict__.get("_qblock")
        if eng is None or eng.fmt != fmt or not eng.current(self):
            eng = GatedEngine(self, fmt)
            self._qblock = eng
        return eng

    def _block_compute(self) -> str:
        kinds = {k._resolve_compute() for k in (self.gate_kan, self.up_kan, self.down_kan)}
        if len(kinds) != 1:
            raise ValueError(f"gate, up and down disagree on compute dtype: {sorted(kinds)}")
        return kinds.pop()

    def _dense_forward(self, x_2d: np.ndarray) -> np.ndarray:
        """gate, up, SwiGLU and down on device activations: one HIP graph per batch size with one H2D and
        one D2H copy (kans_gated_dense_*), in the layers' compute dtype."""
        compute = self._block_compute()
        x_in = np.float16 if (compute == "float16" and x_2d.dtype == np.float16) else np.float32
        x2 = np.ascontiguousarray(x_2d, dtype=x_in)
        if x2.shape[1] != self.d_model:
            raise ValueError(f"Expected d_model={self.d_model}, got {x2.shape[1]}")
        layers = (self.gate_kan, self.up_kan, self.down_kan)
        handles = tuple(device_layer_handle(k, compute) for k in layers)
        lib = device.get_metal_bridge()
        # keyed on the handles' serial numbers and the compute dtype: a layer whose dtype changed got a new
        # handle, possibly at the old address, and the block must not keep the destroyed one
        key = (tuple(k._engine().serial for k in layers), compute)
        if self.__dict__.get("_dense_key") != key:
            self._drop_dense()
            h = ctypes.c_void_p()
            device.check(lib.kans_gated_dense_create(*handles, ctypes.byref(h)), "kans_gated_dense_create")
            self._dense_block = h
            self._dense_key = key
        B = x2.shape[0]
        x_dt = DT_F16 if x2.dtype == np.float16 else DT_F32
        if compute == "bfloat16":
            yb = np.empty((B, self.d_model), dtype=np.uint16)
            device.check(lib.kans_gated_dense_forward_host(self._dense_block, x2.ctypes.data, x_dt, yb.ctypes.data, B),
                         "kans_gated_dense_forward_host")
            return from_bf16_bits(yb).reshape(B, self.d_model)
        y = np.empty((B, self.d_model), dtype=np.float16 if compute == "float16" else np.float32)
        device.check(lib.kans_gated_dense_forward_host(self._dense_block, x2.ctypes.data, x_dt, y.ctypes.data, B),
                     "kans_gated_dense_forward_host")
        return y

    def _drop_dense(self) -> None:
        h = self.__dict__.pop("_dense_block", None)
        self.__dict__.pop("_dense_key", None)
        if h:
            try:
                device.load_library().kans_gated_dense_destroy(h)
            except Exception:
                pass

    def __del__(self):
        self._drop_dense()

    def forward(self, x: np.ndarray) -> np.ndarray:
        orig_shape = x.shape
        x_2d = x.reshape(-1, self.d_model) if len(orig_shape) > 2 else x
        self._saved_x = x_2d
        # the block runs gate, up and down on the device without the layers' own forward: clear what an
        # earlier direct call to a layer saved, so that a layer backward raises instead of differentiating
        # a stale input (the reference's forward saves them, gated_kan.py:97-132)
        for kan in (self.gate_kan, self.up_kan, self.down_kan):
            kan._saved_x = None
        if x_2d.shape[0] > 0:
            eng = self._decode_engine()
            if eng is not None and fused_batch_ok(eng.fmt, self.degree, x_2d.shape[0]):
                if self._packed_compute() == "bfloat16":
                    # the fp16 kernels, gate / up / hidden and the result rounded to bf16
                    out = eng.forward_host(np.asarray(x_2d, np.float32), "bfloat16", 2)
                else:
                    out = eng.forward_host(x_2d if x_2d.dtype == np.float16 else x_2d.astype(np.float32),
                                           np.float16, 1)
                self._saved_gate = self._saved_up = self._saved_hidden = None
                if len(orig_shape) > 2:
                    return out.reshape(*orig_shape[:-1], self.d_model)
                return out
        if x_2d.shape[0] == 0:
            out = self.down_kan(np.zeros((0, self.d_ffn), dtype=x_2d.dtype))
        else:
            out = self._dense_forward(x_2d)
        self._saved_gate = self._saved_up = self._saved_hidden = None
        if len(orig_shape) > 2:
            return out.reshape(*orig_shape[:-1], self.d_model)
        return out

    __call__ = forward

    def freeze_weights(self, frozen: bool = True) -> "GatedKAN":
        """Declare that gate, up and down's weight arrays will not be edited in place (inference loops): the
        forward then checks arrays above 4 MB by identity instead of hashing their bytes on every call (see
        ``KANLayerBase.freeze_weights``)."""
        for kan in (self.gate_kan, self.up_kan, self.down_kan):
            kan.freeze_weights(frozen)
        return self

    def to_int8(self, group_size: int = 64) -> "GatedKAN":
        for kan in (self.gate_kan, self.up_kan, self.down_kan):
            to_int8(kan, group_size=group_size)
        return self

    def to_int4(self, group_size: int = 64) -> "GatedKAN":
        for kan in (self.gate_kan, self.up_kan, self.down_kan):
            to_int4(kan, group_size=group_size)
        return self

    def to_ternary(self, group_size: int = 32) -> "GatedKAN":
        for kan in (self.gate_kan, self.up_kan, self.down_kan):
            to_ternary(kan, group_size=group_size)
        return self

    def parameter_count(self) -> int:
        count = 0
        for kan in (self.gate_kan, self.up_kan, self.down_kan):
            count += kan.w_cheby.size
            if kan.has_base and kan.w_base is not None:
                count += kan.w_base.size
            if kan.has_bias and kan.bias is not None:
                count += kan.bias.size
        return count

    def __repr__(self) -> str:
        return (f"GatedKAN(d_model={self.d_model}, d_ffn={self.d_ffn}, degree={self.degree}, "
                f"has_base={self.has_base}, params={self.parameter_count():,})")

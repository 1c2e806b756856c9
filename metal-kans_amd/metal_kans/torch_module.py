"""PyTorch modules on the fused gfx950 KAN kernels.

Drop-in for the reference ``metal_kans/torch_module.py`` (``TorchMetalKANLinear``,
``TorchMetalKAN``; torch_module.py:19-137): same constructor arguments, the
same NumPy layer built underneath (so ``torch.manual_seed`` / ``np.random.seed``
reproduce the reference weights) and the same ``weight`` / ``bias_param`` /
``metal_layer`` attributes.

Unlike the reference, which copies every tensor to a NumPy array and back
(torch_module.py:22-44), tensors that live on the GPU stay there:

* the forward hands ``data_ptr()`` of x, of the parameters and of a new output
  tensor to the library and runs the fused kernel on torch's current stream;
  the parameters are re-tiled on the device only when one of them changed (its
  pointer or version counter);
* the backward (Chebyshev basis) runs the fused backward kernels on device
  arrays and returns gradients for x **and** for the parameters (``weight``,
  ``base_weight``, ``bias_param``); the reference returns dx only.

CPU tensors take the NumPy layer path, as in the reference.  The base-branch
weight is a trainable parameter here (``base_weight``).  Backward through the
RBF and B-spline bases is not implemented (raises ``NotImplementedError``),
and the ReLU-KAN family is outside this build.
"""
from __future__ import annotations

import ctypes
from typing import Any, Optional, Sequence

import numpy as np
import torch
import torch.nn as nn

from . import device
from ._engine import DT_BF16, DT_F16, DT_F32
from .bspline_kan import BSplineKAN
from .cheby_kan import ChebyKAN
from .fast_kan import FastKAN

_DT = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}


def _aligned_rows(x: torch.Tensor, d_in: int, align: int) -> tuple:
    """x as a contiguous [B, ldx] device buffer: ldx = round_up(d_in, 8) elements and the base
    pointer ``align``-byte aligned, as the fused kernel reads 16-byte rows (padding columns are
    ignored by the kernel)."""
    ldx = (d_in + 7) // 8 * 8
    x = x.contiguous()
    if ldx == d_in and x.data_ptr() % align == 0:
        return x, ldx
    xp = torch.empty((x.shape[0], ldx), dtype=x.dtype, device=x.device)
    xp[:, :d_in] = x
    return xp, ldx


class _KANFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, base_weight, bias, module):
        ctx.module = module
        ctx.save_for_backward(x, weight, base_weight, bias)
        if x.is_cuda:
            return module._forward_device(x, weight, base_weight, bias)
        return module._forward_host(x)

    @staticmethod
    def backward(ctx, grad_out):
        module = ctx.module
        x, weight, base_weight, bias = ctx.saved_tensors
        if module.basis != "cheby":
            raise NotImplementedError("backward is implemented for the Chebyshev basis only "
                                      "(the fused Chebyshev backward kernels)")
        if x.is_cuda:
            dx, dw, dwb, db = module._backward_device(grad_out, x, weight, base_weight, bias)
        else:
            dx, dw, dwb, db = module._backward_host(grad_out, x)
        return dx, dw, dwb, db, None


class TorchMetalKANLinear(nn.Module):
    """KAN layer as a torch module, on the fused gfx950 kernels.

    Args:
        in_features: input dimension
        out_features: output dimension
        basis: "cheby", "fastkan" / "rbf" or "bspline" / "kan"
        degree: Chebyshev coefficients, RBF centres or B-spline grid size
        bias: learnable additive bias
        use_base: SiLU base branch (Chebyshev and RBF)
    """

    def __init__(self, in_features: int, out_features: int, basis: str = "cheby", degree: int = 4,
                 bias: bool = True, use_base: bool = True):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.basis = basis.lower()
        self.degree = degree
        self.use_bias = bias
        if self.basis == "cheby":
            self.metal_layer = ChebyKAN(in_features, out_features, degree=degree, bias=bias, use_base=use_base)
            self._K = degree
        elif self.basis in ("fastkan", "rbf"):
            self.basis = "rbf"
            self.metal_layer = FastKAN(in_features, out_features, num_centers=degree, bias=bias, use_base=use_base)
            self._K = degree
        elif self.basis in ("bspline", "kan"):
            self.basis = "bspline"
            self.metal_layer = BSplineKAN(in_features, out_features, grid_size=degree, bias=bias)
            self._K = degree + 3
        elif self.basis in ("relu", "relukan"):
            raise ValueError("the ReLU-KAN family is outside this build (Chebyshev, RBF, B-spline only)")
        else:
            raise ValueError(f"Unsupported basis type: {basis}")
        L = self.metal_layer
        self.weight = nn.Parameter(torch.from_numpy(getattr(L, L._weight_attr).astype(np.float32).copy()))
        self.base_weight = (nn.Parameter(torch.from_numpy(L.w_base.astype(np.float32).copy()))
                            if L.has_base else None)
        self.bias_param = (nn.Parameter(torch.from_numpy(L.bias.astype(np.float32).copy()))
                           if L.has_bias else None)

    # ---- host (NumPy layer) path ---------------------------------------------
    def _sync_to_metal(self) -> None:
        """Copies the parameters into the NumPy layer (the reference's _sync_to_metal)."""
        L = self.metal_layer
        setattr(L, L._weight_attr, self.weight.detach().cpu().float().numpy().copy())
        if self.base_weight is not None:
            L.w_base = self.base_weight.detach().cpu().float().numpy().copy()
        if self.bias_param is not None:
            L.bias = self.bias_param.detach().cpu().float().numpy().copy()
        L._compute = "float32"

    def _forward_host(self, x: torch.Tensor) -> torch.Tensor:
        self._sync_to_metal()
        y = self.metal_layer.forward(x.detach().contiguous().numpy().astype(np.float32))
        return torch.from_numpy(np.ascontiguousarray(y)).to(dtype=x.dtype)

    def _backward_host(self, grad_out: torch.Tensor, x: torch.Tensor):
        L = self.metal_layer
        self._sync_to_metal()
        L.forward(x.detach().contiguous().numpy().astype(np.float32))  # sets the saved input
        dx = L.backward(grad_out.detach().contiguous().numpy().astype(np.float32))
        to = lambda a, p: None if p is None else torch.from_numpy(np.ascontiguousarray(a)).to(p.dtype)  # noqa: E731
        return (torch.from_numpy(np.ascontiguousarray(dx)).to(x.dtype), to(L.grad_w_cheby, self.weight),
                to(L.grad_w_base, self.base_weight), to(L.grad_bias, self.bias_param))

    # ---- device path ---------------------------------------------------------
    def _forward_device(self, x: torch.Tensor, weight, base_weight, bias) -> torch.Tensor:
        pdt = weight.dtype
        if pdt not in _DT:
            raise TypeError(f"unsupported parameter dtype {pdt}")
        if x.dtype not in (pdt, torch.float32):
            raise TypeError(f"input dtype {x.dtype} does not match the module dtype {pdt}")
        for p in (weight, base_weight, bias):
            if p is not None and (p.dtype != pdt or not p.is_cuda):
                raise TypeError("all parameters must share one dtype and live on the GPU")
        dt = _DT[pdt]
        params = [weight.contiguous()]
        params += [base_weight.contiguous() if base_weight is not None else None,
                   bias.contiguous() if bias is not None else None]
        key = tuple((p.data_ptr(), p._version) if p is not None else None for p in params)
        eng = self.metal_layer._engine()
        if eng.dt != dt or eng.dev_key != key or eng.snaps is not None:
            torch.cuda.current_stream(x.device).synchronize()   # parameter writes done before the re-tiling
        eng.prepare_device(dt, params[0].data_ptr(), params[1].data_ptr() if params[1] is not None else None,
                           params[2].data_ptr() if params[2] is not None else None,
                           self.metal_layer._basis_params(), key)
        shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        if x2.shape[0] == 0:
            return torch.empty((*shape[:-1], self.out_features), dtype=x.dtype, device=x.device)
        xdt = dt if x.dtype == pdt else DT_F32
        xa, ldx = _aligned_rows(x2, self.in_features, 32)
        y = torch.empty((x2.shape[0], self.out_features), dtype=x.dtype, device=x.device)
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        lib = device.get_metal_bridge()
        device.check(lib.kans_layer_forward_ex(eng.handle, ctypes.c_void_p(xa.data_ptr()), xdt, ldx,
                                               ctypes.c_void_p(y.data_ptr()), xdt, self.out_features,
                                               x2.shape[0], stream), "kans_layer_forward_ex")
        return y.reshape(*shape[:-1], self.out_features)

    def _backward_device(self, grad_out, x, weight, base_weight, bias):
        B = grad_out.numel() // self.out_features
        f32 = lambda t: None if t is None else t.detach().float().contiguous()  # noqa: E731
        dy = f32(grad_out).reshape(B, self.out_features)
        xs = f32(x).reshape(B, self.in_features)
        W, Wb = f32(weight), f32(base_weight)
        dev = x.device
        dW = torch.empty_like(W)
        dWb = torch.empty_like(Wb) if Wb is not None else None
        db = torch.empty((self.out_features,), dtype=torch.float32, device=dev) if bias is not None else None
        dX = torch.empty((B, self.in_features), dtype=torch.float32, device=dev)
        ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        device.check(device.get_metal_bridge().kans_cheby_backward(
            ptr(dy), ptr(xs), ptr(W), ptr(Wb), ptr(dW), ptr(dWb), ptr(db), ptr(dX), B, self.in_features,
            self.out_features, self._K, int(Wb is not None), int(db is not None), stream), "kans_cheby_backward")
        cast = lambda g, p: None if g is None else g.to(p.dtype)  # noqa: E731
        return (dX.reshape(x.shape).to(x.dtype), cast(dW, weight), cast(dWb, base_weight), cast(db, bias))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _KANFunction.apply(x, self.weight, self.base_weight, self.bias_param, self)


class TorchMetalKAN(nn.Module):
    """Multi-layer network of ``TorchMetalKANLinear`` (torch_module.py:117-137)."""

    def __init__(self, layers_hidden: Sequence[int], basis: str = "cheby", degree: int = 4, bias: bool = True):
        super().__init__()
        self.layers = nn.ModuleList([
            TorchMetalKANLinear(in_f, out_f, basis=basis, degree=degree, bias=bias)
            for in_f, out_f in zip(layers_hidden, layers_hidden[1:])
        ])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x)
        return x

"""Device management and the ctypes binding of the MI355X HIP library.

Mirrors the reference's ``metal_kans/device.py`` (``get_metal_bridge``,
``is_metal_available``, ``set_async``, ``sync``; device.py:17-494): the shared
library is loaded once into a module global, every export gets explicit
``argtypes``/``restype``, and initialisation failure raises ``RuntimeError``.

Differences by design: the library (``libkans_hip.so``) is built ahead of time
for gfx950 (``python metal-kans_amd/build.py``) instead of on import, and there
is no CPU fallback -- without the library or a gfx950 GPU the layers raise.
``KANS_LIB_PATH`` selects another build of the library.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("KANS_LIB_PATH") or os.path.join(_HERE, "libkans_hip.so")

_lib: Optional[ctypes.CDLL] = None
_initialised = False

c_int = ctypes.c_int
c_long = ctypes.c_long
c_longlong = ctypes.c_longlong
c_float = ctypes.c_float
c_double = ctypes.c_double
c_size_t = ctypes.c_size_t
c_void_p = ctypes.c_void_p
c_char_p = ctypes.c_char_p
P = c_void_p

# name -> (restype, argtypes).  One entry per symbol declared in include/kans_hip.h.
SIGNATURES = {
    "kans_last_error": (c_char_p, []),
    # reference-named surface (device.py:64-474 of the reference)
    "metal_kan_init": (c_int, [c_char_p]),
    "metal_kan_set_async": (c_int, [c_int]),
    "metal_kan_sync": (c_int, []),
    "metal_kan_cheby_forward": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "metal_kan_cheby_forward_fp16": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "metal_kan_cheby_forward_bf16": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "metal_kan_fastkan_forward": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float, c_int, c_int]),
    "metal_kan_fastkan_forward_fp16": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float, c_int, c_int]),
    "metal_kan_fastkan_forward_bf16": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float, c_int, c_int]),
    "metal_kan_bspline_forward": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "metal_kan_bspline_forward_fp16": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "metal_kan_bspline_forward_bf16": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "benchmark_metal_cheby": (c_double, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "benchmark_metal_fastkan": (c_double, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float, c_int, c_int,
                                           c_int, c_int]),
    "benchmark_metal_bspline": (c_double, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                           c_int, c_int]),
    "metal_kan_quantize_int8": (c_int, [P, P, P, P, c_int, c_int]),
    "metal_kan_quantize_int4": (c_int, [P, P, P, P, c_int, c_int]),
    "metal_kan_dequantize_int8": (c_int, [P, P, P, P, c_int, c_int]),
    "metal_kan_dequantize_int4": (c_int, [P, P, P, P, c_int, c_int]),
    "metal_kan_quantize_ternary": (c_int, [P, P, P, c_int, c_int, c_int]),
    "metal_kan_dequantize_ternary": (c_int, [P, P, P, c_int, c_int, c_int]),
    "metal_kan_swiglu_forward": (c_int, [P, P, P, c_int]),
    "metal_kan_forward_ternary_cheby": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int]),
    # device-resident layer API
    "kans_init": (c_int, []),
    "kans_stream": (c_void_p, []),
    "kans_synchronize": (c_int, []),
    "kans_layer_create": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(c_void_p)]),
    "kans_layer_destroy": (c_int, [P]),
    "kans_layer_set_rbf": (c_int, [P, P, c_float]),
    "kans_layer_set_bspline": (c_int, [P, c_int, c_float, c_float]),
    "kans_layer_set_tiling": (c_int, [P, c_int, c_int, c_int]),
    "kans_layer_set_wave_groups": (c_int, [P, c_int]),
    "kans_layer_set_block_pairs": (c_int, [P, c_int]),
    "kans_layer_describe": (c_int, [P, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
    "kans_layer_kernel": (c_int, [P, c_int, ctypes.c_char_p, c_int]),
    "kans_layer_kernel_ex": (c_int, [P, c_int, c_int, c_int, ctypes.c_char_p, c_int]),
    "kans_cheby_backward": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, P]),
    "metal_kan_cheby_backward_fused": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "metal_kan_cheby_backward": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "kans_layer_load_weights": (c_int, [P, P, P, P]),
    "kans_layer_load_weights_device": (c_int, [P, P, P, P]),
    "kans_layer_load_weights_f32": (c_int, [P, P, P, P]),
    "kans_layer_forward": (c_int, [P, P, c_long, P, c_long, c_int, P]),
    "kans_layer_forward_ex": (c_int, [P, P, c_int, c_long, P, c_int, c_long, c_int, P]),
    "kans_layer_forward_host": (c_int, [P, P, P, c_int]),
    "kans_layer_forward_host_ex": (c_int, [P, P, c_int, P, c_int]),
    "kans_layer_time_forward": (c_int, [P, P, c_long, P, c_long, c_int, c_int, c_int, ctypes.POINTER(c_float)]),
    "kans_layer_time_window": (c_int, [P, P, c_long, P, c_long, c_int, c_float, c_int, ctypes.POINTER(c_float),
                                       ctypes.POINTER(c_float)]),
    "metal_kan_chain_pipeline_cheby": (c_int, [P, P, c_int, c_int, P, P, P, P, P]),
    "kans_chain_create": (c_int, [P, c_int, ctypes.POINTER(c_void_p)]),
    "kans_chain_destroy": (c_int, [P]),
    "kans_chain_forward_host": (c_int, [P, P, P, c_int]),
    "kans_chain_forward_host_ex": (c_int, [P, P, c_int, P, c_int]),
    "kans_chain_forward": (c_int, [P, P, c_long, P, c_long, c_int, P]),
    "kans_chain_time": (c_int, [P, c_int, c_int, c_int, c_int, ctypes.POINTER(c_float)]),
    "kans_dequantize_affine_device": (c_int, [P, P, P, P, c_long, c_int, c_int, P]),
    "kans_dequantize_ternary_device": (c_int, [P, P, P, c_int, c_int, c_int, P]),
    "kans_dev_malloc": (c_int, [ctypes.POINTER(c_void_p), c_size_t]),
    "kans_dev_free": (c_int, [P]),
    "kans_memcpy_h2d": (c_int, [P, P, c_size_t]),
    "kans_memcpy_d2h": (c_int, [P, P, c_size_t]),
    "kans_copy_device": (c_int, [P, P, c_size_t, P]),
    # quantized decode path
    "kans_qlayer_create_int4": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, P, P, P, P, P, P, P, c_int, P]),
    "kans_qlayer_create_int8": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, P, P, P, P, P, P, P, c_int, P]),
    "kans_qlayer_create_ternary": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, P, P, P, P, P, c_int, P]),
    "kans_qlayer_destroy": (c_int, [P]),
    "kans_qlayer_set_rbf": (c_int, [P, P, ctypes.c_float]),
    "kans_qlayer_set_bspline": (c_int, [P, c_int, ctypes.c_float, ctypes.c_float]),
    "kans_qlayer_fused": (c_int, [P, c_int]),
    "kans_qlayer_forward": (c_int, [P, P, c_int, c_long, P, c_int, c_long, c_int, P]),
    "kans_qlayer_forward_host": (c_int, [P, P, c_int, P, c_int, c_int]),
    "kans_gated_create": (c_int, [P, P, P, P]),
    "kans_gated_destroy": (c_int, [P]),
    "kans_gated_forward": (c_int, [P, P, c_int, c_long, P, c_int, c_long, c_int, c_int, P]),
    "kans_gated_forward_noalloc": (c_int, [P, P, c_int, c_long, P, c_int, c_long, c_int, c_int, P]),
    "kans_gated_dense_create": (c_int, [P, P, P, P]),
    "kans_gated_dense_destroy": (c_int, [P]),
    "kans_gated_dense_forward": (c_int, [P, P, c_int, c_long, P, c_long, c_int, P]),
    "kans_gated_dense_forward_host": (c_int, [P, P, c_int, P, c_int]),
    "kans_gated_dense_time": (c_int, [P, c_int, c_int, c_int, c_int, ctypes.POINTER(c_float)]),
    "kans_gated_forward_host": (c_int, [P, P, c_int, P, c_int, c_int, c_int]),
    "kans_gated_time": (c_int, [P, P, c_int, P, c_int, c_int, c_int, c_int, c_int, P]),
    "kans_gated_time_rotate": (c_int, [P, c_int, P, c_int, P, c_int, c_int, c_int, c_int, P]),
    "kans_gated_time_step": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, P]),
    "kans_gated_stream_bytes": (c_longlong, [P, c_int]),
    "kans_gated_set_fused_swiglu": (c_int, [c_int]),
    "kans_decode_set_pre_basis": (c_int, [c_int]),
    "kans_decode_set_weight_loads": (c_int, [c_int]),
    "kans_prefill_set_block_pairs": (c_int, [c_int]),
    "kans_mfma_ceiling": (c_int, [c_int, P, P, c_int, P]),
    "kans_stream_ceiling": (c_int, [P, c_size_t, P]),
}


class KansError(RuntimeError):
    """A library call returned a negative code."""


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and attach argtypes (no device access)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"HIP library not found at {path}; build it with `python metal-kans_amd/build.py` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    lib = load_library()
    msg = lib.kans_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(code: int, what: str = "") -> int:
    if code < 0:
        raise KansError(f"{what or 'kans call'} failed with code {code}: {last_error()}")
    return code


def get_metal_bridge() -> ctypes.CDLL:
    """Return the loaded library, initialising the GPU once (reference: device.py:31-482).

    Raises RuntimeError when the library is missing or no gfx950 device is
    visible (the reference raises on non-Darwin platforms, device.py:40-41).
    """
    global _initialised
    lib = load_library()
    if not _initialised:
        code = lib.metal_kan_init(None)
        if code != 0:
            raise RuntimeError(f"MI355X KAN initialization failed with code {code}: {last_error()}")
        _initialised = True
    return lib


def is_metal_available() -> bool:
    """True when the library loads and a gfx950 GPU is visible (name kept for drop-in use)."""
    try:
        return get_metal_bridge() is not None
    except Exception:
        return False


is_gpu_available = is_metal_available


def set_async(enabled: bool = True) -> None:
    """Enable or disable deferred completion of host forwards (reference: device.py:485-488)."""
    get_metal_bridge().metal_kan_set_async(1 if enabled else 0)


def sync() -> None:
    """Wait for pending GPU work and land deferred results (reference: device.py:491-494)."""
    check(get_metal_bridge().metal_kan_sync(), "metal_kan_sync")

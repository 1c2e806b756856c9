"""C-ABI and host-side checks that need no GPU.

* libkans_hip.so loads and exports every function declared in include/kans_hip.h,
  and the ctypes table in metal_kans/device.py binds each of them;
* the native host quantizers (metal_kan_quantize_*) reproduce the reference's
  NumPy-fallback quantizers bit-for-bit (golden vectors + the oracle on random
  data with exact .5 ties);
* argument validation returns negative codes before any HIP call.
"""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import kan_oracle as O

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "kans_hip.h")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if not n.startswith("typedef")))


@pytest.fixture(scope="module")
def lib():
    from metal_kans import device
    return device.load_library()


def test_header_symbols_exported_and_bound(lib):
    from metal_kans import device
    names = declared_functions()
    assert len(names) >= 40, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in kans_hip.h but not exported"
        assert n in device.SIGNATURES, f"{n} has no ctypes signature in device.py"
    assert set(device.SIGNATURES) <= set(names), set(device.SIGNATURES) - set(names)


def _q_native(lib, w, bits, gs):
    out_f, in_f = w.shape
    pad = (gs - in_f % gs) % gs
    padded = np.ascontiguousarray(np.pad(w, ((0, 0), (0, pad))) if pad else w, dtype=np.float32)
    ng = padded.size // gs
    q = np.empty((ng, gs if bits == 8 else gs // 2), dtype=np.uint8)
    s = np.empty((ng, 1), np.float32)
    b = np.empty((ng, 1), np.float32)
    fn = lib.metal_kan_quantize_int8 if bits == 8 else lib.metal_kan_quantize_int4
    assert fn(padded.ctypes.data, q.ctypes.data, s.ctypes.data, b.ctypes.data, ng, gs) == 0
    return q, s, b


def _t_native(lib, w, gs):
    w = np.ascontiguousarray(w, dtype=np.float32)
    D, Kd = w.shape
    p = np.zeros((D, (Kd + 15) // 16), np.uint32)
    s = np.zeros((D, (Kd + gs - 1) // gs), np.float32)
    assert lib.metal_kan_quantize_ternary(w.ctypes.data, p.ctypes.data, s.ctypes.data, D, Kd, gs) == 0
    return p, s


def test_native_quantizers_match_golden(lib):
    g = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in g.files})
    for n in names:
        w = g[f"{n}__w"]
        for bits, gs in ((8, 64), (4, 64), (8, 32), (4, 32)):
            t = f"{n}__int{bits}_g{gs}"
            q, s, b = _q_native(lib, w, bits, gs)
            np.testing.assert_array_equal(q, g[t + "__q"], err_msg=t)
            np.testing.assert_array_equal(s.view(np.uint32), g[t + "__s"].view(np.uint32), err_msg=t)
            np.testing.assert_array_equal(b.view(np.uint32), g[t + "__b"].view(np.uint32), err_msg=t)
        for gs in (32, 16, 64):
            t = f"{n}__tern_g{gs}"
            p, s = _t_native(lib, w, gs)
            np.testing.assert_array_equal(p, g[t + "__p"], err_msg=t)
            np.testing.assert_array_equal(s.view(np.uint32), g[t + "__s"].view(np.uint32), err_msg=t)


@pytest.mark.parametrize("shape,gs", [((64, 640), 64), ((33, 1000), 32), ((5, 129), 64)])
def test_native_quantizers_match_oracle_random(lib, shape, gs):
    rng = np.random.default_rng(shape[1])
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    w[0, :16] = np.float32(0.125) * rng.integers(-8, 8, 16)  # coarse grid: exact ties
    for bits in (8, 4):
        q, s, b = _q_native(lib, w, bits, gs)
        q2, s2, b2, _ = O.quantize_affine(w, bits, gs)
        np.testing.assert_array_equal(q, q2)
        np.testing.assert_array_equal(s.view(np.uint32), s2.view(np.uint32))
        np.testing.assert_array_equal(b.view(np.uint32), b2.view(np.uint32))
    p, s = _t_native(lib, w, gs)
    p2, s2 = O.quantize_ternary(w, gs)
    np.testing.assert_array_equal(p, p2)
    np.testing.assert_array_equal(s.view(np.uint32), s2.view(np.uint32))


def test_argument_validation_without_gpu(lib):
    null = None
    assert lib.metal_kan_quantize_int8(null, null, null, null, 1, 64) == -1
    assert lib.metal_kan_quantize_int4(null, null, null, null, 1, 63) == -1
    assert lib.metal_kan_quantize_ternary(null, null, null, 0, 0, 32) == -1
    h = ctypes.c_void_p()
    assert lib.kans_layer_create(7, 0, 4, 4, 4, 1, 1, ctypes.byref(h)) == -1      # bad basis
    assert lib.kans_layer_create(0, 0, 4, 4, 0, 1, 1, ctypes.byref(h)) == -1      # K = 0
    assert lib.kans_layer_create(0, 0, 4, 4, 33, 1, 1, ctypes.byref(h)) == -1     # K > 32
    assert b"K=" in lib.kans_last_error()
    x = np.zeros(4, np.float32)
    assert lib.metal_kan_cheby_forward(x.ctypes.data, null, null, null, x.ctypes.data, 1, 2, 2, 2, 0, 0) == -1
    assert lib.metal_kan_bspline_forward(x.ctypes.data, x.ctypes.data, null, null, null, x.ctypes.data,
                                         1, 2, 2, 5, 3, 0, 0) == -1   # null grid params


def test_no_device_is_a_clean_error(lib):
    from metal_kans import device
    if device.is_metal_available():
        pytest.skip("a GPU is visible")
    assert lib.metal_kan_init(None) == -1
    with pytest.raises(RuntimeError):
        device.get_metal_bridge()
    import metal_kans as mk
    layer = mk.ChebyKAN(4, 3, degree=3)
    with pytest.raises(RuntimeError):
        layer(np.zeros((2, 4), np.float32))


def test_layer_constructors_match_reference_rng_order():
    """np.random.seed reproduces the reference draws: w_<basis> first, then w_base (cheby_kan.py:39-42)."""
    import metal_kans as mk
    np.random.seed(42)
    layer = mk.ChebyKAN(8, 16, degree=4)
    np.random.seed(42)
    b = 1 / np.sqrt(8)
    w = np.random.uniform(-b, b, (16, 32)).astype(np.float32)
    wb = np.random.uniform(-b, b, (16, 8)).astype(np.float32)
    np.testing.assert_array_equal(layer.w_cheby, w)
    np.testing.assert_array_equal(layer.w_base, wb)
    f = mk.FastKAN(8, 16, num_centers=8, grid_range=(-2, 2))
    assert f.inv_denominator == pytest.approx(49 / 32)
    s = mk.BSplineKAN(8, 16, grid_size=5)
    assert s.w_spline.shape == (16, 64) and s.grid_params.dtype == np.float32
    assert mk.KAN is mk.BSplineKAN

"""GPU parity of the fused Chebyshev backward (run on an MI355X).

Oracle: ``oracle.kan_oracle.cheby_backward`` in float64 (pinned in tests/test_oracle.py against
finite differences, the closed form of T'_k and brute-force loops).  Bar: fp32, max|g - g_ref| /
max|g_ref| <= 1e-4 for every gradient.  Also re-runs the reference's own backward tests:
test_optimizations.py:59-100 (fused vs unfused entry point) and test_training.py:20-71 (finite
differences through the layer API).
"""
import ctypes

import numpy as np
import pytest

from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu


def run_host(lib, fn, dY, X, W, Wb, has_bias):
    B, D_in = X.shape
    D_out = dY.shape[1]
    K = W.shape[1] // D_in
    dW = np.full_like(W, np.nan)
    dWb = np.full_like(Wb, np.nan) if Wb is not None else None
    db = np.full(D_out, np.nan, np.float32) if has_bias else None
    dX = np.full_like(X, np.nan)
    ptr = lambda a: a.ctypes.data if a is not None else None  # noqa: E731
    rc = fn(ptr(dY), ptr(X), ptr(W), ptr(Wb), ptr(dW), ptr(dWb), ptr(db), ptr(dX), B, D_in, D_out, K,
            int(Wb is not None), int(has_bias))
    assert rc == 0, lib.kans_last_error()
    return dW, dWb, db, dX


def case(seed, B, D_in, D_out, K, base, bias, x_lo=-1.3, x_hi=1.3):
    rng = np.random.default_rng(seed)
    X = rng.uniform(x_lo, x_hi, (B, D_in)).astype(np.float32)
    W = rng.normal(0, 1 / np.sqrt(D_in * K), (D_out, D_in * K)).astype(np.float32)
    Wb = rng.normal(0, 1 / np.sqrt(D_in), (D_out, D_in)).astype(np.float32) if base else None
    dY = rng.normal(0, 1, (B, D_out)).astype(np.float32)
    return dY, X, W, Wb


def check(got, ref, tol=1e-4):
    for g, r, name in zip(got, ref, ("dW", "dW_base", "dbias", "dX")):
        if r is None:
            assert g is None
            continue
        e = O.rel_err(g, r)
        assert np.isfinite(g).all(), name
        assert e <= tol, f"{name}: rel err {e:.2e}"


SHAPES = [(1, 3, 5), (37, 24, 70), (130, 33, 64), (300, 16, 9)]


@pytest.mark.parametrize("K", [1, 2, 4, 9, 16, 32])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("base,bias", [(True, True), (False, False), (True, False)])
def test_backward_matches_oracle(gpu, K, shape, base, bias):
    B, D_in, D_out = shape
    dY, X, W, Wb = case(K * 100 + B, B, D_in, D_out, K, base, bias)
    got = run_host(gpu, gpu.metal_kan_cheby_backward_fused, dY, X, W, Wb, bias)
    check(got, O.cheby_backward(dY, X, W, Wb, bias))


def test_backward_device_entry_larger_shape(gpu):
    """kans_cheby_backward on device buffers at 2048 x 512 -> 256, K = 9 (base, bias)."""
    lib = gpu
    B, D_in, D_out, K = 2048, 512, 256, 9
    dY, X, W, Wb = case(77, B, D_in, D_out, K, True, True)
    ref = O.cheby_backward(dY, X, W, Wb, True)
    bufs = {}
    try:
        for name, a in (("dY", dY), ("X", X), ("W", W), ("Wb", Wb)):
            p = ctypes.c_void_p()
            assert lib.kans_dev_malloc(ctypes.byref(p), a.nbytes) == 0
            assert lib.kans_memcpy_h2d(p, a.ctypes.data, a.nbytes) == 0
            bufs[name] = p
        outs = {"dW": np.empty_like(W), "dWb": np.empty_like(Wb), "db": np.empty(D_out, np.float32),
                "dX": np.empty_like(X)}
        for name, a in outs.items():
            p = ctypes.c_void_p()
            assert lib.kans_dev_malloc(ctypes.byref(p), a.nbytes) == 0
            bufs[name] = p
        assert lib.kans_cheby_backward(bufs["dY"], bufs["X"], bufs["W"], bufs["Wb"], bufs["dW"], bufs["dWb"],
                                       bufs["db"], bufs["dX"], B, D_in, D_out, K, 1, 1, None) == 0, \
            lib.kans_last_error()
        assert lib.kans_synchronize() == 0
        for name, a in outs.items():
            assert lib.kans_memcpy_d2h(a.ctypes.data, bufs[name], a.nbytes) == 0
        check((outs["dW"], outs["dWb"], outs["db"], outs["dX"]), ref)
    finally:
        for p in bufs.values():
            lib.kans_dev_free(p)


def test_backward_rejects_bad_arguments(gpu):
    lib = gpu
    dY, X, W, Wb = case(1, 4, 3, 2, 4, True, True)
    z = np.zeros(64, np.float32)
    p = z.ctypes.data
    assert lib.metal_kan_cheby_backward_fused(p, p, p, None, p, None, None, p, 4, 3, 2, 4, 1, 0) < 0  # base, no W_base
    assert lib.metal_kan_cheby_backward_fused(p, p, p, p, p, p, None, p, 4, 3, 2, 4, 1, 1) < 0  # bias, no dbias
    assert lib.metal_kan_cheby_backward_fused(p, p, p, p, p, p, p, p, 0, 3, 2, 4, 1, 1) < 0     # B = 0
    assert lib.metal_kan_cheby_backward_fused(p, p, p, p, p, p, p, p, 4, 3, 2, 33, 1, 1) < 0    # K > 32


def test_reference_fused_vs_unfused(gpu):
    """test_optimizations.py:59-100: both entry points, B=32, 16 -> 8, degree 4, base and bias."""
    lib = gpu
    B, D_in, D_out, degree = 32, 16, 8, 4
    np.random.seed(123)
    dY = np.random.randn(B, D_out).astype(np.float32)
    X = np.random.uniform(-0.9, 0.9, (B, D_in)).astype(np.float32)
    W = np.random.randn(D_out, D_in * degree).astype(np.float32)
    Wb = np.random.randn(D_out, D_in).astype(np.float32)
    a = run_host(lib, lib.metal_kan_cheby_backward, dY, X, W, Wb, True)
    b = run_host(lib, lib.metal_kan_cheby_backward_fused, dY, X, W, Wb, True)
    assert np.max(np.abs(a[0] - b[0])) < 1e-4
    assert np.max(np.abs(a[3] - b[3])) < 1e-4
    assert np.max(np.abs(a[2] - b[2])) < 1e-5
    check(b, O.cheby_backward(dY, X, W, Wb, True))


def test_reference_layer_gradient_numerical_check(gpu):
    """test_training.py:20-71: ChebyKAN(3 -> 2, degree 4) dX and dW against central differences of
    the GPU forward (eps 1e-4, relative error < 1e-3), then zero_grad."""
    import metal_kans as mk
    np.random.seed(42)
    B, D_in, D_out, deg = 4, 3, 2, 4
    layer = mk.ChebyKAN(D_in, D_out, degree=deg, bias=True, use_base=True)
    X = np.random.uniform(-0.8, 0.8, (B, D_in)).astype(np.float32)
    dY = np.random.randn(B, D_out).astype(np.float32)
    layer(X)
    dX = layer.backward(dY)
    eps = 1e-4
    dX_num = np.zeros_like(X)
    for i in range(B):
        for j in range(D_in):
            Xp, Xm = X.copy(), X.copy()
            Xp[i, j] += eps
            Xm[i, j] -= eps
            dX_num[i, j] = (np.sum(layer(Xp) * dY) - np.sum(layer(Xm) * dY)) / (2 * eps)
    rel = np.linalg.norm(dX - dX_num) / (np.linalg.norm(dX) + np.linalg.norm(dX_num) + 1e-7)
    assert rel < 1e-3
    layer(X)
    layer.backward(dY)
    gW = layer.grad_w_cheby.copy()
    dW_num = np.zeros_like(layer.w_cheby)
    for i in range(layer.w_cheby.shape[0]):
        for j in range(layer.w_cheby.shape[1]):
            w0 = layer.w_cheby[i, j]
            layer.w_cheby[i, j] = w0 + eps
            lp = np.sum(layer(X) * dY)
            layer.w_cheby[i, j] = w0 - eps
            lm = np.sum(layer(X) * dY)
            layer.w_cheby[i, j] = w0
            dW_num[i, j] = (lp - lm) / (2 * eps)
    rel = np.linalg.norm(gW - dW_num) / (np.linalg.norm(gW) + np.linalg.norm(dW_num) + 1e-7)
    assert rel < 1e-3
    assert layer.grad_bias.shape == (D_out,) and layer.grad_w_base.shape == (D_out, D_in)
    layer.zero_grad()
    assert not layer.grad_w_cheby.any() and not layer.grad_bias.any()


def test_layer_backward_shapes_and_dtypes(gpu):
    """Layer API: 3-D input, no base / bias, and a half layer differentiated in fp32."""
    import metal_kans as mk
    np.random.seed(7)
    layer = mk.ChebyKAN(24, 10, degree=5, bias=False, use_base=False)
    x = np.random.uniform(-1.2, 1.2, (2, 7, 24)).astype(np.float32)
    y = layer(x)
    dY = np.random.randn(*y.shape).astype(np.float32)
    dX = layer.backward(dY)
    assert dX.shape == x.shape
    assert layer.grad_w_base.shape == (1,) and layer.grad_bias.shape == (1,)
    ref = O.cheby_backward(dY.reshape(14, 10), x.reshape(14, 24), layer.w_cheby, None, False)
    assert O.rel_err(layer.grad_w_cheby, ref[0]) <= 1e-4
    assert O.rel_err(dX.reshape(14, 24), ref[3]) <= 1e-4

    h = mk.ChebyKAN(16, 8, degree=4).half()
    xh = np.random.uniform(-1, 1, (9, 16)).astype(np.float16)
    h(xh)
    dYh = np.random.randn(9, 8).astype(np.float32)
    dXh = h.backward(dYh)
    ref = O.cheby_backward(dYh, xh.astype(np.float32), h.w_cheby.astype(np.float32),
                           h.w_base.astype(np.float32), True)
    assert O.rel_err(dXh, ref[3]) <= 1e-4 and O.rel_err(h.grad_w_cheby, ref[0]) <= 1e-4

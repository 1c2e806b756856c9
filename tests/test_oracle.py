"""Pins the CPU oracle (oracle/kan_oracle.py) before it is trusted as the checker.

Each oracle function is checked against something it does not restate:
closed forms (T_k(cos t) = cos(k t)), invariants (B-spline partition of unity),
an independent textbook algorithm (Cox-de Boor recursion), brute-force loops,
special cases that reduce to plain linear algebra, and golden vectors written
by the reference's own NumPy-fallback quantizers (tests/golden/).
"""
import os

import math

import numpy as np
import pytest

from oracle import kan_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


# ---------------------------------------------------------------- Chebyshev
def test_cheby_cosine_identity():
    th = np.linspace(0, np.pi, 257)
    phi = O.cheby_basis(np.cos(th), 14)
    for k in range(14):
        np.testing.assert_allclose(phi[:, k], np.cos(k * th), atol=1e-12)


def test_cheby_endpoints_and_clamp():
    phi = O.cheby_basis(np.array([1.0, -1.0, 3.0, -7.5]), 10)
    k = np.arange(10)
    np.testing.assert_array_equal(phi[0], np.ones(10))
    np.testing.assert_array_equal(phi[1], (-1.0) ** k)
    np.testing.assert_array_equal(phi[2], np.ones(10))       # clamp, not extrapolation
    np.testing.assert_array_equal(phi[3], (-1.0) ** k)


def test_cheby_K_means_coefficients():
    assert O.cheby_basis(np.zeros(3), 9).shape == (3, 9)   # degree 8 -> 9 coefficients


# ---------------------------------------------------------------- RBF
def test_rbf_grid_and_cfg3_constant():
    grid, inv_den = O.rbf_grid((-2.0, 2.0), 8)
    np.testing.assert_allclose(grid, np.linspace(-2, 2, 8), rtol=0, atol=1e-7)
    assert inv_den == pytest.approx(49.0 / 32.0, rel=1e-15)   # h = 4/7 -> 1/(2h^2)


def test_rbf_peak_and_symmetry():
    grid, inv_den = O.rbf_grid((-1.0, 1.0), 6)
    phi = O.rbf_basis(grid.astype(np.float64), grid, inv_den)
    np.testing.assert_allclose(np.diag(phi), 1.0)
    d = 0.37
    a = O.rbf_basis(grid + d, grid, inv_den)
    b = O.rbf_basis(grid - d, grid, inv_den)
    np.testing.assert_allclose(np.diag(a), np.diag(b))
    np.testing.assert_allclose(np.diag(a), np.exp(-d * d * inv_den))


# ---------------------------------------------------------------- B-spline
def _cox_de_boor(x, knots, p):
    """Textbook Cox-de Boor recursion for all B-splines of degree p on `knots`."""
    n = len(knots) - 1
    N = np.array([1.0 if knots[j] <= x < knots[j + 1] else 0.0 for j in range(n)])
    for d in range(1, p + 1):
        M = np.zeros(n - d)
        for j in range(n - d):
            a = 0.0 if knots[j + d] == knots[j] else (x - knots[j]) / (knots[j + d] - knots[j]) * N[j]
            b = 0.0 if knots[j + d + 1] == knots[j + 1] else (knots[j + d + 1] - x) / (knots[j + d + 1] - knots[j + 1]) * N[j + 1]
            M[j] = a + b
        N = M
    return N


@pytest.mark.parametrize("G,lo,hi", [(5, -1.0, 1.0), (3, -2.0, 0.5), (8, 0.0, 4.0)])
def test_bspline_matches_cox_de_boor_inside_grid(G, lo, hi):
    params = O.bspline_params(G, (lo, hi))
    h = (hi - lo) / G
    knots = lo + (np.arange(G + 7) - 3) * h          # 3 extension knots each side
    xs = np.linspace(lo, hi, 401)[:-1]
    phi = O.bspline_basis(xs, G, float(params[0]), float(params[1]))
    for x, row in zip(xs, phi):
        ref = _cox_de_boor(x, knots, 3)
        assert ref.shape == (G + 3,)
        np.testing.assert_allclose(row, ref, atol=1e-6)


def test_bspline_partition_knots_and_saturation():
    G = 5
    p = O.bspline_params(G)
    xs = np.linspace(-3, 3, 1001)
    phi = O.bspline_basis(xs, G, float(p[0]), float(p[1]))
    np.testing.assert_allclose(phi.sum(-1), 1.0, atol=1e-12)
    assert (np.count_nonzero(phi, axis=-1) <= 4).all()
    at_knot = O.bspline_basis(np.array([-1.0 + 2 * 0.4]), G, float(p[0]), float(p[1]))[0]  # pos = 2 exactly
    np.testing.assert_allclose(at_knot[2:5], [1 / 6, 2 / 3, 1 / 6])
    left = O.bspline_basis(np.array([-1.0, -1.1, -9.0]), G, float(p[0]), float(p[1]))
    np.testing.assert_array_equal(left[1], left[0])
    np.testing.assert_array_equal(left[2], left[0])
    right = O.bspline_basis(np.array([1.0, 1.2, 50.0]), G, float(p[0]), float(p[1]))
    np.testing.assert_allclose(right[1], right[0], atol=1e-15)
    np.testing.assert_allclose(right[2], right[0], atol=1e-15)
    np.testing.assert_allclose(right[0][-3:], [1 / 6, 2 / 3, 1 / 6])


# ---------------------------------------------------------------- SiLU
def test_silu_identities():
    x = np.linspace(-30, 30, 601)
    s = O.silu(x)
    np.testing.assert_allclose(s - O.silu(-x), x, atol=1e-12)
    assert O.silu(np.array(0.0)) == 0.0
    np.testing.assert_allclose(O.silu(np.array([40.0])), [40.0])


# ---------------------------------------------------------------- contraction
def _brute(kind, x, W, Wb, bias, params):
    B, D_in = x.shape
    D_out = W.shape[0]
    phi = O.basis(kind, x, params)
    K = phi.shape[-1]
    y = np.zeros((B, D_out))
    for b in range(B):
        for o in range(D_out):
            acc = 0.0 if bias is None else float(bias[o])
            for i in range(D_in):
                if Wb is not None:
                    acc += x[b, i] / (1 + np.exp(-x[b, i])) * Wb[o, i]
                for k in range(K):
                    acc += phi[b, i, k] * W[o, i * K + k]
            y[b, o] = acc
    return y


def _params(kind, K):
    if kind == "cheby":
        return {"K": K}
    if kind == "rbf":
        grid, inv = O.rbf_grid((-1.5, 1.5), K)
        return {"grid": grid, "inv_den": inv}
    G = K - 3
    p = O.bspline_params(G)
    return {"G": G, "grid_min": float(p[0]), "inv_h": float(p[1])}


@pytest.mark.parametrize("kind,K", [("cheby", 3), ("cheby", 9), ("rbf", 5), ("bspline", 8)])
@pytest.mark.parametrize("base,bias", [(True, True), (False, False), (True, False)])
def test_forward_matches_brute_force(kind, K, base, bias):
    rng = np.random.default_rng(7)
    B, D_in, D_out = 3, 4, 5
    x = rng.uniform(-1.3, 1.3, (B, D_in))
    W = rng.normal(size=(D_out, D_in * K))
    Wb = rng.normal(size=(D_out, D_in)) if base else None
    bb = rng.normal(size=D_out) if bias else None
    p = _params(kind, K)
    np.testing.assert_allclose(O.kan_forward(kind, x, W, Wb, bb, p), _brute(kind, x, W, Wb, bb, p), atol=1e-12)


def test_forward_special_cases():
    rng = np.random.default_rng(3)
    x = rng.uniform(-2, 2, (6, 7))
    W1 = rng.normal(size=(4, 7))
    Wb = rng.normal(size=(4, 7))
    bias = rng.normal(size=4)
    # K = 1 Chebyshev: phi_0 = 1 -> y = bias + silu(x) Wb^T + row sums of W
    y = O.kan_forward("cheby", x, W1, Wb, bias, {"K": 1})
    np.testing.assert_allclose(y, bias + (x / (1 + np.exp(-x))) @ Wb.T + W1.sum(1), atol=1e-12)
    # W = 0 -> pure base branch
    y0 = O.kan_forward("cheby", x, np.zeros((4, 21)), Wb, None, {"K": 3})
    np.testing.assert_allclose(y0, (x / (1 + np.exp(-x))) @ Wb.T, atol=1e-12)
    # linearity in W
    Wa, Wc = rng.normal(size=(4, 21)), rng.normal(size=(4, 21))
    ya = O.kan_forward("cheby", x, Wa, None, None, {"K": 3})
    yc = O.kan_forward("cheby", x, Wc, None, None, {"K": 3})
    np.testing.assert_allclose(O.kan_forward("cheby", x, 2 * Wa - Wc, None, None, {"K": 3}), 2 * ya - yc,
                               atol=1e-10)


def test_fp32_stage_mode_close_to_float64():
    rng = np.random.default_rng(11)
    x = np.tanh(rng.uniform(-1, 1, (256, 64))).astype(np.float32)
    W = rng.normal(0, (1 / (64 * 9)) ** 0.5, (64, 64 * 9)).astype(np.float32)
    Wb = rng.uniform(-1 / 8, 1 / 8, (64, 64)).astype(np.float32)
    y32 = O.kan_forward("cheby", x, W, Wb, None, {"K": 9}, acc=np.float32)
    y64 = O.kan_forward("cheby", x, W, Wb, None, {"K": 9})
    assert y32.dtype == np.float32
    assert O.rel_err(y32, y64) < 1e-5


def test_gated_forward_against_affine_closed_form():
    # K = 2 without base: each layer is affine in clamp(x): y = sum_i W[o,2i] + W[:,1::2] @ clamp(x)
    rng = np.random.default_rng(5)
    d, h = 6, 10
    x = rng.uniform(-1.5, 1.5, (4, d))
    L = {n: {"W": rng.normal(size=(o, i * 2)), "K": 2} for n, (i, o) in
         {"g": (d, h), "u": (d, h), "d": (h, d)}.items()}

    def aff(Lw, z):
        W = Lw["W"]
        return W[:, 0::2].sum(1) + np.clip(z, -1, 1) @ W[:, 1::2].T
    g, u = aff(L["g"], x), aff(L["u"], x)
    # hidden = SiLU(g) * u, SiLU from the tanh identity x * sigmoid(x) = x/2 (1 + tanh(x/2)) (|g| < 20 here)
    assert np.abs(g).max() < 20
    hidden = 0.5 * g * (1.0 + np.tanh(0.5 * g)) * u
    np.testing.assert_allclose(O.gated_forward(x, L["g"], L["u"], L["d"]), aff(L["d"], hidden), atol=1e-10)


def _silu_tanh(x):
    """x * sigmoid(x) through the identity sigmoid(x) = (1 + tanh(x/2)) / 2, in float64."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(0.5 * x))


def test_silu_clipped_and_swiglu_closed_forms():
    """gated_kan.py:15-16 and fused_kan.metal:2284-2296 clip the exponent argument at +-20, not g itself:
    inside [-20, 20] both equal x * sigmoid(x) (tanh identity, independent of the exp form), beyond it the
    exact saturated forms g / (1 + e^-+20) hold, and SwiGLU(0, u) = 0.  A clip of g itself, a clip at another
    bound, a sign error in the exponent or a dropped factor u fails one of these."""
    rng = np.random.default_rng(11)
    g = np.concatenate([rng.uniform(-20, 20, 4000), [-20.0, -19.99, -1e-3, 0.0, 1e-3, 19.99, 20.0]])
    u = rng.normal(0, 2, g.size)
    # (absolute bar: 1 + tanh(x/2) cancels near x = -20, where the values are ~1e-7)
    np.testing.assert_allclose(O.silu_clipped(g), _silu_tanh(g), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(O.swiglu(g, u), (_silu_tanh(g) * u).astype(np.float32), rtol=3e-6, atol=1e-12)
    # beyond the clip: SiLU_clipped(g) = g / (1 + e^-20) for g > 20 and g / (1 + e^20) for g < -20
    hi = rng.uniform(20.001, 500, 500)
    lo = -rng.uniform(20.001, 500, 500)
    uu = rng.normal(0, 2, 500)
    np.testing.assert_allclose(O.silu_clipped(hi), hi / (1.0 + math.exp(-20.0)), rtol=1e-15)
    np.testing.assert_allclose(O.silu_clipped(lo), lo / (1.0 + math.exp(20.0)), rtol=1e-15)
    np.testing.assert_allclose(O.swiglu(hi, uu), (hi * uu / (1.0 + math.exp(-20.0))).astype(np.float32), rtol=3e-6)
    np.testing.assert_allclose(O.swiglu(lo, uu), (lo * uu / (1.0 + math.exp(20.0))).astype(np.float32), rtol=3e-6)
    # not the unclipped SiLU: at g = -30 the unclipped value is -30 e^-30 ~ -2.8e-12, the clipped one -6.2e-8
    assert abs(O.silu_clipped(np.array([-30.0]))[0] - (-30.0 / (1.0 + math.exp(20.0)))) < 1e-20
    assert O.swiglu(np.zeros(7), rng.normal(size=7)).tolist() == [0.0] * 7
    assert O.swiglu(np.array([3.0]), np.array([0.0]))[0] == 0.0


# ---------------------------------------------------------------- quantizers
def _golden():
    return np.load(GOLDEN)


def test_quantizers_match_reference_golden_vectors():
    g = _golden()
    names = sorted({k.split("__")[0] for k in g.files})
    assert len(names) >= 6
    for n in names:
        w = g[f"{n}__w"]
        for bits, gs in ((8, 64), (4, 64), (8, 32), (4, 32)):
            t = f"{n}__int{bits}_g{gs}"
            q, s, b, pin = O.quantize_affine(w, bits, gs)
            np.testing.assert_array_equal(q, g[t + "__q"], err_msg=t)
            np.testing.assert_array_equal(s.view(np.uint32), g[t + "__s"].view(np.uint32), err_msg=t)
            np.testing.assert_array_equal(b.view(np.uint32), g[t + "__b"].view(np.uint32), err_msg=t)
            dq = O.dequantize_affine(q, s, b, bits, gs, w.shape, pin)
            np.testing.assert_array_equal(dq.view(np.uint32), g[t + "__dq"].view(np.uint32), err_msg=t)
        for gs in (32, 16, 64):
            t = f"{n}__tern_g{gs}"
            p, s = O.quantize_ternary(w, gs)
            np.testing.assert_array_equal(p, g[t + "__p"], err_msg=t)
            np.testing.assert_array_equal(s.view(np.uint32), g[t + "__s"].view(np.uint32), err_msg=t)
            dq = O.dequantize_ternary(p, s, w.shape, gs)
            np.testing.assert_array_equal(dq.view(np.uint32), g[t + "__dq"].view(np.uint32), err_msg=t)


def test_quantizer_invariants():
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, (37, 150)).astype(np.float32)
    for bits in (8, 4):
        q, s, b, pin = O.quantize_affine(w, bits, 64)
        assert pin == 192 and q.shape[0] == 37 * 3
        dq = O.dequantize_affine(q, s, b, bits, 64, w.shape, pin)
        srow = np.repeat(s[:, 0], 64).reshape(37, 192)[:, :150]
        assert (np.abs(dq - w) <= srow / 2 * (1 + 1e-5) + 1e-8).all()
    p, s = O.quantize_ternary(w, 32)
    assert p.shape == (37, 10) and s.shape == (37, 5)
    dq = O.dequantize_ternary(p, s, w.shape, 32)
    sc = s[:, np.arange(150) // 32]
    assert np.isin(dq / sc, [-1.0, 0.0, 1.0]).all()
    c = O.ternary_codes(p, 150)
    assert c.max() <= 2
    # code of weight k sits at bits 2*(k%16) of word k//16
    assert ((p[:, 3] >> 10) & 3 == c[:, 53]).all()


def test_bf16_rounding():
    v = np.array([1.0, -2.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.inf], dtype=np.float32)
    bits = O.bf16_round(v)
    np.testing.assert_array_equal(bits, [0x3F80, 0xC000, 0x3F80, 0x3F82, 0x7F80])  # ties to even
    np.testing.assert_array_equal(O.bf16_to_f32(bits)[:2], [1.0, -2.0])


# ---- Chebyshev backward --------------------------------------------------------

def test_cheby_derivative_closed_form():
    """T'_k(cos t) = k sin(k t) / sin t inside (-1, 1); T'_k(+-1) = (+-1)^(k+1) k^2; 0 outside."""
    th = np.linspace(0.05, np.pi - 0.05, 37)
    d = O.cheby_basis_deriv(np.cos(th), 12)
    for k in range(12):
        np.testing.assert_allclose(d[:, k], k * np.sin(k * th) / np.sin(th), rtol=1e-10, atol=1e-10)
    e = O.cheby_basis_deriv(np.array([1.0, -1.0, 1.3, -2.0]), 9)
    ks = np.arange(9)
    np.testing.assert_allclose(e[0], ks ** 2)
    np.testing.assert_allclose(e[1], (-1.0) ** (ks + 1) * ks ** 2)
    assert not e[2:].any()


def test_silu_derivative_matches_difference_quotient():
    x = np.linspace(-8, 8, 41)
    h = 1e-6
    np.testing.assert_allclose(O.silu_deriv(x), (O.silu(x + h) - O.silu(x - h)) / (2 * h), rtol=1e-7, atol=1e-9)


@pytest.mark.parametrize("base,bias", [(True, True), (False, False)])
def test_cheby_backward_matches_finite_differences(base, bias):
    """Every gradient of L = sum(y * dY) against central differences of the float64 forward, with
    inputs inside (-1, 1) and outside it (where the clamp makes the basis flat)."""
    rng = np.random.default_rng(5)
    B, Di, Do, K = 5, 4, 3, 6
    x = rng.uniform(-0.95, 0.95, (B, Di))
    x[0, 1], x[3, 2] = 1.4, -1.7
    W = rng.normal(0, 1, (Do, Di * K))
    Wb = rng.normal(0, 1, (Do, Di)) if base else None
    bv = rng.normal(0, 1, Do) if bias else None
    dY = rng.normal(0, 1, (B, Do))
    dW, dWb, db, dX = O.cheby_backward(dY, x, W, Wb, bias)

    def loss(x_, W_, Wb_, b_):
        return float(np.sum(O.kan_forward("cheby", x_, W_, Wb_, b_, {"K": K}) * dY))

    def num(arr, f):
        g = np.zeros_like(arr)
        h = 1e-6
        for idx in np.ndindex(arr.shape):
            a, b = arr.copy(), arr.copy()
            a[idx] += h
            b[idx] -= h
            g[idx] = (f(a) - f(b)) / (2 * h)
        return g

    np.testing.assert_allclose(dX, num(x, lambda a: loss(a, W, Wb, bv)), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(dW, num(W, lambda a: loss(x, a, Wb, bv)), rtol=1e-6, atol=1e-7)
    if base:
        np.testing.assert_allclose(dWb, num(Wb, lambda a: loss(x, W, a, bv)), rtol=1e-6, atol=1e-7)
    else:
        assert dWb is None
    if bias:
        np.testing.assert_allclose(db, num(bv, lambda a: loss(x, W, Wb, a)), rtol=1e-6, atol=1e-7)
    else:
        assert db is None


def test_cheby_backward_brute_force_loops():
    rng = np.random.default_rng(9)
    B, Di, Do, K = 3, 2, 2, 4
    x = rng.uniform(-1, 1, (B, Di))
    W = rng.normal(0, 1, (Do, Di * K))
    Wb = rng.normal(0, 1, (Do, Di))
    dY = rng.normal(0, 1, (B, Do))
    dW, dWb, db, dX = O.cheby_backward(dY, x, W, Wb, True)
    for o in range(Do):
        for i in range(Di):
            for k in range(K):
                ref = sum(dY[b, o] * np.cos(k * np.arccos(x[b, i])) for b in range(B))
                assert abs(dW[o, i * K + k] - ref) < 1e-12
            assert abs(dWb[o, i] - sum(dY[b, o] * x[b, i] / (1 + np.exp(-x[b, i])) for b in range(B))) < 1e-12
        assert abs(db[o] - dY[:, o].sum()) < 1e-12

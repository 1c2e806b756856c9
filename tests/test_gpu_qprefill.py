"""GPU parity of the fused quantized prefill path (batches above 32 rows).

The quantized forward of the reference is forward(x, dequant(quant(W))) in fp32
(quantization.py:152-188); the fused kernel decodes the packed codes into fp16
MFMA operands on the GPU.  Each case is checked two ways against the float64
oracle on the oracle-dequantized weights:

* at the 16-bit bar, max|y - y_ref| / max|y_ref| <= 2e-2;
* tightly (<= 2e-3) against the oracle that rounds exactly the operands the
  kernel feeds its MFMAs to fp16 (the dequantized weights, T_k(clamp x) and
  SiLU(x)): a wrong code, nibble order, group parameter, slot or feature index
  moves the output by far more than that.

Shapes cover ragged D_in (the last feature block is partly padding, inside an
affine group), ragged D_out (N-tile padding), several feature blocks per
split, feature splits (few row tiles, a split size rounded up to the kernel's
phase period), K = 1 .. 9 (Chebyshev: at K in {3, 5, 6, 7, 9} the 8 codes of a
chunk straddle quantization groups, and where they straddle depends on the
feature block and lane half), {3, 4, 5, 7, 8} (Gaussian RBF on uniform centres)
and {4, 8} (cubic B-spline), with and without the base / bias branches, fp16
and fp32 inputs and fp32 / fp16 / bf16 outputs.  The same RBF / B-spline layers
are checked through the decode GEMVs (B <= 32, every K).
"""
import ctypes

import numpy as np
import pytest

from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu

DT = {"float32": 0, "float16": 1, "bfloat16": 2}


def quantize(lib, fmt, W):
    """Packed arrays of W (D_out x kd) in the reference format (native host quantizers), and the
    oracle's dequantization of them."""
    rows, kd = W.shape
    if fmt in ("int4", "int8"):
        bits = 4 if fmt == "int4" else 8
        pad = (kd + 63) // 64 * 64
        Wp = np.zeros((rows, pad), np.float32)
        Wp[:, :kd] = W
        ng = rows * pad // 64
        q = np.empty((ng, 64 * bits // 8), np.uint8)
        s = np.empty(ng, np.float32)
        b = np.empty(ng, np.float32)
        fn = lib.metal_kan_quantize_int4 if bits == 4 else lib.metal_kan_quantize_int8
        assert fn(Wp.ctypes.data, q.ctypes.data, s.ctypes.data, b.ctypes.data, ng, 64) == 0
        dq = O.dequantize_affine(q, s.reshape(-1, 1), b.reshape(-1, 1), bits, 64, W.shape, pad)
        return (q, s, b), dq
    p = np.zeros((rows, (kd + 15) // 16), np.uint32)
    s = np.zeros((rows, (kd + 31) // 32), np.float32)
    assert lib.metal_kan_quantize_ternary(W.ctypes.data, p.ctypes.data, s.ctypes.data, rows, kd, 32) == 0
    return (p, s), O.dequantize_ternary(p, s, W.shape, 32)


def basis_params(kind, K, rng=None, uniform=True):
    """Oracle parameters of a layer of `kind` with K basis functions: RBF centres on [-1.5, 1.5] (uniform, or
    moved off the grid) with the reference's inv_den = 1 / (2 h^2); B-spline G = K - 3 on [-1, 1]."""
    if kind == "cheby":
        return {"K": K}
    if kind == "rbf":
        c = np.linspace(-1.5, 1.5, K).astype(np.float32)
        if not uniform:
            c = c + np.linspace(0.0, 0.4, K).astype(np.float32) ** 2
        h = 3.0 / (K - 1)
        return {"grid": c.astype(np.float64), "inv_den": float(np.float32(1.0 / (2.0 * h * h)))}
    G = K - 3
    return {"G": G, "grid_min": -1.0, "inv_h": float(np.float32(G / 2.0))}


def set_basis(lib, h, kind, params):
    if kind == "rbf":
        c = np.ascontiguousarray(params["grid"], np.float32)
        assert lib.kans_qlayer_set_rbf(h, c.ctypes.data, params["inv_den"]) == 0, lib.kans_last_error()
    elif kind == "bspline":
        assert lib.kans_qlayer_set_bspline(h, params["G"], params["grid_min"], params["inv_h"]) == 0, \
            lib.kans_last_error()


def make_qlayer(lib, fmt, d_in, d_out, K, base, bias, seed, kind="cheby", uniform=True):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.5 / np.sqrt(d_in * K), (d_out, d_in * K)).astype(np.float32)
    Wb = rng.normal(0, 0.5 / np.sqrt(d_in), (d_out, d_in)).astype(np.float32)
    bv = rng.normal(0, 0.1, d_out).astype(np.float32)
    pw, dw = quantize(lib, fmt, W)
    pb, db = quantize(lib, fmt, Wb) if base else ((None,) * len(pw), None)
    h = ctypes.c_void_p()
    ptr = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    if fmt == "ternary":
        rc = lib.kans_qlayer_create_ternary(d_in, d_out, K, int(base), int(bias), 32, ptr(pw[0]), ptr(pw[1]),
                                            ptr(pb[0]), ptr(pb[1]), ptr(bv) if bias else None, 0, ctypes.byref(h))
    else:
        fn = lib.kans_qlayer_create_int4 if fmt == "int4" else lib.kans_qlayer_create_int8
        rc = fn(d_in, d_out, K, int(base), int(bias), 64, *[ptr(a) for a in pw], *[ptr(a) for a in pb],
                ptr(bv) if bias else None, 0, ctypes.byref(h))
    assert rc == 0, lib.kans_last_error()
    params = basis_params(kind, K, uniform=uniform)
    set_basis(lib, h, kind, params)
    return h, {"W": dw, "W_base": db, "bias": bv if bias else None, "K": K, "kind": kind, "params": params}


def oracle(L, x):
    """float64 forward on the original inputs and the dequantized weights."""
    return O.kan_forward(L.get("kind", "cheby"), x, L["W"], L["W_base"], L["bias"], L.get("params", {"K": L["K"]}))


def _oracle_rounded(L, x, weights16=True):
    """float64 forward with the fp16 MFMA operands: the basis values and SiLU(x) (evaluated from x in fp32,
    as the kernel does) rounded to fp16, and the dequantized weights rounded to fp16 too (prefill; the
    decode GEMVs apply the group parameters in fp32 and feed the weights exactly: weights16=False)."""
    r16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float64)  # noqa: E731
    rw = r16 if weights16 else (lambda a: np.asarray(a, np.float64))  # noqa: E731
    x32 = np.asarray(x, np.float32)
    B, d_in = x32.shape
    kind = L.get("kind", "cheby")
    phi = r16(O.basis(kind, x32, L.get("params", {"K": L["K"]}), np.float32).reshape(B, -1))
    y = phi @ rw(L["W"]).T
    if L["W_base"] is not None:
        y += r16(O.silu(x32)) @ rw(L["W_base"]).T
    if L["bias"] is not None:
        y += L["bias"].astype(np.float64)
    return y


def prefill_built(fmt, kind, K, base):
    """Whether the fused prefill kernel is built for a layer (the rest runs the dense kernels on the dequantized
    weights above 32 rows): not INT8 with the base branch at K = 7, nor INT8 B-spline at K = 8 (both spill)."""
    return not ((fmt == "int8" and K == 7 and base) or (fmt, kind, K) == ("int8", "bspline", 8))


def run(lib, h, x, d_out, y_dt="float32"):
    B = x.shape[0]
    xdt = DT["float16"] if x.dtype == np.float16 else DT["float32"]
    y = np.zeros((B, d_out), np.float32 if y_dt == "float32" else np.uint16)
    rc = lib.kans_qlayer_forward_host(h, x.ctypes.data, xdt, y.ctypes.data, DT[y_dt], B)
    assert rc == 0, lib.kans_last_error()
    if y_dt == "float16":
        return y.view(np.float16).astype(np.float32)
    if y_dt == "bfloat16":
        return O.bf16_to_f32(y)
    return y


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8, 9])
@pytest.mark.parametrize("base,bias", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("B,d_in,d_out", [(300, 100, 70), (40, 256, 300), (600, 48, 33), (64, 328, 40)])
def test_qlayer_prefill(gpu, fmt, K, base, bias, B, d_in, d_out):
    lib = gpu
    print(f"case {fmt} K={K} base={base} bias={bias} B={B} {d_in}->{d_out}", flush=True)
    h, L = make_qlayer(lib, fmt, d_in, d_out, K, base, bias, seed=B + d_in + K)
    try:
        x = np.random.default_rng(K * 7 + d_out).uniform(-1.3, 1.3, (B, d_in)).astype(np.float32)
        if not prefill_built(fmt, "cheby", K, base):
            assert lib.kans_qlayer_fused(h, B) == 0
            y = np.zeros((B, d_out), np.float32)
            assert lib.kans_qlayer_forward_host(h, x.ctypes.data, 0, y.ctypes.data, 0, B) == -5
            return
        assert lib.kans_qlayer_fused(h, B) == 1
        y = run(lib, h, x, d_out)
        e16 = O.rel_err(y, oracle(L, x))
        eop = O.rel_err(y, _oracle_rounded(L, x))
        print(f"  rel err {e16:.2e} (16-bit bar), {eop:.2e} vs operand-rounded oracle")
        assert e16 <= 2e-2 and eop <= 2e-3, (e16, eop)
        y2 = run(lib, h, x, d_out)
        np.testing.assert_array_equal(y.view(np.uint32), y2.view(np.uint32))
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
@pytest.mark.parametrize("base", [True, False])
@pytest.mark.parametrize("B,d_in,d_out", [(300, 100, 70), (40, 256, 300), (600, 16, 33), (64, 48, 40), (2000, 112, 256)])
def test_qlayer_prefill_block_pairs(gpu, fmt, base, B, d_in, d_out):
    """Chebyshev K = 4 prefill with two feature blocks per LDS stage against one block per stage, bit for
    bit (7, 16, 1, 3 and 7 feature blocks; the batch sizes give 1 to several feature splits), and the
    GatedKAN prefill block (column-paired gate|up launch, then down) the same way."""
    lib = gpu
    h, L = make_qlayer(lib, fmt, d_in, d_out, 4, base, True, seed=B + d_in)
    try:
        x = np.random.default_rng(d_out).uniform(-1.3, 1.3, (B, d_in)).astype(np.float32)
        assert lib.kans_qlayer_fused(h, B) == 1
        ys = []
        for on in (1, 0):
            prev = lib.kans_prefill_set_block_pairs(on)
            assert prev in (0, 1)
            ys.append(run(lib, h, x, d_out))
        assert lib.kans_prefill_set_block_pairs(1) == 0
        np.testing.assert_array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))
        assert O.rel_err(ys[0], oracle(L, x)) <= 2e-2
    finally:
        lib.kans_prefill_set_block_pairs(1)
        lib.kans_qlayer_destroy(h)
    if (B, d_in) == (300, 100):
        blk, layers, specs = make_block(lib, fmt, 96, 200, K=4, bias=base, seed=3)
        try:
            xb = np.random.default_rng(1).normal(0, 1, (B, 96)).astype(np.float16)
            outs = []
            for on in (1, 0):
                lib.kans_prefill_set_block_pairs(on)
                y = np.zeros((B, 96), np.float16)
                assert lib.kans_gated_forward_host(blk, xb.ctypes.data, 1, y.ctypes.data, 1, B, 1) == 0
                outs.append(y)
            np.testing.assert_array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
            assert O.rel_err(outs[0].astype(np.float32), gated_oracle(specs, xb.astype(np.float64), 1)) <= 2e-2
        finally:
            lib.kans_prefill_set_block_pairs(1)
            lib.kans_gated_destroy(blk)
            for hnd in layers:
                lib.kans_qlayer_destroy(hnd)
    assert lib.kans_prefill_set_block_pairs(2) < 0


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
@pytest.mark.parametrize("kind,K", [("rbf", 8), ("rbf", 4), ("rbf", 3), ("rbf", 5), ("rbf", 7), ("bspline", 8),
                                    ("bspline", 4)])
@pytest.mark.parametrize("base,bias", [(True, True), (False, False)])
@pytest.mark.parametrize("B,d_in,d_out", [(300, 100, 70), (40, 256, 300)])
def test_qlayer_prefill_bases(gpu, fmt, kind, K, base, bias, B, d_in, d_out):
    """Quantized FastKAN (uniform centres: the RBF recurrence) and BSplineKAN layers on the fused prefill
    kernel (K = 8: B-spline basis table), inputs beyond the grid included."""
    lib = gpu
    print(f"case {kind} K={K} {fmt} base={base} bias={bias} B={B} {d_in}->{d_out}", flush=True)
    h, L = make_qlayer(lib, fmt, d_in, d_out, K, base, bias, seed=B + d_in + 3 * K, kind=kind)
    try:
        x = np.random.default_rng(K + d_out).uniform(-2.0, 2.0, (B, d_in)).astype(np.float32)
        if not prefill_built(fmt, kind, K, base):
            assert lib.kans_qlayer_fused(h, B) == 0
            y = np.zeros((B, d_out), np.float32)
            assert lib.kans_qlayer_forward_host(h, x.ctypes.data, 0, y.ctypes.data, 0, B) == -5
            return
        assert lib.kans_qlayer_fused(h, B) == 1
        y = run(lib, h, x, d_out)
        e16 = O.rel_err(y, oracle(L, x))
        eop = O.rel_err(y, _oracle_rounded(L, x))
        print(f"  rel err {e16:.2e} (16-bit bar), {eop:.2e} vs operand-rounded oracle")
        assert e16 <= 2e-2 and eop <= 2e-3, (e16, eop)
        y2 = run(lib, h, x, d_out)
        np.testing.assert_array_equal(y.view(np.uint32), y2.view(np.uint32))
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
@pytest.mark.parametrize("kind,K,uniform", [("rbf", 8, True), ("rbf", 5, False), ("bspline", 8, True),
                                            ("bspline", 6, True), ("cheby", 9, True)])
def test_qlayer_decode_bases(gpu, fmt, kind, K, uniform):
    """The decode GEMVs (B <= 32) for every basis and K: the activation basis (k_prep) evaluates the RBF and
    B-spline functions; against the oracle with the fp16 basis operands and exact weights."""
    lib = gpu
    h, L = make_qlayer(lib, fmt, 90, 70, K, True, True, seed=K + 11, kind=kind, uniform=uniform)
    try:
        for B in (1, 2, 5, 32):
            assert lib.kans_qlayer_fused(h, B) == 1
            x = np.random.default_rng(B + K).uniform(-2.0, 2.0, (B, 90)).astype(np.float32)
            y = run(lib, h, x, 70)
            e16 = O.rel_err(y, oracle(L, x))
            eop = O.rel_err(y, _oracle_rounded(L, x, weights16=False))
            print(f"{kind} K={K} {fmt} B={B}: rel err {e16:.2e}, {eop:.2e} vs fp16-basis oracle")
            assert e16 <= 2e-2 and eop <= 3e-4, (e16, eop)
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", ["int4", "ternary"])
@pytest.mark.parametrize("kind,K,uniform", [("rbf", 8, False), ("rbf", 9, True), ("bspline", 5, True),
                                            ("bspline", 6, True)])
def test_qlayer_prefill_bases_unsupported(gpu, fmt, kind, K, uniform):
    """RBF on non-uniform centres, RBF whose centres span more than the recurrence's guard (9 centres at
    the reference's inv_den = 1 / (2 h^2): scaled span 6.8 > 6) and B-spline K outside {4, 8}: decode
    batches run, larger ones report KANS_ERR_UNSUPPORTED (-5) and kans_qlayer_fused says so."""
    lib = gpu
    h, L = make_qlayer(lib, fmt, 40, 24, K, True, False, seed=2, kind=kind, uniform=uniform)
    try:
        assert lib.kans_qlayer_fused(h, 33) == 0 and lib.kans_qlayer_fused(h, 32) == 1
        x = np.random.default_rng(0).uniform(-1, 1, (33, 40)).astype(np.float32)
        y = np.zeros((33, 24), np.float32)
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, 0, y.ctypes.data, 0, 33) == -5
        assert O.rel_err(run(lib, h, x[:8], 24), _oracle_rounded(L, x[:8], weights16=False)) <= 3e-4
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
def test_qlayer_prefill_io_dtypes(gpu, fmt):
    """fp16 input used as given, fp32 input unrounded; fp16 / bf16 outputs are the fp32 output rounded."""
    lib = gpu
    h, L = make_qlayer(lib, fmt, 72, 96, 4, True, True, seed=5)
    try:
        x = np.random.default_rng(1).uniform(-1.1, 1.1, (130, 72)).astype(np.float32)
        y32 = run(lib, h, x, 96)
        assert O.rel_err(y32, _oracle_rounded(L, x)) <= 2e-3
        x16 = x.astype(np.float16)
        y16in = run(lib, h, x16, 96)
        assert O.rel_err(y16in, _oracle_rounded(L, x16.astype(np.float32))) <= 2e-3
        yh = run(lib, h, x, 96, "float16")
        np.testing.assert_array_equal(yh.astype(np.float16), y32.astype(np.float16))
        yb = run(lib, h, x, 96, "bfloat16")
        np.testing.assert_array_equal(O.bf16_round(yb), O.bf16_round(y32))
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
def test_qlayer_prefill_rejects_unsupported_K(gpu, fmt):
    """K = 10 (past the prefill kernel's 9): the layer decodes small batches (any K) and reports
    KANS_ERR_UNSUPPORTED (-5) for batches the prefill kernel would take."""
    lib = gpu
    rng = np.random.default_rng(0)
    h, L = make_qlayer(lib, fmt, 24, 40, 10, True, False, seed=1)
    try:
        x = rng.uniform(-1, 1, (33, 24)).astype(np.float32)
        y = np.zeros((33, 40), np.float32)
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, 0, y.ctypes.data, 0, 33) == -5
        y8 = run(lib, h, x[:8], 40)          # decode path: any K
        assert O.rel_err(y8, _oracle_rounded(L, x[:8])) <= 2e-3
        assert lib.kans_qlayer_fused(h, 33) == 0 and lib.kans_qlayer_fused(h, 8) == 1
    finally:
        lib.kans_qlayer_destroy(h)


# ---------------------------------------------------------------- GatedKAN block
def make_block(lib, fmt, d, hdim, K=4, bias=False, seed=0):
    layers, specs = [], []
    for i, (di, do) in enumerate(((d, hdim), (d, hdim), (hdim, d))):
        hnd, L = make_qlayer(lib, fmt, di, do, K, True, bias, seed=seed + 17 * i)
        layers.append(hnd)
        specs.append(L)
    blk = ctypes.c_void_p()
    assert lib.kans_gated_create(*layers, ctypes.byref(blk)) == 0
    return blk, layers, specs


def gated_oracle(specs, x, round16):
    """float64 oracle block on the dequantized weights; with round16 the gate / up / hidden activations are
    rounded to fp16 (1) or bf16 (2), as a 16-bit model stores them."""
    if round16 == 2:
        r = lambda a: O.bf16_to_f32(O.bf16_round(a.astype(np.float32))).astype(np.float64)  # noqa: E731
    else:
        r = (lambda a: a.astype(np.float16).astype(np.float64)) if round16 else (lambda a: a)  # noqa: E731
    f = lambda L, z: O.kan_forward("cheby", z, L["W"], L["W_base"], L["bias"], {"K": L["K"]})  # noqa: E731
    g, u = r(f(specs[0], x)), r(f(specs[1], x))
    return f(specs[2], r(O.silu_clipped(g) * u))


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
@pytest.mark.parametrize("B", [33, 300])
@pytest.mark.parametrize("d,hdim,bias,K", [(64, 160, False, 4), (96, 150, True, 4), (256, 520, False, 4),
                                           (96, 200, True, 8), (80, 200, False, 3), (96, 136, True, 9)])
@pytest.mark.parametrize("round16", [1, 0])
def test_gated_prefill(gpu, fmt, B, d, hdim, bias, K, round16):
    """gate|up in one launch (column-paired tile, SwiGLU epilogue), then down: against the oracle block."""
    lib = gpu
    print(f"case gated {fmt} B={B} d={d} h={hdim} bias={bias} K={K} round16={round16}", flush=True)
    blk, layers, specs = make_block(lib, fmt, d, hdim, K=K, bias=bias, seed=B + d)
    try:
        x = np.random.default_rng(B).normal(0, 1, (B, d)).astype(np.float16)
        y = np.zeros((B, d), np.float16)
        assert lib.kans_gated_forward_host(blk, x.ctypes.data, 1, y.ctypes.data, 1, B, round16) == 0, \
            lib.kans_last_error()
        ref = gated_oracle(specs, x.astype(np.float64), round16)
        e = O.rel_err(y.astype(np.float32), ref)
        print(f"  rel err {e:.2e}")
        assert np.isfinite(y.astype(np.float32)).all()
        assert e <= 2e-2
        y2 = np.zeros_like(y)
        assert lib.kans_gated_forward_host(blk, x.ctypes.data, 1, y2.ctypes.data, 1, B, round16) == 0
        np.testing.assert_array_equal(y.view(np.uint16), y2.view(np.uint16))
    finally:
        lib.kans_gated_destroy(blk)
        for hnd in layers:
            lib.kans_qlayer_destroy(hnd)


@pytest.mark.parametrize("fmt", ["int4", "ternary"])
def test_gated_decode_and_prefill_agree(gpu, fmt):
    """The same rows through the decode block (B = 32) and the prefill block (B = 33, one extra row) give the
    same outputs to fp16 rounding."""
    lib = gpu
    blk, layers, specs = make_block(lib, fmt, 128, 256, seed=9)
    try:
        x = np.random.default_rng(3).normal(0, 1, (33, 128)).astype(np.float16)
        yd = np.zeros((32, 128), np.float16)
        yp = np.zeros((33, 128), np.float16)
        assert lib.kans_gated_forward_host(blk, x.ctypes.data, 1, yd.ctypes.data, 1, 32, 1) == 0
        assert lib.kans_gated_forward_host(blk, x.ctypes.data, 1, yp.ctypes.data, 1, 33, 1) == 0
        assert O.rel_err(yp[:32].astype(np.float32), yd.astype(np.float32)) <= 5e-3
    finally:
        lib.kans_gated_destroy(blk)
        for hnd in layers:
            lib.kans_qlayer_destroy(hnd)


# ---------------------------------------------------------------- Python layer API
@pytest.mark.parametrize("quant", ["int8", "int4", "ternary"])
@pytest.mark.parametrize("degree", [4, 9, 3])
def test_python_quantized_fp16_layer_uses_packed_weights(gpu, quant, degree):
    """ChebyKAN(...).half().to_<quant>() keeps fp16 compute and runs on its packed weights at every batch
    (decode GEMV up to 32 rows, the prefill kernel above), including degrees whose code chunks straddle
    quantization groups (3, and the north star's 9)."""
    import metal_kans as mk
    np.random.seed(7)
    L = mk.ChebyKAN(80, 50, degree=degree)
    L.bias = np.random.normal(0, 0.1, 50).astype(np.float32)
    L.half()
    getattr(mk, f"to_{quant}")(L)
    spec = {"W": L.w_cheby, "W_base": L.w_base, "bias": L.bias.astype(np.float32), "K": degree}
    for B in (5, 300):
        x = np.random.default_rng(B).uniform(-1.1, 1.1, (B, 80)).astype(np.float32)
        y = L(x)
        assert y.dtype == np.float16 and y.shape == (B, 50)
        eng = L.__dict__.get("_qlayer_engine")
        assert eng is not None and eng.fused(B)
        assert O.rel_err(y.astype(np.float32), _oracle_rounded(spec, x)) <= 2e-3
        assert O.rel_err(y.astype(np.float32), oracle(spec, x)) <= 2e-2


@pytest.mark.parametrize("quant", ["int8", "int4", "ternary"])
@pytest.mark.parametrize("kind", ["cheby4", "cheby3", "rbf", "bspline"])
def test_python_quantized_bf16_layer_uses_packed_weights(gpu, quant, kind):
    """A bf16 layer quantized with to_<quant>() keeps bf16 compute and runs on its packed weights: the
    same kernels as the fp16 layer (fp16 basis values and decoded weights, fp32 accumulation) with the
    result rounded to bf16, at the decode (B = 5) and prefill (B = 300) sizes."""
    import metal_kans as mk
    from metal_kans._engine import from_bf16_bits, to_bf16_bits
    np.random.seed(11)
    if kind.startswith("cheby"):
        L = mk.ChebyKAN(80, 48, degree=int(kind[-1]))
    elif kind == "rbf":
        L = mk.FastKAN(80, 48, num_centers=8, grid_range=(-2.0, 2.0))
    else:
        L = mk.BSplineKAN(80, 48, grid_size=5)
    L.bias = np.random.normal(0, 0.1, 48).astype(np.float32)
    L.bfloat16()
    getattr(mk, f"to_{quant}")(L)
    if kind.startswith("cheby"):
        spec = {"W": L.w_cheby, "W_base": L.w_base, "bias": L.bias.astype(np.float32), "K": L.degree}
    else:
        params = ({"G": L.grid_size, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])}
                  if kind == "bspline" else {"grid": np.asarray(L.grid, np.float64), "inv_den": L.inv_denominator})
        spec = {"W": getattr(L, L._weight_attr), "W_base": L.w_base, "bias": L.bias.astype(np.float32),
                "K": L._num_basis(), "kind": L._basis, "params": params}
    for B in (5, 300):
        x = np.random.default_rng(B).normal(0, 1, (B, 80)).astype(np.float32)
        y = L(x)
        assert y.shape == (B, 48)
        eng = L.__dict__.get("_qlayer_engine")
        assert eng is not None
        if not eng.fused(B):
            assert B > 32 and (kind, quant) == ("bspline", "int8")  # not built: dequantized weights
        y32 = np.asarray(y, np.float32)
        assert np.array_equal(from_bf16_bits(to_bf16_bits(y32)).reshape(y32.shape), y32)  # bf16 values
        assert O.rel_err(y32, oracle(spec, x)) <= 2e-2
        if eng.fused(B):
            # against the fp16-operand forward: only the bf16 rounding of the output (2^-9 of |y|) apart
            assert O.rel_err(y32, _oracle_rounded(spec, x, weights16=B > 32)) <= 5e-3


@pytest.mark.parametrize("quant", ["int8", "int4", "ternary"])
def test_python_gatedkan_prefill(gpu, quant):
    """GatedKAN(dtype=float16).to_<quant>() at B > 32 runs the fused prefill block."""
    import metal_kans as mk
    np.random.seed(4)
    blk = mk.GatedKAN(d_model=96, d_ffn=200, degree=4, dtype=np.float16)
    getattr(blk, f"to_{quant}")()
    x = np.random.default_rng(2).normal(0, 1, (3, 50, 96)).astype(np.float16)
    out = blk(x)
    assert blk.__dict__.get("_qblock") is not None
    assert out.shape == (3, 50, 96) and out.dtype == np.float16
    specs = [{"W": k.w_cheby, "W_base": k.w_base, "bias": None, "K": 4}
             for k in (blk.gate_kan, blk.up_kan, blk.down_kan)]
    ref = gated_oracle(specs, x.reshape(-1, 96).astype(np.float64), 1)
    assert O.rel_err(out.reshape(-1, 96).astype(np.float32), ref) <= 2e-2


@pytest.mark.parametrize("quant", ["int8", "int4", "ternary"])
def test_python_gatedkan_bf16_packed(gpu, quant):
    """A GatedKAN whose layers were made bf16 before to_<quant>() runs the packed-weight block (decode at
    B = 6, prefill at B = 150) with gate, up, hidden and the result rounded to bf16."""
    import metal_kans as mk
    from metal_kans._engine import from_bf16_bits, to_bf16_bits
    np.random.seed(5)
    blk = mk.GatedKAN(d_model=96, d_ffn=200, degree=4)
    for k in (blk.gate_kan, blk.up_kan, blk.down_kan):
        k.bfloat16()
    getattr(blk, f"to_{quant}")()
    specs = [{"W": k.w_cheby, "W_base": k.w_base, "bias": None, "K": 4}
             for k in (blk.gate_kan, blk.up_kan, blk.down_kan)]
    for B in (6, 150):
        x = np.random.default_rng(B).normal(0, 1, (B, 96)).astype(np.float32)
        out = blk(x)
        assert blk.__dict__.get("_qblock") is not None
        assert out.shape == (B, 96) and out.dtype == np.float32
        assert np.array_equal(from_bf16_bits(to_bf16_bits(out)).reshape(out.shape), out)
        ref = gated_oracle(specs, x.astype(np.float64), 2)
        assert O.rel_err(out, ref) <= 2e-2


@pytest.mark.parametrize("quant", ["int8", "int4", "ternary"])
@pytest.mark.parametrize("kind", ["rbf", "bspline", "rbf5", "rbf9"])
def test_python_quantized_fastkan_bsplinekan(gpu, quant, kind):
    """FastKAN(...).half().to_<quant>() and BSplineKAN(...).half().to_<quant>() keep fp16 compute and run on
    their packed weights: the decode GEMVs at B = 5 and the prefill kernel at B = 300 (K = 8, and 5 centres);
    a 9-centre FastKAN (its centres span more than the RBF recurrence allows at the default width) takes
    the packed path at B = 5 and the dequantized weights at B = 300, equally correct."""
    import metal_kans as mk
    np.random.seed(8)
    if kind == "bspline":
        L = mk.BSplineKAN(72, 40, grid_size=5)
    else:
        L = mk.FastKAN(72, 40, num_centers={"rbf5": 5, "rbf9": 9}.get(kind, 8), grid_range=(-2.0, 2.0))
    L.bias = np.random.normal(0, 0.1, 40).astype(np.float32)
    L.half()
    getattr(mk, f"to_{quant}")(L)
    params = ({"G": L.grid_size, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])}
              if kind == "bspline" else {"grid": np.asarray(L.grid, np.float64), "inv_den": L.inv_denominator})
    spec = {"W": getattr(L, L._weight_attr), "W_base": L.w_base, "bias": L.bias.astype(np.float32),
            "K": L._num_basis(), "kind": L._basis, "params": params}
    for B in (5, 300):
        x = np.random.default_rng(B).normal(0, 1, (B, 72)).astype(np.float32)
        y = L(x)
        assert y.dtype == np.float16 and y.shape == (B, 40)
        eng = L.__dict__.get("_qlayer_engine")
        assert eng is not None
        assert eng.fused(B) == (B <= 32 or (kind != "rbf9" and (kind, quant) != ("bspline", "int8")))
        assert O.rel_err(y.astype(np.float32), oracle(spec, x)) <= 2e-2
        if eng.fused(B):
            # fp16 output: its own rounding is up to 2^-12 of |y| (the C-level tests above check fp32 outputs)
            ref = _oracle_rounded(spec, x, weights16=B > 32)
            assert O.rel_err(y.astype(np.float32), ref) <= (2e-3 if B > 32 else 1e-3)

"""GPU parity at the BASELINE.json configurations' own shapes (run on an MI355X).

Config 1 (256 x 64 -> 64) and config 3 (16384 x 1024 -> 1024) are covered by
test_gpu_parity.py (test_layer_parity, test_full_size_sampled_rows); this file
runs the others at their full sizes, where the tile choice, the feature splits
and the decode split-K differ from every smaller test:

* config 2: the fp16 ChebyKAN chain 784 -> 256 -> 256 -> 10 (K = 9) on the full
  B = 4096 batch, against the float64 oracle chain on every row;
* config 4: the cubic B-spline layer 8192 x 1024 -> 4096 (G = 5, base branch),
  fp32 and bf16, on a seeded sample of rows (rows are independent) plus a
  bitwise rerun;
* config 5: the GatedKAN block d_model = 4096, h = 11008, K = 4, INT4 (group 64)
  and ternary (group 32), plus INT8 (group 64), through the fused decode block
  at B = 1 and 32 and the fused prefill block at B = 8192 (sampled rows),
  against the float64 oracle block on the dequantized weights
  (quantization.py:168-171: quantized forward = forward on dequant(quant(W))).

Metric and tolerances as everywhere: max|y - y_ref| / max|y_ref| <= 1e-4 (fp32),
2e-2 (fp16 / bf16).
"""
import ctypes
import concurrent.futures as cf

import numpy as np
import pytest

from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu

TOL = {"float32": 1e-4, "float16": 2e-2, "bfloat16": 2e-2}


def normal_block(rng, std, n=1 << 24, pad=1 << 16):
    """n + pad float32 N(0, std^2) values shared by normal_matrix."""
    return rng.standard_normal(n + pad, dtype=np.float32) * np.float32(std)


def normal_matrix(rng, base, shape):
    """A float32 matrix of N(0, std^2) values: each row is a window of the shared normal block ``base``
    at a seeded random offset (drawing ~10^9 fresh normals would take most of a minute)."""
    rows, cols = shape
    n = base.size - cols
    offs = rng.integers(0, n, rows)
    out = np.empty(shape, np.float32)
    for r, o in enumerate(offs.tolist()):
        out[r] = base[o:o + cols]
    return out


# ---------------------------------------------------------------- config 2
def test_cfg2_chain_full_batch(gpu):
    """x ~ U(0,1) 4096 x 784, W_l ~ N(0, 1/(D_in*9)), fp16 via .half(), one HIP graph."""
    import metal_kans as mk
    rng = np.random.default_rng(1002)
    B = 4096
    x = rng.uniform(0, 1, (B, 784)).astype(np.float32)
    net = mk.MetalKAN([784, 256, 256, 10], basis_type="cheby", degree=9)
    for layer in net.layers:
        layer.w_cheby = rng.normal(0, np.sqrt(1.0 / (layer.in_features * 9)), layer.w_cheby.shape).astype(np.float32)

    def spec(ops=None):
        return [{"kind": "cheby", "W": l.w_cheby, "W_base": l.w_base, "bias": l.bias, "params": {"K": 9}}
                for l in net.layers]
    ref32 = O.chain_forward(spec(), x)                 # fp32 weights, float64 arithmetic
    net.half()
    y = net(x)
    y2 = net(x)                                        # graph replay
    np.testing.assert_array_equal(y.view(np.uint16), y2.view(np.uint16))
    ref_ops = O.chain_forward(spec(), x, operands="float16")   # fp16 weights and MFMA operands
    for l in net.layers:
        wm, nb, sp = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        assert gpu.kans_layer_describe(l._engine().handle, B, ctypes.byref(wm), ctypes.byref(nb), ctypes.byref(sp)) == 0
        print(f"cfg2 layer {l.in_features}->{l.out_features}: tile ({wm.value},{nb.value}) x {sp.value} splits")
    e32, eops = O.rel_err(y, ref32), O.rel_err(y, ref_ops)
    print(f"cfg2 fp16 B=4096: rel err {e32:.3e} vs fp32 weights, {eops:.3e} vs operand-rounded oracle")
    assert e32 <= TOL["float16"]
    assert eops <= 5e-3


# ---------------------------------------------------------------- config 4
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_cfg4_bspline_full_shape(gpu, dtype):
    """BSplineKAN G = 5 on [-1, 1] (8 bases) + SiLU base, 8192 x 1024 -> 4096,
    x ~ U(-1.2, 1.2) (about 8 % of the inputs outside the grid)."""
    import metal_kans as mk
    rng = np.random.default_rng(1004)
    B, di, do = 8192, 1024, 4096
    x = rng.uniform(-1.2, 1.2, (B, di)).astype(np.float32)
    L = mk.BSplineKAN(di, do, grid_size=5, spline_order=3, grid_range=(-1.0, 1.0))
    L.w_spline = rng.normal(0, np.sqrt(1.0 / (di * 8)), (do, di * 8)).astype(np.float32)
    L.w_base = rng.uniform(-1 / 32, 1 / 32, (do, di)).astype(np.float32)
    L.bias = rng.normal(0, 0.1, do).astype(np.float32)
    rows = np.sort(rng.choice(B, 64, replace=False))
    y_ref = O.kan_forward("bspline", x[rows], L.w_spline, L.w_base, L.bias,
                          {"G": 5, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])})
    if dtype == "bfloat16":
        L.bfloat16()
    y = L(x)
    y2 = L(x)
    assert y.shape == (B, do)
    np.testing.assert_array_equal(y.view(np.uint32), y2.view(np.uint32))
    name = ctypes.create_string_buffer(160)
    assert gpu.kans_layer_kernel(L._engine().handle, B, name, 160) == 0
    e = O.rel_err(y[rows], y_ref)
    print(f"cfg4 {dtype}: {name.value.decode()}: rel err {e:.3e} on {rows.size} rows")
    assert e <= TOL[dtype]


# ---------------------------------------------------------------- config 5
D_MODEL, D_FFN, K5 = 4096, 11008, 4


def _quantize(lib, fmt, W):
    """Packed arrays of W in the reference format (native host quantizers; the row lengths here are
    multiples of the group, so no padding)."""
    if fmt in ("int4", "int8"):
        ng = W.size // 64
        q = np.empty((ng, 32 if fmt == "int4" else 64), np.uint8)
        s = np.empty(ng, np.float32)
        b = np.empty(ng, np.float32)
        fn = lib.metal_kan_quantize_int4 if fmt == "int4" else lib.metal_kan_quantize_int8
        assert fn(W.ctypes.data, q.ctypes.data, s.ctypes.data, b.ctypes.data, ng, 64) == 0
        return (q, s, b)
    rows, kd = W.shape
    p = np.zeros((rows, (kd + 15) // 16), np.uint32)
    s = np.zeros((rows, (kd + 31) // 32), np.float32)
    assert lib.metal_kan_quantize_ternary(W.ctypes.data, p.ctypes.data, s.ctypes.data, rows, kd, 32) == 0
    return (p, s)


def _dequant_rows(fmt, packed, shape, r0, r1):
    """Oracle dequantization of rows r0 .. r1-1 (groups never straddle rows: the row lengths here are
    multiples of the group)."""
    rows, kd = shape
    if fmt in ("int4", "int8"):
        q, s, b = packed
        gpr = kd // 64
        sl = slice(r0 * gpr, r1 * gpr)
        return O.dequantize_affine(q[sl], s[sl], b[sl], 4 if fmt == "int4" else 8, 64, (r1 - r0, kd), kd)
    p, s = packed
    return O.dequantize_ternary(p[r0:r1], s[r0:r1], (r1 - r0, kd), 32)


def _oracle_layer(fmt, pk_w, pk_b, shape_w, shape_b, xs):
    """float64 oracle of one Chebyshev K = 4 layer with base branch, no bias, on the dequantized weights
    (row blocks dequantized in a thread pool, so no full-size float64 copy exists)."""
    rows = shape_w[0]
    phi = O.cheby_basis(xs, K5).reshape(xs.shape[0], -1)
    sx = O.silu(xs)
    out = np.empty((xs.shape[0], rows), np.float64)

    def block(r0):
        r1 = min(rows, r0 + 512)
        Wd = _dequant_rows(fmt, pk_w, shape_w, r0, r1).astype(np.float64)
        Wbd = _dequant_rows(fmt, pk_b, shape_b, r0, r1).astype(np.float64)
        out[:, r0:r1] = phi @ Wd.T + sx @ Wbd.T
    with cf.ThreadPoolExecutor(8) as ex:
        list(ex.map(block, range(0, rows, 512)))
    return out


@pytest.fixture(scope="module")
def cfg5_weights():
    """The six cfg5 matrices ~ N(0, 0.02): gate / up (11008 x 16384, base 11008 x 4096), down (4096 x 44032,
    base 4096 x 11008)."""
    rng = np.random.default_rng(1005)
    base = normal_block(rng, 0.02)
    mats = []
    for (di, do) in ((D_MODEL, D_FFN), (D_MODEL, D_FFN), (D_FFN, D_MODEL)):
        mats.append((normal_matrix(rng, base, (do, di * K5)), normal_matrix(rng, base, (do, di))))
    xs = {B: rng.standard_normal((B, D_MODEL), dtype=np.float32).astype(np.float16) for B in (1, 32, 8192)}
    return mats, xs


def _qlayer(lib, fmt, pk_w, pk_b, di, do):
    h = ctypes.c_void_p()
    if fmt in ("int4", "int8"):
        fn = lib.kans_qlayer_create_int4 if fmt == "int4" else lib.kans_qlayer_create_int8
        rc = fn(di, do, K5, 1, 0, 64, *[a.ctypes.data for a in pk_w + pk_b], None, 0, ctypes.byref(h))
    else:
        rc = lib.kans_qlayer_create_ternary(di, do, K5, 1, 0, 32, *[a.ctypes.data for a in pk_w + pk_b], None, 0,
                                            ctypes.byref(h))
    assert rc == 0, lib.kans_last_error()
    return h


@pytest.mark.parametrize("fmt", ["int4", "ternary", "int8"])
def test_cfg5_gatedkan_full_shape(gpu, cfg5_weights, fmt):
    """the fused quantized GatedKAN block at B = 1 and 32 (decode: one HIP graph of prep,
    gate|up GEMV with the SwiGLU epilogue at B = 1, down GEMV, reduce) and at B = 8192
    (prefill: gate|up in one launch with the SwiGLU epilogue, then down), against the float64 oracle block
    out = Down(SiLU(Gate(x)) * Up(x)) (gated_kan.py:86-138) on the dequantized weights.  At B = 8192 a seeded
    sample of 48 rows is checked (rows are independent), plus a bitwise rerun of the whole batch."""
    lib = gpu
    mats, xs = cfg5_weights
    packed = [(_quantize(lib, fmt, W), _quantize(lib, fmt, Wb)) for (W, Wb) in mats]
    dims = [(D_MODEL, D_FFN), (D_MODEL, D_FFN), (D_FFN, D_MODEL)]
    layers = [_qlayer(lib, fmt, pw, pb, di, do) for (pw, pb), (di, do) in zip(packed, dims)]
    blk = ctypes.c_void_p()
    assert lib.kans_gated_create(*layers, ctypes.byref(blk)) == 0
    rows8k = np.sort(np.random.default_rng(58).choice(8192, 48, replace=False))
    checked = {1: xs[1], 32: xs[32], 8192: xs[8192][rows8k]}
    try:
        # float64 oracle block on every checked row at once (rows are independent)
        xall = np.concatenate([checked[B] for B in (1, 32, 8192)]).astype(np.float64)
        g = _oracle_layer(fmt, *packed[0], mats[0][0].shape, mats[0][1].shape, xall)
        u = _oracle_layer(fmt, *packed[1], mats[1][0].shape, mats[1][1].shape, xall)
        ref_all = _oracle_layer(fmt, *packed[2], mats[2][0].shape, mats[2][1].shape, O.silu_clipped(g) * u)
        r0 = 0
        for B in (1, 32, 8192):
            x = xs[B]
            n = checked[B].shape[0]
            ref = ref_all[r0:r0 + n]
            r0 += n
            y = np.empty((B, D_MODEL), np.float16)
            print(f"cfg5 {fmt} B={B}", flush=True)
            assert lib.kans_gated_forward_host(blk, x.ctypes.data, 1, y.ctypes.data, 1, B, 1) == 0, \
                lib.kans_last_error()
            y2 = np.empty_like(y)
            assert lib.kans_gated_forward_host(blk, x.ctypes.data, 1, y2.ctypes.data, 1, B, 1) == 0
            np.testing.assert_array_equal(y.view(np.uint16), y2.view(np.uint16))
            ys = y if B < 8192 else y[rows8k]
            e = O.rel_err(ys.astype(np.float32), ref)
            print(f"cfg5 {fmt} B={B}: rel err {e:.3e}")
            assert np.isfinite(ys.astype(np.float32)).all()
            assert e <= TOL["float16"]
        # fp32 x at B = 1 and 2: the in-kernel basis (each workgroup's range holds 4096 base inputs here)
        # equals the separate basis kernel bit for bit
        for B in (1, 2):
            x32 = xs[32][:B].astype(np.float32)
            outs = []
            for mode in (2, 0):
                prev = lib.kans_decode_set_pre_basis(mode)
                try:
                    y = np.empty((B, D_MODEL), np.float16)
                    assert lib.kans_gated_forward_host(blk, x32.ctypes.data, 0, y.ctypes.data, 1, B, 1) == 0, \
                        lib.kans_last_error()
                finally:
                    lib.kans_decode_set_pre_basis(prev)
                outs.append(y)
            print(f"cfg5 {fmt} fp32 x B={B}: in-kernel basis vs separate kernel", flush=True)
            np.testing.assert_array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
    finally:
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)

"""GPU parity of the fused HIP path against the CPU oracle (run on an MI355X).

Metric: max|y - y_ref| / max|y_ref| with y_ref the float64 oracle on the
original fp32 inputs and weights (the reference's fp16 test compares against
its fp32 path the same way, tests/test_metal_kans.py:257-308).
Tolerances: fp32 <= 1e-4, fp16 / bf16 <= 2e-2.
Dequantization: bit-exact.
"""
import ctypes

import numpy as np
import pytest

from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu

TOL = {"float32": 1e-4, "float16": 2e-2, "bfloat16": 2e-2}


def make_layer(mk, kind, d_in, d_out, K, bias=True, base=True, seed=0, grid_range=(-1.0, 1.0)):
    np.random.seed(seed)
    if kind == "cheby":
        L = mk.ChebyKAN(d_in, d_out, degree=K, bias=bias, use_base=base)
    elif kind == "rbf":
        L = mk.FastKAN(d_in, d_out, num_centers=K, grid_range=grid_range, bias=bias, use_base=base)
    else:
        L = mk.BSplineKAN(d_in, d_out, grid_size=K - 3, grid_range=grid_range, bias=bias, use_base=base)
    if bias:
        L.bias = np.random.normal(0, 0.1, d_out).astype(np.float32)
    return L


def oracle_of(L, x):
    kind = L._basis
    W = getattr(L, L._weight_attr).astype(np.float64)
    Wb = L.w_base.astype(np.float64) if L.has_base else None
    bias = L.bias.astype(np.float64) if L.has_bias else None
    if kind == "cheby":
        p = {"K": L.degree}
    elif kind == "rbf":
        p = {"grid": np.asarray(L.grid, np.float64), "inv_den": L.inv_denominator}
    else:
        p = {"G": L.grid_size, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])}
    return O.kan_forward(kind, x.astype(np.float64), W, Wb, bias, p)


def cast(L, dtype):
    if dtype == "float16":
        L.half()
    elif dtype == "bfloat16":
        L.bfloat16()
    return L


SHAPES = [
    (1, 3, 5),        # single row, D_in not a multiple of 8
    (37, 24, 70),     # ragged rows / columns, D_in % 16 == 8
    (256, 64, 64),    # config 1 shape
    (300, 130, 200),  # several feature blocks, ragged everything
]
KINDS = [("cheby", 9), ("cheby", 4), ("rbf", 8), ("bspline", 8)]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("kind,K", KINDS)
@pytest.mark.parametrize("B,d_in,d_out", SHAPES)
def test_layer_parity(gpu, dtype, kind, K, B, d_in, d_out):
    import metal_kans as mk
    print(f"case {kind} K={K} {dtype} B={B} {d_in}->{d_out}", flush=True)
    L = make_layer(mk, kind, d_in, d_out, K, seed=B + d_in, grid_range=(-1.5, 1.5) if kind == "rbf" else (-1, 1))
    rng = np.random.default_rng(B * 7 + d_out)
    x = rng.uniform(-1.2, 1.2, (B, d_in)).astype(np.float32)
    y_ref = oracle_of(L, x)
    y = cast(L, dtype)(x)
    assert y.shape == (B, d_out)
    assert np.isfinite(y).all()
    assert O.rel_err(y, y_ref) <= TOL[dtype], O.rel_err(y, y_ref)


@pytest.mark.parametrize("base,bias", [(False, False), (False, True), (True, False)])
@pytest.mark.parametrize("kind,K", [("cheby", 5), ("rbf", 6), ("bspline", 7)])
def test_branch_flags(gpu, kind, K, base, bias):
    import metal_kans as mk
    L = make_layer(mk, kind, 40, 33, K, bias=bias, base=base, seed=3)
    x = np.random.default_rng(1).uniform(-1.1, 1.1, (65, 40)).astype(np.float32)
    assert O.rel_err(L(x), oracle_of(L, x)) <= 1e-4


@pytest.mark.parametrize("wm,nb,splits", [(64, 4, 1), (32, 8, 1), (32, 4, 1), (32, 1, 1), (64, 4, 3), (32, 4, 5),
                                          (32, 8, 4)])
@pytest.mark.parametrize("dtype", ["float32", "float16"])
@pytest.mark.parametrize("kind,K", [("cheby", 6), ("rbf", 8), ("bspline", 8), ("rbf", 12)])
def test_tilings_and_splits(gpu, wm, nb, splits, dtype, kind, K):
    import metal_kans as mk
    L = make_layer(mk, kind, 200, 150, K, seed=11)
    L.set_tiling(wm, nb, splits)
    x = np.random.default_rng(2).uniform(-1, 1, (333, 200)).astype(np.float32)
    y_ref = oracle_of(L, x)
    assert O.rel_err(cast(L, dtype)(x), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("wm,nb", [(32, 4), (32, 8), (32, 1)])
@pytest.mark.parametrize("d_out", [200, 64])
def test_split_reduce_vector_path(gpu, dtype, wm, nb, d_out):
    """Feature splits on layers whose output width is a multiple of 4 take the 4-column split reduce
    (16-byte partial loads, one vector store); splits of 2, 3 and 5, ragged rows."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", 120, d_out, 6, seed=17)
    x = np.random.default_rng(12).uniform(-1, 1, (201, 120)).astype(np.float32)
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    for splits in (2, 3, 5):
        L.set_tiling(wm, nb, splits)
        assert O.rel_err(L(x), y_ref) <= TOL[dtype], splits


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("kind,K", [("rbf", 8), ("bspline", 8), ("rbf", 5), ("bspline", 6), ("cheby", 9),
                                    ("cheby", 4)])
@pytest.mark.parametrize("base,bias", [(True, True), (False, False), (False, True)])
def test_block_kernel_256x256_tile(gpu, dtype, kind, K, base, bias):
    """16-bit layers on the (32, 8) tile take the 8-wave block kernel (K + base <= 9 for RBF, 10 otherwise): ragged
    rows, a feature count that is not a multiple of 16, output columns that end inside an N-tile,
    with and without a feature split."""
    import metal_kans as mk
    L = make_layer(mk, kind, 200, 150, K, bias=bias, base=base, seed=21, grid_range=(-1.5, 1.5))
    x = np.random.default_rng(5).uniform(-1.7, 1.7, (300, 200)).astype(np.float32)
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    for splits in (1, 3):
        L.set_tiling(32, 8, splits)
        assert O.rel_err(L(x), y_ref) <= TOL[dtype]
        name = ctypes.create_string_buffer(160)
        assert gpu.kans_layer_kernel(L._engine().handle, 300, name, 160) == 0
        assert name.value.startswith(b"kans::kan_fused_block<") and b"32, 8, 8 waves>" in name.value, name.value


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("K,base,bias", [(4, True, True), (4, False, False), (2, True, False), (1, False, True)])
@pytest.mark.parametrize("d_in", [112, 200, 16, 40])
def test_block_kernel_two_blocks_per_stage(gpu, dtype, K, base, bias, d_in):
    """8-wave Chebyshev block kernel with K + base <= 5: two feature blocks per LDS stage (one barrier per
    pair) against one block per stage, bit for bit, and against the oracle; 7, 13 (ragged), 1 and 3
    feature blocks, with and without feature splits (odd and one-block splits)."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", d_in, 300, K, bias=bias, base=base, seed=23)
    x = np.random.default_rng(7).uniform(-1.3, 1.3, (520, d_in)).astype(np.float32)
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    for splits in (1, 2, 3):
        L.set_tiling(32, 8, splits)
        L(x)  # the device layer exists after its first forward
        h = L._engine().handle
        outs = []
        for on in (1, 0):
            assert gpu.kans_layer_set_block_pairs(h, on) == 0
            y = np.asarray(L(x), np.float32)
            assert O.rel_err(y, y_ref) <= TOL[dtype], (splits, on)
            name = ctypes.create_string_buffer(200)
            assert gpu.kans_layer_kernel(h, 520, name, 200) == 0
            assert b"32, 8, 8 waves>" in name.value, name.value
            assert (b"2 feature blocks per stage" in name.value) == bool(on), name.value
            outs.append(y)
        assert np.array_equal(outs[0], outs[1]), splits
    assert gpu.kans_layer_set_block_pairs(h, 2) < 0
    assert gpu.kans_layer_set_block_pairs(h, 1) == 0


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("K,base,bias", [(9, True, True), (4, False, True), (1, True, False)])
@pytest.mark.parametrize("d_in", [200, 64, 16])
def test_block_kernel_small_tile_stages(gpu, dtype, K, base, bias, d_in):
    """16-bit Chebyshev on the (32, 1) tile takes the 4-wave block kernel: feature counts of 13, 4
    and 1 blocks (one not a multiple of 16), feature splits of 1, 2, 3 and 5 (empty and one-block
    splits), K + base from 2 to 10."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", d_in, 70, K, bias=bias, base=base, seed=31)
    x = np.random.default_rng(9).uniform(-1.2, 1.2, (150, d_in)).astype(np.float32)
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    for splits in (1, 2, 3, 5):
        L.set_tiling(32, 1, splits)
        assert O.rel_err(L(x), y_ref) <= TOL[dtype], splits
        name = ctypes.create_string_buffer(160)
        assert gpu.kans_layer_kernel(L._engine().handle, 150, name, 160) == 0
        assert name.value.startswith(b"kans::kan_fused_block<") and b"32, 1, 4 waves>" in name.value, name.value


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("wm,nb,groups", [(32, 1, 2), (32, 1, 4), (32, 4, 2)])
@pytest.mark.parametrize("K,base,bias", [(9, True, True), (4, False, True), (1, True, False)])
@pytest.mark.parametrize("d_in", [200, 64, 16])
def test_block_kernel_wave_groups(gpu, dtype, wm, nb, groups, K, base, bias, d_in):
    """The 4-wave Chebyshev block kernel with 2 or 4 wave groups per workgroup splitting a tile's
    feature blocks (13, 4 and 1 blocks: uneven runs and groups with no block), alone and under a
    3-way feature split, ragged rows and columns; the groups' sums are added in a fixed order, so
    a rerun is bit-identical."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", d_in, 70, K, bias=bias, base=base, seed=31)
    x = np.random.default_rng(9).uniform(-1.2, 1.2, (150, d_in)).astype(np.float32)
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    for splits in (1, 3):
        L.set_tiling(wm, nb, splits, groups)
        y = L(x)
        assert O.rel_err(y, y_ref) <= TOL[dtype], splits
        assert np.array_equal(L(x).view(np.uint16), y.view(np.uint16))
        name = ctypes.create_string_buffer(160)
        assert gpu.kans_layer_kernel(L._engine().handle, 150, name, 160) == 0
        tag = f"{wm}, {nb}, 4 waves x {groups} groups>".encode()
        assert name.value.startswith(b"kans::kan_fused_block<") and tag in name.value, name.value


def test_rbf_arbitrary_centres(gpu):
    import metal_kans as mk
    L = make_layer(mk, "rbf", 48, 40, 5, seed=4)
    L.grid = np.array([-1.7, -0.2, 0.0, 0.9, 2.4], np.float32)   # non-uniform centres
    x = np.random.default_rng(3).normal(0, 1, (90, 48)).astype(np.float32)
    assert O.rel_err(L(x), oracle_of(L, x)) <= 1e-4
    # reference layers always carry inv_denominator = 1/(2h^2) >= 0; a negative one is refused loudly
    L.inv_denominator = -1.0
    with pytest.raises(RuntimeError, match="inv_denominator"):
        L(x)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("case", ["uniform8", "uniform5_wide", "uniform9_span", "nonuniform8"])
def test_block_rbf_recurrence_and_table(gpu, dtype, case):
    """The 8-wave block kernel evaluates RBF layers on uniform centres whose scaled span is at most 6 by the
    phi_{k+1} = phi_k * r_k recurrence (BASIS_RBF_REC) and every other grid by exp2 per value
    (BASIS_RBF_TABLE).  Both against the oracle, with inputs far outside the grid (where the recurrence
    clamps) and on the centres."""
    import metal_kans as mk
    K, rng_, path = {"uniform8": (8, (-2, 2), b"BASIS_RBF_REC"), "uniform5_wide": (5, (-1, 1), b"BASIS_RBF_REC"),
                     "uniform9_span": (9, (-2, 2), b"BASIS_RBF_TABLE"),
                     "nonuniform8": (8, (-2, 2), b"BASIS_RBF_TABLE")}[case]
    # K + base <= 9 slots keeps the layer on the block kernel
    L = make_layer(mk, "rbf", 72, 300, K, seed=31, grid_range=rng_, base=K < 9)
    if case == "uniform5_wide":
        L.inv_denominator = np.float32(0.3)   # wide Gaussians: scaled span 1.3
    if case == "nonuniform8":
        L.grid = np.array([-2.0, -1.3, -0.9, 0.0, 0.2, 0.9, 1.6, 2.0], np.float32)
    x = np.random.default_rng(6).normal(0, 1.5, (260, 72)).astype(np.float32)
    x[0, :10] = [1e4, -1e4, 7.5, -7.5, 3.0, -3.0, 0.0, 2.0, -2.0, 1e-3]
    x[1, :K] = np.asarray(L.grid, np.float32)   # exactly on the centres
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    L.set_tiling(32, 8, 1)
    y = L(x)
    assert np.isfinite(y).all()
    assert O.rel_err(y, y_ref) <= TOL[dtype]
    name = ctypes.create_string_buffer(160)
    assert gpu.kans_layer_kernel(L._engine().handle, 260, name, 160) == 0
    assert path in name.value, name.value


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("base", [True, False])
def test_block_bspline_table(gpu, dtype, base):
    """16-bit B-spline layers with G = 5 on the block kernel place each input's eight basis values into a
    register table once per feature block (BASIS_BSPLINE_TAB / _TAB0): against the oracle with inputs on
    every knot, just inside and outside the grid, far outside it, and a bias-free layer."""
    import metal_kans as mk
    L = make_layer(mk, "bspline", 40, 280, 8, bias=base, base=base, seed=41, grid_range=(-1.0, 1.0))
    x = np.random.default_rng(9).uniform(-1.3, 1.3, (300, 40)).astype(np.float32)
    x[0, :6] = np.linspace(-1, 1, 6)                       # the knots (span boundaries)
    x[1, :8] = [-1.0000001, 0.9999999, 1.0000001, -0.9999999, 1e4, -1e4, 3.0, -3.0]
    x[2, :6] = np.linspace(-1, 1, 6) + np.float32(1e-7)
    y_ref = oracle_of(L, x)
    cast(L, dtype)
    L.set_tiling(32, 8, 1)
    y = L(x)
    assert np.isfinite(y).all()
    assert O.rel_err(y, y_ref) <= TOL[dtype]
    name = ctypes.create_string_buffer(160)
    assert gpu.kans_layer_kernel(L._engine().handle, 300, name, 160) == 0
    assert (b"BASIS_BSPLINE_TAB," if base else b"BASIS_BSPLINE_TAB0,") in name.value, name.value


def test_inputs_outside_grid_and_extremes(gpu):
    import metal_kans as mk
    x = np.random.default_rng(8).uniform(-6, 6, (64, 32)).astype(np.float32)
    x[0, :8] = [0.0, 1.0, -1.0, 1e4, -1e4, 1.0000001, -0.99999, 5.0]
    for kind, K in (("cheby", 9), ("bspline", 8), ("rbf", 8)):
        L = make_layer(mk, kind, 32, 48, K, seed=5)
        y = L(x)
        assert np.isfinite(y).all()
        assert O.rel_err(y, oracle_of(L, x)) <= 1e-4, kind


def test_multi_dim_input_and_dtype_cast(gpu):
    import metal_kans as mk
    L = make_layer(mk, "cheby", 16, 8, 4)
    x = np.random.default_rng(0).uniform(-1, 1, (2, 5, 16))
    y = L(x)                      # float64 input is cast to float32 as in the reference
    assert y.shape == (2, 5, 8) and y.dtype == np.float32
    assert O.rel_err(y.reshape(10, 8), oracle_of(L, x.reshape(10, 16).astype(np.float32))) <= 1e-4
    with pytest.raises(ValueError):
        L(np.zeros((3, 15), np.float32))


def test_in_place_weight_edit_is_seen(gpu):
    """The reference's finite-difference tests edit weights in place (test_training.py:59-67)."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", 3, 2, 4)
    x = np.random.default_rng(0).uniform(-0.8, 0.8, (4, 3)).astype(np.float32)
    y0 = L(x).copy()
    L.w_cheby[1, 5] += 1e-2
    y1 = L(x)
    assert O.rel_err(y1, oracle_of(L, x)) <= 1e-4
    assert not np.array_equal(y0, y1)


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_in_place_edit_of_large_weights_is_seen(gpu, dtype):
    """An optimizer step edits parameters in place (the reference's optim.py: param -= lr * update):
    arrays over 4 MB are checked by a hash of their bytes, so the next forward sees the edit.  With
    freeze_weights() (opt-in) only identity is checked until invalidate()."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", 512, 512, 5, seed=4)     # w_cheby 512 x 2560 fp32 = 5.2 MB
    cast(L, dtype)
    assert getattr(L, L._weight_attr).nbytes > (4 << 20) or dtype == "float16"
    x = np.random.default_rng(1).uniform(-1, 1, (64, 512)).astype(np.float32)
    y0 = np.array(L(x), np.float32)
    L.w_cheby -= (0.05 * np.sign(L.w_cheby)).astype(L.w_cheby.dtype)
    y1 = np.array(L(x), np.float32)
    assert not np.array_equal(y0, y1)
    assert O.rel_err(y1, oracle_of(L, x)) <= TOL[dtype]
    L.freeze_weights()
    L.w_cheby *= np.asarray(0.5, L.w_cheby.dtype)
    y_frozen = np.array(L(x), np.float32)
    if L.w_cheby.nbytes > (4 << 20):
        np.testing.assert_array_equal(y_frozen, y1)        # frozen: the large array is not re-read
    L.invalidate()
    assert O.rel_err(np.array(L(x), np.float32), oracle_of(L, x)) <= TOL[dtype]
    L.freeze_weights(False)


def test_gradients_exist_from_construction(gpu):
    """cheby_kan.py:44-46: gradient arrays are zeros before the first backward."""
    import metal_kans as mk
    L = mk.ChebyKAN(6, 4, degree=3)
    assert L.grad_w_cheby.shape == L.w_cheby.shape and not L.grad_w_cheby.any()
    assert L.grad_w_base.shape == L.w_base.shape and L.grad_bias.shape == (4,)
    L2 = mk.ChebyKAN(6, 4, degree=3, bias=False, use_base=False)
    assert L2.grad_w_base is None and L2.grad_bias is None


# ---------------------------------------------------------------- reference tests, on this build
def test_reference_fp16_vs_fp32(gpu):
    """tests/test_metal_kans.py:257-308: fp16 output within atol 1e-2 of fp32."""
    import metal_kans as mk
    np.random.seed(42)
    for ctor, xr in ((lambda: mk.ChebyKAN(8, 16, degree=4), 1.0), (lambda: mk.FastKAN(8, 16, num_centers=8), 1.0),
                     (lambda: mk.BSplineKAN(8, 16, grid_size=5, spline_order=3), 0.9)):
        layer = ctor()
        x = np.random.uniform(-xr, xr, (64, 8)).astype(np.float32)
        y32 = layer(x)
        layer.half()
        y16 = layer(x.astype(np.float16))
        assert y16.dtype == np.float16
        np.testing.assert_allclose(y16.astype(np.float32), y32, atol=1e-2)


def test_reference_fp16_boundary(gpu):
    """tests/test_optimizations.py:17-26: fp16 Chebyshev at x = +-1, K = 8 stays finite."""
    import metal_kans as mk
    layer = mk.ChebyKAN(in_features=8, out_features=4, degree=8).half()
    X = np.array([[-1.0, -0.999, 0.0, 0.999, 1.0, -0.5, 0.5, 0.0] for _ in range(4)], dtype=np.float16)
    Y = layer(X)
    assert Y.shape == (4, 4) and np.isfinite(Y.astype(np.float32)).all()


def test_reference_chain_vs_layers(gpu):
    """tests/test_metal_kans.py:145-160: chained network equals per-layer dispatch (abs < 1e-4)."""
    import metal_kans as mk
    np.random.seed(42)
    net = mk.MetalKAN([4, 16, 8, 2], basis_type="cheby", degree=4, pipeline=True)
    x = np.random.uniform(-1.0, 1.0, (128, 4)).astype(np.float32)
    y_chain = net(x)
    h = x
    for layer in net.layers:
        h = layer(h)
    assert np.max(np.abs(y_chain - h)) < 1e-4
    ref = O.chain_forward([{"kind": "cheby", "W": l.w_cheby, "W_base": l.w_base, "bias": l.bias,
                            "params": {"K": 4}} for l in net.layers], x)
    assert O.rel_err(y_chain, ref) <= 1e-4


def test_reference_quantization_error_bounds(gpu):
    """tests/test_metal_kans.py:163-181."""
    import metal_kans as mk
    np.random.seed(42)
    w = np.random.normal(0.0, 1.0, (32, 64)).astype(np.float32)
    assert np.max(np.abs(w - mk.QuantizedWeight(w, bits=8, group_size=32).dequantize())) < 0.05
    assert np.max(np.abs(w - mk.QuantizedWeight(w, bits=4, group_size=32).dequantize())) < 0.35
    net = mk.MetalKAN([8, 16, 4], basis_type="cheby")
    mk.to_int8(net)
    assert net(np.random.uniform(-1, 1, (16, 8)).astype(np.float32)).shape == (16, 4)


def test_reference_ternary_cosine(gpu):
    """tests/test_optimizations.py:104-120."""
    import metal_kans as mk
    np.random.seed(42)
    layer = mk.ChebyKAN(in_features=16, out_features=8, degree=4)
    x = np.random.uniform(-0.8, 0.8, (4, 16)).astype(np.float32)
    out32 = layer(x)
    mk.to_ternary(layer, group_size=32)
    assert hasattr(layer, "_w_cheby_ternary")
    out_t = layer(x)
    cos = np.dot(out32.ravel(), out_t.ravel()) / (np.linalg.norm(out32) * np.linalg.norm(out_t) + 1e-8)
    assert cos > 0.4


def test_reference_async_stream(gpu):
    """tests/test_metal_kans.py:318-332."""
    import metal_kans as mk
    np.random.seed(42)
    net = mk.MetalKAN([8, 16, 2], basis_type="fastkan", degree=8)
    batches = [np.random.uniform(-1.0, 1.0, (32, 8)).astype(np.float32) for _ in range(8)]
    y_sync = [net(b) for b in batches]
    y_async = net.async_stream(batches)
    for a, s in zip(y_async, y_sync):
        np.testing.assert_allclose(a, s, atol=1e-5)


# ---------------------------------------------------------------- quantization on device
@pytest.mark.parametrize("bits", [8, 4])
def test_dequant_affine_bit_exact(gpu, bits):
    import metal_kans as mk
    w = np.random.default_rng(bits).normal(0, 0.02, (70, 300)).astype(np.float32)
    qw = mk.QuantizedWeight(w, bits=bits, group_size=64)
    dq = qw.dequantize()
    ref = O.dequantize_affine(qw.qweight, qw.scales, qw.biases, bits, 64, w.shape, qw.padded_in_features)
    np.testing.assert_array_equal(dq.view(np.uint32), ref.view(np.uint32))


def test_dequant_ternary_bit_exact(gpu):
    import metal_kans as mk
    w = np.random.default_rng(3).normal(0, 0.02, (50, 1000)).astype(np.float32)
    tq = mk.TernaryQuantizedWeight(w, group_size=32)
    ref = O.dequantize_ternary(tq.w_packed, tq.scales, w.shape, 32)
    np.testing.assert_array_equal(tq.dequantize().view(np.uint32), ref.view(np.uint32))


def test_dequant_golden_bit_exact(gpu, request):
    import os
    from metal_kans import device
    lib = device.get_metal_bridge()
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz"))
    for n in sorted({k.split("__")[0] for k in g.files}):
        for bits, gs in ((8, 64), (4, 32)):
            t = f"{n}__int{bits}_g{gs}"
            q, s, b = g[t + "__q"], g[t + "__s"], g[t + "__b"]
            out = np.empty(s.shape[0] * gs, np.float32)
            fn = lib.metal_kan_dequantize_int8 if bits == 8 else lib.metal_kan_dequantize_int4
            assert fn(q.ctypes.data, s.ctypes.data, b.ctypes.data, out.ctypes.data, s.shape[0], gs) == 0
            w = g[f"{n}__w"]
            dq = out.reshape(w.shape[0], -1)[:, : w.shape[1]]
            np.testing.assert_array_equal(dq.view(np.uint32), g[t + "__dq"].view(np.uint32), err_msg=t)
        t = f"{n}__tern_g32"
        p, s = g[t + "__p"], g[t + "__s"]
        w = g[f"{n}__w"]
        out = np.empty(w.shape, np.float32)
        assert lib.metal_kan_dequantize_ternary(p.ctypes.data, s.ctypes.data, out.ctypes.data, w.shape[0],
                                                w.shape[1], 32) == 0
        np.testing.assert_array_equal(out.view(np.uint32), g[t + "__dq"].view(np.uint32), err_msg=t)


@pytest.mark.parametrize("quant", ["int8", "int4", "ternary"])
def test_quantized_layer_forward(gpu, quant):
    """Quantized forward = forward(x, dequant(quant(W))) (quantization.py:168-171)."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", 64, 48, 4, seed=9)
    getattr(mk, f"to_{quant}")(L)
    assert L.w_cheby.dtype == np.float32
    x = np.random.default_rng(4).uniform(-1, 1, (40, 64)).astype(np.float32)
    assert O.rel_err(L(x), oracle_of(L, x)) <= 1e-4


def test_swiglu(gpu):
    from metal_kans import device
    lib = device.get_metal_bridge()
    rng = np.random.default_rng(0)
    g = rng.normal(0, 8, 1000).astype(np.float32)
    u = rng.normal(0, 1, 1000).astype(np.float32)
    out = np.empty_like(g)
    assert lib.metal_kan_swiglu_forward(g.ctypes.data, u.ctypes.data, out.ctypes.data, g.size) == 0
    np.testing.assert_allclose(out, O.swiglu(g, u), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_gated_kan(gpu, dtype):
    import metal_kans as mk
    np.random.seed(1)
    blk = mk.GatedKAN(d_model=32, d_ffn=64, degree=4, dtype=np.float16 if dtype == "float16" else np.float32)
    x = np.random.uniform(-0.8, 0.8, (6, 32)).astype(np.float32)
    ref = O.gated_forward(x, *[{"W": k.w_cheby, "W_base": k.w_base, "K": 4}
                               for k in (blk.gate_kan, blk.up_kan, blk.down_kan)])
    out = blk(x)
    assert out.shape == (6, 32)
    assert O.rel_err(out, ref) <= TOL[dtype]
    out3 = blk(x.reshape(2, 3, 32))
    assert out3.shape == (2, 3, 32)


# ---------------------------------------------------------------- reference-named C-ABI entry points
def test_reference_named_entry_points(gpu):
    lib = gpu
    rng = np.random.default_rng(6)
    B, Di, Do = 50, 20, 30
    x = rng.uniform(-1.1, 1.1, (B, Di)).astype(np.float32)
    Wb = rng.normal(0, 0.2, (Do, Di)).astype(np.float32)
    bias = rng.normal(0, 0.1, Do).astype(np.float32)
    y = np.empty((B, Do), np.float32)
    # Chebyshev fp32 / fp16
    W = rng.normal(0, 0.1, (Do, Di * 5)).astype(np.float32)
    assert lib.metal_kan_cheby_forward(x.ctypes.data, W.ctypes.data, Wb.ctypes.data, bias.ctypes.data,
                                       y.ctypes.data, B, Di, Do, 5, 1, 1) == 0
    ref = O.kan_forward("cheby", x, W, Wb, bias, {"K": 5})
    assert O.rel_err(y, ref) <= 1e-4
    h = [a.astype(np.float16) for a in (x, W, Wb, bias)]
    y16 = np.empty((B, Do), np.float16)
    assert lib.metal_kan_cheby_forward_fp16(h[0].ctypes.data, h[1].ctypes.data, h[2].ctypes.data, h[3].ctypes.data,
                                            y16.ctypes.data, B, Di, Do, 5, 1, 1) == 0
    assert O.rel_err(y16, ref) <= 2e-2
    # FastKAN fp32
    grid, inv = O.rbf_grid((-1.0, 1.0), 6)
    W6 = rng.normal(0, 0.1, (Do, Di * 6)).astype(np.float32)
    assert lib.metal_kan_fastkan_forward(x.ctypes.data, W6.ctypes.data, Wb.ctypes.data, grid.ctypes.data,
                                         bias.ctypes.data, y.ctypes.data, B, Di, Do, 6, ctypes.c_float(inv),
                                         1, 1) == 0
    assert O.rel_err(y, O.kan_forward("rbf", x, W6, Wb, bias, {"grid": grid, "inv_den": inv})) <= 1e-4
    # B-spline fp32 (grid = [min, inv_h], read on the host)
    gp = O.bspline_params(5)
    W8 = rng.normal(0, 0.1, (Do, Di * 8)).astype(np.float32)
    assert lib.metal_kan_bspline_forward(x.ctypes.data, W8.ctypes.data, Wb.ctypes.data, gp.ctypes.data,
                                         bias.ctypes.data, y.ctypes.data, B, Di, Do, 5, 3, 1, 1) == 0
    assert O.rel_err(y, O.kan_forward("bspline", x, W8, Wb, bias,
                                      {"G": 5, "grid_min": float(gp[0]), "inv_h": float(gp[1])})) <= 1e-4
    # in-place edit between calls is honoured (host arrays are read every call)
    W[0, 0] += 0.5
    assert lib.metal_kan_cheby_forward(x.ctypes.data, W.ctypes.data, Wb.ctypes.data, bias.ctypes.data,
                                       y.ctypes.data, B, Di, Do, 5, 1, 1) == 0
    assert O.rel_err(y, O.kan_forward("cheby", x, W, Wb, bias, {"K": 5})) <= 1e-4
    ms = lib.benchmark_metal_cheby(x.ctypes.data, W.ctypes.data, Wb.ctypes.data, bias.ctypes.data, y.ctypes.data,
                                   B, Di, Do, 5, 1, 1, 1, 3)
    assert ms > 0


def test_reference_named_16bit_entry_points(gpu):
    """The fp16 entry points of the reference (device.py:227-237,263-267; metal_kan_bridge.mm:1890-2151) and
    their bf16 counterparts, called through the C-ABI with 16-bit bit patterns, against the float64 oracle on
    the original fp32 arrays at the 16-bit bar: the FastKAN grid travels as fp16 bits (_fp16) or fp32 (_bf16),
    the B-spline grid as host fp32 [grid_min, inv_h] in both."""
    from metal_kans._engine import from_bf16_bits, to_bf16_bits
    lib = gpu
    rng = np.random.default_rng(16)
    B, Di, Do = 70, 40, 45
    x = rng.uniform(-1.15, 1.15, (B, Di)).astype(np.float32)
    Wb = rng.normal(0, 0.2, (Do, Di)).astype(np.float32)
    bias = rng.normal(0, 0.1, Do).astype(np.float32)
    grid, inv = O.rbf_grid((-1.2, 1.2), 7)
    gp = O.bspline_params(5)
    cases = {
        "cheby": (5, {"K": 5}),
        "rbf": (7, {"grid": grid, "inv_den": inv}),
        "bspline": (8, {"G": 5, "grid_min": float(gp[0]), "inv_h": float(gp[1])}),
    }
    for kind, (K, params) in cases.items():
        W = rng.normal(0, 0.15, (Do, Di * K)).astype(np.float32)
        ref = O.kan_forward(kind, x, W, Wb, bias, params)
        for dt in ("fp16", "bf16"):
            if dt == "fp16":
                enc = lambda a: np.ascontiguousarray(a, np.float16).view(np.uint16)  # noqa: E731
                dec = lambda a: a.view(np.float16).astype(np.float32)  # noqa: E731
            else:
                enc = lambda a: to_bf16_bits(a)  # noqa: E731
                dec = lambda a: from_bf16_bits(a)  # noqa: E731
            hx, hW, hWb, hb = (enc(a) for a in (x, W, Wb, bias))
            y = np.zeros((B, Do), np.uint16)
            args = (hx.ctypes.data, hW.ctypes.data, hWb.ctypes.data)
            if kind == "cheby":
                fn = getattr(lib, f"metal_kan_cheby_forward_{dt}")
                rc = fn(*args, hb.ctypes.data, y.ctypes.data, B, Di, Do, K, 1, 1)
            elif kind == "rbf":
                g = enc(grid) if dt == "fp16" else np.ascontiguousarray(grid, np.float32)
                fn = getattr(lib, f"metal_kan_fastkan_forward_{dt}")
                rc = fn(*args, g.ctypes.data, hb.ctypes.data, y.ctypes.data, B, Di, Do, K, ctypes.c_float(inv), 1, 1)
            else:
                fn = getattr(lib, f"metal_kan_bspline_forward_{dt}")
                rc = fn(*args, gp.ctypes.data, hb.ctypes.data, y.ctypes.data, B, Di, Do, 5, 3, 1, 1)
            assert rc == 0, (kind, dt, lib.kans_last_error())
            e = O.rel_err(dec(y), ref)
            print(f"{kind} {dt}: rel err {e:.2e}")
            assert e <= 2e-2, (kind, dt, e)
            # without the base / bias branches (dummy pointers are not read)
            ref0 = O.kan_forward(kind, x, W, None, None, params)
            y0 = np.zeros((B, Do), np.uint16)
            if kind == "cheby":
                rc = fn(*args, hb.ctypes.data, y0.ctypes.data, B, Di, Do, K, 0, 0)
            elif kind == "rbf":
                rc = fn(*args, g.ctypes.data, hb.ctypes.data, y0.ctypes.data, B, Di, Do, K, ctypes.c_float(inv), 0, 0)
            else:
                rc = fn(*args, gp.ctypes.data, hb.ctypes.data, y0.ctypes.data, B, Di, Do, 5, 3, 0, 0)
            assert rc == 0
            assert O.rel_err(dec(y0), ref0) <= 2e-2, (kind, dt)


def test_layer_benchmark_method(gpu):
    """layer.benchmark(x, warmup, iters) (cheby_kan.py:233-257, fast_kan.py:223-247, bspline_kan.py:227-251):
    mean ms per full host call of the fp32 reference-named forward, for fp32 and converted 16-bit layers;
    the timed calls compute what the fp32 entry point computes."""
    import metal_kans as mk
    np.random.seed(11)
    x = np.random.default_rng(11).uniform(-1, 1, (96, 40)).astype(np.float32)
    for L in (mk.ChebyKAN(40, 24, degree=4), mk.FastKAN(40, 24, num_centers=8), mk.BSplineKAN(40, 24, grid_size=5)):
        y_ref = L(x)
        ms = L.benchmark(x, warmup=2, iters=5)
        assert np.isfinite(ms) and ms > 0
        assert np.array_equal(L(x), y_ref)
        L.half()
        assert L.benchmark(x, warmup=1, iters=2) > 0


def test_reference_chain_entry_point(gpu):
    lib = gpu
    rng = np.random.default_rng(12)
    dims = [12, 24, 24, 7]
    degs = [3, 6, 4]
    Ws = [rng.normal(0, 0.2, (dims[l + 1], dims[l] * degs[l])).astype(np.float32) for l in range(3)]
    Wbs = [rng.normal(0, 0.2, (dims[l + 1], dims[l])).astype(np.float32) for l in range(3)]
    bs = [rng.normal(0, 0.1, dims[l + 1]).astype(np.float32) for l in range(3)]
    x = rng.uniform(-1, 1, (77, 12)).astype(np.float32)
    y = np.empty((77, 7), np.float32)
    P = ctypes.c_void_p * 3
    rc = lib.metal_kan_chain_pipeline_cheby(x.ctypes.data, y.ctypes.data, 77, 3, (ctypes.c_int * 4)(*dims),
                                            (ctypes.c_int * 3)(*degs), P(*[w.ctypes.data for w in Ws]),
                                            P(Wbs[0].ctypes.data, None, Wbs[2].ctypes.data),
                                            P(None, bs[1].ctypes.data, bs[2].ctypes.data))
    assert rc == 0
    layers = [{"kind": "cheby", "W": Ws[0], "W_base": Wbs[0], "bias": None, "params": {"K": 3}},
              {"kind": "cheby", "W": Ws[1], "W_base": None, "bias": bs[1], "params": {"K": 6}},
              {"kind": "cheby", "W": Ws[2], "W_base": Wbs[2], "bias": bs[2], "params": {"K": 4}}]
    assert O.rel_err(y, O.chain_forward(layers, x)) <= 1e-4


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_metal_kan_chain(gpu, dtype):
    """Config-2 shape (784 -> 256 -> 256 -> 10, K = 9) on a smaller batch.

    With K = 9 this network amplifies 16-bit rounding (T_k'(+-1) = k^2 at the
    clamp edge): exact arithmetic on fp16 weights alone is ~1.4% away from the
    fp32 network, and the MFMA's 16-bit basis operands add more; an fp16 input
    would cost another ~7%, so the input stays fp32.  Checked: (a) against the
    oracle on the same (rounded) weights with the BASELINE tolerance, and (b)
    tightly against the oracle that also rounds the contraction operands to the
    MFMA type, which is what the kernel computes."""
    import metal_kans as mk
    np.random.seed(2)
    net = mk.MetalKAN([784, 256, 256, 10], basis_type="cheby", degree=9)
    x = np.random.default_rng(1).uniform(0, 1, (512, 784)).astype(np.float32)
    if dtype == "float16":
        net.half()
    elif dtype == "bfloat16":
        net.bfloat16()
    ref = O.chain_forward([{"kind": "cheby", "W": l.w_cheby, "W_base": l.w_base, "bias": l.bias,
                            "params": {"K": 9}} for l in net.layers], x)
    y1 = net(x)
    y2 = net(x)   # graph replay
    np.testing.assert_array_equal(np.asarray(y1), np.asarray(y2))
    ops = None if dtype == "float32" else dtype
    ref_ops = O.chain_forward([{"kind": "cheby", "W": l.w_cheby, "W_base": l.w_base, "bias": l.bias,
                                "params": {"K": 9}} for l in net.layers], x, operands=ops)
    e_same, e_ops = O.rel_err(y1, ref), O.rel_err(y1, ref_ops)
    print(f"chain {dtype}: rel err vs same weights {e_same:.2e}, vs operand-rounded oracle {e_ops:.2e}")
    assert e_ops <= (1e-4 if dtype == "float32" else 5e-3)
    if dtype != "bfloat16":  # bf16's 8-bit mantissa: ~6% here, inherent to bf16 operands at K = 9
        assert e_same <= TOL[dtype]


def test_fp16_layer_input_semantics(gpu):
    """fp16 input: used as given (the reference casts x to the weight dtype);
    fp32 input to an fp16 layer: read unrounded by the kernel."""
    import metal_kans as mk
    L = make_layer(mk, "cheby", 64, 32, 9, seed=13)
    x = np.random.default_rng(5).uniform(0.9, 1.0, (50, 64)).astype(np.float32)  # near the clamp edge
    L.half()
    W = {"kind": "cheby", "W": L.w_cheby, "W_base": L.w_base, "bias": L.bias, "params": {"K": 9}}
    y16 = L(x.astype(np.float16))
    assert y16.dtype == np.float16
    assert O.rel_err(y16, O.chain_forward([W], x.astype(np.float16))) <= 2e-2
    y32in = L(x)
    assert y32in.dtype == np.float16
    assert O.rel_err(y32in, O.chain_forward([W], x)) <= 2e-2


# ---------------------------------------------------------------- full-size properties
@pytest.mark.parametrize("kind,K", [("cheby", 9), ("rbf", 8), ("bspline", 8)])
def test_full_size_sampled_rows(gpu, kind, K):
    """16384 x 1024 -> 1024 fp16 (north-star shape): rows are independent, so a
    seeded sample of rows is checked against the float64 oracle; a second run
    must be bitwise identical."""
    import metal_kans as mk
    L = make_layer(mk, kind, 1024, 1024, K, bias=False, seed=21, grid_range=(-2, 2) if kind == "rbf" else (-1, 1))
    rng = np.random.default_rng(100)
    x = (rng.normal(0, 1, (16384, 1024)) if kind == "rbf" else rng.uniform(-1.2, 1.2, (16384, 1024))).astype(np.float32)
    rows = np.sort(rng.choice(16384, 48, replace=False))
    y_ref = oracle_of(L, x[rows])
    L.half()
    y = L(x)
    y2 = L(x)
    np.testing.assert_array_equal(y.view(np.uint16), y2.view(np.uint16))
    assert O.rel_err(y[rows], y_ref) <= 2e-2


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_host_staging_large_ragged(gpu, dtype):
    """Host arrays large enough for the pipelined, multi-threaded staging (several ~2 MB pieces, a short
    last one) and for the chunked synchronous forward (four row chunks of whole 256-row tiles, the last
    one ragged: 3 x 2304 + 1283 rows) with D_in = 1001, so every staged row is padded to 1008 columns:
    the synchronous and the async host call equal the device-array forward of the same layer and batch
    bit for bit, and sampled rows match the float64 oracle."""
    import bench
    import metal_kans as mk
    B, d_in, d_out = 8195, 1001, 515
    L = make_layer(mk, "cheby", d_in, d_out, 4, seed=5)
    rng = np.random.default_rng(7)
    x = rng.uniform(-1.1, 1.1, (B, d_in)).astype(np.float32)
    rows = np.sort(rng.choice(B, 32, replace=False))
    y_ref = oracle_of(L, x[rows])
    if dtype == "float16":
        L.half()
        x = x.astype(np.float16)
    y = L(x)
    mk.set_async(True)
    try:
        ya = L(x)
        mk.sync()
    finally:
        mk.set_async(False)
    np.testing.assert_array_equal(ya, y)
    ldx = 1008
    xp = np.zeros((B, ldx), x.dtype)
    xp[:, :d_in] = x
    xd, yd = bench.DevBuf(gpu, xp.nbytes), bench.DevBuf(gpu, y.nbytes)
    try:
        xd.upload(xp)
        assert gpu.kans_layer_forward(L._engine().handle, xd.p, ldx, yd.p, d_out, B, None) == 0, gpu.kans_last_error()
        assert gpu.kans_synchronize() == 0
        y_dev = yd.download(np.empty_like(y))
    finally:
        xd.free()
        yd.free()
    np.testing.assert_array_equal(y_dev, y)
    assert O.rel_err(y[rows].astype(np.float64), y_ref) <= TOL[dtype]


def test_host_staging_large_chain(gpu):
    """The chain's host path through the same staging (fp32 x of 16.5 MB, D_in = 1001): async equals
    sync bit for bit, sampled rows match the float64 oracle chain."""
    import metal_kans as mk
    np.random.seed(11)
    net = mk.MetalKAN([1001, 96, 40], basis_type="cheby", degree=4)
    rng = np.random.default_rng(12)
    x = rng.uniform(-1, 1, (4099, 1001)).astype(np.float32)
    y = net(x)
    mk.set_async(True)
    try:
        ya = net(x)
        mk.sync()
    finally:
        mk.set_async(False)
    np.testing.assert_array_equal(ya, y)
    rows = np.sort(rng.choice(4099, 24, replace=False))
    h = x[rows].astype(np.float64)
    for L in net.layers:
        h = oracle_of(L, h)
    assert O.rel_err(y[rows].astype(np.float64), h) <= 1e-4


# ---------------------------------------------------------------- GatedKAN on device activations
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("B", [1, 40, 300])
def test_gated_kan_dense_block(gpu, dtype, B):
    """Unquantized GatedKAN: gate, up, SwiGLU and down on device activations in one graph
    (kans_gated_dense_forward_host), against the float64 oracle block on the same weights; the 16-bit
    blocks store gate / up / hidden in their dtype, as the reference's layers output them."""
    import metal_kans as mk
    np.random.seed(B)
    blk = mk.GatedKAN(d_model=72, d_ffn=130, degree=4, has_bias=True, dtype=np.float32)
    for k in (blk.gate_kan, blk.up_kan, blk.down_kan):
        k.bias = np.random.normal(0, 0.1, k.out_features).astype(np.float32)
    specs = [{"W": k.w_cheby, "W_base": k.w_base, "bias": k.bias, "K": 4}
             for k in (blk.gate_kan, blk.up_kan, blk.down_kan)]
    if dtype == "float16":
        for k in (blk.gate_kan, blk.up_kan, blk.down_kan):
            k.half()
        blk.dtype = np.dtype(np.float16)
    elif dtype == "bfloat16":
        for k in (blk.gate_kan, blk.up_kan, blk.down_kan):
            k.bfloat16()
    x = np.random.default_rng(B).uniform(-1.5, 1.5, (B, 72)).astype(np.float32)
    ref = O.gated_forward(x, *specs)
    out = blk(x)
    assert out.shape == (B, 72)
    assert blk.__dict__.get("_dense_block") is not None
    e = O.rel_err(np.asarray(out, np.float32), ref)
    print(f"gated dense {dtype} B={B}: rel err {e:.2e}")
    assert e <= TOL[dtype]
    out2 = blk(x)   # graph replay
    np.testing.assert_array_equal(np.asarray(out), np.asarray(out2))
    if dtype == "float32":
        # the same as the per-layer composition with the reference-named SwiGLU entry point
        g, u = blk.gate_kan(x), blk.up_kan(x)
        hid = np.empty_like(g)
        assert gpu.metal_kan_swiglu_forward(g.ctypes.data, u.ctypes.data, hid.ctypes.data, g.size) == 0
        np.testing.assert_array_equal(out, blk.down_kan(hid))


def test_gated_kan_dense_block_async(gpu):
    """Async mode (metal_kan_set_async): results land at metal_kan_sync(), equal to the synchronous ones."""
    import metal_kans as mk
    np.random.seed(3)
    blk = mk.GatedKAN(d_model=40, d_ffn=64, degree=4)
    xs = [np.random.uniform(-1, 1, (50, 40)).astype(np.float32) for _ in range(4)]
    sync = [blk(x) for x in xs]
    mk.set_async(True)
    try:
        outs = [blk(x) for x in xs]
        mk.sync()
    finally:
        mk.set_async(False)
    for a, b in zip(outs, sync):
        np.testing.assert_array_equal(a, b)

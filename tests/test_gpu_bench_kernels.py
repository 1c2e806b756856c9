"""Parity of the exact kernels bench.py times: 16-bit device x into the 8-wave block kernel.

bench.py uploads x in the layer's own 16-bit type (fp16 bits, or bf16 bits for a bf16 layer) and runs
``kans_layer_forward`` on device buffers, so its launches use the ``kan_fused_block<T, TX = T, TY = T, ...>``
instantiation -- the reference's ``.half()`` semantics, where the layer casts x to the weight dtype
(cheby_kan.py:97-101; the reference's own fp16 test, tests/test_metal_kans.py:257-308).  These tests build
each timed workload with bench.py's own helpers (same seeds, draw order, input transforms and upload),
run the same entry point, and check:

* the kernel that ran, through ``kans_layer_kernel_ex`` (T, TX and TY in template order, basis variant,
  tile, waves, no feature split);
* seeded sampled rows against the float64 oracle on the 16-bit-rounded x with the original fp32 weights
  (max|y - y_ref| / max|y_ref| <= 2e-2);
* the same rows against the oracle with the layer's 16-bit weights, grid and MFMA operands rounded as the
  kernel feeds them (fp16 <= 2e-3: one output rounding of 2^-11 plus fp32 accumulation; bf16 <= 1e-2: one
  output rounding of 2^-8);
* a second launch bitwise equal to the first.

Each workload also runs on a ragged 300 x 200 -> 150 layer (the last 16-feature block half padding, the
last 32-column block partly padding) forced onto the same (32, 8) 8-wave tile.
"""
import ctypes

import numpy as np
import pytest

import bench
from metal_kans._engine import to_bf16_bits
from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu

DT_NAME = {"f16": "float16", "bf16": "bfloat16"}
T_NAME = {"f16": "_Float16", "bf16": "__bf16"}
DT_CODE = {"f16": 1, "bf16": 2}


def _ln_normal(rng, B, d):
    return O.layer_norm(rng.normal(0, 1, (B, d)).astype(np.float32))


def _unif(lo, hi):
    return lambda rng, B, d: rng.uniform(lo, hi, (B, d)).astype(np.float32)


# (name, basis, B, D_in, D_out, K, dtype, seed, x draw, W std, grid range, basis variant): bench.py's workloads
WORKLOADS = [
    ("cfg3_fastkan_fp16", "rbf", 16384, 1024, 1024, 8, "f16", 1003, _ln_normal, np.sqrt(1.0 / (1024 * 8)),
     (-2.0, 2.0), "BASIS_RBF_REC"),
    ("ns_cheby_fp16", "cheby", 16384, 1024, 1024, 9, "f16", 2001, _unif(-1, 1), np.sqrt(1 / (1024 * 9)),
     (-1.0, 1.0), "BASIS_CHEBY"),
    ("ns_bspline_fp16", "bspline", 16384, 1024, 1024, 8, "f16", 2002, _unif(-1.2, 1.2), np.sqrt(1 / (1024 * 8)),
     (-1.0, 1.0), "BASIS_BSPLINE_TAB"),
    ("cfg4_bspline_bf16", "bspline", 8192, 1024, 4096, 8, "bf16", 1004, _unif(-1.2, 1.2), np.sqrt(1 / (1024 * 8)),
     (-1.0, 1.0), "BASIS_BSPLINE_TAB"),
]


def _params(L, kind):
    if kind == "cheby":
        return {"K": L.degree}
    if kind == "rbf":
        return {"grid": np.asarray(L.grid, np.float64), "inv_den": float(L.inv_denominator)}
    return {"G": L.grid_size, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])}


def _to16(a, dtype):
    """fp32 values rounded to the 16-bit type, returned as float64."""
    a = np.asarray(a, np.float32)
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float64)
    return O.bf16_to_f32(to_bf16_bits(a)).reshape(a.shape).astype(np.float64)


def _from_bits(u16, dtype):
    return (u16.view(np.float16).astype(np.float32) if dtype == "f16"
            else O.bf16_to_f32(u16).reshape(u16.shape))


def _run_case(gpu, kind, B, d_in, d_out, K, dtype, seed, x_fn, w_std, grid_range, variant, force_tile, nrows):
    import metal_kans as mk
    rng = np.random.default_rng(seed)
    x = x_fn(rng, B, d_in)
    # bench.make_layer draws W then W_base from the same generator after x; cast afterwards so the fp32
    # originals stay available for the oracle
    L = bench.make_layer(mk, kind, d_in, d_out, K, "f32", rng, w_std, grid_range)
    W32 = np.array(getattr(L, L._weight_attr), np.float64)
    Wb32 = np.array(L.w_base, np.float64)
    bias32 = np.array(L.bias, np.float64)
    p32 = _params(L, kind)
    if dtype == "f16":
        L.half()
    else:
        L.bfloat16()
    p16 = _params(L, kind)
    eng = bench.device_layer(L, dtype)
    if force_tile:
        assert gpu.kans_layer_set_tiling(eng.handle, 32, 8, 1) == 0
    name = ctypes.create_string_buffer(200)
    assert gpu.kans_layer_kernel_ex(eng.handle, B, DT_CODE[dtype], DT_CODE[dtype], name, 200) == 0
    t = T_NAME[dtype]
    assert name.value.decode() == f"kans::kan_fused_block<{t}, {t}, {t}, {variant}, 32, 8, 8 waves>", name.value

    xh = bench.host_input(x, dtype)            # the 16-bit bits bench.py uploads
    xd = bench.DevBuf(gpu, xh.nbytes)
    yd = bench.DevBuf(gpu, B * d_out * 2)
    try:
        xd.upload(xh)
        outs = []
        for _ in range(2):
            assert gpu.kans_layer_forward(eng.handle, xd.p, d_in, yd.p, d_out, B, None) == 0, gpu.kans_last_error()
            assert gpu.kans_synchronize() == 0
            outs.append(yd.download(np.empty((B, d_out), np.uint16)))
    finally:
        xd.free()
        yd.free()
    np.testing.assert_array_equal(outs[0], outs[1])
    y = _from_bits(outs[0], dtype)
    assert np.isfinite(y).all()

    rows = np.sort(np.random.default_rng(seed + 77).choice(B, min(nrows, B), replace=False))
    x16 = _to16(x[rows], dtype)
    y_ref = O.kan_forward(kind, x16, W32, Wb32, bias32, p32)
    ops = DT_NAME[dtype]
    W16 = np.asarray(getattr(L, L._weight_attr), np.float32).astype(np.float64)
    Wb16 = np.asarray(L.w_base, np.float32).astype(np.float64)
    b16 = np.asarray(L.bias, np.float32).astype(np.float64)
    y_ops = O.kan_forward(kind, x16, W16, Wb16, b16, p16, operands=ops)
    e_ref, e_ops = O.rel_err(y[rows], y_ref), O.rel_err(y[rows], y_ops)
    print(f"{kind} {dtype} {B}x{d_in}->{d_out}: rel err vs fp32 weights {e_ref:.2e}, "
          f"vs operand-rounded oracle {e_ops:.2e}", flush=True)
    assert e_ref <= 2e-2
    assert e_ops <= (2e-3 if dtype == "f16" else 1e-2)


@pytest.mark.parametrize("wl", WORKLOADS, ids=[w[0] for w in WORKLOADS])
def test_bench_workload_full_shape(gpu, wl):
    """The timed workload itself: its shape, seed, input transform and 16-bit device x."""
    name, kind, B, di, do, K, dt, seed, xf, ws, gr, variant = wl
    print(f"case {name}", flush=True)
    _run_case(gpu, kind, B, di, do, K, dt, seed, xf, ws, gr, variant, force_tile=False, nrows=48)


@pytest.mark.parametrize("wl", WORKLOADS, ids=[w[0] for w in WORKLOADS])
def test_bench_kernel_ragged(gpu, wl):
    """The same instantiation on 300 x 200 -> 150 (ragged rows, half-padded last feature block, partly
    padded last column block), forced onto the (32, 8) 8-wave tile; every row checked."""
    name, kind, _, _, _, K, dt, seed, xf, ws, gr, variant = wl
    print(f"case {name} ragged", flush=True)
    _run_case(gpu, kind, 300, 200, 150, K, dt, seed + 5, xf, ws, gr, variant, force_tile=True, nrows=300)

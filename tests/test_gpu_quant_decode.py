"""GPU parity of the fused quantized decode path (INT4 / INT8 group 64, ternary group 32).

Parity target (quantization.py:168-171): the forward on the dequantized weights,
dequant(quant(W)), evaluated by the float64 oracle.  The decode kernel feeds the
basis values to the MFMAs in fp16, so the bar is the 16-bit one, 2e-2 (the
measured error is ~1e-3); the reference-named fp32 ternary entry point keeps the
fp32 bar, 1e-4.  Packed weights come from the oracle's quantizers (pinned
against the reference's NumPy fallback in tests/test_oracle.py).
"""
import ctypes

import numpy as np
import pytest

from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu

DT_F32, DT_F16, DT_BF16 = 0, 1, 2


def _quant_int4(W):
    q, s, b, pad = O.quantize_affine(W, 4, 64)
    deq = O.dequantize_affine(q, s, b, 4, 64, W.shape, pad)
    return (np.ascontiguousarray(q), np.ascontiguousarray(s, np.float32).ravel(),
            np.ascontiguousarray(b, np.float32).ravel()), deq


def _quant_int8(W):
    q, s, b, pad = O.quantize_affine(W, 8, 64)
    deq = O.dequantize_affine(q, s, b, 8, 64, W.shape, pad)
    return (np.ascontiguousarray(q), np.ascontiguousarray(s, np.float32).ravel(),
            np.ascontiguousarray(b, np.float32).ravel()), deq


def _quant_tern(W):
    p, s = O.quantize_ternary(W, 32)
    deq = O.dequantize_ternary(p, s, W.shape, 32)
    return (np.ascontiguousarray(p), np.ascontiguousarray(s, np.float32)), deq


def make_qlayer(lib, fmt, d_in, d_out, K, base, bias, seed, bias_dtype=DT_F32):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.05, (d_out, d_in * K)).astype(np.float32)
    Wb = rng.normal(0, 0.1, (d_out, d_in)).astype(np.float32) if base else None
    bv = rng.normal(0, 0.1, d_out).astype(np.float32) if bias else None
    h = ctypes.c_void_p()
    bdev = None
    if bv is not None:
        bdev = bv.astype(np.float16) if bias_dtype == DT_F16 else bv
        bv = bdev.astype(np.float32)   # the values the layer holds
    bptr = bdev.ctypes.data if bdev is not None else None
    if fmt in ("int4", "int8"):
        qf = _quant_int4 if fmt == "int4" else _quant_int8
        pw, dW = qf(W)
        pb, dWb = qf(Wb) if base else ((None, None, None), None)
        keep = (pw, pb)
        cfn = lib.kans_qlayer_create_int4 if fmt == "int4" else lib.kans_qlayer_create_int8
        rc = cfn(d_in, d_out, K, int(base), int(bias), 64, *[a.ctypes.data if a is not None else None for a in pw + pb],
                 bptr, bias_dtype, ctypes.byref(h))
    else:
        pw, dW = _quant_tern(W)
        pb, dWb = _quant_tern(Wb) if base else ((None, None), None)
        keep = (pw, pb)
        rc = lib.kans_qlayer_create_ternary(d_in, d_out, K, int(base), int(bias), 32,
                                            *[a.ctypes.data if a is not None else None for a in pw + pb],
                                            bptr, bias_dtype, ctypes.byref(h))
    assert rc == 0, lib.kans_last_error()
    del keep
    return h, {"W": dW, "W_base": dWb, "bias": bv, "K": K}


SHAPES = [(100, 70, 4, True, True), (256, 130, 3, True, False), (64, 48, 4, False, True), (33, 17, 5, True, True)]
FMTS = ["int4", "int8", "ternary"]


def _oracle_phi16(L, x):
    """float64 forward on the exact dequantized weights with the basis operands the decode kernel feeds its
    MFMAs: T_k(clamp x) and SiLU(x) evaluated in fp32 and rounded to fp16.  The kernel then only adds fp32
    rounding of its accumulations, so a wrong code, byte / nibble order, group parameter or index shows far
    above the bar this is checked at."""
    r16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float64)  # noqa: E731
    x32 = np.asarray(x, np.float32)
    B = x32.shape[0]
    y = r16(O.cheby_basis(x32, L["K"], np.float32).reshape(B, -1)) @ np.asarray(L["W"], np.float64).T
    if L["W_base"] is not None:
        y += r16(O.silu(x32)) @ np.asarray(L["W_base"], np.float64).T
    if L["bias"] is not None:
        y += L["bias"].astype(np.float64)
    return y


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}K{s[2]}b{int(s[3])}{int(s[4])}")
def test_qlayer_decode(gpu, fmt, shape):
    lib = gpu
    d_in, d_out, K, base, bias = shape
    h, ref_l = make_qlayer(lib, fmt, d_in, d_out, K, base, bias, seed=d_in + d_out)
    try:
        rng = np.random.default_rng(7)
        for B in (1, 2, 3, 4, 16, 17, 32):  # B <= 2: k_qgemv (SR = B); 2 < B <= 32: k_qgemv_wg (MT = 1, 2)
            x = rng.uniform(-1.3, 1.3, (B, d_in)).astype(np.float32)
            ref = O.kan_forward("cheby", x, ref_l["W"], ref_l["W_base"], ref_l["bias"], {"K": K})
            for xdt, xin in ((DT_F32, x), (DT_F16, x.astype(np.float16))):
                y = np.empty((B, d_out), np.float32)
                assert lib.kans_qlayer_forward_host(h, xin.ctypes.data, xdt, y.ctypes.data, DT_F32, B) == 0, \
                    lib.kans_last_error()
                r = ref if xdt == DT_F32 else O.kan_forward("cheby", xin.astype(np.float32), ref_l["W"],
                                                            ref_l["W_base"], ref_l["bias"], {"K": K})
                e = O.rel_err(y, r)
                eop = O.rel_err(y, _oracle_phi16(ref_l, xin.astype(np.float32)))
                print(f"{fmt} {shape} B={B} x_dtype={xdt}: rel err {e:.2e}, {eop:.2e} vs fp16-operand oracle")
                assert e <= 2e-2
                assert e <= 5e-3  # fp16 basis operands: observed ~1e-3
                assert eop <= 1e-4
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("B", [1, 2, 5, 32])
def test_qlayer_decode_io_dtypes(gpu, fmt, B):
    """Every input and output dtype of the decode path.  The split-K reduce adds the partial sums in
    fp32 and converts once, so fp16 / bf16 outputs equal the fp32 output rounded to that type bit for
    bit; bf16 inputs (RNE bit patterns) match the oracle on the rounded inputs."""
    lib = gpu
    d_in, d_out, K = 100, 70, 4
    h, ref_l = make_qlayer(lib, fmt, d_in, d_out, K, True, True, seed=41 + B)
    try:
        x = np.random.default_rng(B).uniform(-1.2, 1.2, (B, d_in)).astype(np.float32)
        y32 = np.empty((B, d_out), np.float32)
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, DT_F32, y32.ctypes.data, DT_F32, B) == 0, \
            lib.kans_last_error()
        y16 = np.empty((B, d_out), np.float16)
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, DT_F32, y16.ctypes.data, DT_F16, B) == 0
        assert np.array_equal(y16, y32.astype(np.float16))
        yb = np.empty((B, d_out), np.uint16)
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, DT_F32, yb.ctypes.data, DT_BF16, B) == 0
        assert np.array_equal(yb, O.bf16_round(y32))
        xb = O.bf16_round(x)
        xbf = (xb.astype(np.uint32) << 16).view(np.float32)
        yx = np.empty((B, d_out), np.float32)
        assert lib.kans_qlayer_forward_host(h, xb.ctypes.data, DT_BF16, yx.ctypes.data, DT_F32, B) == 0
        ref = O.kan_forward("cheby", xbf, ref_l["W"], ref_l["W_base"], ref_l["bias"], {"K": K})
        assert O.rel_err(yx, ref) <= 2e-2
    finally:
        lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", FMTS)
def test_weight_load_modes_identical(gpu, fmt):
    """Plain and non-temporal weight-record loads (kans_decode_set_weight_loads 1 / 2) change only the
    cache policy: a single layer and a GatedKAN block give the same output bit for bit in both modes,
    through the small-batch kernel (B = 1, 2) and the workgroup kernel (B = 5, 32).  The call
    returns the previous mode and refuses modes outside 0..2."""
    lib = gpu
    d, hdim = 96, 200
    layers = [make_qlayer(lib, fmt, di, do, 4, True, True, seed=300 + i)[0]
              for i, (di, do) in enumerate(((d, hdim), (d, hdim), (hdim, d)))]
    single, _ = make_qlayer(lib, fmt, 130, 70, 3, True, True, seed=310)
    blk = ctypes.c_void_p()
    assert lib.kans_gated_create(*layers, ctypes.byref(blk)) == 0, lib.kans_last_error()
    try:
        assert lib.kans_decode_set_weight_loads(3) < 0 and lib.kans_decode_set_weight_loads(-1) < 0
        for B in (1, 2, 5, 32):
            xg = np.random.default_rng(B).normal(0, 1, (B, d)).astype(np.float16)
            xs = np.random.default_rng(B + 1).uniform(-1.2, 1.2, (B, 130)).astype(np.float32)
            outs = []
            for mode in (1, 2):
                assert lib.kans_decode_set_weight_loads(mode) in (0, 1, 2)
                try:
                    yg = np.empty((B, d), np.float32)
                    assert lib.kans_gated_forward_host(blk, xg.ctypes.data, DT_F16, yg.ctypes.data, DT_F32, B,
                                                       0) == 0, lib.kans_last_error()
                    ys = np.empty((B, 70), np.float32)
                    assert lib.kans_qlayer_forward_host(single, xs.ctypes.data, DT_F32, ys.ctypes.data, DT_F32,
                                                        B) == 0, lib.kans_last_error()
                finally:
                    prev = lib.kans_decode_set_weight_loads(0)
                assert prev == mode
                outs.append((yg, ys))
            assert np.isfinite(outs[0][0]).all() and np.isfinite(outs[0][1]).all()
            assert np.array_equal(outs[0][0], outs[1][0]), B
            assert np.array_equal(outs[0][1], outs[1][1]), B
    finally:
        lib.kans_decode_set_weight_loads(0)
        lib.kans_gated_destroy(blk)
        for h in layers + [single]:
            lib.kans_qlayer_destroy(h)


def test_qlayer_rejects(gpu):
    lib = gpu
    h, _ = make_qlayer(lib, "int4", 64, 32, 4, True, False, seed=1)
    try:
        x = np.zeros((33, 64), np.float32)
        y = np.empty((33, 32), np.float32)
        # B > 32 runs the prefill kernel, B = 0 does nothing, B < 0 and bad dtypes are refused
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, DT_F32, y.ctypes.data, DT_F32, 33) == 0
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, DT_F32, y.ctypes.data, DT_F32, 0) == 0
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, DT_F32, y.ctypes.data, DT_F32, -1) < 0
        assert lib.kans_qlayer_forward_host(h, x.ctypes.data, 7, y.ctypes.data, DT_F32, 4) < 0
    finally:
        lib.kans_qlayer_destroy(h)
    out = ctypes.c_void_p()
    q = np.zeros(64 * 32, np.uint8)
    s = np.ones(64, np.float32)
    assert lib.kans_qlayer_create_int4(64, 32, 1, 0, 0, 32, q.ctypes.data, s.ctypes.data, s.ctypes.data,
                                       None, None, None, None, DT_F32, ctypes.byref(out)) < 0  # group 32


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("B,biased", [(1, False), (8, False), (32, False), (1, True), (17, True)])
def test_gated_block_decode(gpu, fmt, B, biased):
    """Fused GatedKAN block vs down(SiLU(gate(x)) * up(x)) on dequantized weights; the biased case
    gives gate an fp32 bias, up an fp16 bias and down an fp32 bias."""
    lib = gpu
    d, hdim, K = 96, 200, 4
    layers, refs = [], []
    for i, (di, do) in enumerate(((d, hdim), (d, hdim), (hdim, d))):
        h, r = make_qlayer(lib, fmt, di, do, K, True, biased, seed=100 + i,
                           bias_dtype=DT_F16 if (biased and i == 1) else DT_F32)
        layers.append(h)
        refs.append(r)
    blk = ctypes.c_void_p()
    assert lib.kans_gated_create(*layers, ctypes.byref(blk)) == 0, lib.kans_last_error()
    try:
        x = np.random.default_rng(B).normal(0, 1, (B, d)).astype(np.float16)
        ref = O.gated_forward(x.astype(np.float32), *refs)
        for round16 in (0, 1):
            y = np.empty((B, d), np.float32)
            assert lib.kans_gated_forward_host(blk, x.ctypes.data, DT_F16, y.ctypes.data, DT_F32, B, round16) == 0, \
                lib.kans_last_error()
            e = O.rel_err(y, ref)
            print(f"gated {fmt} B={B} round16={round16}: rel err {e:.2e}")
            assert e <= 2e-2
        ms = ctypes.c_float()
        xd, yd = ctypes.c_void_p(), ctypes.c_void_p()
        assert lib.kans_dev_malloc(ctypes.byref(xd), x.nbytes) == 0
        assert lib.kans_dev_malloc(ctypes.byref(yd), B * d * 2) == 0
        try:
            assert lib.kans_memcpy_h2d(xd, x.ctypes.data, x.nbytes) == 0
            outs = []
            for graph in (0, 1):
                assert lib.kans_gated_time(blk, xd, DT_F16, yd, DT_F16, B, 1, 3, graph, ctypes.byref(ms)) == 0, \
                    lib.kans_last_error()
                y16 = np.empty((B, d), np.float16)
                assert lib.kans_memcpy_d2h(y16.ctypes.data, yd, y16.nbytes) == 0
                assert O.rel_err(y16.astype(np.float32), ref) <= 2e-2
                outs.append(y16)
            assert np.array_equal(outs[0], outs[1])  # graph replays give the eager result
            # a decode step of one block captured as one graph (kans_gated_time_step): X -> Y
            arr = (ctypes.c_void_p * 1)(blk.value)
            assert lib.kans_gated_time_step(arr, 1, xd, yd, DT_F16, B, 1, 3, ctypes.byref(ms)) == 0, \
                lib.kans_last_error()
            assert ms.value > 0
            y16 = np.empty((B, d), np.float16)
            assert lib.kans_memcpy_d2h(y16.ctypes.data, yd, y16.nbytes) == 0
            assert np.array_equal(y16, outs[0])
            assert lib.kans_gated_time_step(arr, 1, xd, yd, DT_F16, 0, 1, 3, ctypes.byref(ms)) == -1  # bad B
        finally:
            lib.kans_dev_free(xd)
            lib.kans_dev_free(yd)
        assert lib.kans_gated_stream_bytes(blk, B) > 0
    finally:
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("B", [1, 2, 32])
def test_gated_decode_step_graph(gpu, fmt, B):
    """kans_gated_time_step: three blocks chained x -> y -> x -> y (x = X's buffer, y = Y's).  The
    uncaptured step leaves x2 = f2(f1(x)) in X; one graph replay then leaves f2(f1(x2)) in X and
    f3(f2(f1(x2))) in Y, bit for bit the eager block forwards (round16 on, fp16 activations, as the
    step runs them)."""
    lib = gpu
    d, hdim, K = 96, 200, 4
    layers, blocks = [], []
    for bi in range(3):
        ls = []
        for i, (di, do) in enumerate(((d, hdim), (d, hdim), (hdim, d))):
            h, _ = make_qlayer(lib, fmt, di, do, K, True, bi == 1, seed=300 + 10 * bi + i)
            ls.append(h)
        blk = ctypes.c_void_p()
        assert lib.kans_gated_create(*ls, ctypes.byref(blk)) == 0, lib.kans_last_error()
        layers += ls
        blocks.append(blk)
    xd, yd = ctypes.c_void_p(), ctypes.c_void_p()
    try:
        x = np.random.default_rng(40 + B).normal(0, 1, (B, d)).astype(np.float16)
        chain = [x]
        for blk in blocks:
            y = np.empty((B, d), np.float16)
            assert lib.kans_gated_forward_host(blk, chain[-1].ctypes.data, DT_F16, y.ctypes.data, DT_F16, B, 1) == 0, \
                lib.kans_last_error()
            chain.append(y)
        assert lib.kans_dev_malloc(ctypes.byref(xd), x.nbytes) == 0
        assert lib.kans_dev_malloc(ctypes.byref(yd), x.nbytes) == 0
        assert lib.kans_memcpy_h2d(xd, x.ctypes.data, x.nbytes) == 0
        arr = (ctypes.c_void_p * 3)(*[b.value for b in blocks])
        ms = ctypes.c_float()
        # no warm-up, one timed replay
        assert lib.kans_gated_time_step(arr, 3, xd, yd, DT_F16, B, 0, 1, ctypes.byref(ms)) == 0, \
            lib.kans_last_error()
        assert ms.value > 0
        got_x, got_y = np.empty_like(x), np.empty_like(x)
        assert lib.kans_memcpy_d2h(got_x.ctypes.data, xd, x.nbytes) == 0
        assert lib.kans_memcpy_d2h(got_y.ctypes.data, yd, x.nbytes) == 0
        print(f"step {fmt} B={B}: {ms.value * 1e3:.1f} us per block")
        assert np.isfinite(chain[3].astype(np.float32)).all()
        x2 = chain[2]
        ref = [x2]
        for blk in blocks:
            y = np.empty((B, d), np.float16)
            assert lib.kans_gated_forward_host(blk, ref[-1].ctypes.data, DT_F16, y.ctypes.data, DT_F16, B, 1) == 0
            ref.append(y)
        assert np.array_equal(got_x, ref[2])
        assert np.array_equal(got_y, ref[3])
        assert lib.kans_gated_time_step(arr, 3, xd, yd, 9, B, 0, 1, ctypes.byref(ms)) < 0  # bad dtype
    finally:
        for p_ in (xd, yd):
            if p_.value:
                lib.kans_dev_free(p_)
        for blk in blocks:
            lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


GATED_EDGE = [  # d, h, K of gate/up, K of down, down has base, biased
    (96, 200, 4, 4, True, True), (40, 65, 3, 5, False, False), (128, 64, 4, 1, True, True),
    (72, 130, 2, 32, True, False), (512, 1000, 4, 4, True, True), (2048, 256, 4, 4, True, True)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("cfg", GATED_EDGE, ids=lambda c: "d{}h{}K{}-{}b{}{}".format(*c[:4], int(c[4]), int(c[5])))
def test_gated_fused_epilogue_matches_unfused(gpu, fmt, cfg):
    """SwiGLU and the down layer's basis in one step -- the gate|up GEMV's epilogue at B <= 2 (the
    last wave of each 64-feature group reduces the split-K partials), k_swiglu_basis at B > 2: the
    output must equal the separate-kernel path bit for bit, also on a repeated call (the arrival
    counters reset themselves), for h not a multiple of 64, odd K, K = 1 and K = 32 in the down
    layer, with and without its base branch, with 1 to 20 split-K waves per matrix and group."""
    lib = gpu
    d, hdim, Kg, Kd, base_d, biased = cfg
    layers, refs = [], []
    for i, (di, do, K, base) in enumerate(((d, hdim, Kg, True), (d, hdim, Kg, True), (hdim, d, Kd, base_d))):
        h, r = make_qlayer(lib, fmt, di, do, K, base, biased, seed=200 + i,
                           bias_dtype=DT_F16 if (biased and i == 1) else DT_F32)
        layers.append(h)
        refs.append(r)
    blk = ctypes.c_void_p()
    assert lib.kans_gated_create(*layers, ctypes.byref(blk)) == 0, lib.kans_last_error()

    def run(x, B, round16):
        y = np.full((B, d), np.nan, np.float32)
        assert lib.kans_gated_forward_host(blk, x.ctypes.data, DT_F16, y.ctypes.data, DT_F32, B, round16) == 0, \
            lib.kans_last_error()
        return y

    try:
        for B in (1, 2, 5, 32):  # B <= 2: GEMV epilogue; B > 2: k_swiglu_basis
            x = np.random.default_rng(B + d).normal(0, 1, (B, d)).astype(np.float16)
            ref = O.gated_forward(x.astype(np.float32), *refs)
            for round16 in (0, 1, 2):
                assert lib.kans_gated_set_fused_swiglu(1) == 1
                try:
                    y1, y1b = run(x, B, round16), run(x, B, round16)
                    lib.kans_gated_set_fused_swiglu(0)
                    y0 = run(x, B, round16)
                finally:
                    lib.kans_gated_set_fused_swiglu(1)
                print(f"{fmt} {cfg} B={B} round16={round16}: rel err {O.rel_err(y1, ref):.2e}")
                assert np.isfinite(y1).all()
                assert np.array_equal(y1, y0), np.max(np.abs(y1 - y0))
                assert np.array_equal(y1, y1b)
                if round16 < 2:
                    assert O.rel_err(y1, ref) <= 2e-2
    finally:
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


PRE_CFGS = [  # d, h, K and base branch of gate / up (K = 4 and 8 take the whole-block basis path)
    (96, 200, 1, True), (100, 70, 5, False), (130, 64, 32, True), (2048, 256, 4, True), (33, 17, 3, True),
    (1000, 96, 8, True), (333, 80, 4, False), (3001, 64, 4, True)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("cfg", PRE_CFGS, ids=lambda c: "d{}h{}K{}b{}".format(*c[:3], int(c[3])))
def test_gated_pre_basis_matches_kprep(gpu, fmt, cfg):
    """The gate|up GEMV can compute the basis of x itself, each wave for its own superchunk range
    in LDS (kans_decode_set_pre_basis: mode 1, the default, at B = 1; mode 2 at B <= 2).  It must
    equal the separate basis kernel (k_prep, mode 0) bit for bit, for every input dtype, with and
    without the base branch, K = 1 to 32 (a feature's basis values split across two waves'
    ranges), and on a repeated call."""
    lib = gpu
    d, hdim, K, base = cfg
    layers = []
    for i, (di, do, k, b) in enumerate(((d, hdim, K, base), (d, hdim, K, base), (hdim, d, 4, True))):
        layers.append(make_qlayer(lib, fmt, di, do, k, b, True, seed=400 + i)[0])
    blk = ctypes.c_void_p()
    assert lib.kans_gated_create(*layers, ctypes.byref(blk)) == 0, lib.kans_last_error()
    try:
        for B in (1, 2):
            x32 = np.random.default_rng(B + d + K).normal(0, 1, (B, d)).astype(np.float32)
            x32[0, :3] = (1.5, -1.5, 0.0)  # clamped and zero inputs
            xs = {DT_F32: x32, DT_F16: x32.astype(np.float16),
                  DT_BF16: (x32.view(np.uint32) >> 16).astype(np.uint16)}
            for xdt, x in xs.items():
                outs = []
                for pre in (2, 0, 1):
                    prev = lib.kans_decode_set_pre_basis(pre)
                    try:
                        y = np.full((B, d), np.nan, np.float32)
                        assert lib.kans_gated_forward_host(blk, x.ctypes.data, xdt, y.ctypes.data, DT_F32, B, 0) == 0, \
                            lib.kans_last_error()
                    finally:
                        lib.kans_decode_set_pre_basis(prev)
                    outs.append(y)
                assert np.isfinite(outs[0]).all()
                assert np.array_equal(outs[0], outs[1]), (B, xdt, float(np.max(np.abs(outs[0] - outs[1]))))
                assert np.array_equal(outs[0], outs[2])
    finally:
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("quant", FMTS)
def test_gatedkan_python_decode(gpu, quant):
    """GatedKAN(dtype=float16).to_int8() / .to_int4() / .to_ternary() takes the fused block for B <= 32."""
    import metal_kans as mk
    np.random.seed(3)
    blk = mk.GatedKAN(d_model=64, d_ffn=160, degree=4, dtype=np.float16)
    getattr(blk, f"to_{quant}")()
    x = np.random.default_rng(2).normal(0, 1, (5, 64)).astype(np.float16)
    out = blk(x)
    assert blk.__dict__.get("_qblock") is not None
    assert out.shape == (5, 64) and out.dtype == np.float16
    ref = O.gated_forward(x.astype(np.float32), *[{"W": k.w_cheby, "W_base": k.w_base, "K": 4}
                                                   for k in (blk.gate_kan, blk.up_kan, blk.down_kan)])
    assert O.rel_err(out.astype(np.float32), ref) <= 2e-2
    # larger batches take the per-layer path on the dequantized weights
    xb = np.random.default_rng(3).normal(0, 1, (40, 64)).astype(np.float16)
    refb = O.gated_forward(xb.astype(np.float32), *[{"W": k.w_cheby, "W_base": k.w_base, "K": 4}
                                                     for k in (blk.gate_kan, blk.up_kan, blk.down_kan)])
    assert O.rel_err(blk(xb).astype(np.float32), refb) <= 2e-2
    # re-quantizing rebuilds the device block from the new packed weights
    old = blk._qblock
    blk.to_int4() if quant == "ternary" else blk.to_ternary()
    out2 = blk(x)
    assert blk._qblock is not old and blk._qblock.fmt != old.fmt
    ref2 = O.gated_forward(x.astype(np.float32), *[{"W": k.w_cheby, "W_base": k.w_base, "K": 4}
                                                    for k in (blk.gate_kan, blk.up_kan, blk.down_kan)])
    assert O.rel_err(out2.astype(np.float32), ref2) <= 2e-2
    # the dequantized weights stay writeable, as in the reference: an in-place edit (an optimizer's
    # param -= lr * update) retires the packed path for that layer, which then runs on the edited weights
    blk.down_kan.w_cheby[0, :] += np.float32(0.5)
    assert blk._decode_engine() is None
    refe = O.gated_forward(x.astype(np.float32), *[{"W": k.w_cheby, "W_base": k.w_base, "K": 4}
                                                    for k in (blk.gate_kan, blk.up_kan, blk.down_kan)])
    assert O.rel_err(blk(x).astype(np.float32), refe) <= 2e-2
    assert O.rel_err(refe, ref2) > 1e-2      # the edit changed the result
    # so does a new array
    getattr(blk, f"to_{quant}")()
    assert blk._decode_engine() is not None
    w = blk.down_kan.w_cheby.copy()
    w[0, 0] += 1.0
    blk.down_kan.w_cheby = w
    assert blk._decode_engine() is None
    refe = O.gated_forward(x.astype(np.float32), *[{"W": k.w_cheby, "W_base": k.w_base, "K": 4}
                                                    for k in (blk.gate_kan, blk.up_kan, blk.down_kan)])
    assert O.rel_err(blk(x).astype(np.float32), refe) <= 2e-2


def test_reference_ternary_entry_point(gpu):
    """metal_kan_forward_ternary_cheby (metal_kan_bridge.mm:4684-4733): fp32, no base."""
    lib = gpu
    rng = np.random.default_rng(11)
    B, Di, Do, deg = 9, 40, 24, 5
    W = rng.normal(0, 0.1, (Do, Di * deg)).astype(np.float32)
    p, s = O.quantize_ternary(W, 32)
    bias = rng.normal(0, 0.1, Do).astype(np.float32)
    x = rng.uniform(-1.2, 1.2, (B, Di)).astype(np.float32)
    y = np.empty((B, Do), np.float32)
    for hb in (0, 1):
        assert lib.metal_kan_forward_ternary_cheby(x.ctypes.data, p.ctypes.data, s.ctypes.data, bias.ctypes.data,
                                                   y.ctypes.data, B, Di, Do, deg, 32, hb) == 0, lib.kans_last_error()
        ref = O.kan_forward("cheby", x, O.dequantize_ternary(p, s, W.shape, 32), None, bias if hb else None,
                            {"K": deg})
        assert O.rel_err(y, ref) <= 1e-4

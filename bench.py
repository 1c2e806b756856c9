#!/usr/bin/env python3
"""Benchmark of the fused KAN layer forward on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 100] [--quick] [--only cfg5,...]

Prints ONE JSON line.  A "step" is one fused forward over one batch with the
inputs already resident in HBM.  The headline workload is BASELINE config 3
(FastKAN Gaussian-RBF, 16384 x 1024 -> 1024, 8 centres on [-2, 2], fp16,
x = LayerNorm(N(0,1)), W ~ N(0, 1/(1024*8))): the north-star MFMA-bound shape.
``value`` is its whole-job throughput in TFLOP/s of algorithmic work
F = 2*B*D_out*D_in*(K + has_base).  The other BASELINE configs are reported
under ``workloads`` (same timing method).  ``roofline`` uses the dominant
kernel's mean duration measured with HIP events on the launch stream;
``cpu_baseline`` times this repo's NumPy restatement of the reference's
four-stage fp32 CPU path on a bounded row sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "metal-kans_amd"))
sys.path.insert(0, ROOT)

PEAK = {"f16": 2516.6, "bf16": 2516.6, "f32": 157.3}   # dense MFMA TFLOP/s (MI355X datasheet)
# Committed summary of the headline kernel's two
# rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) scaled by a copy-kernel
# calibration: the source of roofline.traffic (PMC counters cannot be read
# from inside the timed process).
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_kan_fused_block_cfg3_fastkan_fp16.txt")
SECONDARY = ("python_api", "ns_cheby_fp16", "ns_bspline_fp16", "cfg4_bspline_bf16", "cfg4_bspline_fp32",
             "cfg1_cheby_fp32", "cfg2", "cfg5", "ref_published")
HBM_PEAK_GBS = 8000.0
METRIC = "fused KAN fwd TFLOP/s + % MFMA peak; quantized-weight HBM GB/s (1 MI355X)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class DevBuf:
    def __init__(self, lib, nbytes):
        self.lib = lib
        self.p = ctypes.c_void_p()
        rc = lib.kans_dev_malloc(ctypes.byref(self.p), nbytes)
        if rc:
            raise RuntimeError(lib.kans_last_error().decode())

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert self.lib.kans_memcpy_h2d(self.p, a.ctypes.data, a.nbytes) == 0

    def download(self, a: np.ndarray):
        assert self.lib.kans_memcpy_d2h(a.ctypes.data, self.p, a.nbytes) == 0
        return a

    def free(self):
        if self.p:
            self.lib.kans_dev_free(self.p)
            self.p = ctypes.c_void_p()


def make_layer(mk, kind, d_in, d_out, K, dtype, rng, w_std, grid_range=(-1.0, 1.0)):
    """Layer with weights drawn in the BASELINE order (x drawn first by the caller): W, then W_base."""
    if kind == "cheby":
        L = mk.ChebyKAN(d_in, d_out, degree=K)
    elif kind == "rbf":
        L = mk.FastKAN(d_in, d_out, num_centers=K, grid_range=grid_range)
    else:
        L = mk.BSplineKAN(d_in, d_out, grid_size=K - 3, grid_range=grid_range)
    setattr(L, L._weight_attr, rng.normal(0, w_std, (d_out, d_in * K)).astype(np.float32))
    bound = 1.0 / np.sqrt(d_in)
    L.w_base = rng.uniform(-bound, bound, (d_out, d_in)).astype(np.float32)
    L.bias = np.zeros(d_out, np.float32)
    if dtype == "f16":
        L.half()
    elif dtype == "bf16":
        L.bfloat16()
    return L


def device_layer(L, dtype):
    """Upload the layer's weights; returns the engine (device handle)."""
    from metal_kans._engine import DT_BF16, DT_F16, DT_F32
    eng = L._engine()
    W = getattr(L, L._weight_attr)
    if dtype == "bf16":
        eng.prepare_f32(DT_BF16, W, L.w_base, L.bias, L._basis_params())
    else:
        eng.prepare(DT_F16 if dtype == "f16" else DT_F32, W, L.w_base, L.bias, L._basis_params())
    return eng


def host_input(x: np.ndarray, dtype):
    from metal_kans._engine import to_bf16_bits
    if dtype == "f16":
        return np.ascontiguousarray(x, dtype=np.float16)
    if dtype == "bf16":
        return to_bf16_bits(x)
    return np.ascontiguousarray(x, dtype=np.float32)


# Wall time every timed window is preceded by (GPU busy with the same forward): the first ~60 launches of a
# fresh process run 3-8 % slow while the clock settles, whatever --warmup asks for.
SETTLE_MS = 400.0


def time_layer(lib, eng, xd, yd, B, d_in, d_out, warmup, iters):
    """(kernel_ms, wall_ms): HIP-event and wall-clock means over the same `iters` launches, after `warmup`
    launches and a clock settle of at least SETTLE_MS (kans_layer_time_window)."""
    kms, wms = ctypes.c_float(), ctypes.c_float()
    if warmup:
        rc = lib.kans_layer_time_forward(eng.handle, xd.p, d_in, yd.p, d_out, B, 0, warmup, ctypes.byref(kms))
        if rc:
            raise RuntimeError(lib.kans_last_error().decode())
    rc = lib.kans_layer_time_window(eng.handle, xd.p, d_in, yd.p, d_out, B, ctypes.c_float(SETTLE_MS), iters,
                                    ctypes.byref(kms), ctypes.byref(wms))
    if rc:
        raise RuntimeError(lib.kans_last_error().decode())
    return kms.value, wms.value


def run_layer_workload(lib, mk, name, kind, B, d_in, d_out, K, dtype, seed, x_fn, w_std, warmup, iters,
                       grid_range=(-1.0, 1.0)):
    rng = np.random.default_rng(seed)
    x = x_fn(rng, B, d_in)
    L = make_layer(mk, kind, d_in, d_out, K, dtype, rng, w_std, grid_range)
    eng = device_layer(L, dtype)
    es = 4 if dtype == "f32" else 2
    xd = DevBuf(lib, B * d_in * es)
    yd = DevBuf(lib, B * d_out * es)
    xd.upload(host_input(x, dtype))
    ms, wall = time_layer(lib, eng, xd, yd, B, d_in, d_out, warmup, iters)
    flops = 2.0 * B * d_out * d_in * (K + 1)
    out = {"ms": round(ms, 5), "ms_wall": round(wall, 5), "tflops": round(flops / ms / 1e9, 2),
           "frac_mfma_peak": round(flops / ms / 1e9 / PEAK[dtype], 4),
           "shape": f"{B}x{d_in}->{d_out}", "K": K, "basis": kind, "dtype": dtype}
    if dtype != "f32":
        ceil = mfma_ceiling_same_data(lib, L, x, kind, dtype)
        out["mfma_ceiling_same_data_tflops"] = ceil
        out["frac_of_data_ceiling"] = round(flops / ms / 1e9 / ceil, 4)
    log(f"[bench] {name}: {out}")
    state = {"x": x, "L": L, "eng": eng, "xd": xd, "yd": yd, "flops": flops}
    return out, state


def _bits16(a, dtype):
    """fp32 values -> uint16 bit patterns of the layer's 16-bit operand type."""
    from metal_kans._engine import to_bf16_bits
    a = np.asarray(a, np.float32)
    return to_bf16_bits(a) if dtype == "bf16" else a.astype(np.float16).view(np.uint16)


def _basis_values(L, kind, xs, k):
    """Basis k of the layer at the values xs (fp32): the operand values the fused kernel feeds MFMA."""
    xs = np.asarray(xs, np.float32)
    if kind == "cheby":
        t = np.clip(xs, -1.0, 1.0)
        a, b = np.ones_like(t), t
        for _ in range(k):
            a, b = b, 2.0 * t * b - a
        return a
    if kind == "rbf":
        c = np.float32(np.asarray(L.grid, np.float32).ravel()[k])
        return np.exp(-((xs - c) ** 2) * np.float32(L.inv_denominator))
    gmin, inv_h = (float(v) for v in np.asarray(L.grid_params, np.float64).ravel()[:2])
    G = L.grid_size
    pos = (xs - gmin) * inv_h
    span = np.clip(np.floor(pos), 0, G - 1)
    u = np.clip(pos - span, 0.0, 1.0)
    w = [(1 - u) ** 3 / 6, (3 * u ** 3 - 6 * u ** 2 + 4) / 6, (-3 * u ** 3 + 3 * u ** 2 + 3 * u + 1) / 6, u ** 3 / 6]
    d = k - span
    return sum(np.where(d == j, w[j], 0.0) for j in range(4)).astype(np.float32)


def mfma_ceiling_same_data(lib, L, x, kind, dtype, seed=7, iters=2000):
    """TFLOP/s of back-to-back MFMAs (kans_mfma_ceiling) on 16 A and 16 B operand fragments sampled from
    this layer's own MFMA operands: A = the basis / SiLU values of 32 consecutive rows x 16 features of x
    for one slot, B = the matching W' tile (W for slot k >= 1, W_base for slot 0), in the kernel's fragment
    layout.  The MFMA rate depends on the operand data, so this is the ceiling the fused kernel is measured
    against beside the published peak."""
    rng = np.random.default_rng(seed)
    B, d_in = x.shape
    W = np.asarray(getattr(L, L._weight_attr), np.float32)
    K = W.shape[1] // d_in
    Wb = np.asarray(L.w_base, np.float32)
    d_out = Wb.shape[0]
    lane = np.arange(64)
    a = np.empty((16, 64, 8), np.uint16)
    b = np.empty((16, 64, 8), np.uint16)
    for f in range(16):
        r0 = int(rng.integers(0, B // 32)) * 32
        fb = int(rng.integers(0, d_in // 16))
        s = int(rng.integers(0, K + 1))
        rows = r0 + (lane % 32)
        feats = fb * 16 + 8 * (lane // 32)[:, None] + np.arange(8)[None, :]
        xv = x[rows[:, None], feats]
        av = xv / (1.0 + np.exp(-xv)) if s == 0 else _basis_values(L, kind, xv, s - 1)
        a[f] = _bits16(av, dtype)
        ob = int(rng.integers(0, d_out // 32))
        outs = ob * 32 + (lane % 32)
        bv = Wb[outs[:, None], feats] if s == 0 else W[outs[:, None], feats * K + (s - 1)]
        b[f] = _bits16(bv, dtype)
    t = ctypes.c_double()
    rc = lib.kans_mfma_ceiling(1 if dtype == "f16" else 2, a.ctypes.data, b.ctypes.data, iters, ctypes.byref(t))
    if rc:
        raise RuntimeError(lib.kans_last_error().decode())
    return round(t.value, 1)


def measured_traffic(kernel):
    """HBM bytes per launch of ``kernel`` from the committed PMC summary (``key: value`` lines), or None
    when the summary is missing or was measured on another kernel."""
    try:
        kv = {}
        with open(TRAFFIC_FILE) as f:
            for line in f:
                k, sep, v = line.partition(":")
                if sep and not line.startswith((" ", "#", "|")):
                    kv[k.strip()] = v.strip()
        if kv.get("kernel") != kernel:
            return None
        return int(float(kv["traffic_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


def cpu_env():
    """(cores, description) of the host the CPU baselines run on: BLAS threads = the process's CPU share
    (capped by OMP_NUM_THREADS), CPU model and BLAS library."""
    try:
        from threadpoolctl import threadpool_info
    except Exception:  # pragma: no cover
        threadpool_info = lambda: []  # noqa: E731
    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        cores = min(cores, int(env))
    blas = ""
    try:
        info = threadpool_info()
        blas = ", ".join(f"{i.get('internal_api')} {i.get('version')}" for i in info if i.get("user_api") == "blas")
    except Exception:
        pass
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except Exception:
        pass
    return cores, f"CPU {cpu_model}; BLAS {blas}"


def cpu_time(fn, min_runs=3, budget_s=8.0, max_runs=20, warm=None):
    """Median wall seconds of fn() over at least min_runs calls (more while within budget_s), after one
    warm-up call (``warm``, default fn itself), with BLAS threads = cpu_env()'s cores."""
    try:
        from threadpoolctl import threadpool_limits
    except Exception:  # pragma: no cover
        threadpool_limits = None
    cores, _ = cpu_env()
    ctx = threadpool_limits(limits=cores) if threadpool_limits else None
    times = []
    try:
        (warm or fn)()
        t_start = time.perf_counter()
        while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < max_runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    return float(np.median(times)), len(times)


def _layer_params(L, kind):
    if kind == "cheby":
        return {"K": L.degree}
    if kind == "rbf":
        return {"grid": np.asarray(L.grid, np.float32), "inv_den": L.inv_denominator}
    return {"G": L.grid_size, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])}


def cpu_layer_baseline(name, kind, x, L, dtype, rows, budget_s=8.0):
    """The oracle's fp32 four-stage NumPy forward (SiLU+bias, silu(x)W_base^T, Phi, Phi W^T: the reference's
    stage order, metal_kan_bridge.mm:472-523) on rows 0..rows-1 of the workload's input as the GPU received
    it (16-bit inputs and weights upcast to fp32: NumPy has no fast fp16 GEMM)."""
    from oracle import kan_oracle as O
    B = x.shape[0]
    rows = min(rows, B)
    xs = np.asarray(x[:rows], np.float32)
    if dtype == "f16":
        xs = xs.astype(np.float16).astype(np.float32)
    elif dtype == "bf16":
        xs = O.bf16_to_f32(O.bf16_round(xs)).reshape(xs.shape)
    W = np.asarray(getattr(L, L._weight_attr), dtype=np.float32)
    Wb = np.asarray(L.w_base, dtype=np.float32)
    bias = np.asarray(L.bias, dtype=np.float32)
    params = _layer_params(L, kind)
    fwd = lambda: O.kan_forward(kind, xs, W, Wb, bias, params, acc=np.float32)  # noqa: E731
    t, n = cpu_time(fwd, budget_s=budget_s, warm=lambda: O.kan_forward(kind, xs[:min(rows, 64)], W, Wb, bias, params,
                                                                       acc=np.float32))
    d_out, d_in = Wb.shape
    K = W.shape[1] // d_in
    flops = 2.0 * rows * d_out * d_in * (K + 1)
    cores, env = cpu_env()
    frac = "the whole batch" if rows == B else f"1/{B // rows} of the batch"
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "ms": round(t * 1e3, 3),
            "tokens_per_s": round(rows / t, 1), "cores": cores, "kind": "port",
            "sample": f"{name} rows 0..{rows - 1} of {B} ({frac}), fp32 NumPy four-stage forward "
                      f"(SiLU+bias, silu(x)W_base^T, Phi, Phi W^T), median of {n} runs ({t * 1e3:.1f} ms each); "
                      f"{env}"}


def run_python_api(L, x, flops, kernel_ms, iters=20):
    """The drop-in API end to end at cfg3: ``layer(x)`` on host fp16 arrays, as a user of the reference calls
    it (cheby_kan.py:92-141; the reference times whole host calls the same way, metal_kan_bridge.mm:1250-1371).
    Each call checks the weights for in-place edits (content hash of the weight arrays above 4 MB), stages x
    through pinned memory, copies it to the device, runs the fused kernel and copies y back; ``frozen``
    repeats it after ``layer.freeze_weights()``, which skips the hash."""
    x16 = np.ascontiguousarray(x, dtype=np.float16)

    def med(n):
        L(x16)
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            L(x16)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)) * 1e3
    ms = med(iters)
    L.freeze_weights(True)
    try:
        ms_frozen = med(iters)
    finally:
        L.freeze_weights(False)
    wbytes = int(np.asarray(L.w_rbf).nbytes + np.asarray(L.w_base).nbytes)
    out = {"ms_per_call": round(ms, 3), "ms_per_call_frozen": round(ms_frozen, 3), "kernel_ms": round(kernel_ms, 5),
           "tflops_per_call": round(flops / ms / 1e9, 2), "tflops_per_call_frozen": round(flops / ms_frozen / 1e9, 2),
           "tokens_per_s": round(x16.shape[0] / ms * 1e3, 1), "weight_bytes_checked": wbytes,
           "io_bytes": int(2 * x16.nbytes), "calls": iters,
           "what": "FastKAN.__call__ on a host fp16 x (16384 x 1024) returning a host fp16 y: weight check "
                   "(xxh3 hash of w_rbf and w_base; skipped when frozen), pinned staging, H2D, kernel, D2H, median "
                   "wall clock per call"}
    log(f"[bench] cfg3_python_api_host_call: {out}")
    return out


def run_chain_cfg2(lib, mk, warmup, iters, cpu=True):
    """ChebyKAN MLP 784 -> 256 -> 256 -> 10, K = 9, fp16, B = 4096, one HIP graph."""
    rng = np.random.default_rng(1002)
    B = 4096
    x = rng.uniform(0, 1, (B, 784)).astype(np.float32)
    net = mk.MetalKAN([784, 256, 256, 10], basis_type="cheby", degree=9)
    for layer in net.layers:
        layer.w_cheby = rng.normal(0, np.sqrt(1.0 / (layer.in_features * 9)),
                                   layer.w_cheby.shape).astype(np.float32)
    net.half()
    y = net(x)  # builds the chain and uploads weights
    assert y.shape == (B, 10) and np.isfinite(y.astype(np.float32)).all()
    ms_dev = ctypes.c_float()
    ms_host = ctypes.c_float()
    assert lib.kans_chain_time(net._chain, B, warmup, iters, 0, ctypes.byref(ms_dev)) == 0
    assert lib.kans_chain_time(net._chain, B, warmup, iters, 1, ctypes.byref(ms_host)) == 0
    flops = sum(2.0 * B * l.out_features * l.in_features * 10 for l in net.layers)
    out = {"ms_graph_device": round(ms_dev.value, 5), "ms_graph_with_pcie": round(ms_host.value, 5),
           "tflops": round(flops / ms_dev.value / 1e9, 2),
           "frac_mfma_peak": round(flops / ms_dev.value / 1e9 / PEAK["f16"], 4),
           "tokens_per_s": round(B / ms_dev.value * 1e3, 1), "shape": "4096x[784,256,256,10]", "K": 9,
           "dtype": "f16"}
    if cpu:
        from oracle import kan_oracle as O
        specs = [{"kind": "cheby", "W": np.asarray(l.w_cheby, np.float32), "W_base": np.asarray(l.w_base, np.float32),
                  "bias": np.asarray(l.bias, np.float32), "params": {"K": 9}} for l in net.layers]
        xs = np.asarray(x, np.float32)
        t, n = cpu_time(lambda: O.chain_forward(specs, xs, acc=np.float32),
                        warm=lambda: O.chain_forward(specs, xs[:64], acc=np.float32))
        cores, env = cpu_env()
        out["cpu_baseline"] = {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "ms": round(t * 1e3, 3),
                               "tokens_per_s": round(B / t, 1), "cores": cores, "kind": "port",
                               "sample": f"cfg2 whole batch (4096 rows), fp32 NumPy forward of the three layers "
                                         f"(four stages each), median of {n} runs; {env}"}
    log(f"[bench] cfg2_chain: {out}")
    return out


def _pack(lib, fmt, W, Wb):
    """A float32 (W, W_base) pair packed in the reference format by the native quantizers."""
    arrs = []
    if fmt in ("int4", "int8"):
        for A in (W, Wb):
            ng = A.size // 64
            q = np.empty((ng, 32 if fmt == "int4" else 64), np.uint8)
            s_ = np.empty(ng, np.float32)
            b_ = np.empty(ng, np.float32)
            qfn = lib.metal_kan_quantize_int4 if fmt == "int4" else lib.metal_kan_quantize_int8
            assert qfn(A.ctypes.data, q.ctypes.data, s_.ctypes.data, b_.ctypes.data, ng, 64) == 0
            arrs += [q, s_, b_]
    else:
        for A in (W, Wb):
            kd = A.shape[1]
            p_ = np.zeros((A.shape[0], (kd + 15) // 16), np.uint32)
            s_ = np.zeros((A.shape[0], (kd + 31) // 32), np.float32)
            assert lib.metal_kan_quantize_ternary(A.ctypes.data, p_.ctypes.data, s_.ctypes.data, A.shape[0], kd, 32) == 0
            arrs += [p_, s_]
    return arrs


def _quantized_layer(lib, fmt, W, Wb, K):
    """kans_qlayer from a float32 (W, W_base) pair packed in the reference format (native quantizers)."""
    return _create_qlayer(lib, fmt, Wb.shape, K, _pack(lib, fmt, W, Wb))


def _create_qlayer(lib, fmt, shape, K, arrs):
    d_out, d_in = shape
    h = ctypes.c_void_p()
    if fmt in ("int4", "int8"):
        cfn = lib.kans_qlayer_create_int4 if fmt == "int4" else lib.kans_qlayer_create_int8
        rc = cfn(d_in, d_out, K, 1, 0, 64, *[a.ctypes.data for a in arrs], None, 0, ctypes.byref(h))
    else:
        rc = lib.kans_qlayer_create_ternary(d_in, d_out, K, 1, 0, 32, *[a.ctypes.data for a in arrs], None, 0,
                                            ctypes.byref(h))
    if rc:
        raise RuntimeError(lib.kans_last_error().decode())
    return h


def _dense_dequant_block(lib, packed, shapes, K):
    """Dense fp16 GatedKAN block (kan_fused_block) on INT4 weights dequantized by the library's own
    metal_kan_dequantize_int4 (fp32, then rounded to fp16 on upload): the same weight values the fused INT4
    prefill feeds its MFMAs, moved as 2 bytes per weight."""
    layers = []
    for (d_out, d_in), arrs in zip(shapes, packed):
        q, s_, b_, qb, sb, bb = arrs
        W = np.empty((d_out, d_in * K), np.float32)
        Wb = np.empty((d_out, d_in), np.float32)
        assert lib.metal_kan_dequantize_int4(q.ctypes.data, s_.ctypes.data, b_.ctypes.data, W.ctypes.data,
                                             s_.size, 64) == 0, lib.kans_last_error()
        assert lib.metal_kan_dequantize_int4(qb.ctypes.data, sb.ctypes.data, bb.ctypes.data, Wb.ctypes.data,
                                             sb.size, 64) == 0, lib.kans_last_error()
        h = ctypes.c_void_p()
        assert lib.kans_layer_create(0, 1, d_in, d_out, K, 1, 0, ctypes.byref(h)) == 0, lib.kans_last_error()
        assert lib.kans_layer_load_weights_f32(h, W.ctypes.data, Wb.ctypes.data, None) == 0, lib.kans_last_error()
        layers.append(h)
        del W, Wb
    blk = ctypes.c_void_p()
    assert lib.kans_gated_dense_create(*layers, ctypes.byref(blk)) == 0, lib.kans_last_error()
    return blk, layers


def _dequantized(lib, fmt, arrs, shape, K):
    """fp32 (W, W_base) of one layer from its reference-format packed arrays (library dequantizers,
    bit-identical to quantization.py:136-148 / :275-286)."""
    d_out, d_in = shape
    res = []
    for j, kd in enumerate((d_in * K, d_in)):
        out = np.empty((d_out, kd), np.float32)
        if fmt == "ternary":
            p_, s_ = arrs[2 * j], arrs[2 * j + 1]
            assert lib.metal_kan_dequantize_ternary(p_.ctypes.data, s_.ctypes.data, out.ctypes.data, d_out, kd,
                                                    32) == 0, lib.kans_last_error()
        else:
            q, s_, b_ = arrs[3 * j:3 * j + 3]
            fn = lib.metal_kan_dequantize_int4 if fmt == "int4" else lib.metal_kan_dequantize_int8
            assert fn(q.ctypes.data, s_.ctypes.data, b_.ctypes.data, out.ctypes.data, s_.size, 64) == 0, \
                lib.kans_last_error()
        res.append(out)
    return res


def cpu_cfg5(lib, fmt, packed, shapes, K, xs, out, batches):
    """CPU baseline of the cfg5 lines in the reference's quantized semantics (quantization.py:152-178,
    gated_kan.py:86-138): the weights dequantized to fp32 once (not timed), then the fp32 NumPy GatedKAN
    forward (four stages per layer, SwiGLU with the +-20 clip) on the line's own x, timed per batch."""
    from oracle import kan_oracle as O
    specs = []
    for arrs, shape in zip(packed, shapes):
        W, Wb = _dequantized(lib, fmt, arrs, shape, K)
        specs.append({"W": W, "W_base": Wb, "K": K})
    cores, env = cpu_env()
    for B in batches:
        x = np.asarray(xs[B], np.float32)
        fwd = lambda: O.gated_forward(x, *specs, acc=np.float32)  # noqa: E731
        if B >= 8192:   # one run (about 10-20 s), after a one-row warm-up
            t, n = cpu_time(fwd, min_runs=1, budget_s=0.0, warm=lambda: O.gated_forward(x[:1], *specs, acc=np.float32))
        else:
            t, n = cpu_time(fwd, min_runs=3, budget_s=3.0)
        key = f"cfg5_{fmt}_prefill_b8192" if B >= 8192 else f"cfg5_{fmt}_decode_b{B}"
        line = {"ms": round(t * 1e3, 3), "tokens_per_s": round(B / t, 2), "cores": cores, "kind": "port",
                "sample": f"cfg5 {fmt} GatedKAN at B={B} (the line's own x), weights dequantized to fp32 once "
                          f"(reference semantics), fp32 NumPy forward, median of {n} runs; {env}"}
        if B >= 8192:
            line["value"] = round(2.0 * B * sum(sp["W_base"].size for sp in specs) * (K + 1) / t / 1e12, 4)
            line["unit"] = "TFLOP/s"
        else:
            wb = 4 * sum(sp["W"].size + sp["W_base"].size for sp in specs)
            line["value"] = round(wb / t / 1e9, 1)
            line["unit"] = "GB/s of fp32 weights read"
        out[key]["cpu_baseline"] = line
        log(f"[bench] {key} cpu_baseline: {line}")
    del specs


# Weight copies the decode lines rotate over: each call's weights were last read COPIES - 1 calls earlier,
# so even the ternary block (254 MB, within the 256 MB MALL) streams from HBM, as in a model whose layers
# together exceed the MALL.
COPIES = 3
DECODE_ITERS, DECODE_REPS = 40, 5


def run_cfg5(lib, warmup, iters, cpu=True):
    """GatedKAN d=4096, h=11008, K=4 (base on, no bias), all six weight matrices
    ~N(0, 0.02) then INT4 (group 64) or ternary (group 32), plus the north star's INT8 (group 64); x ~ N(0,1)
    fp16.  Every line times whole block forwards (gate, up, SwiGLU, down) captured in HIP graphs on
    device-resident x / y, with HIP events.  Decode B in {1, 32} (INT4 / ternary GEMVs over the packed
    weights): COPIES blocks with separate device weights (weights from HBM, not the MALL) chained x -> y -> x
    as one decode step captured in ONE graph, time per block (median of DECODE_REPS timings); GB/s = algorithmic bytes (packed codes + group
    parameters + x + y) / time.  Beside it: each block as its own graph, calls cycling through the copies
    (ms_graph_per_block, which also carries one graph launch per block), and the same block replayed alone
    (the MALL-warm rate).  Prefill B = 8192 (fused kernels decoding
    the packed weights into fp16 MFMA tiles, gate|up in one launch with the SwiGLU epilogue): TFLOP/s of
    2*B*(2*h*d + d*h)*(K + 1), and the packed bytes per forward."""
    d, hdim, K = 4096, 11008, 4
    rng = np.random.default_rng(1005)
    t0 = time.perf_counter()
    xs = {B: rng.standard_normal((B, d), dtype=np.float32).astype(np.float16) for B in (1, 32, 8192)}
    mats = []
    for (di, do) in ((d, hdim), (d, hdim), (hdim, d)):
        W = rng.standard_normal((do, di * K), dtype=np.float32) * np.float32(0.02)
        Wb = rng.standard_normal((do, di), dtype=np.float32) * np.float32(0.02)
        mats.append((W, Wb))
    out = {}
    stream_ceiling = {}
    prefill_flops = 2.0 * 8192 * (2 * hdim * d + d * hdim) * (K + 1)
    for fmt in ("int4", "ternary", "int8"):
        packed = [_pack(lib, fmt, W, Wb) for (W, Wb) in mats]
        ncopy = COPIES
        layers, blocks = [], []
        for _ in range(ncopy):
            ls = [_create_qlayer(lib, fmt, Wb.shape, K, arrs) for (W, Wb), arrs in zip(mats, packed)]
            blk = ctypes.c_void_p()
            assert lib.kans_gated_create(*ls, ctypes.byref(blk)) == 0
            layers += ls
            blocks.append(blk)
        blk = blocks[0]
        for B, x in xs.items():
            xd, yd = DevBuf(lib, x.nbytes), DevBuf(lib, x.nbytes)
            xd.upload(x)
            ms = ctypes.c_float()
            it = iters if B < 8192 else max(5, iters // 10)
            rc = lib.kans_gated_time(blk, xd.p, 1, yd.p, 1, B, min(warmup, it), it, 1, ctypes.byref(ms))
            if rc:
                raise RuntimeError(lib.kans_last_error().decode())
            nbytes = lib.kans_gated_stream_bytes(blk, B)
            if B == 8192:
                out[f"cfg5_{fmt}_prefill_b8192"] = {
                    "ms": round(ms.value, 4), "tflops": round(prefill_flops / ms.value / 1e9, 2),
                    "tokens_per_s": round(B / ms.value * 1e3, 1),
                    "frac_mfma_peak": round(prefill_flops / ms.value / 1e9 / PEAK["f16"], 4),
                    "packed_weight_bytes": int(nbytes - 2 * 2 * B * d), "batch": B,
                    "path": "fused prefill: packed weights decoded into fp16 MFMA tiles; gate|up one launch "
                            "with the SwiGLU epilogue, then down"}
            else:
                warm = ms.value
                arr = (ctypes.c_void_p * ncopy)(*[b.value for b in blocks])
                # decode lines are tens of microseconds: median of DECODE_REPS timings of >= DECODE_ITERS
                # replays each, so that one slow stretch (clock, another engine) does not set the line
                dit = max(it, DECODE_ITERS)

                def median_ms(call):
                    vals = []
                    for _ in range(DECODE_REPS):
                        if call():
                            raise RuntimeError(lib.kans_last_error().decode())
                        vals.append(ms.value)
                    return float(np.median(vals))

                per_graph = median_ms(lambda: lib.kans_gated_time_rotate(
                    arr, ncopy, xd.p, 1, yd.p, 1, B, max(ncopy, min(warmup, dit)), dit, ctypes.byref(ms)))
                # the decode step a serving loop replays: the ncopy blocks chained (x -> y -> x ...) in ONE graph
                step = median_ms(lambda: lib.kans_gated_time_step(
                    arr, ncopy, xd.p, yd.p, 1, B, max(2, min(warmup, dit)), dit, ctypes.byref(ms)))
                ms.value = step
                gbs = nbytes / ms.value / 1e6
                if fmt not in stream_ceiling:
                    # one read-only streaming kernel (kans_stream_ceiling) over ncopy times the block's bytes, so
                    # that its repeated launches, like the rotating calls, read from HBM and not the MALL
                    cb = ncopy * ((nbytes + 15) // 16 * 16)
                    sb = DevBuf(lib, cb)
                    g = ctypes.c_double()
                    assert lib.kans_stream_ceiling(sb.p, cb, ctypes.byref(g)) == 0, lib.kans_last_error()
                    sb.free()
                    stream_ceiling[fmt] = round(g.value, 1)
                out[f"cfg5_{fmt}_decode_b{B}"] = {"ms": round(ms.value, 5), "GB_per_s": round(gbs, 1),
                                                  "tokens_per_s": round(B / ms.value * 1e3, 1),
                                                  "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                                  "stream_ceiling_GB_per_s": stream_ceiling[fmt],
                                                  "frac_of_stream_ceiling": round(gbs / stream_ceiling[fmt], 4),
                                                  "bytes": int(nbytes), "batch": B,
                                                  "timing": f"decode step of {ncopy} blocks with separate weights "
                                                            "(from HBM), chained and captured as one HIP graph; "
                                                            "time per block",
                                                  "ms_graph_per_block": round(per_graph, 5),
                                                  "GB_per_s_graph_per_block": round(nbytes / per_graph / 1e6, 1),
                                                  "ms_mall_warm": round(warm, 5),
                                                  "GB_per_s_mall_warm": round(nbytes / warm / 1e6, 1)}
            xd.free()
            yd.free()
        for b in blocks:
            lib.kans_gated_destroy(b)
        for hnd in layers:
            lib.kans_qlayer_destroy(hnd)
        if cpu and fmt in ("int4", "ternary"):
            cpu_cfg5(lib, fmt, packed, [Wb.shape for (W, Wb) in mats], K, xs, out,
                     batches=(1, 32, 8192) if fmt == "int4" else (1, 32))
        if fmt == "int4":
            # reference point measured in the same run: the dense fp16 kernel on the dequantized weights
            dblk, dlayers = _dense_dequant_block(lib, packed, [Wb.shape for (W, Wb) in mats], K)
            x, B = xs[8192], 8192
            y = np.empty_like(x)
            assert lib.kans_gated_dense_forward_host(dblk, x.ctypes.data, 1, y.ctypes.data, B) == 0
            ms = ctypes.c_float()
            it = max(5, iters // 10)
            assert lib.kans_gated_dense_time(dblk, B, min(warmup, it), it, 0, ctypes.byref(ms)) == 0, \
                lib.kans_last_error()
            out["cfg5_int4_dequant_fp16_prefill_b8192"] = {
                "ms": round(ms.value, 4), "tflops": round(prefill_flops / ms.value / 1e9, 2),
                "frac_mfma_peak": round(prefill_flops / ms.value / 1e9 / PEAK["f16"], 4), "batch": B,
                "path": "reference point: dense fp16 GatedKAN (kan_fused_block) on the INT4 weights dequantized "
                        "by metal_kan_dequantize_int4 and rounded to fp16 (2 bytes per weight), same run"}
            lib.kans_gated_dense_destroy(dblk)
            for hnd in dlayers:
                lib.kans_layer_destroy(hnd)
    log(f"[bench] cfg5 ({time.perf_counter() - t0:.1f} s): {out}")
    return out


# The reference's own published points (README.md:147-162, scripts/render_figures.py:29-37): 64 -> 64 fp32
# layers with the SiLU base branch, host wall clock per full call (Apple GPU, unified memory), ms per B.
REF_PUBLISHED_MS = {
    "cheby": {64: 0.279, 1024: 0.362, 4096: 0.812, 16384: 1.659, 65536: 8.995},
    "rbf": {64: 0.268, 1024: 0.318, 4096: 0.710, 16384: 2.366, 65536: 14.815},
    "bspline": {64: 0.258, 1024: 0.339, 4096: 0.782, 16384: 2.347, 65536: 14.857},
}


def run_ref_published(mk, iters):
    """The reference's published benchmark shape: ChebyKAN(64, 64, degree=4), FastKAN(64, 64, 8 centres),
    BSplineKAN(64, 64, grid 5), fp32, timed as the reference times it (layer.benchmark: mean host wall clock
    per full synchronous call, here including the PCIe copies of x and y that unified memory does not need).
    Context beside the published Apple-GPU numbers, not a roofline measurement."""
    rng = np.random.default_rng(1100)
    out = {}
    for kind, K in (("cheby", 4), ("rbf", 8), ("bspline", 8)):
        np.random.seed(1100)
        L = {"cheby": lambda: mk.ChebyKAN(64, 64, degree=4), "rbf": lambda: mk.FastKAN(64, 64, num_centers=8),
             "bspline": lambda: mk.BSplineKAN(64, 64, grid_size=5)}[kind]()
        rows = []
        for B, ref_ms in REF_PUBLISHED_MS[kind].items():
            x = rng.uniform(-1, 1, (B, 64)).astype(np.float32)
            ms = L.benchmark(x, warmup=5, iters=max(10, min(iters, 50)))
            flops = 2.0 * B * 64 * 64 * (K + 1)
            rows.append({"B": B, "ms_per_call": round(ms, 4), "gflops": round(flops / ms / 1e6, 1),
                         "reference_published_ms": ref_ms, "reference_over_this": round(ref_ms / ms, 2)})
        out[kind] = rows
    log(f"[bench] ref_published: {out}")
    return {"ref_published_64x64_fp32_host_call": out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--quick", action="store_true", help="headline only, no secondary workloads / CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", metavar="NAMES",
                    help="comma-separated secondary workloads to run (default all): " + ",".join(SECONDARY))
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="only run kans_copy_device over MIB MiB, 5 times (byte-counter calibration)")
    a = ap.parse_args()
    only = set(filter(None, a.only.split(",")))
    if only - set(SECONDARY):
        ap.error(f"unknown workloads {sorted(only - set(SECONDARY))}")
    want = lambda name: not only or name in only  # noqa: E731
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build measures one GPU only: the layer shards along the batch "
                                   "(rows independent, weights replicated), so N GPUs would each run this "
                                   "benchmark's workload on B/N rows; run with --gpus 1", "n_gpus": a.gpus}))
        sys.exit(2)
    import metal_kans as mk
    lib = mk.get_metal_bridge()
    iters = max(a.steps, 1)
    if a.calib_copy:
        nbytes = a.calib_copy << 20
        src, dst = DevBuf(lib, nbytes), DevBuf(lib, nbytes)
        for _ in range(5):
            assert lib.kans_copy_device(dst.p, src.p, nbytes, None) == 0
        lib.kans_synchronize()
        print(json.dumps({"calib_copy_bytes_read": nbytes, "calib_copy_bytes_written": nbytes, "dispatches": 5}))
        return

    # ---- headline: config 3 ------------------------------------------------
    def ln_normal(rng, B, d):
        from oracle.kan_oracle import layer_norm
        return layer_norm(rng.normal(0, 1, (B, d)).astype(np.float32))

    head, st = run_layer_workload(lib, mk, "cfg3_fastkan_fp16", "rbf", 16384, 1024, 1024, 8, "f16", 1003,
                                  ln_normal, np.sqrt(1.0 / (1024 * 8)), a.warmup, iters, grid_range=(-2.0, 2.0))
    F = st["flops"]
    wall_ms = head["ms_wall"]
    name = ctypes.create_string_buffer(200)
    assert lib.kans_layer_kernel_ex(st["eng"].handle, 16384, 1, 1, name, 200) == 0   # fp16 x and y, as timed
    head_kernel = name.value.decode()
    value = F / wall_ms / 1e9
    kernel_ms = head["ms"]
    assert kernel_ms <= wall_ms * 1.0001, (kernel_ms, wall_ms)   # same window: events inside the wall bracket
    achieved = F / kernel_ms / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": iters,
        "warmup": a.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded NumPy; random-init weights of the BASELINE shapes)",
        "config": {"workload": "cfg3: FastKAN Gaussian-RBF layer, B=16384, 1024->1024, 8 centres on [-2,2], "
                               "fp16, x=LayerNorm(N(0,1)), inputs resident in HBM",
                   "batch": 16384, "d_in": 1024, "d_out": 1024, "K": 8, "has_base": 1,
                   "flops_per_step": F},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK["f16"], "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK["f16"], 4), "traffic": measured_traffic(head_kernel),
                     "traffic_unit": "bytes per launch", "kernel": head_kernel, "kernel_ms": kernel_ms,
                     "timing": f"value and achieved from the same {iters} launches (wall clock between stream "
                               f"synchronisations, and HIP events on the launch stream inside it), after "
                               f"{a.warmup} warm-up launches and >= {SETTLE_MS:.0f} ms of clock-settling launches",
                     "measured_ceiling": {"what": "back-to-back MFMAs on operand fragments sampled from this "
                                                  "layer's own basis values and weights (kans_mfma_ceiling)",
                                          "tflops": head["mfma_ceiling_same_data_tflops"],
                                          "frac": round(achieved / head["mfma_ceiling_same_data_tflops"], 4)}},
    }
    workloads = {"cfg3_fastkan_fp16": head}
    cpu = not (a.quick or a.no_cpu)
    cpu_rows = {"cfg3_fastkan_fp16": 2048, "ns_cheby_fp16": 2048, "ns_bspline_fp16": 2048, "cfg4_bspline_bf16": 1024,
                "cfg4_bspline_fp32": 1024, "cfg1_cheby_fp32": 256}
    if cpu:
        head["cpu_baseline"] = cpu_layer_baseline("cfg3", "rbf", st["x"], st["L"], "f16", cpu_rows["cfg3_fastkan_fp16"])
        log(f"[bench] cfg3 cpu_baseline: {head['cpu_baseline']}")
    if not a.quick and want("python_api"):
        workloads["cfg3_python_api_host_call"] = run_python_api(st["L"], st["x"], F, kernel_ms)
    # the host-call lines run before the workloads that free large device allocations: once a process has
    # freed about 1 GB of device memory, this part's DMA device-to-host copies run at half their rate
    if not a.quick and want("ref_published"):
        workloads.update(run_ref_published(mk, iters))
    if not a.quick:
        unif = lambda lo, hi: (lambda rng, B, d: rng.uniform(lo, hi, (B, d)).astype(np.float32))  # noqa: E731
        for name, kind, B, di, do, K, dt, seed, xf, ws in [
            ("ns_cheby_fp16", "cheby", 16384, 1024, 1024, 9, "f16", 2001, unif(-1, 1), np.sqrt(1 / (1024 * 9))),
            ("ns_bspline_fp16", "bspline", 16384, 1024, 1024, 8, "f16", 2002, unif(-1.2, 1.2), np.sqrt(1 / (1024 * 8))),
            ("cfg4_bspline_bf16", "bspline", 8192, 1024, 4096, 8, "bf16", 1004, unif(-1.2, 1.2), np.sqrt(1 / (1024 * 8))),
            ("cfg4_bspline_fp32", "bspline", 8192, 1024, 4096, 8, "f32", 1004, unif(-1.2, 1.2), np.sqrt(1 / (1024 * 8))),
            ("cfg1_cheby_fp32", "cheby", 256, 64, 64, 9, "f32", 1001, lambda rng, B, d: np.tanh(rng.uniform(-1, 1, (B, d))).astype(np.float32), np.sqrt(1 / (64 * 9))),
        ]:
            if not want(name):
                continue
            out, s2 = run_layer_workload(lib, mk, name, kind, B, di, do, K, dt, seed, xf, ws, a.warmup, iters)
            if cpu:
                out["cpu_baseline"] = cpu_layer_baseline(name, kind, s2["x"], s2["L"], dt, cpu_rows[name])
                log(f"[bench] {name} cpu_baseline: {out['cpu_baseline']}")
            workloads[name] = out
            s2["xd"].free()
            s2["yd"].free()
            del s2
        if want("cfg2"):
            workloads["cfg2_chain_fp16_graph"] = run_chain_cfg2(lib, mk, a.warmup, iters, cpu=cpu)
        if want("cfg5"):
            workloads.update(run_cfg5(lib, a.warmup, iters, cpu=cpu))
    result["workloads"] = workloads
    result["cpu_baseline"] = head.get("cpu_baseline")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

"""kans_gated_forward_noalloc: the zero-allocation variant of kans_gated_forward.

Both entry points run the same kernels on the same inputs, so their outputs must
be identical bit for bit.  Two calls in a row share the scratch array (the
second with a smaller batch, so it reads a prefix the first call left
behind), on the decode GEMVs with the fused SwiGLU epilogue (B <= 2, arrival
counters in the scratch), the workgroup GEMVs (B <= 32) and the prefill
kernels (B > 32).  A call whose workspace exceeds the scratch is refused.
Calls leave the device's free memory unchanged (hipMemGetInfo), and the entry
point can be captured into a HIP graph whose replays, with eager work and
synchronisations between them, equal the eager result.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _block(lib, fmt, d, hdim, seed):
    from test_gpu_qprefill import make_block
    return make_block(lib, fmt, d, hdim, seed=seed)


def _dev(lib, a):
    p = ctypes.c_void_p()
    assert lib.kans_dev_malloc(ctypes.byref(p), a.nbytes) == 0
    assert lib.kans_memcpy_h2d(p, a.ctypes.data, a.nbytes) == 0
    return p


@pytest.mark.parametrize("fmt", ["int4", "int8", "ternary"])
def test_noalloc_matches_allocating_entry_point(gpu, fmt):
    lib = gpu
    d, hdim = 256, 640
    blk, layers, _ = _block(lib, fmt, d, hdim, seed=31)
    bufs = []
    try:
        for pair in ((32, 5), (2, 1), (300, 40)):
            print(f"case {fmt} B={pair}", flush=True)
            for B in pair:
                x = np.random.default_rng(B).normal(0, 1, (B, d)).astype(np.float16)
                xd = _dev(lib, x)
                ya = _dev(lib, np.zeros((B, d), np.float16))
                yb = _dev(lib, np.full((B, d), np.nan, np.float16))
                bufs += [xd, ya, yb]
                assert lib.kans_gated_forward(blk, xd, 1, d, ya, 1, d, B, 1, None) == 0, lib.kans_last_error()
                assert lib.kans_gated_forward_noalloc(blk, xd, 1, d, yb, 1, d, B, 1, None) == 0, \
                    lib.kans_last_error()
                assert lib.kans_synchronize() == 0
                ha = np.empty((B, d), np.float16)
                hb = np.empty((B, d), np.float16)
                assert lib.kans_memcpy_d2h(ha.ctypes.data, ya, ha.nbytes) == 0
                assert lib.kans_memcpy_d2h(hb.ctypes.data, yb, hb.nbytes) == 0
                assert np.isfinite(ha.astype(np.float32)).all()
                np.testing.assert_array_equal(ha.view(np.uint16), hb.view(np.uint16))
    finally:
        for p in bufs:
            lib.kans_dev_free(p)
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


def test_noalloc_refuses_oversized_workspace(gpu):
    """The prefill hidden state of B = 16384 rows x 1024 features (fp32) alone is 64 MiB."""
    lib = gpu
    d, hdim = 64, 1024
    blk, layers, _ = _block(lib, "int4", d, hdim, seed=3)
    bufs = []
    try:
        B = 16384
        xd = _dev(lib, np.zeros((B, d), np.float16))
        yd = _dev(lib, np.zeros((B, d), np.float16))
        bufs += [xd, yd]
        rc = lib.kans_gated_forward_noalloc(blk, xd, 1, d, yd, 1, d, B, 0, None)
        assert rc == -1
        assert b"scratch" in lib.kans_last_error()
    finally:
        for p in bufs:
            lib.kans_dev_free(p)
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    return hip


def _free_bytes(hip):
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _d2h(lib, p, shape):
    h = np.empty(shape, np.float16)
    assert lib.kans_memcpy_d2h(h.ctypes.data, p, h.nbytes) == 0
    return h


@pytest.mark.parametrize("fmt", ["int4", "ternary"])
def test_noalloc_allocates_nothing(gpu, fmt):
    """After one call per batch size, further calls (decode with the fused epilogue, workgroup decode,
    prefill) leave the device's free memory exactly as it was."""
    lib = gpu
    hip = _hip()
    d, hdim = 128, 384
    blk, layers, _ = _block(lib, fmt, d, hdim, seed=41)
    bufs = []
    try:
        io = {}
        for B in (1, 17, 64):
            x = np.random.default_rng(B).normal(0, 1, (B, d)).astype(np.float16)
            io[B] = (_dev(lib, x), _dev(lib, np.zeros((B, d), np.float16)))
            bufs += list(io[B])
        for B, (xd, yd) in io.items():   # first calls: any lazy set-up happens here
            assert lib.kans_gated_forward_noalloc(blk, xd, 1, d, yd, 1, d, B, 1, None) == 0, lib.kans_last_error()
        assert lib.kans_synchronize() == 0
        before = _free_bytes(hip)
        for _ in range(3):
            for B, (xd, yd) in io.items():
                assert lib.kans_gated_forward_noalloc(blk, xd, 1, d, yd, 1, d, B, 1, None) == 0
        assert lib.kans_synchronize() == 0
        assert _free_bytes(hip) == before
    finally:
        for p in bufs:
            lib.kans_dev_free(p)
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)


@pytest.mark.parametrize("fmt", ["int4", "ternary"])
@pytest.mark.parametrize("B", [1, 20, 40])
def test_noalloc_graph_capture(gpu, fmt, B):
    """The entry point captured on a stream into a HIP graph (no allocation, no memset inside), replayed four
    times with eager calls of the allocating entry point and synchronisations between the replays: every
    replay equals the eager result bit for bit."""
    lib = gpu
    hip = _hip()
    d, hdim = 128, 384
    blk, layers, _ = _block(lib, fmt, d, hdim, seed=B + 3)
    bufs = []
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    try:
        x = np.random.default_rng(B).normal(0, 1, (B, d)).astype(np.float16)
        xd, ye, yg = _dev(lib, x), _dev(lib, np.zeros((B, d), np.float16)), _dev(lib, np.zeros((B, d), np.float16))
        bufs += [xd, ye, yg]
        assert lib.kans_gated_forward(blk, xd, 1, d, ye, 1, d, B, 1, None) == 0, lib.kans_last_error()
        assert lib.kans_synchronize() == 0
        eager = _d2h(lib, ye, (B, d))
        assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
        # one eager call on the stream first (lazy set-up outside the capture)
        assert lib.kans_gated_forward_noalloc(blk, xd, 1, d, yg, 1, d, B, 1, stream) == 0
        assert hip.hipStreamSynchronize(stream) == 0
        np.testing.assert_array_equal(_d2h(lib, yg, (B, d)).view(np.uint16), eager.view(np.uint16))
        assert hip.hipStreamBeginCapture(stream, 1) == 0   # hipStreamCaptureModeThreadLocal
        rc = lib.kans_gated_forward_noalloc(blk, xd, 1, d, yg, 1, d, B, 1, stream)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rc == 0, lib.kans_last_error()
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep in range(4):
            zero = np.zeros((B, d), np.float16)
            assert lib.kans_memcpy_h2d(yg, zero.ctypes.data, zero.nbytes) == 0
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            got = _d2h(lib, yg, (B, d))
            np.testing.assert_array_equal(got.view(np.uint16), eager.view(np.uint16), err_msg=f"replay {rep}")
            # eager work of the program between replays
            assert lib.kans_gated_forward(blk, xd, 1, d, ye, 1, d, B, 1, None) == 0
            assert lib.kans_synchronize() == 0
    finally:
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        if stream:
            hip.hipStreamDestroy(stream)
        for p in bufs:
            lib.kans_dev_free(p)
        lib.kans_gated_destroy(blk)
        for h in layers:
            lib.kans_qlayer_destroy(h)

"""kans_gated_forward_noalloc: the zero-allocation variant of kans_gated_forward.

Both entry points run the same kernels on the same inputs, so their outputs must
be identical bit for bit.  Two calls in a row share the scratch array (the
second with a smaller batch, so it reads a prefix the first call left
behind), on the decode GEMVs with the fused SwiGLU epilogue (B <= 2, arrival
counters in the scratch), the workgroup GEMVs (B <= 32) and the prefill
kernels (B > 32).  A call whose workspace exceeds the scratch is refused.
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

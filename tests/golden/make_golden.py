"""Write golden quantizer vectors from the reference's own NumPy fallback.

Run in the build container only (the reference tree is absent on GPU boxes):

    python tests/golden/make_golden.py [/root/reference]

The reference's quantizers (``metal_kans/quantization.py``) fall back to NumPy
when its Metal bridge is unavailable (``quantization.py:37-42,73-99,136-148,
212-217,231-246,250-255,275-286``), which is always the case on Linux.  Their
bit-level behaviour -- half-to-even ties of ``np.round``, the pairwise float32
summation inside ``np.mean``, fp32 true division, two separate roundings in
``q * scale + bias`` -- is not fixed by any invariant, so it is captured here as
data: inputs and the reference's outputs, nothing else.  The fixtures are
``quant_golden.npz`` beside this script.

Only data is written; no reference source is copied.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def cases():
    rng = np.random.default_rng(20261201)
    out = {}
    # Plain Gaussian weights, several shapes, including an input dim that needs padding.
    out["gauss_32x64"] = rng.normal(0.0, 1.0, (32, 64)).astype(np.float32)
    out["gauss_7x100"] = rng.normal(0.0, 0.02, (7, 100)).astype(np.float32)
    out["gauss_5x70"] = rng.normal(0.0, 0.5, (5, 70)).astype(np.float32)
    # Values on a coarse grid so that (w - min) / scale lands exactly on .5 ties.
    ties = (rng.integers(0, 31, (6, 128)).astype(np.float32) * np.float32(0.5)) - np.float32(7.5)
    out["ties_6x128"] = ties
    # A constant row (range floor 1e-7) and an all-zero row (ternary 1e-4 scale).
    cz = rng.normal(0.0, 1.0, (4, 64)).astype(np.float32)
    cz[1, :] = 0.25
    cz[2, :] = 0.0
    out["const_zero_4x64"] = cz
    # fp16 input weights (quantize() is applied to .half() layers too).
    out["half_8x96"] = rng.normal(0.0, 0.1, (8, 96)).astype(np.float16)
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from metal_kans.quantization import QuantizedWeight, TernaryQuantizedWeight  # noqa: E402

    arrays = {}
    for name, w in cases().items():
        arrays[f"{name}__w"] = w
        for bits, gs in ((8, 64), (4, 64), (8, 32), (4, 32)):
            qw = QuantizedWeight(w, bits=bits, group_size=gs)
            tag = f"{name}__int{bits}_g{gs}"
            arrays[f"{tag}__q"] = qw.qweight
            arrays[f"{tag}__s"] = qw.scales
            arrays[f"{tag}__b"] = qw.biases
            arrays[f"{tag}__dq"] = qw.dequantize()
        for gs in (32, 16, 64):
            tq = TernaryQuantizedWeight(w, group_size=gs)
            tag = f"{name}__tern_g{gs}"
            arrays[f"{tag}__p"] = tq.w_packed
            arrays[f"{tag}__s"] = tq.scales
            arrays[f"{tag}__dq"] = tq.dequantize()
    path = os.path.join(HERE, "quant_golden.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(arrays)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

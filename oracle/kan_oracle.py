"""CPU oracle for the fused KAN layer forward -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``metal-kans_amd/metal_kans`` + the HIP library)
must not import, call or fall back to anything here.

It restates, in NumPy, what the reference computes on the hot path:

* basis evaluators          -- ``metal_kans/kernels/fused_kan.metal:13-16,116-166,205-276``
                               and the fp16 variants ``:1373-1450,1476-1512``
* four-stage forward order  -- ``metal_kans/kernels/metal_kan_bridge.mm:443-625,1069-1164``
                               (SiLU+bias, SiLU(x)@W_base^T, Phi, Phi@W^T)
* layer parameters          -- ``metal_kans/cheby_kan.py:38-42``, ``fast_kan.py:40-47``,
                               ``bspline_kan.py:40-54``
* INT8/INT4 quantizer       -- NumPy fallback ``metal_kans/quantization.py:24-35,73-99``
* INT8/INT4 dequantizer     -- NumPy fallback ``quantization.py:136-148``
* ternary (de)quantizer     -- NumPy fallback ``quantization.py:196-246,275-286``
* GatedKAN block            -- ``metal_kans/gated_kan.py:15-16,86-138``
* Chebyshev backward        -- ``metal_kan_bridge.mm:4532-4632``, ``fused_kan.metal:2053-2163``
* SwiGLU kernel             -- ``fused_kan.metal:2284-2296``

Two accumulation modes exist for the forward: ``acc=np.float64`` (the
correctness reference: float64 arithmetic on the original inputs) and
``acc=np.float32`` (the reference's own four fp32 stages, used as the timed CPU
baseline).

Pinning (what checks each function, beyond retyping it) lives in
``tests/test_oracle.py``: Chebyshev against cos(k*theta) and T_k(+-1),
B-spline against partition of unity / knot values / a textbook Cox-de Boor
recursion on the extended uniform knot vector, RBF against phi(c_k)=1 and the
cfg3 constant inv_den=49/32, the contraction against brute-force loops and the
K=1 / W=0 reductions, and the quantizers bit-for-bit against golden vectors
written by the reference's own NumPy fallback (``tests/golden/``).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np

LOG2E = 1.4426950408889634


# ----------------------------------------------------------------------------
# Basis evaluators.  All return Phi with shape (B, D_in, K) in ``dtype``.
# ----------------------------------------------------------------------------

def silu(x: np.ndarray) -> np.ndarray:
    """x / (1 + e^-x) on the raw (unclamped) input (fused_kan.metal:13-16,132-133).

    For very negative x, e^-x overflows to inf and the quotient is the exact limit -0, so
    the overflow is expected and not reported."""
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-x))


def cheby_basis(x: np.ndarray, K: int, dtype=np.float64) -> np.ndarray:
    """T_0..T_{K-1}(clamp(x,-1,1)) by the 3-term recurrence (fused_kan.metal:205-238).

    ``K`` is the number of coefficients (the reference's ``degree`` argument,
    cheby_kan.py:40).
    """
    t = np.clip(np.asarray(x, dtype=dtype), -1.0, 1.0)
    out = np.empty(t.shape + (K,), dtype=dtype)
    out[..., 0] = 1.0
    if K > 1:
        out[..., 1] = t
    for k in range(2, K):
        out[..., k] = 2.0 * t * out[..., k - 1] - out[..., k - 2]
    return out


def rbf_grid(grid_range: Tuple[float, float], num_centers: int):
    """Centres and 1/(2h^2) exactly as FastKAN.__init__ builds them (fast_kan.py:40-42)."""
    grid = np.linspace(grid_range[0], grid_range[1], num_centers, dtype=np.float32)
    h = (grid_range[1] - grid_range[0]) / (num_centers - 1)
    inv_den = float(1.0 / (2.0 * (h ** 2)))
    return grid, inv_den


def rbf_basis(x: np.ndarray, grid: np.ndarray, inv_den: float, dtype=np.float64) -> np.ndarray:
    """exp(-(x - c_k)^2 * inv_den) (fused_kan.metal:140-166)."""
    xv = np.asarray(x, dtype=dtype)[..., None]
    c = np.asarray(grid, dtype=dtype)
    d = xv - c
    return np.exp(-(d * d) * dtype(inv_den)).astype(dtype)


def bspline_params(grid_size: int, grid_range: Sequence[float] = (-1.0, 1.0)):
    """[grid_min, inv_h] in fp32 as BSplineKAN.__init__ stores them (bspline_kan.py:44-49)."""
    gmin = float(grid_range[0])
    gmax = float(grid_range[1])
    inv_h = float(grid_size) / (gmax - gmin)
    return np.array([gmin, inv_h], dtype=np.float32)


def bspline_basis(x: np.ndarray, grid_size: int, grid_min: float, inv_h: float,
                  dtype=np.float64) -> np.ndarray:
    """Clamped closed-form uniform cubic B-spline, G+3 bases (fused_kan.metal:240-276).

    span = clamp(floor(pos), 0, G-1), u = clamp(pos - span, 0, 1); the four
    non-zero values sit at span..span+3, everything else is 0.  Outside the grid
    the reference saturates (it does not extrapolate).
    """
    xv = np.asarray(x, dtype=dtype)
    nb = grid_size + 3
    pos = (xv - dtype(grid_min)) * dtype(inv_h)
    span = np.clip(np.floor(pos), 0, grid_size - 1).astype(np.int64)
    u = np.clip(pos - span, 0.0, 1.0)
    om = 1.0 - u
    b0 = om * om * om / 6.0
    b1 = (3.0 * u ** 3 - 6.0 * u ** 2 + 4.0) / 6.0
    b2 = (-3.0 * u ** 3 + 3.0 * u ** 2 + 3.0 * u + 1.0) / 6.0
    b3 = u ** 3 / 6.0
    out = np.zeros(xv.shape + (nb,), dtype=dtype)
    idx = np.indices(xv.shape)
    for j, bj in enumerate((b0, b1, b2, b3)):
        out[tuple(idx) + (span + j,)] = bj
    return out


def basis(kind: str, x: np.ndarray, params: dict, dtype=np.float64) -> np.ndarray:
    if kind == "cheby":
        return cheby_basis(x, params["K"], dtype)
    if kind == "rbf":
        return rbf_basis(x, params["grid"], params["inv_den"], dtype)
    if kind == "bspline":
        return bspline_basis(x, params["G"], params["grid_min"], params["inv_h"], dtype)
    raise ValueError(kind)


# ----------------------------------------------------------------------------
# Forward.
# ----------------------------------------------------------------------------

def round_to(a: np.ndarray, kind: Optional[str]) -> np.ndarray:
    """Round values to fp16 / bf16 (RNE) and return them widened back; None = unchanged."""
    if kind is None:
        return a
    if kind == "float16":
        return np.asarray(a).astype(np.float16).astype(np.asarray(a).dtype)
    if kind == "bfloat16":
        return bf16_to_f32(bf16_round(np.asarray(a, dtype=np.float32))).astype(np.asarray(a).dtype)
    raise ValueError(kind)


def kan_forward(kind: str, x: np.ndarray, W: np.ndarray, W_base: Optional[np.ndarray],
                bias: Optional[np.ndarray], params: dict, acc=np.float64,
                operands: Optional[str] = None) -> np.ndarray:
    """y = bias + SiLU(x) @ W_base^T + Phi(x) @ W^T, in the reference's stage order.

    Follows metal_kan_bridge.mm:472-523: (1) Y = bias (or 0), (2) Y += SiLU(x)
    W_base^T, (3) Phi = basis(x) laid out [B, D_in*K] k-fastest, (4) Y += Phi W^T.
    ``W`` has shape (D_out, D_in*K); ``W_base`` (D_out, D_in) or None; ``bias``
    (D_out,) or None.  ``operands`` ('float16' / 'bfloat16') rounds SiLU(x) and
    Phi to that type before the contraction, as a 16-bit GEMM stage does (the
    reference's fp16 path stores Phi in half, fused_kan.metal:1399-1426).
    """
    x = np.asarray(x)
    B, D_in = x.shape
    Wf = np.asarray(W, dtype=acc)
    D_out = Wf.shape[0]
    xa = x.astype(acc)
    y = np.zeros((B, D_out), dtype=acc)
    if bias is not None:
        y += np.asarray(bias, dtype=acc)[None, :]
    if W_base is not None:
        y += round_to(silu(xa), operands) @ np.asarray(W_base, dtype=acc).T
    phi = round_to(basis(kind, xa, params, acc).reshape(B, -1), operands)
    y += phi @ Wf.T
    return y


def rel_err(y: np.ndarray, y_ref: np.ndarray) -> float:
    """Norm-wise max|y - y_ref| / max|y_ref| (the parity metric)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    den = float(np.max(np.abs(y_ref)))
    num = float(np.max(np.abs(y - y_ref)))
    return num / den if den > 0 else num


def chain_forward(layers: Sequence[dict], x: np.ndarray, acc=np.float64,
                  operands: Optional[str] = None) -> np.ndarray:
    """Sequential layers (metal_kan.py:133-135; chain at metal_kan_bridge.mm:1168-1248)."""
    h = np.asarray(x, dtype=acc)
    for L in layers:
        h = kan_forward(L["kind"], h, L["W"], L.get("W_base"), L.get("bias"), L["params"], acc, operands)
    return h


def cheby_basis_deriv(x: np.ndarray, K: int, dtype=np.float64) -> np.ndarray:
    """d/dx of phi_k(x) = T_k(clamp(x, -1, 1)), k < K, shape (B, D_in, K).

    As the reference backward (fused_kan.metal:2098-2162): T'_0 = 0, T'_1 = 1,
    T'_k = 2 T_{k-1} + 2t T'_{k-1} - T'_{k-2} at t = clamp(x), and 0 wherever the
    raw input lies outside [-1, 1] (the clamp is flat there; x = +-1 counts as
    inside).
    """
    x = np.asarray(x, dtype=dtype)
    t = np.clip(x, -1.0, 1.0)
    T = cheby_basis(x, K, dtype)
    d = np.zeros(x.shape + (K,), dtype=dtype)
    if K > 1:
        d[..., 1] = 1.0
    for k in range(2, K):
        d[..., k] = 2.0 * T[..., k - 1] + 2.0 * t * d[..., k - 1] - d[..., k - 2]
    d[(x < -1.0) | (x > 1.0)] = 0.0
    return d


def silu_deriv(x: np.ndarray) -> np.ndarray:
    """d/dx x*sigmoid(x) = s (1 + x (1 - s)), s = sigmoid(x) (fused_kan.metal:2152-2153)."""
    s = 1.0 / (1.0 + np.exp(-x))
    return s * (1.0 + x * (1.0 - s))


def cheby_backward(dY: np.ndarray, x: np.ndarray, W: np.ndarray, W_base: Optional[np.ndarray],
                   has_bias: bool, acc=np.float64):
    """Gradients of y = bias + SiLU(x) W_base^T + Phi W^T for a Chebyshev layer given dL/dy.

    Returns (dW [D_out, D_in*K], dW_base [D_out, D_in] or None, dbias [D_out] or None,
    dX [B, D_in]), the quantities of metal_kan_cheby_backward_fused
    (metal_kan_bridge.mm:4532-4632; kernels fused_kan.metal:2053-2163):
      dW[o, i*K+k]   = sum_b dY[b,o] T_k(clamp x[b,i])
      dW_base[o, i]  = sum_b dY[b,o] SiLU(x[b,i])
      dbias[o]       = sum_b dY[b,o]
      dX[b, i]       = sum_k (dY W)[b, i*K+k] T'_k(x[b,i]) + (dY W_base)[b,i] SiLU'(x[b,i])
    """
    dY = np.asarray(dY, dtype=acc)
    x = np.asarray(x, dtype=acc)
    B, D_in = x.shape
    D_out = dY.shape[1]
    K = W.shape[1] // D_in
    Wa = np.asarray(W, dtype=acc)
    Phi = cheby_basis(x, K, acc).reshape(B, D_in * K)
    dW = dY.T @ Phi
    dPhi = (dY @ Wa).reshape(B, D_in, K)
    dX = np.sum(dPhi * cheby_basis_deriv(x, K, acc), axis=2)
    dWb = None
    if W_base is not None:
        dWb = dY.T @ silu(x)
        dX = dX + (dY @ np.asarray(W_base, dtype=acc)) * silu_deriv(x)
    db = dY.sum(axis=0) if has_bias else None
    return dW, dWb, db, dX


def silu_clipped(x: np.ndarray) -> np.ndarray:
    """GatedKAN's SiLU with the +-20 clip in the exponent (gated_kan.py:15-16, fused_kan.metal:2284-2296)."""
    return x / (1.0 + np.exp(-np.clip(x, -20.0, 20.0)))


def gated_forward(x: np.ndarray, gate: dict, up: dict, down: dict, acc=np.float64) -> np.ndarray:
    """out = Down(SiLU(Gate(x)) * Up(x)) (gated_kan.py:86-138); dicts hold W, W_base, bias, K."""
    def f(L, h):
        return kan_forward("cheby", h, L["W"], L.get("W_base"), L.get("bias"), {"K": L["K"]}, acc)
    g = f(gate, x)
    u = f(up, x)
    hidden = silu_clipped(g) * u
    return f(down, hidden)


# ----------------------------------------------------------------------------
# Quantizers / dequantizers (NumPy-fallback semantics of quantization.py).
# ----------------------------------------------------------------------------

def quantize_affine(weight: np.ndarray, bits: int, group_size: int):
    """Block-affine min/max quantizer: returns (qweight, scales, biases, padded_in).

    quantization.py:24-35 (zero padding of the input dim to a multiple of the
    group), :74-99 (min/max, range floor 1e-7, scale = range / (2^bits - 1),
    q = round-half-even((w - min) / scale) clipped, INT4: even index -> low nibble).
    All arithmetic in fp32, as NumPy does on fp32 arrays.
    """
    w = np.asarray(weight)
    out_f, in_f = w.shape
    pad_in = (group_size - (in_f % group_size)) % group_size
    if pad_in > 0:
        padded = np.pad(w, ((0, 0), (0, pad_in)), mode="constant", constant_values=0.0)
    else:
        padded = w.copy()
    padded = np.ascontiguousarray(padded, dtype=np.float32)
    grouped = padded.reshape(-1, group_size)
    min_vals = grouped.min(axis=1, keepdims=True)
    max_vals = grouped.max(axis=1, keepdims=True)
    range_vals = np.maximum(max_vals - min_vals, np.float32(1e-7))
    max_int = (1 << bits) - 1
    scales = range_vals / np.float32(max_int)
    biases = min_vals
    q = np.round((grouped - biases) / scales).astype(np.int32)
    q = np.clip(q, 0, max_int)
    scales = scales.astype(np.float32)
    biases = biases.astype(np.float32)
    if bits == 8:
        qweight = q.astype(np.uint8)
    elif bits == 4:
        qweight = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    else:
        raise ValueError(bits)
    return qweight, scales, biases, padded.shape[1]


def dequantize_affine(qweight: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
                      group_size: int, shape: Tuple[int, int], padded_in: int) -> np.ndarray:
    """q * scale + bias with two separate fp32 roundings (quantization.py:136-148).

    Evaluated in place on one fp32 array (multiply, then add: the same two roundings as
    ``q * scales + biases``), so full-size matrices need no large temporaries."""
    ng = qweight.shape[0]
    if bits == 8:
        q = qweight.astype(np.float32)
    elif bits == 4:
        nib = np.empty((ng, group_size // 2, 2), dtype=np.uint8)
        np.bitwise_and(qweight, 0x0F, out=nib[:, :, 0])     # even index: low nibble
        np.right_shift(qweight, 4, out=nib[:, :, 1])        # odd index: high nibble
        q = nib.reshape(ng, group_size).astype(np.float32)
        del nib
    else:
        raise ValueError(bits)
    np.multiply(q, np.asarray(scales, np.float32).reshape(ng, 1), out=q)
    np.add(q, np.asarray(biases, np.float32).reshape(ng, 1), out=q)
    restored = q.reshape(-1, padded_in)
    if restored.shape == tuple(shape):
        return restored
    return np.ascontiguousarray(restored[: shape[0], : shape[1]])


def quantize_ternary(weight: np.ndarray, group_size: int = 32):
    """Absmean ternary quantizer: returns (w_packed uint32 (D_out, ceil(K/16)), scales (D_out, ceil(K/g))).

    quantization.py:196-246: per (row, group) sc = float32 mean(|w|) (1e-4 if the
    mean is 0), codes 0 (w/sc < -0.5), 2 (> 0.5) else 1, 16 codes per uint32 at bit
    2*(k % 16).  Vectorised; per-group means are bitwise identical to the
    reference's per-slice np.mean (checked in tests/test_oracle.py).
    """
    w = np.ascontiguousarray(weight, dtype=np.float32)
    D_out, K_dim = w.shape
    words = (K_dim + 15) // 16
    gpr = (K_dim + group_size - 1) // group_size
    scales = np.zeros((D_out, gpr), dtype=np.float32)
    codes = np.empty((D_out, K_dim), dtype=np.uint32)
    nfull = K_dim // group_size
    absw = np.abs(w)

    def group_scale(mean32):
        sc = mean32.astype(np.float32)
        return np.where(sc > 0, sc, np.float32(1e-4)).astype(np.float32)

    if nfull > 0:
        blk = w[:, : nfull * group_size].reshape(D_out, nfull, group_size)
        m = np.mean(absw[:, : nfull * group_size].reshape(D_out * nfull, group_size), axis=1)
        sc = group_scale(m).reshape(D_out, nfull)
        scales[:, :nfull] = sc
        norm = blk / sc[:, :, None]
        codes[:, : nfull * group_size] = np.where(norm < -0.5, 0, np.where(norm > 0.5, 2, 1)).reshape(
            D_out, nfull * group_size)
    if K_dim % group_size:
        start = nfull * group_size
        tail = np.ascontiguousarray(absw[:, start:])
        m = np.mean(tail, axis=1)
        sc = group_scale(m)
        scales[:, nfull] = sc
        norm = w[:, start:] / sc[:, None]
        codes[:, start:] = np.where(norm < -0.5, 0, np.where(norm > 0.5, 2, 1))
    pad = words * 16 - K_dim
    if pad:
        codes = np.pad(codes, ((0, 0), (0, pad)), constant_values=0)
    c = codes.reshape(D_out, words, 16)
    shifts = (np.arange(16, dtype=np.uint32) * 2)[None, None, :]
    packed = np.bitwise_or.reduce(c << shifts, axis=2).astype(np.uint32)
    return packed, scales


def ternary_codes(w_packed: np.ndarray, K_dim: int) -> np.ndarray:
    """Unpack 2-bit codes, code k at bits 2*(k%16) of word k//16 (quantization.py:279-281)."""
    D_out, words = w_packed.shape
    shifts = (np.arange(16, dtype=np.uint32) * 2)[None, None, :]
    c = (w_packed[:, :, None] >> shifts) & np.uint32(3)
    return c.reshape(D_out, words * 16)[:, :K_dim]


# value of each 2-bit code {0: -1, 1: 0, 2: +1, 3: 0}, for the four codes of every byte value
# (code of bits 2t..2t+1 at column t: little-endian uint32 words hold codes 4b..4b+3 in byte b)
_TERN_LUT = np.array([[(-1.0, 0.0, 1.0, 0.0)[(v >> (2 * t)) & 3] for t in range(4)] for v in range(256)],
                     dtype=np.float32)


def dequantize_ternary(w_packed: np.ndarray, scales: np.ndarray, shape: Tuple[int, int],
                       group_size: int = 32) -> np.ndarray:
    """{0:-1, 1:0, 2:+1, 3:0}[code] * scale in fp32 (quantization.py:275-286).

    Codes are expanded through a per-byte table (``_TERN_LUT``); the product with the scale is exact
    (the value is -1, 0 or +1)."""
    D_out, K_dim = shape
    wp = np.ascontiguousarray(w_packed, dtype=np.uint32)
    words = wp.shape[1]
    val = _TERN_LUT[wp.view(np.uint8).reshape(D_out, words * 4)].reshape(D_out, words * 16)
    if words * 16 != K_dim:
        val = np.ascontiguousarray(val[:, :K_dim])
    sc = np.asarray(scales, np.float32)
    if K_dim % group_size == 0:
        v3 = val.reshape(D_out, K_dim // group_size, group_size)
        np.multiply(v3, sc[:, :, None], out=v3)
        return val
    g = np.arange(K_dim) // group_size
    return (val * sc[:, g]).astype(np.float32)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """(g * sigmoid(clamp(g, +-20))) * u in fp32 (fused_kan.metal:2284-2296)."""
    g = np.asarray(gate, dtype=np.float32)
    u = np.asarray(up, dtype=np.float32)
    sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-np.clip(g, -20.0, 20.0)))
    return ((g * sig) * u).astype(np.float32)


# ----------------------------------------------------------------------------
# Synthetic workloads named in BASELINE.json (seeded: rng = default_rng(1000+cfg),
# draw order x, W, W_base, bias).
# ----------------------------------------------------------------------------

def layer_norm(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """Non-affine LayerNorm over the feature axis in fp32 (cfg3 input conditioning)."""
    x = np.asarray(x, dtype=np.float32)
    mu = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    return ((x - mu) / np.sqrt(var + np.float32(eps))).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16) with round-to-nearest-even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((u >> 16) & 1) + np.uint32(0x7FFF)
    out = ((u + rounding) >> 16).astype(np.uint16)
    nan = np.isnan(np.ascontiguousarray(x, dtype=np.float32))
    out[nan] = 0x7FC0
    return out


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)

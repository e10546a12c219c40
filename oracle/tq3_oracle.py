"""ORACLE -- test infrastructure only (see ``oracle/__init__.py``).

Numpy restatement of the reference's TQ3 codebook format (kandiga/tq3/quantize.py) for checking
the TQ3 GEMV kernels:

* the randomized Walsh-Hadamard transform of a 32-weight block (quantize.py:55-86):
  forward ``H (S x) / sqrt(32)``, inverse ``S (H r) / sqrt(32)``, H the unnormalised
  32-point Hadamard butterfly, S the sign table;
* the TQ3_1S block with per-half means, 20 bytes per 32 weights (quantize.py:120-143,
  466-486): fp16 d0, d1, m0, m1, then 12 bytes of 3-bit indices (4 groups of 3 bytes, index r
  of group g = bits 3r..3r+2 of ``b0 | b1<<8 | b2<<16``, quantize.py:98-117); weights
  ``iWHT(C[q] * d + m)`` with d, m of the block's half (elements 0-15, 16-31);
* ``x @ W.T`` over such blocks in float64.

The centroid, boundary and sign tables are the format's own (quantize.py:29-46).
"""
from __future__ import annotations

import numpy as np

BLOCK = 32
BLOCK_BYTES = 20
CENTROIDS = np.array([-1.996684, -1.291398, -0.740341, -0.247508,
                      0.230106, 0.725222, 1.277503, 1.988943], dtype=np.float32)
BOUNDARIES = np.array([-1.644041, -1.015870, -0.493924, -0.008701,
                       0.477664, 1.001362, 1.633223], dtype=np.float32)
SIGNS = np.array([+1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1,
                  -1, -1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1], dtype=np.float32)


def hadamard_butterfly(v: np.ndarray) -> np.ndarray:
    """Unnormalised 32-point Hadamard transform of the last axis (5 butterfly stages)."""
    out = np.array(v, dtype=np.float64, copy=True)
    step = 1
    while step < BLOCK:
        o = out.reshape(*out.shape[:-1], BLOCK // (2 * step), 2, step)
        a, b = o[..., 0, :].copy(), o[..., 1, :].copy()
        o[..., 0, :], o[..., 1, :] = a + b, a - b
        step *= 2
    return out


def wht_forward(x: np.ndarray) -> np.ndarray:
    return hadamard_butterfly(np.asarray(x, np.float64) * SIGNS) / np.sqrt(32.0)


def wht_inverse(r: np.ndarray) -> np.ndarray:
    return hadamard_butterfly(r) * SIGNS / np.sqrt(32.0)


def unpack_indices(qs: np.ndarray) -> np.ndarray:
    """[..., 12] bytes -> [..., 32] indices (quantize.py:109-117)."""
    q = np.asarray(qs, dtype=np.uint32).reshape(*np.shape(qs)[:-1], 4, 3)
    p = q[..., 0] | (q[..., 1] << 8) | (q[..., 2] << 16)
    r = np.arange(8, dtype=np.uint32)
    return ((p[..., None] >> (3 * r)) & 7).reshape(*np.shape(qs)[:-1], 32).astype(np.uint8)


def block_fields(raw: np.ndarray):
    """Blocks ``[N, 20]`` uint8 -> (d [N,2], m [N,2] float64, q [N,32])."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    f = raw[:, :8].copy().view(np.float16).astype(np.float64)
    return f[:, 0:2], f[:, 2:4], unpack_indices(raw[:, 8:20])


def dequantize_blocks(raw: np.ndarray) -> np.ndarray:
    """Weights of the blocks (quantize.py:466-486): ``[N, 32]`` float64."""
    d, m, q = block_fields(raw)
    rot = CENTROIDS[q].astype(np.float64)
    rot[:, :16] = rot[:, :16] * d[:, :1] + m[:, :1]
    rot[:, 16:] = rot[:, 16:] * d[:, 1:] + m[:, 1:]
    return wht_inverse(rot)


def dequantize_matrix(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    return dequantize_blocks(raw).reshape(rows, cols)


def gemv_f64(raw: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """``x @ W.T`` for a TQ3 matrix ``W [rows, cols]`` (row-major blocks), float64."""
    xs = np.atleast_2d(np.asarray(x, dtype=np.float64))
    return xs @ dequantize_matrix(raw, rows, cols).T


def expert_mlp_f64(expert_raw: np.ndarray, hidden: int, inter: int, x: np.ndarray) -> np.ndarray:
    """SwiGLU expert over one TQ3X expert body (gate, up, down blocks in turn)."""
    ng = inter * hidden // BLOCK * BLOCK_BYTES
    g = gemv_f64(expert_raw[:ng], inter, hidden, x)
    u = gemv_f64(expert_raw[ng:2 * ng], inter, hidden, x)
    a = g / (1.0 + np.exp(-g)) * u
    return gemv_f64(expert_raw[2 * ng:3 * ng], hidden, inter, a)

"""Bit-exact per-output-row symmetric int8 quantizer (numpy float32 IEEE ops).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates src/kernels/quantize.cu:8-44 of visheshnarayan/llm.cu:
  scale = max_c |w[row, c]| / 127            (fp32 division, :30)
  inv   = scale > 0 ? 1 / scale : 0          (fp32 division, :35)
  q     = (int8) rint(clamp(w * inv, -127, 127))   (round half to even, :37-40)
and the dequantised GEMM semantics of src/kernels/quantize.cu:55-70,
C[m, n] = (sum_k a[m, k] * q[n, k]) * scale[n].

Config C4 stores the scale as fp16 (the int8 integers still come from the fp32
scale above); ``dequant`` takes whichever scale array it is handed.
Pinned in tests by an element-wise brute force in Python float32 scalars and
by the round-half-even special cases (0.5 -> 0, 1.5 -> 2, -2.5 -> -2).
"""
from __future__ import annotations

import numpy as np


def quantize_rows(w: np.ndarray):
    """w: float32 [rows, cols] -> (q int8 [rows, cols], scale float32 [rows])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=1).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scale > 0, np.float32(1.0) / np.where(scale > 0, scale, np.float32(1.0)),
                       np.float32(0.0)).astype(np.float32)
    val = (w * inv[:, None]).astype(np.float32)
    val = np.minimum(np.maximum(val, np.float32(-127.0)), np.float32(127.0))
    q = np.rint(val).astype(np.int8)
    return q, scale


def dequant(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """float32 [rows, cols] = q * scale[row] (scale fp32 or fp16)."""
    return q.astype(np.float32) * scale.astype(np.float32)[:, None]

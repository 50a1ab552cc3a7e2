"""CPU oracle of the int8 weight-only GEMV -- TEST INFRASTRUCTURE, never shipped.

The reference plans int8 weights dequantised inside its hand-written decode
GEMV (``TODO.md:58-63``) and has no kernel or format for it yet, so there is
no reference output to match. What pins these two functions instead:

* ``quantize_i8_ref``: the round-trip bound ``|W - s q| <= s / 2``, ``max |q|
  == 127`` on every non-zero row, and exact results on matrices that are
  already integer multiples of their scale (``tests/test_quant.py``).
* ``gemv_i8_ref``: a brute-force double loop on small inputs, one-hot rows
  that pick ``s[n] x[k]``, and linearity in x (``tests/test_quant.py``).

Arithmetic is float64 (the scale in float32, as the kernel's input holds it).
"""

from __future__ import annotations

import numpy as np


def quantize_i8_ref(W: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8: scale = max|W[n]| / 127 (float32, 0 for a zero
    row), q = round-half-even(W / scale) clipped to [-127, 127]."""
    w = np.asarray(W, dtype=np.float32)
    scale = (np.abs(w).max(axis=1) / np.float32(127.0)).astype(np.float32)
    div = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / div[:, None]), -127, 127).astype(np.int8)
    return q, scale


def gemv_i8_ref(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """y[n] = scale[n] * sum_k x[k] q[n, k], in float64."""
    acc = q.astype(np.float64) @ np.asarray(x, dtype=np.float64)
    return np.asarray(scale, dtype=np.float64) * acc


def gemv_i8_abs_ref(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """scale[n] * sum_k |x[k] q[n, k]|: the size of the terms, which bounds
    the rounding error of an fp32 sum of them."""
    acc = np.abs(q.astype(np.float64)) @ np.abs(np.asarray(x, dtype=np.float64))
    return np.abs(np.asarray(scale, dtype=np.float64)) * acc

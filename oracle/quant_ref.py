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

any4 (the reference names it beside int8, same plan, no kernel or format
either): ``dequant_any4_ref`` / ``gemv_any4_ref`` restate the format -- per
row a 16-entry table, one 4-bit code per weight, column 2j in the low nibble
of byte j and 2j+1 in the high nibble. Pinned by a per-element brute-force
loop, one-hot codes that pick single table entries, constant tables (y =
c * sum(x)) and linearity in x (``tests/test_quant.py``).
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


def dequant_any4_ref(codes: np.ndarray, lut: np.ndarray) -> np.ndarray:
    """W[n, 2j] = lut[n, codes[n, j] & 15], W[n, 2j + 1] = lut[n, codes[n, j] >> 4], float64."""
    c = np.asarray(codes, dtype=np.uint8)
    t = np.asarray(lut, dtype=np.float64)
    N, half = c.shape
    idx = np.empty((N, 2 * half), dtype=np.int64)
    idx[:, 0::2] = c & 15
    idx[:, 1::2] = c >> 4
    return np.take_along_axis(t, idx, axis=1)


def gemv_any4_ref(x: np.ndarray, codes: np.ndarray, lut: np.ndarray) -> np.ndarray:
    """y[n] = sum_k x[k] lut[n, code(n, k)], float64."""
    return dequant_any4_ref(codes, lut) @ np.asarray(x, dtype=np.float64)


def gemv_any4_abs_ref(x: np.ndarray, codes: np.ndarray, lut: np.ndarray) -> np.ndarray:
    """sum_k |x[k] lut[n, code(n, k)]|: the size of the terms."""
    return np.abs(dequant_any4_ref(codes, lut)) @ np.abs(np.asarray(x, dtype=np.float64))

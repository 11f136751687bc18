"""Oracle: restatement of the reference's MX (microscaling) weight formats.
Test infrastructure only (see ``oracle/__init__.py``).

e8m0_to_float  reference python/ccut/quant/kernels.py:240-256
dequant_mxfp8  reference python/ccut/quant/mx.py:60-73
dequant_mxfp4  reference python/ccut/quant/mx.py:75-94 (MXFP4 and NVFP4)
apply          reference python/ccut/quant/mx.py:37-58 (x @ W.T, here in float64)

The 4-bit table is the reference's own (codes & 7 -> 0, .5, 1, 1.5, -0, -.5,
-1, -1.5), not OCP E2M1; E8M0 byte 0 decodes to 0, not 2^-127.
"""

from __future__ import annotations

import numpy as np

from oracle.ref_quant import fp8_e4m3_to_float32

LUT4 = np.array([0.0, 0.5, 1.0, 1.5, -0.0, -0.5, -1.0, -1.5] * 2, dtype=np.float32)


def e8m0_to_float(e8m0) -> np.ndarray:
    e = np.asarray(e8m0).reshape(-1).astype(np.int64)
    out = np.empty(e.shape[0], np.float32)
    for i, v in enumerate(e.tolist()):
        out[i] = np.nan if v == 255 else (0.0 if v == 0 else 2.0 ** (v - 127))
    return out


def _group_scale(scale_e8m0, rows: int, cols: int, group_size: int) -> np.ndarray:
    """[rows, cols] float32 of each element's group scale."""
    gpr = (cols + group_size - 1) // group_size
    s = e8m0_to_float(scale_e8m0)[: rows * gpr].reshape(rows, gpr)
    return np.repeat(s, group_size, axis=1)[:, :cols]


def dequant_mxfp8(w_fp8: np.ndarray, scale_e8m0, group_size: int) -> np.ndarray:
    m, n = w_fp8.shape
    vals = fp8_e4m3_to_float32(np.asarray(w_fp8, np.uint8).reshape(-1)).reshape(m, n)
    return (vals * _group_scale(scale_e8m0, m, n, group_size)).astype(np.float32)


def dequant_mxfp4(packed: np.ndarray, scale_e8m0, group_size: int, scale2: float | None = None) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    m, n2 = p.shape
    w = np.empty((m, 2 * n2), np.float32)
    w[:, 0::2] = LUT4[p & 0x0F]
    w[:, 1::2] = LUT4[(p >> 4) & 0x0F]
    if scale_e8m0 is not None:
        w = (w * _group_scale(scale_e8m0, m, 2 * n2, group_size)).astype(np.float32)
    if scale2 is not None:
        w = (w * np.float32(scale2)).astype(np.float32)
    return w


def apply(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """x @ W.T in float64, returned float32."""
    return (np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32)

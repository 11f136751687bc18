"""Oracle: restatement of the reference's INT8 linear layer.  Test
infrastructure only (see ``oracle/__init__.py``).

quantize_per_token  reference python/ccut/quant/int8.py:65-77
int8_matmul         reference python/ccut/quant/int8.py:80-100 (exact int64 sums)
w8a8                reference python/ccut/quant/int8.py:52-62
dequant_row         reference python/ccut/quant/kernels.py:180-189
w8a16               reference python/ccut/quant/int8.py:38-50, with the
                    product written x @ W.T (the reference's ``out @ x`` at
                    :49 only type-checks when in_features == batch; its
                    LinearMethod at quant/method.py:106-111 writes x @ w.T)

numpy casts NaN to int8 as 0 (x86's truncating convert gives 0x80000000,
whose low byte is 0); the restatement keeps numpy's cast.
"""

from __future__ import annotations

import warnings

import numpy as np


def quantize_per_token(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(xq int8 [M, K], x_scale float32 [M])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=1).astype(np.float32)  # raises on K == 0, as the reference does
    amax = np.where(amax > 0, amax, 1.0).astype(np.float32)
    x_scale = (amax / 127.0).astype(np.float32)
    factor = (127.0 / x_scale).astype(np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RuntimeWarning)
        xq = np.clip(np.round(x * factor[:, None]), -127, 127).astype(np.int8)
    return xq, x_scale


def int8_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a [M, K] int8 @ b [K, N] int8 -> int64 [M, N], exact."""
    return a.astype(np.int64) @ b.astype(np.int64)


def w8a8(w: np.ndarray, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y [M, N] float32 for w int8 [N, K], scale float32 [N], x float32 [M, K]."""
    xq, x_scale = quantize_per_token(x)
    acc = int8_matmul(xq, np.asarray(w, np.int8).T)
    with np.errstate(invalid="ignore", over="ignore"):
        return acc.astype(np.float32) * x_scale[:, None] * np.asarray(scale, np.float32)[None, :]


def dequant_row(w: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """out[r, c] = w[r, c] * scale[r] (float32)."""
    return np.asarray(w, np.int8).astype(np.float32) * np.asarray(scale, np.float32)[:, None]


def w8a16(w: np.ndarray, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """x @ dequant_row(w, scale).T in float64, returned float32."""
    return (np.asarray(x, np.float64) @ dequant_row(w, scale).astype(np.float64).T).astype(np.float32)


def quantize_cols(x: np.ndarray, amax: np.ndarray) -> np.ndarray:
    """int8_quantize_row (reference python/ccut/quant/kernels.py:192-211):
    per column inv = 127 / amax[c] in float64 (0 when amax[c] is not > 0),
    q = round-half-even(float64(x) * inv) clamped to +-127.  NaN -> 0 and
    +-inf -> +-127, which the reference leaves undefined (numba fastmath)."""
    x = np.asarray(x, np.float32)
    a = np.asarray(amax, np.float32).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(a > 0, 127.0 / np.where(a > 0, a, 1.0), 0.0)
        q = np.rint(x.astype(np.float64) * inv[None, :])
    q = np.where(np.isnan(q), 0.0, np.clip(q, -127, 127))
    return q.astype(np.int8)

"""Oracle: AWQ int4 GEMM format (pack / unpack / dequant / linear).

Test infrastructure only (see ``oracle/__init__.py``).

The reference does not implement AWQ: its group strategy maps to FP8 only
(reference ``python/ccut/quant/compressed_tensors.py:61-70``) and for group
layers it only names the ``.scales`` / ``.zero_points`` tensors
(``compressed_tensors.py:209-211``); ``GroupShape.rows`` is the group size
along the input dimension (``quant/spec.py:57-69``).  The format restated here
is the public AutoAWQ "GEMM" packing (AutoAWQ v0.2.x, ``awq/utils/
packing_utils.py``: ``AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]``,
``AWQ_REVERSE_ORDER = [0, 4, 1, 5, 2, 6, 3, 7]``):

* ``qweight`` int32 ``[K, N/8]``: nibble ``i`` (bits ``4i..4i+3``) of word
  ``[k, c]`` holds column ``8c + AWQ_ORDER[i]``; so column ``8c + j`` sits at
  shift ``4 * AWQ_REVERSE_ORDER[j]``.
* ``qzeros`` int32 ``[K/G, N/8]``: 4-bit zero points, packed the same way.
* ``scales`` fp16 ``[K/G, N]``.
* ``W[k, n] = (q[k, n] - z[k//G, n]) * s[k//G, n]`` -- exact in float32
  (a 5-bit integer times an 11-bit significand).
* ``y = x @ W`` (``W`` is ``[in, out]``).

Parity against the reference is unpinned (the format is absent there); the
tests pin this restatement by the format's own invariants.
"""

from __future__ import annotations

import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def pack(q: np.ndarray) -> np.ndarray:
    """``q [R, N]`` values 0..15 -> int32 ``[R, N/8]`` in AWQ order."""
    q = np.asarray(q).astype(np.uint32)
    R, N = q.shape
    assert N % 8 == 0
    q8 = q.reshape(R, N // 8, 8)
    word = np.zeros((R, N // 8), dtype=np.uint32)
    for i in range(8):
        word |= (q8[:, :, AWQ_ORDER[i]] & 0xF) << np.uint32(4 * i)
    return word.view(np.int32)


def unpack(packed: np.ndarray) -> np.ndarray:
    """int32 ``[R, N/8]`` -> uint8 ``[R, N]`` (inverse of :func:`pack`)."""
    w = np.asarray(packed).view(np.uint32)
    R, C = w.shape
    out = np.empty((R, C, 8), dtype=np.uint8)
    for j in range(8):
        out[:, :, j] = (w >> np.uint32(4 * AWQ_REVERSE_ORDER[j])) & 0xF
    return out.reshape(R, C * 8)


def dequant(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """``W [K, N] f32 = (q - z) * s`` with the group index ``k // G``.  q - z
    is an integer in [-15, 15] and s an fp16/bf16 value, so the float32
    product is exact."""
    q = unpack(qweight)
    z = unpack(qzeros)
    K, N = q.shape
    G = int(group_size)
    s = np.asarray(scales).astype(np.float32)
    d = q.reshape(K // G, G, N).astype(np.float32) - z.astype(np.float32)[:, None, :]
    return (d * s[:, None, :]).reshape(K, N)


def linear(x: np.ndarray, qweight, qzeros, scales, group_size: int) -> np.ndarray:
    """Dequantize-then-matmul in float32 (the reference's W4A16 semantics,
    ``quant/weight_only.py:37-54``, applied to the AWQ format)."""
    w = dequant(qweight, qzeros, scales, group_size)
    return np.asarray(x, dtype=np.float32) @ w

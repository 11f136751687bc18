"""Oracle: restatement of the reference's load-time and KV-cache FP8
quantizers.  Test infrastructure only (see ``oracle/__init__.py``).

quantize_buffer_inplace  reference python/ccut/quant/online.py:37-64
quantize_kv_token        reference python/ccut/quant/kv.py:70-90
dequantize_kv_token      reference python/ccut/quant/kv.py:93-101

numpy divides a float32 row by a Python float in float32 (the scalar is
rounded to float32 first); the scale arithmetic before that is float64.
"""

from __future__ import annotations

import numpy as np

from oracle.ref_quant import float32_to_fp8_e4m3, fp8_e4m3_to_float32


def quantize_buffer(raw_bf16, scale, in_features: int) -> np.ndarray:
    """e4m3 codes [out, in] of a BF16 weight, one scale per output row."""
    w16 = np.frombuffer(bytes(raw_bf16) if isinstance(raw_bf16, (bytes, bytearray)) else
                        np.ascontiguousarray(raw_bf16).tobytes(), dtype=np.uint16).reshape(-1, in_features)
    w32 = (w16.astype(np.uint32) << 16).view(np.float32)
    amax = np.abs(w32).max(axis=1)
    out = np.empty(w32.shape, dtype=np.uint8)
    for r in range(w32.shape[0]):
        s = float(scale[r]) if scale is not None else (float(amax[r]) / 448.0 or 1.0)
        s = s if s > 0 else 1.0
        out[r] = float32_to_fp8_e4m3(np.clip(w32[r] / np.float32(s), -448.0, 448.0).astype(np.float32))
    return out


def kv_quant(kv: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """codes [..., dim] and one scale byte per row of a float32 KV block."""
    kv = np.asarray(kv, dtype=np.float32)
    rows = kv.reshape(-1, kv.shape[-1])
    codes = np.zeros(rows.shape, dtype=np.uint8)
    scales = np.zeros(rows.shape[0], dtype=np.uint8)
    for i, x in enumerate(rows):
        amax = float(np.abs(x).max())
        if amax <= 0:
            continue
        s = amax / 448.0
        codes[i] = float32_to_fp8_e4m3(np.clip(x / np.float32(s), -448.0, 448.0).astype(np.float32))
        scales[i] = float32_to_fp8_e4m3(np.array([s], dtype=np.float32))[0]
    return codes.reshape(kv.shape), scales.reshape(kv.shape[:-1])


def kv_dequant(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8)
    rows = c.reshape(-1, c.shape[-1])
    sc = np.asarray(scales, dtype=np.uint8).reshape(-1)
    out = np.zeros(rows.shape, dtype=np.float32)
    for i in range(rows.shape[0]):
        s = float(fp8_e4m3_to_float32(sc[i:i + 1])[0])
        out[i] = fp8_e4m3_to_float32(rows[i]) * np.float32(s) if s > 0 else 0.0
    return out.reshape(c.shape)

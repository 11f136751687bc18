"""MX (microscaling) Linear method (reference ``python/ccut/quant/mx.py:21-94``).

Format: weights ``[out, in]`` in groups of ``group_size`` consecutive input
columns per output row (32 for MXFP8 / MXFP4, 16 for NVFP4), one E8M0 scale
byte per group (``2^(e-127)``; 0 -> 0, 255 -> NaN), scales ``[out,
ceil(in / group_size)]``.  MXFP8 holds e4m3fn bytes; MXFP4 / NVFP4 hold two
4-bit codes per byte (low nibble first) decoded by the reference's table
``{0, .5, 1, 1.5, -0, -.5, -1, -1.5}`` (codes & 7), NVFP4 times the mean of
its per-tensor second scale.  ``apply`` is ``x @ W.T`` in float32 with W
formed on the fly on the GPU (``ccq_mx_linear_f32``).
"""

from __future__ import annotations

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call
from ccut.quant.method import QuantizeMethodBase
from ccut.quant.spec import LayerQuantSpec, QuantDType

__all__ = ["MxLinearMethod", "e8m0_bytes", "mx_linear", "mx_dequant"]

FMT_MXFP8, FMT_MXFP4 = 0, 1


def e8m0_bytes(scale) -> torch.Tensor:
    """E8M0 scales as a uint8 device tensor.  The reference reads them with
    ``astype(np.float32)`` and ``int()``; values must be whole numbers in
    0..255 here (a byte's range), anything else is rejected."""
    if isinstance(scale, torch.Tensor) and scale.dtype == torch.uint8:
        return _dev.to_device(scale).reshape(-1)
    if isinstance(scale, torch.Tensor):
        v = scale.detach().float().cpu().numpy()
    else:
        v = np.asarray(scale).astype(np.float32)
    v = v.reshape(-1)
    if v.size and not (np.all(np.isfinite(v)) and v.min() >= 0 and v.max() <= 255 and np.all(v == np.floor(v))):
        raise ValueError("E8M0 scales must be whole numbers in 0..255")
    return _dev.to_device(v.astype(np.uint8))


def _fmt(weight_dtype: str) -> int:
    if weight_dtype == QuantDType.MXFP8:
        return FMT_MXFP8
    if weight_dtype in (QuantDType.MXFP4, QuantDType.NVFP4):
        return FMT_MXFP4
    raise ValueError(f"MX method does not support weight dtype {weight_dtype}")


def _args(weight_bytes, scale, rows_hint: int | None, cols: int, fmt: int, group_size: int):
    raw = _dev.raw_u8(weight_bytes)
    row_bytes = cols if fmt == FMT_MXFP8 else cols // 2
    if cols <= 0 or (fmt == FMT_MXFP4 and cols % 2) or raw.numel() % row_bytes:
        raise ValueError(f"weight of {raw.numel()} bytes does not hold rows of {cols} columns")
    rows = raw.numel() // row_bytes
    if rows_hint is not None and rows != rows_hint:
        raise ValueError(f"weight holds {rows} rows, expected {rows_hint}")
    sc = None
    if scale is not None:
        sc = e8m0_bytes(scale)
        need = rows * ((cols + group_size - 1) // group_size)
        if sc.numel() < need:
            raise ValueError(f"E8M0 scales hold {sc.numel()} entries, {need} needed")
    elif fmt == FMT_MXFP8:
        raise ValueError("MXFP8 layer is missing its E8M0 scales")
    return raw, sc, rows


def mx_linear(weight_bytes, scale, x, weight_dtype: str, group_size: int = 32, scale2: float | None = None):
    """``x @ W.T`` (float32) for MX weights; numpy in -> numpy out."""
    fmt = _fmt(weight_dtype)
    xd = _dev.to_device(x, torch.float32)
    if xd.dim() != 2:
        raise ValueError(f"x must be [batch, in_features], got shape {tuple(xd.shape)}")
    batch, in_f = xd.shape
    raw, sc, rows = _args(weight_bytes, scale, None, in_f, fmt, group_size)
    s2 = float(1.0 if scale2 is None else np.float32(scale2))
    # one call for every batch size: W formed in registers; from 8 rows on,
    # in_features % 256 == 0, the products run on the matrix cores
    y = torch.empty((batch, rows), dtype=torch.float32, device=xd.device)
    call("ccq_mx_linear_f32", xd.contiguous().data_ptr(), raw.data_ptr(), sc.data_ptr() if sc is not None else None,
         y.data_ptr(), batch, in_f, rows, fmt, group_size, s2, _dev.stream_ptr())
    return _dev.to_host(y) if _dev.is_host(x) else y


def mx_dequant(weight_bytes, scale, cols: int, weight_dtype: str, group_size: int = 32,
               scale2: float | None = None, like=None):
    """W [rows, cols] float32 as the layer forms it."""
    fmt = _fmt(weight_dtype)
    raw, sc, rows = _args(weight_bytes, scale, None, cols, fmt, group_size)
    out = torch.empty((rows, cols), dtype=torch.float32, device=raw.device)
    call("ccq_mx_dequant", raw.data_ptr(), sc.data_ptr() if sc is not None else None, out.data_ptr(), rows, cols,
         fmt, group_size, float(1.0 if scale2 is None else np.float32(scale2)), _dev.stream_ptr())
    return _dev.to_host(out) if _dev.is_host(weight_bytes if like is None else like) else out


def _scale2(s) -> np.float32:
    """NVFP4's factor: the float32 mean of the second scale tensor
    (reference ``mx.py:55-56``)."""
    if isinstance(s, torch.Tensor):
        s = s.detach().cpu().numpy()
    return np.float32(np.float32(s).mean())


class MxLinearMethod(QuantizeMethodBase):
    """MX layer: W dequantized on the fly, float32 product."""

    compute_path = "w8a16"

    def __init__(self, spec: LayerQuantSpec):
        self.spec = spec
        key = spec.effective_key()
        self.weight_dtype = key.weight_dtype
        self.group_size = key.group_shape.group_size or 32
        self.scale_name = spec.scales[0].name if spec.scales else None
        self.scale2_name = spec.scales[1].name if len(spec.scales) > 1 else None

    def create_weights(self, spec: LayerQuantSpec) -> None:
        QuantizeMethodBase.create_weights(self, spec)

    def apply(self, weight_bytes, scales: dict, x):
        scale = scales.get(self.scale_name) if self.scale_name else None
        if self.weight_dtype == QuantDType.MXFP8 and scale is None:
            raise ValueError(f"MXFP8 layer is missing its E8M0 scale ({self.scale_name})")
        s2 = None
        if self.weight_dtype == QuantDType.NVFP4 and self.scale2_name:
            s2 = _scale2(scales[self.scale2_name])
        return mx_linear(weight_bytes, scale, x, self.weight_dtype, self.group_size, s2)

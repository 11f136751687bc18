"""Load-time (online) FP8 quantization of BF16 weights (reference
``python/ccut/quant/online.py:37-64``), on the GPU."""

from __future__ import annotations

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call

__all__ = ["quantize_buffer_inplace"]


def quantize_buffer_inplace(raw_bf16, scale, out, in_features: int | None = None) -> None:
    """BF16 ``[out, in]`` bytes (or uint16 / bfloat16 array) -> e4m3 codes
    written into ``out`` (uint8 ``[out, in]``, numpy or device tensor), one
    scale per output row: ``scale[r]`` when given, else ``amax / 448``
    (``ccq_quantize_rows_fp8``)."""
    if in_features is None:
        in_features = out.shape[1]
    if isinstance(raw_bf16, torch.Tensor):
        w = raw_bf16.view(torch.int16) if raw_bf16.dtype == torch.bfloat16 else raw_bf16
        w = w.to(_dev.require_gpu()).contiguous().view(torch.int16)
    else:
        buf = raw_bf16 if isinstance(raw_bf16, (bytes, bytearray)) else np.ascontiguousarray(raw_bf16)
        w = torch.from_numpy(np.frombuffer(buf, dtype=np.int16).copy()).to(_dev.require_gpu())
    if w.numel() % in_features:
        raise ValueError(f"{w.numel()} bf16 values are not rows of {in_features}")
    rows = w.numel() // in_features
    sd = None if scale is None else _dev.to_device(scale, torch.float32).reshape(-1).contiguous()
    if sd is not None and sd.numel() < rows:
        raise ValueError(f"{sd.numel()} scales for {rows} rows")
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()) else \
        torch.empty((rows, in_features), dtype=torch.uint8, device=w.device)
    call("ccq_quantize_rows_fp8", w.data_ptr(), sd.data_ptr() if sd is not None else None, dst.data_ptr(), rows,
         in_features, _dev.stream_ptr())
    if dst is not out:
        if isinstance(out, torch.Tensor):
            out.copy_(dst.reshape(out.shape))
        else:
            np.copyto(out, dst.cpu().numpy().reshape(out.shape))

"""Online quantization: load-time FP8 quantization of BF16 weights
(reference ``python/ccut/quant/online.py:37-64``) on the GPU, and the
``OnlineQuantConfig`` a shorthand of ``resolve_checkpoint_quant`` selects
(reference ``online.py:67-122``)."""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call
from ccut.quant.registry import QuantizationConfig
from ccut.quant.spec import K_BF16, LayerQuantSpec, ScaleDesc, get_quant_key

__all__ = ["quantize_buffer_inplace", "OnlineQuantConfig"]


class OnlineQuantConfig(QuantizationConfig):
    """Every layer quantized at load time with the shorthand's weight key,
    except those matching an ignore regex (BF16 passthrough); the scales are
    computed at load, so each spec names a placeholder scale tensor
    ``<layer>.online_scale``."""

    name = "online"

    def __init__(self, shorthand: dict, weight_key_name: str, ignore_patterns: list[str]):
        self.shorthand = shorthand
        self.weight_key_name = weight_key_name
        self.ignore_patterns = [re.compile(p) for p in (ignore_patterns or [])]
        self._specs: dict[str, LayerQuantSpec] = {}

    @classmethod
    def from_config(cls, shorthand: dict, model_dir: str | Path | None = None,
                    ignore_patterns: list[str] | None = None) -> "OnlineQuantConfig":
        return cls(shorthand, shorthand["weight"], ignore_patterns or [])

    def is_layer_skipped(self, layer_name: str) -> bool:
        return any(rx.search(layer_name) for rx in self.ignore_patterns)

    def get_layer_spec(self, layer_name: str) -> LayerQuantSpec:
        spec = self._specs.get(layer_name)
        if spec is None:
            if self.is_layer_skipped(layer_name):
                spec = LayerQuantSpec(layer_name, get_quant_key(K_BF16), skipped=True, quant_method=self.name)
            else:
                spec = LayerQuantSpec(layer_name, get_quant_key(self.weight_key_name),
                                      scales=(ScaleDesc(f"{layer_name}.online_scale", "F32", ()),),
                                      quant_method=self.name)
            self._specs[layer_name] = spec
        return spec


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

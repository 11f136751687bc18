"""Quantization method base class and per-layer dispatch (same API as the
reference's ``python/ccut/quant/method.py``).

A method is a stateless compute strategy: the caller supplies the raw weight
bytes and the scale tensors, the method decides how to read and multiply
them.  Every quantized path here runs in libccq_hip.so on the GPU; inputs
given as numpy arrays are uploaded and the result is returned as numpy
(float32, the reference's contract), inputs given as CUDA tensors stay on the
device.
"""

from __future__ import annotations

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call, lib
from ccut.quant.spec import LayerQuantSpec, QuantDType, QuantKey

__all__ = ["QuantizeMethodBase", "LinearMethod", "UnquantizedMethod", "make_method_for_spec"]


class QuantizeMethodBase:
    """Base of all layer methods (reference ``method.py:29-62``)."""

    compute_path: str = "bf16"

    def create_weights(self, spec: LayerQuantSpec) -> None:
        """Validate the spec; a quantized layer without scales is an error
        (reference ``method.py:35-43``)."""
        if spec.skipped:
            return
        key = spec.effective_key()
        if key.is_quantized() and not spec.scales:
            raise ValueError(f"{spec.layer_name}: quantized layer has no scale tensors")
        self.spec = spec

    def apply(self, weight_bytes, scales: dict, x):
        """``y = x @ dequant(W).T``: ``weight_bytes`` raw ``[out, in]`` bytes,
        ``scales`` ``{name: array}``, ``x [batch, in]`` -> ``[batch, out]``."""
        raise NotImplementedError

    def process_weights_after_loading(self) -> None:
        return None


def _f32_input(x) -> torch.Tensor:
    xd = _dev.to_device(x, torch.float32)
    if xd.dim() != 2:
        raise ValueError(f"x must be [batch, in_features], got shape {tuple(xd.shape)}")
    return xd


def _return(y: torch.Tensor, x):
    return _dev.to_host(y) if _dev.is_host(x) else y


class UnquantizedMethod(QuantizeMethodBase):
    """BF16/FP16/FP32 pass-through (reference ``method.py:65-75``): the
    weight widened to float32, ``x @ W.T`` on ``ccq_f32_gemm``."""

    compute_path = "bf16"

    def __init__(self, weight_dtype: str = QuantDType.BF16):
        self.weight_dtype = weight_dtype

    def apply(self, weight_bytes, scales, x):
        xd = _f32_input(x)
        w = _unpack_weight(weight_bytes, self.weight_dtype).reshape(-1, xd.shape[1])
        return _return(f32_linear(xd, w), x)


def f32_linear(xd: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``xd [batch, in] @ w.T`` for a float32 device weight ``w [out, in]``
    (``ccq_f32_gemm``: float32 products on the fp32 matrix cores)."""
    xd = xd.contiguous()
    w = w.contiguous()
    batch, in_f = xd.shape
    out_f = w.shape[0]
    if w.dim() != 2 or w.shape[1] != in_f:
        raise ValueError(f"weight {tuple(w.shape)} does not match in_features={in_f}")
    y = torch.empty((batch, out_f), dtype=torch.float32, device=xd.device)
    nbytes = lib().ccq_f32_gemm_workspace_size(batch, in_f, out_f)
    ws = _dev.workspace("f32_gemm", nbytes, xd.device) if nbytes else None
    call("ccq_f32_gemm", xd.data_ptr(), w.data_ptr(), y.data_ptr(), batch, in_f, out_f, 1,
         ws.data_ptr() if ws is not None else None, nbytes, _dev.stream_ptr(xd.device))
    return y


def _unpack_weight(weight_bytes, dtype: str) -> torch.Tensor:
    """Raw bytes -> float32 device matrix for the unquantized dtypes
    (reference ``method.py:143-154``)."""
    raw = _dev.raw_u8(weight_bytes)
    if dtype == QuantDType.BF16:
        return raw.view(torch.bfloat16).float()
    if dtype == QuantDType.FP32:
        return raw.view(torch.float32)
    if dtype == QuantDType.FP16:
        return raw.view(torch.float16).float()
    return raw.float()


class LinearMethod(QuantizeMethodBase):
    """Per-key dispatch, W8A16 by default (reference ``method.py:78-140``).

    ``compute_mode="w8a8"`` is numerically identical to W8A16 in the
    reference (``method.py:133-140``: activations are not quantized), and so
    it is here."""

    def __init__(self, key: QuantKey, scale_name: str | None = None, compute_mode: str = "w8a16"):
        self.key = key
        self.compute_mode = (compute_mode or "w8a16").casefold()
        self.scale_name = scale_name
        if key.is_w8a8() and self.compute_mode != "w8a8":
            self.compute_path = "w8a16"
        else:
            self.compute_path = key.compute_path()

    def create_weights(self, spec: LayerQuantSpec) -> None:
        super().create_weights(spec)
        key = spec.effective_key()
        if key.weight_dtype != self.key.weight_dtype:
            raise ValueError(f"{spec.layer_name}: weight dtype mismatch {key.weight_dtype} != {self.key.weight_dtype}")

    def apply(self, weight_bytes, scales, x):
        path = self.compute_path
        if path == "w4a16":
            raise NotImplementedError(f"{path}: W4 weight-only is served by weight_only.WeightOnlyMethod")
        if path in ("w8a16", "w8a8"):
            if self.key.weight_dtype not in (QuantDType.FP8_E4M3, QuantDType.INT8):
                raise ValueError(f"w8a16 on the GPU path supports fp8_e4m3 and int8 weights, "
                                 f"not {self.key.weight_dtype}")
            scale = scales.get(self.scale_name) if self.scale_name else None
            if self.key.weight_dtype == QuantDType.INT8:
                from ccut.quant.int8 import w8a16_linear

                return w8a16_linear(weight_bytes, scale, x)
            if scale is None:
                raise ValueError(f"FP8 layer is missing its scale tensor ({self.scale_name})")
            return fp8_linear_f32(weight_bytes, scale, x)
        xd = _f32_input(x)
        w = _unpack_weight(weight_bytes, self.key.weight_dtype).reshape(-1, xd.shape[1])
        return _return(f32_linear(xd, w), x)


def fp8_linear_f32(weight_bytes, scale, x):
    """``x @ (fp8(w) * s[:, None]).T`` in float32 with ``w [out, in]`` and one
    scale per output row (reference ``method.py:109-111,120-125``)."""
    xd = _f32_input(x)
    batch, in_f = xd.shape
    raw = _dev.raw_u8(weight_bytes)
    if raw.numel() % in_f:
        raise ValueError(f"weight of {raw.numel()} bytes is not a multiple of in_features={in_f}")
    out_f = raw.numel() // in_f
    s = _dev.to_device(np.asarray(scale, dtype=np.float32) if not isinstance(scale, torch.Tensor) else scale,
                       torch.float32).reshape(-1)
    if s.numel() != out_f:
        raise ValueError(f"per-channel scale has {s.numel()} entries for {out_f} output rows")
    y = torch.empty((batch, out_f), dtype=torch.float32, device=xd.device)
    call("ccq_fp8_linear_f32", xd.data_ptr(), raw.data_ptr(), s.data_ptr(), y.data_ptr(), batch, in_f, out_f,
         _dev.stream_ptr())
    return _return(y, x)


def make_method_for_spec(spec: LayerQuantSpec) -> QuantizeMethodBase:
    """``LayerQuantSpec`` -> method (reference ``method.py:157-183``):
    skipped -> Unquantized; otherwise by weight dtype."""
    if spec.skipped:
        return UnquantizedMethod(weight_dtype=spec.effective_key().weight_dtype)
    key = spec.effective_key()
    wd = key.weight_dtype
    if wd in (QuantDType.FP8_E4M3, QuantDType.FP8_E5M2):
        from ccut.quant.fp8 import Fp8LinearMethod

        return Fp8LinearMethod(spec)
    if wd in (QuantDType.INT4, QuantDType.NF4):
        from ccut.quant.weight_only import WeightOnlyMethod

        return WeightOnlyMethod(spec)
    if wd == QuantDType.INT8:
        from ccut.quant.int8 import Int8LinearMethod

        return Int8LinearMethod(spec)
    if wd in (QuantDType.MXFP8, QuantDType.MXFP4, QuantDType.NVFP4):
        from ccut.quant.mx import MxLinearMethod

        return MxLinearMethod(spec)
    return UnquantizedMethod(weight_dtype=wd)

"""INT8 Linear method (reference ``python/ccut/quant/int8.py:20-62``).

Format: weights ``w [out, in]`` int8 (row = output channel), one float32
scale per output row, ``W[r, c] = w[r, c] * scale[r]``.

- ``compute_path="w8a16"`` (default): ``y = x @ W.T`` in float32, W formed
  on the fly (``ccq_int8_linear_f32``).  The reference writes ``out @ x``
  (``int8.py:49``), which only type-checks when ``in_features == batch``;
  this is the product its generic ``LinearMethod`` computes
  (``quant/method.py:106-111``).
- ``compute_path="w8a8"`` (``compute_mode="w8a8"`` and a key with an
  activation scale): per-token activation quantization
  (``_quantize_per_token``, ``int8.py:65-77``), exact int32 sums of the
  int8 products on MFMA, ``y = (float(acc) * x_scale) * scale`` in float32
  (``int8.py:52-62``) -- bit-identical to the reference.
"""

from __future__ import annotations

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call, lib
from ccut.quant.method import QuantizeMethodBase
from ccut.quant.spec import LayerQuantSpec

__all__ = ["Int8LinearMethod", "quantize_per_token", "int8_linear", "w8a8_linear", "w8a16_linear"]


def _weights(weight_bytes, scale, in_features: int) -> tuple[torch.Tensor, torch.Tensor]:
    raw = _dev.raw_u8(weight_bytes)
    if in_features <= 0 or raw.numel() % in_features:
        raise ValueError(f"weight of {raw.numel()} bytes is not a multiple of in_features={in_features}")
    out_f = raw.numel() // in_features
    if scale is None:
        raise ValueError("INT8 layer is missing its per-channel scale tensor")
    s = _dev.to_device(scale if isinstance(scale, torch.Tensor) else np.asarray(scale, np.float32),
                       torch.float32).reshape(-1)
    if s.numel() != out_f:
        raise ValueError(f"per-channel scale has {s.numel()} entries for {out_f} output rows")
    return raw.view(torch.int8).reshape(out_f, in_features), s


def quantize_per_token(x) -> tuple[torch.Tensor, torch.Tensor]:
    """``x [M, K]`` -> ``(xq int8 [M, K], x_scale float32 [M])`` on the device
    (reference ``int8.py:65-77``)."""
    xd = _dev.to_device(x, torch.float32)
    if xd.dim() != 2:
        raise ValueError(f"x must be [batch, in_features], got shape {tuple(xd.shape)}")
    M, K = xd.shape
    xq = torch.empty((M, K), dtype=torch.int8, device=xd.device)
    xs = torch.empty((M,), dtype=torch.float32, device=xd.device)
    call("ccq_int8_act_quant", xd.data_ptr(), xq.data_ptr(), xs.data_ptr(), M, K, _dev.stream_ptr())
    return xq, xs


def int8_linear(xq: torch.Tensor, x_scale: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor) -> torch.Tensor:
    """``(float(xq @ w.T) * x_scale[:, None]) * w_scale[None, :]`` with exact
    int32 sums; all operands device tensors (``xq [M, K]``, ``w [N, K]`` int8)."""
    if xq.dtype != torch.int8 or w.dtype != torch.int8 or xq.dim() != 2 or w.dim() != 2:
        raise ValueError("int8_linear needs int8 xq [M, K] and w [N, K]")
    M, K = xq.shape
    N = w.shape[0]
    if w.shape[1] != K or x_scale.numel() != M or w_scale.numel() != N:
        raise ValueError(f"shape mismatch: xq {tuple(xq.shape)}, w {tuple(w.shape)}, "
                         f"x_scale {x_scale.numel()}, w_scale {w_scale.numel()}")
    xq, w = xq.contiguous(), w.contiguous()
    x_scale = x_scale.contiguous().float()
    w_scale = w_scale.contiguous().float()
    y = torch.empty((M, N), dtype=torch.float32, device=xq.device)
    nbytes = int(lib().ccq_int8_linear_workspace_size(M, K, N))
    ws = _dev.workspace("int8_linear", nbytes, xq.device) if nbytes else None
    call("ccq_int8_linear", xq.data_ptr(), x_scale.data_ptr(), w.data_ptr(), w_scale.data_ptr(), y.data_ptr(),
         M, K, N, ws.data_ptr() if ws is not None else None, nbytes, _dev.stream_ptr())
    return y


def w8a8_linear(weight_bytes, scale, x):
    """The reference's ``Int8LinearMethod._w8a8`` on the GPU: one call of
    ``ccq_int8_w8a8_linear`` (the activation quantization fused into the GEMM
    for up to 4 rows)."""
    xd = _dev.to_device(x, torch.float32)
    if xd.dim() != 2:
        raise ValueError(f"x must be [batch, in_features], got shape {tuple(xd.shape)}")
    M, K = xd.shape
    w, s = _weights(weight_bytes, scale, K)
    xs = torch.empty((M,), dtype=torch.float32, device=xd.device)
    y = torch.empty((M, w.shape[0]), dtype=torch.float32, device=xd.device)
    nbytes = int(lib().ccq_int8_w8a8_workspace_size(M, K, w.shape[0]))
    ws = _dev.workspace("int8_w8a8", nbytes, xd.device) if nbytes else None
    call("ccq_int8_w8a8_linear", xd.data_ptr(), xs.data_ptr(), w.data_ptr(), s.data_ptr(), y.data_ptr(), M, K,
         w.shape[0], ws.data_ptr() if ws is not None else None, nbytes, _dev.stream_ptr())
    return _dev.to_host(y) if _dev.is_host(x) else y


def w8a16_linear(weight_bytes, scale, x):
    """``x @ (w * scale[:, None]).T`` in float32."""
    xd = _dev.to_device(x, torch.float32)
    if xd.dim() != 2:
        raise ValueError(f"x must be [batch, in_features], got shape {tuple(xd.shape)}")
    batch, in_f = xd.shape
    w, s = _weights(weight_bytes, scale, in_f)
    y = torch.empty((batch, w.shape[0]), dtype=torch.float32, device=xd.device)
    call("ccq_int8_linear_f32", xd.data_ptr(), w.data_ptr(), s.data_ptr(), y.data_ptr(), batch, in_f, w.shape[0],
         _dev.stream_ptr())
    return _dev.to_host(y) if _dev.is_host(x) else y


class Int8LinearMethod(QuantizeMethodBase):
    """INT8 per-channel weights, per-token activations (W8A8 semantics)."""

    def __init__(self, spec: LayerQuantSpec, compute_mode: str = "w8a16"):
        self.spec = spec
        self.compute_mode = compute_mode.casefold()
        key = spec.effective_key()
        self.compute_path = "w8a8" if self.compute_mode == "w8a8" and key.act_scale != "none" else "w8a16"
        self.scale_name = spec.scales[0].name if spec.scales else None

    def create_weights(self, spec: LayerQuantSpec) -> None:
        QuantizeMethodBase.create_weights(self, spec)

    def apply(self, weight_bytes, scales: dict, x):
        scale = scales.get(self.scale_name) if self.scale_name else None
        if self.compute_path == "w8a8":
            return w8a8_linear(weight_bytes, scale, x)
        return w8a16_linear(weight_bytes, scale, x)

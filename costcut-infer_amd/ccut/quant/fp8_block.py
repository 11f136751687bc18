"""FP8 e4m3fn with 128x128 block weight scales on the GPU (DeepSeek-V3-style
block FP8): per-token-per-128 activation quantization, the load-time weight
re-pack, and the block-scaled linear on FP8 MFMA.

Format: weights ``w [N, K]`` e4m3fn bytes (row = output channel),
``s_w [N/128, K/128]`` float32, ``W[n, k] = fp8(w[n, k]) * s_w[n//128,
k//128]``; activations quantized per token per 128 channels,
``s_a = max(amax, 1e-12) / 448``, ``q = RNE(x / s_a)`` saturated to +-448;
``y = dequant(q) @ W.T`` accumulated in float32.  The reference's FP8 has one
scale per output row only (``python/ccut/quant/kernels.py:150-171``) and its
"w8a8" path leaves activations unquantized (``quant/method.py:133-140``);
this module serves the block-scaled layout behind the same
``Fp8LinearMethod.apply`` boundary (``quant/fp8.py:33``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call, lib

BLOCK = 128

__all__ = ["act_quant", "Fp8BlockWeights", "prepare", "unpack", "dequant", "linear"]


def act_quant(x) -> tuple[torch.Tensor, torch.Tensor]:
    """``x [rows, K]`` (float32/float16/bfloat16) -> ``(q uint8 [rows, K]
    e4m3fn, s float32 [rows, K/128])`` on the device."""
    xd = _dev.to_device(x)
    if xd.dtype not in _dev.DTYPE_CODE:
        xd = xd.float()
    if xd.dim() != 2 or xd.shape[1] % BLOCK:
        raise ValueError(f"act_quant needs [rows, K] with K % 128 == 0, got {tuple(xd.shape)}")
    rows, K = xd.shape
    q = torch.empty((rows, K), dtype=torch.uint8, device=xd.device)
    s = torch.empty((rows, K // BLOCK), dtype=torch.float32, device=xd.device)
    call("ccq_fp8_act_quant", xd.data_ptr(), _dev.DTYPE_CODE[xd.dtype], rows, K, q.data_ptr(), s.data_ptr(),
         _dev.stream_ptr(xd.device))
    return q, s


@dataclass
class Fp8BlockWeights:
    """One block-FP8 linear resident in HBM: ``w_tiled`` holds the bytes of
    ``w [N, K]`` in the MFMA tile layout of ``ccq_fp8_block_repack``."""

    w_tiled: torch.Tensor
    s_w: torch.Tensor
    N: int
    K: int

    @property
    def nbytes(self) -> int:
        return self.w_tiled.numel() + self.s_w.numel() * 4


def _repack(w: torch.Tensor, N: int, K: int) -> torch.Tensor:
    out = torch.empty_like(w)
    call("ccq_fp8_block_repack", w.data_ptr(), out.data_ptr(), N, K, _dev.stream_ptr(w.device))
    return out


def prepare(weight_bytes, s_w, K: int | None = None) -> Fp8BlockWeights:
    """Upload (if needed) and re-pack ``w [N, K]`` with its block scales.
    ``K`` is taken from the scale shape when not given."""
    s = _dev.to_device(np.asarray(s_w, dtype=np.float32) if not isinstance(s_w, torch.Tensor) else s_w,
                       torch.float32)
    if s.dim() != 2:
        raise ValueError(f"block scales must be [N/128, K/128], got {tuple(s.shape)}")
    raw = _dev.raw_u8(weight_bytes)
    K = K or s.shape[1] * BLOCK
    if raw.numel() % K:
        raise ValueError(f"weight of {raw.numel()} bytes is not a multiple of K={K}")
    N = raw.numel() // K
    if N % BLOCK or K % BLOCK:
        raise ValueError(f"block FP8 needs N and K multiples of 128 (N={N}, K={K})")
    if tuple(s.shape) != (N // BLOCK, K // BLOCK):
        raise ValueError(f"block scales of shape {tuple(s.shape)} do not match w [{N}, {K}]")
    return Fp8BlockWeights(_repack(raw.reshape(N, K).contiguous(), N, K), s.contiguous(), N, K)


def unpack(w: Fp8BlockWeights) -> torch.Tensor:
    """Tiled bytes -> ``w [N, K]`` uint8 (inverse of the re-pack)."""
    out = torch.empty((w.N, w.K), dtype=torch.uint8, device=w.w_tiled.device)
    call("ccq_fp8_block_unpack", w.w_tiled.data_ptr(), out.data_ptr(), w.N, w.K, _dev.stream_ptr(out.device))
    return out


def dequant(w, s_w) -> torch.Tensor:
    """``W [N, K] float32 = fp8(w) * s_w[n//128, k//128]`` on the device (any
    N, K; ``s_w [ceil(N/128), ceil(K/128)]``), bit-exact."""
    wd = w if isinstance(w, torch.Tensor) else _dev.to_device(np.ascontiguousarray(w).view(np.uint8))
    wd = wd.to(_dev.require_gpu()).contiguous().view(torch.uint8)
    if wd.dim() != 2:
        raise ValueError(f"block FP8 weight must be [N, K], got {tuple(wd.shape)}")
    N, K = wd.shape
    s = _dev.to_device(s_w, torch.float32).contiguous()
    if tuple(s.shape) != (-(-N // BLOCK), -(-K // BLOCK)):
        raise ValueError(f"block scales of shape {tuple(s.shape)} do not match w [{N}, {K}]")
    out = torch.empty((N, K), dtype=torch.float32, device=wd.device)
    call("ccq_fp8_block_dequant", wd.data_ptr(), s.data_ptr(), out.data_ptr(), N, K, _dev.stream_ptr(wd.device))
    return out


def linear(weight, s_w, x, out_dtype: torch.dtype | None = None):
    """``y = dequant(act_quant(x)) @ W.T``.  ``weight`` is raw ``[N, K]``
    bytes / array / tensor or a prepared :class:`Fp8BlockWeights`.  numpy
    ``x`` -> numpy float32 (the reference's contract); CUDA ``x`` -> CUDA
    tensor of ``out_dtype`` (default: x's dtype, float32 for float32)."""
    w = weight if isinstance(weight, Fp8BlockWeights) else prepare(weight, s_w)
    xd = _dev.to_device(x)
    if xd.dtype not in _dev.DTYPE_CODE:
        xd = xd.float()
    if xd.dim() != 2 or xd.shape[1] != w.K:
        raise ValueError(f"x must be [batch, {w.K}], got {tuple(xd.shape)}")
    M = xd.shape[0]
    host = _dev.is_host(x)
    od = torch.float32 if host else (out_dtype or xd.dtype)
    y = torch.empty((M, w.N), dtype=od, device=xd.device)
    nbytes = lib().ccq_fp8_block_linear_workspace_size(M, w.K)
    ws = _dev.workspace("fp8_block_linear", nbytes, xd.device) if nbytes else None
    call("ccq_fp8_block_linear", xd.data_ptr(), _dev.DTYPE_CODE[xd.dtype], w.w_tiled.data_ptr(), w.s_w.data_ptr(),
         y.data_ptr(), _dev.DTYPE_CODE[od], M, w.K, w.N, ws.data_ptr() if ws is not None else None, nbytes,
         _dev.stream_ptr(xd.device))
    return _dev.to_host(y) if host else y

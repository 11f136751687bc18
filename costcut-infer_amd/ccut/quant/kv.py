"""FP8 KV cache quantization (reference ``python/ccut/quant/kv.py:29-101``):
mode resolution and byte budget on the host, per-token quantization and
read-back on the GPU."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call

__all__ = ["KVQuantMode", "resolve_kv_dtype", "kv_bytes_per_token", "quantize_kv_token", "dequantize_kv_token"]


class KVQuantMode:
    BF16 = "bf16"
    FP8 = "fp8"


def resolve_kv_dtype(model_dir: str | Path | None, requested: str = "auto") -> str:
    """``bf16`` / ``fp8`` as requested; ``auto`` reads ``kv_cache_scheme``
    from the checkpoint's ``config.json`` (its text config first): fp8 when
    the scheme names fp8, else bf16.  ``ValueError`` for other requests."""
    req = (requested or "auto").casefold()
    if req in (KVQuantMode.BF16, KVQuantMode.FP8):
        return req
    if req != "auto":
        raise ValueError(f"unknown kv_cache_dtype {requested!r} (auto, bf16 or fp8)")
    if model_dir is None:
        return KVQuantMode.BF16
    cfg_path = Path(model_dir) / "config.json"
    if cfg_path.exists():
        cfg = json.loads(cfg_path.read_text())
        scheme = cfg.get("text_config", cfg).get("kv_cache_scheme") or cfg.get("kv_cache_scheme")
        if scheme and "fp8" in str(scheme).casefold():
            return KVQuantMode.FP8
    return KVQuantMode.BF16


def kv_bytes_per_token(num_kv_heads: int, head_dim: int, mode: str) -> int:
    """KV bytes per token per attention layer: K and V, 2 B per element for
    bf16; 1 B per element plus one scale byte per head and side for fp8."""
    if mode == KVQuantMode.BF16:
        return 2 * num_kv_heads * head_dim * 2
    if mode == KVQuantMode.FP8:
        return 2 * num_kv_heads * head_dim + 2 * num_kv_heads
    raise ValueError(f"unknown KV quantization mode {mode!r}")


def _fill(out, dev_tensor: torch.Tensor) -> None:
    if isinstance(out, torch.Tensor):
        if out.data_ptr() != dev_tensor.data_ptr():
            out.copy_(dev_tensor.reshape(out.shape))
    else:
        np.copyto(out, dev_tensor.cpu().numpy().reshape(out.shape))


def quantize_kv_token(kv, out, scales) -> None:
    """``kv [2, heads, seq, dim]`` float32 -> e4m3 codes ``out`` (uint8, same
    shape) and one e4m3 scale byte per (side, head, token) in ``scales``
    (``ccq_kv_quant_fp8``)."""
    k = _dev.to_device(kv, torch.float32).contiguous()
    dim = k.shape[-1]
    rows = k.numel() // dim if dim else 0
    codes = torch.empty(k.shape, dtype=torch.uint8, device=k.device)
    sc = torch.empty(k.shape[:-1], dtype=torch.uint8, device=k.device)
    call("ccq_kv_quant_fp8", k.data_ptr(), codes.data_ptr(), sc.data_ptr(), rows, dim, _dev.stream_ptr())
    _fill(out, codes)
    _fill(scales, sc)


def dequantize_kv_token(fp8_kv, scales, out) -> None:
    """Inverse of ``quantize_kv_token`` into ``out`` (float32, same shape as
    the codes) (``ccq_kv_dequant_fp8``)."""
    c = _dev.to_device(fp8_kv, torch.uint8).contiguous()
    s = _dev.to_device(scales, torch.uint8).contiguous()
    dim = c.shape[-1]
    rows = c.numel() // dim if dim else 0
    if s.numel() != rows:
        raise ValueError(f"{s.numel()} scales for {rows} rows of {dim}")
    y = torch.empty(c.shape, dtype=torch.float32, device=c.device)
    call("ccq_kv_dequant_fp8", c.data_ptr(), s.data_ptr(), y.data_ptr(), rows, dim, _dev.stream_ptr())
    _fill(out, y)

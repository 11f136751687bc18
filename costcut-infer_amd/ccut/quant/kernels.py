"""GPU versions of the reference's quant kernels (``python/ccut/quant/
kernels.py``), same names and argument meaning.

Each function accepts numpy arrays (then returns / fills numpy, like the
reference) or CUDA tensors (then stays on the device).  The work runs in
libccq_hip.so; results are bit-identical to the reference for the codecs and
dequantizers.
"""

from __future__ import annotations

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call

__all__ = [
    "fp8_e4m3_to_float32",
    "float32_to_fp8_e4m3",
    "fp8_dequant_row",
    "fp8_dequant_mat",
    "int4_dequant_row",
    "int8_dequant_row",
    "int8_quantize_row",
    "mx_e8m0_to_float",
    "nf4_dequant_row",
    "silu_mul_fused",
    "group_broadcast_scale",
]


def _finish(out_dev: torch.Tensor, like, out=None):
    """Return on the caller's side: numpy in -> numpy out (or fill ``out``)."""
    if out is not None:
        if isinstance(out, torch.Tensor):
            if out.data_ptr() != out_dev.data_ptr():
                out.copy_(out_dev.reshape(out.shape))
            return out
        np.copyto(out, _dev.to_host(out_dev).reshape(out.shape))
        return out
    return _dev.to_host(out_dev) if _dev.is_host(like) else out_dev


def fp8_e4m3_to_float32(code):
    """e4m3fn bytes -> float32 (reference ``kernels.py:52-74``)."""
    c = _dev.to_device(code, torch.uint8).reshape(-1)
    out = torch.empty(c.numel(), dtype=torch.float32, device=c.device)
    call("ccq_fp8_to_f32", c.data_ptr(), out.data_ptr(), c.numel(), _dev.stream_ptr())
    return _finish(out, code)


def float32_to_fp8_e4m3(x):
    """float32 -> e4m3fn, round-half-up, saturating (reference ``kernels.py:77-123``)."""
    v = _dev.to_device(x, torch.float32).reshape(-1)
    out = torch.empty(v.numel(), dtype=torch.uint8, device=v.device)
    call("ccq_f32_to_fp8", v.data_ptr(), out.data_ptr(), v.numel(), _dev.stream_ptr())
    return _finish(out, x)


def fp8_dequant_mat(w, scale, out):
    """``out[i,j] = fp8(w[i,j]) * scale[i]`` (reference ``kernels.py:150-171``)."""
    wd = _dev.to_device(w, torch.uint8)
    rows, cols = wd.shape
    sd = _dev.to_device(scale, torch.float32).reshape(-1)
    if sd.numel() != rows:
        raise ValueError(f"fp8_dequant_mat: scale has {sd.numel()} entries for {rows} rows")
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()
                  and out.dtype == torch.float32) else torch.empty((rows, cols), dtype=torch.float32,
                                                                  device=wd.device)
    call("ccq_fp8_dequant", wd.data_ptr(), sd.data_ptr(), dst.data_ptr(), rows, cols, _dev.stream_ptr())
    return _finish(dst, w, out)


fp8_dequant_row = fp8_dequant_mat  # identical arithmetic (reference kernels.py:126-147)


def int4_dequant_row(packed, scale, out):
    """Signed-nibble int4 with per-input-column scale (reference ``kernels.py:276-295``)."""
    pd = _dev.to_device(packed, torch.uint8)
    sd = _dev.to_device(scale, torch.float32).reshape(-1)
    rows, cols = pd.shape[0], sd.numel()
    if cols % 2 or pd.shape[1] < cols // 2:
        raise ValueError(f"int4_dequant_row: packed {tuple(pd.shape)} does not hold {cols} columns")
    pd = pd[:, : cols // 2].contiguous()
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()
                  and out.dtype == torch.float32) else torch.empty((rows, cols), dtype=torch.float32,
                                                                  device=pd.device)
    call("ccq_int4_dequant", pd.data_ptr(), sd.data_ptr(), dst.data_ptr(), rows, cols, _dev.stream_ptr())
    return _finish(dst, packed, out)


def int8_dequant_row(w, scale, out):
    """``out[r, c] = w[r, c] * scale[r]`` for int8 ``w [out, in]`` and one
    scale per output row (reference ``kernels.py:180-189``)."""
    wd = _dev.to_device(w).view(torch.int8)
    if wd.dim() != 2:
        raise ValueError(f"int8_dequant_row: w must be [rows, cols], got {tuple(wd.shape)}")
    rows, cols = wd.shape
    sd = _dev.to_device(scale, torch.float32).reshape(-1)
    if sd.numel() != rows:
        raise ValueError(f"int8_dequant_row: scale has {sd.numel()} entries for {rows} rows")
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()
                  and out.dtype == torch.float32) else torch.empty((rows, cols), dtype=torch.float32,
                                                                  device=wd.device)
    call("ccq_int8_dequant", wd.data_ptr(), sd.data_ptr(), dst.data_ptr(), rows, cols, _dev.stream_ptr())
    return _finish(dst, w, out)


def int8_quantize_row(x, amax, out):
    """Per-column int8 quantization ``q = clip(round(x * 127 / amax[c]),
    -127, 127)`` (float64 arithmetic; 0 where amax is not > 0) of ``x [rows,
    cols]`` (reference ``kernels.py:192-211``); fills and returns ``out``."""
    xd = _dev.to_device(x, torch.float32)
    if xd.dim() != 2:
        raise ValueError(f"int8_quantize_row: x must be [rows, cols], got {tuple(xd.shape)}")
    rows, cols = xd.shape
    ad = _dev.to_device(amax, torch.float32).reshape(-1)
    if ad.numel() != cols:
        raise ValueError(f"int8_quantize_row: amax has {ad.numel()} entries for {cols} columns")
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()
                  and out.dtype == torch.int8) else torch.empty((rows, cols), dtype=torch.int8, device=xd.device)
    call("ccq_int8_quantize_cols", xd.data_ptr(), ad.data_ptr(), dst.data_ptr(), rows, cols, _dev.stream_ptr())
    return _finish(dst, x, out)


def nf4_dequant_row(packed, scale, table, out):
    """NF4 dequant: the int4 layout (low nibble first, one scale per input
    column) with each code looked up in ``table`` (reference
    ``kernels.py:305-322``; codes past the table give NaN)."""
    pd = _dev.to_device(packed, torch.uint8)
    sd = _dev.to_device(scale, torch.float32).reshape(-1)
    tb = _dev.to_device(np.asarray(table, np.float32) if not isinstance(table, torch.Tensor) else table,
                        torch.float32).reshape(-1)
    rows, cols = pd.shape[0], sd.numel()
    if cols % 2 or pd.shape[1] < cols // 2 or tb.numel() > 16:
        raise ValueError(f"nf4_dequant_row: packed {tuple(pd.shape)}, {cols} scales, {tb.numel()} table entries")
    pd = pd[:, : cols // 2].contiguous()
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()
                  and out.dtype == torch.float32) else torch.empty((rows, cols), dtype=torch.float32,
                                                                  device=pd.device)
    call("ccq_nf4_dequant", pd.data_ptr(), sd.data_ptr(), tb.data_ptr(), tb.numel(), dst.data_ptr(), rows, cols,
         _dev.stream_ptr())
    return _finish(dst, packed, out)


def mx_e8m0_to_float(e8m0):
    """E8M0 bytes -> float32 ``2^(e-127)``, 0 -> 0, 255 -> NaN (reference
    ``kernels.py:240-256``)."""
    from ccut.quant.mx import e8m0_bytes

    e = e8m0_bytes(e8m0)
    out = torch.empty(e.numel(), dtype=torch.float32, device=e.device)
    call("ccq_e8m0_to_f32", e.data_ptr(), out.data_ptr(), e.numel(), _dev.stream_ptr())
    return _finish(out, e8m0)


def silu_mul_fused(gate, up, out):
    """``out = silu(gate) * up`` computed in float64, stored float32
    (reference ``kernels.py:219-231``)."""
    g = _dev.to_device(gate, torch.float32)
    u = _dev.to_device(up, torch.float32)
    if g.shape != u.shape:
        raise ValueError(f"silu_mul_fused: shapes {tuple(g.shape)} and {tuple(u.shape)} differ")
    dst = out if (isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous()
                  and out.dtype == torch.float32) else torch.empty(g.shape, dtype=torch.float32, device=g.device)
    call("ccq_silu_mul", g.data_ptr(), u.data_ptr(), dst.data_ptr(), g.numel(), _dev.stream_ptr())
    return _finish(dst, gate, out)


def group_broadcast_scale(scale_groups, group_size: int, out):
    """``out[i*G + j] = s[i]`` for the ``groups * G`` leading elements of
    ``out`` (reference ``kernels.py:258-268``: ``out`` is written in place,
    elements past ``groups * G`` are left alone; ``ccq_group_broadcast_scale``).
    Returns ``out``; with ``out=None`` a new ``[groups * G]`` array (numpy in
    -> numpy out)."""
    s = _dev.to_device(scale_groups, torch.float32).reshape(-1).contiguous()
    G = int(group_size)
    if G < 0:
        raise ValueError(f"group_broadcast_scale: group_size={G} < 0")
    n = s.numel() * G
    if out is not None and int(np.prod(np.shape(out))) < n:
        raise ValueError(f"group_broadcast_scale: out has {int(np.prod(np.shape(out)))} elements, {n} needed")
    if isinstance(out, torch.Tensor) and out.is_cuda and out.is_contiguous() and out.dtype == torch.float32:
        call("ccq_group_broadcast_scale", s.data_ptr(), s.numel(), G, out.data_ptr(), _dev.stream_ptr(out.device))
        return out
    dst = torch.empty(n, dtype=torch.float32, device=s.device)
    call("ccq_group_broadcast_scale", s.data_ptr(), s.numel(), G, dst.data_ptr(), _dev.stream_ptr())
    if out is None:
        return _dev.to_host(dst) if _dev.is_host(scale_groups) else dst
    if isinstance(out, torch.Tensor):
        out.reshape(-1)[:n].copy_(dst.to(out.device, out.dtype))
        return out
    if not out.flags.c_contiguous:
        raise ValueError("group_broadcast_scale: out must be C-contiguous (it is written in place)")
    out.reshape(-1)[:n] = _dev.to_host(dst)
    return out

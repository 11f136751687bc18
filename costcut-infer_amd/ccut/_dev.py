"""Device plumbing shared by the Python front end: tensors in HBM, streams,
dtype codes.  torch is used only for device memory and streams here; every
computation runs in libccq_hip.so."""

from __future__ import annotations

import warnings

import numpy as np
import torch

from ccut._lib import CCQ_BF16, CCQ_F16, CCQ_F32

DTYPE_CODE = {torch.float32: CCQ_F32, torch.float16: CCQ_F16, torch.bfloat16: CCQ_BF16}


def require_gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("the quantized expert path runs on a ROCm GPU only (no CPU fallback); "
                           "torch.cuda.is_available() is False")
    return torch.device("cuda", torch.cuda.current_device())


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def is_host(a) -> bool:
    return not (isinstance(a, torch.Tensor) and a.is_cuda)


def to_device(a, dtype: torch.dtype | None = None) -> torch.Tensor:
    """numpy / bytes / torch -> contiguous tensor on the current GPU."""
    dev = require_gpu()
    if isinstance(a, (bytes, bytearray, memoryview)):
        a = np.frombuffer(a, dtype=np.uint8)
    if isinstance(a, np.ndarray):
        with warnings.catch_warnings():
            # read-only arrays (np.frombuffer over weight bytes) are only read here: uploaded, never written
            warnings.filterwarnings("ignore", message="The given NumPy array is not writable")
            t = torch.from_numpy(np.ascontiguousarray(a))
    elif isinstance(a, torch.Tensor):
        t = a
    else:
        t = torch.as_tensor(a)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.to(dev, non_blocking=False).contiguous()


def half_for_mfma(x_f32: torch.Tensor, host=None) -> torch.dtype:
    """The 16-bit type float32 activations take into a bf16 / fp16 MFMA:
    float16 (11 significant bits) when every |x| is finite and fits its
    range, else bfloat16 (8 bits, float32's range).  ``host``: the same
    values as a host array, when the caller has them (no device read)."""
    if x_f32.numel() == 0:
        amax = 0.0
    elif host is not None:
        amax = float(np.abs(np.asarray(host, np.float32)).max())
    else:
        amax = float(x_f32.abs().amax().item())
    return torch.float16 if np.isfinite(amax) and amax <= 65504.0 else torch.bfloat16


def to_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def raw_u8(weight_bytes) -> torch.Tensor:
    """The reference passes weights as raw bytes or any ndarray (reinterpreted
    as uint8, ``quant/method.py:103-106``); return a uint8 device view."""
    if isinstance(weight_bytes, torch.Tensor):
        t = weight_bytes if weight_bytes.is_cuda else to_device(weight_bytes)
        return t.contiguous().view(torch.uint8).reshape(-1)
    if isinstance(weight_bytes, (bytes, bytearray, memoryview)):
        return to_device(np.frombuffer(weight_bytes, dtype=np.uint8))
    arr = np.ascontiguousarray(np.asarray(weight_bytes))
    return to_device(arr.reshape(-1).view(np.uint8))


_WS: dict[tuple, torch.Tensor] = {}


def workspace(tag: str, nbytes: int, device: torch.device | None = None) -> torch.Tensor:
    """Per-device, per-tag zero-initialised scratch that only grows.  Kernels
    that use counters in it leave them at zero after every call, so the buffer
    is zeroed only when (re)allocated."""
    dev = device or require_gpu()
    key = (tag, dev.index)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)
        _WS[key] = buf
    return buf

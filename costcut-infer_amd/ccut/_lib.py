"""ctypes binding of ``libccq_hip.so`` (the C ABI in ``include/ccq.h``).

torch is imported before the library is opened: torch ships its own HIP
runtime whose soname (``libamdhip64.so.7``) is the one the library links
against, so both share one runtime (one set of streams, one allocator).

There is no fallback: if the library is missing or fails to load, every
entry point raises :class:`CcqLibraryError`.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(os.environ.get("CCQ_LIB", Path(__file__).resolve().parent / "_lib" / "libccq_hip.so"))

CCQ_F32, CCQ_F16, CCQ_BF16 = 0, 1, 2
CCQ_EINVAL, CCQ_EUNSUPPORTED, CCQ_EWORKSPACE = -1, -2, -3
CCQ_MOE_W4_NOALLOC_BYTES = 32 << 20  # the per-GPU scratch array of ccq_moe_w4_forward_noalloc

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t


class CcqLibraryError(RuntimeError):
    """libccq_hip.so is missing or unusable."""


class ccq_w4_experts(ctypes.Structure):
    _fields_ = [
        ("w_gate", _vp), ("sz_gate", _vp),
        ("w_up", _vp), ("sz_up", _vp),
        ("w_down", _vp), ("sz_down", _vp),
        ("scale_dtype", _int),
        ("num_experts", _i64), ("hidden", _i64), ("inter", _i64), ("group_size", _i64),
    ]


class ccq_fp8_experts(ctypes.Structure):
    _fields_ = [
        ("w_gate", _vp), ("s_gate", _vp),
        ("w_up", _vp), ("s_up", _vp),
        ("w_down", _vp), ("s_down", _vp),
        ("num_experts", _i64), ("hidden", _i64), ("inter", _i64),
    ]


class ccq_fp8row_experts(ctypes.Structure):
    _fields_ = [
        ("w_gate", _vp), ("s_gate", _vp),
        ("w_up", _vp), ("s_up", _vp),
        ("w_down", _vp), ("s_down", _vp),
        ("num_experts", _i64), ("hidden", _i64), ("inter", _i64),
    ]


# name -> (restype, argtypes); the order follows include/ccq.h
SIGNATURES: dict[str, tuple] = {
    "ccq_version": (_int, []),
    "ccq_last_error": (ctypes.c_char_p, []),
    "ccq_launch_timer": (_int, [_vp, _vp]),
    "ccq_fp8_to_f32": (_int, [_vp, _vp, _i64, _vp]),
    "ccq_f32_to_fp8": (_int, [_vp, _vp, _i64, _vp]),
    "ccq_fp8_dequant": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_quantize_rows_fp8": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_kv_quant_fp8": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_kv_dequant_fp8": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_group_broadcast_scale": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "ccq_silu_mul": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "ccq_int4_dequant": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_int4_linear_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "ccq_fp8_linear_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "ccq_int8_linear_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "ccq_int8_dequant": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_int8_act_quant": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_int8_linear_workspace_size": (_sz, [_i64, _i64, _i64]),
    "ccq_int8_linear": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "ccq_int8_w8a8_workspace_size": (_sz, [_i64, _i64, _i64]),
    "ccq_int8_w8a8_linear": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "ccq_e8m0_to_f32": (_int, [_vp, _vp, _i64, _vp]),
    "ccq_nf4_dequant": (_int, [_vp, _vp, _vp, _int, _vp, _i64, _i64, _vp]),
    "ccq_nf4_linear_f32": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _i64, _i64, _i64, _vp]),
    "ccq_int8_quantize_cols": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_moe_combine_shared": (_int, [_vp, _vp, _vp, ctypes.c_float, _vp, _int, _i64, _i64, _i64, _vp]),
    "ccq_shared_expert_add": (_int, [_vp, _vp, ctypes.c_float, _i64, _vp]),
    "ccq_moe_w4_ffn_shared": (_int, [_vp, _int, _vp, _vp, _vp, ctypes.c_float, _vp, _int, _i64, _i64,
                                     ctypes.POINTER(ccq_w4_experts), _vp, _sz, _vp]),
    "ccq_moe_fp8_ffn_shared": (_int, [_vp, _int, _vp, _vp, _vp, ctypes.c_float, _vp, _int, _i64, _i64,
                                      ctypes.POINTER(ccq_fp8_experts), _vp, _sz, _vp]),
    "ccq_mx_dequant": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _int, ctypes.c_float, _vp]),
    "ccq_mx_linear_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, ctypes.c_float, _vp]),
    "ccq_wq_mfma_linear_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, ctypes.c_float, _vp]),
    "ccq_awq_dequant": (_int, [_vp, _vp, _vp, _int, _vp, _i64, _i64, _i64, _vp]),
    "ccq_awq_repack": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "ccq_awq_unpack_tiled": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "ccq_awq_sz_words": (_i64, [_i64, _i64]),
    "ccq_awq_pack_sz": (_int, [_vp, _vp, _int, _vp, _i64, _i64, _i64, _vp]),
    "ccq_w4_gemm_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "ccq_w4_gemm": (_int, [_vp, _int, _vp, _vp, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "ccq_topk_softmax": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "ccq_moe_align_max_tiles": (_i64, [_i64, _i64, _i64]),
    "ccq_moe_align": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "ccq_moe_combine": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _vp]),
    "ccq_moe_w4_gate_up": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _i64, _vp, ctypes.POINTER(ccq_w4_experts),
                                  _vp]),
    "ccq_moe_w4_down": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _vp, ctypes.POINTER(ccq_w4_experts), _vp]),
    "ccq_moe_w4_workspace_size": (_sz, [_i64, _i64, ctypes.POINTER(ccq_w4_experts)]),
    "ccq_moe_w4_ffn": (_int, [_vp, _int, _vp, _vp, _vp, _int, _i64, _i64,
                              ctypes.POINTER(ccq_w4_experts), _vp, _sz, _vp]),
    "ccq_moe_w4_forward": (_int, [_vp, _int, _vp, _i64, _i64, _int, _vp, _vp, _vp, _int,
                                  ctypes.POINTER(ccq_w4_experts), _vp, _sz, _vp]),
    "ccq_moe_w4_route_gate_up": (_int, [_vp, _int, _vp, _i64, _i64, _int, _vp, _vp,
                                        ctypes.POINTER(ccq_w4_experts), _vp, _sz, _vp]),
    "ccq_moe_w4_forward_shared": (_int, [_vp, _int, _vp, _i64, _i64, _int, ctypes.c_float, _vp, _vp, _vp, _int,
                                         ctypes.POINTER(ccq_w4_experts), _vp, _sz, _vp]),
    "ccq_moe_w4_forward_noalloc": (_int, [_vp, _int, _vp, _i64, _i64, _int, _vp, _vp, _vp, _int,
                                          ctypes.POINTER(ccq_w4_experts), _vp]),
    "ccq_fp8_act_quant": (_int, [_vp, _int, _i64, _i64, _vp, _vp, _vp]),
    "ccq_fp8_block_repack": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "ccq_fp8_block_unpack": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "ccq_fp8_block_dequant": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "ccq_fp8_block_linear_workspace_size": (_sz, [_i64, _i64]),
    "ccq_fp8_block_linear": (_int, [_vp, _int, _vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _sz, _vp]),
    "ccq_moe_fp8_workspace_size": (_sz, [_i64, _i64, ctypes.POINTER(ccq_fp8_experts)]),
    "ccq_moe_fp8_ffn": (_int, [_vp, _int, _vp, _vp, _vp, _int, _i64, _i64,
                               ctypes.POINTER(ccq_fp8_experts), _vp, _sz, _vp]),
    "ccq_moe_fp8row_workspace_size": (_sz, [_i64, _i64, ctypes.POINTER(ccq_fp8row_experts)]),
    "ccq_moe_fp8row_ffn": (_int, [_vp, _vp, _vp, _vp, _int, _i64, _i64, ctypes.POINTER(ccq_fp8row_experts), _vp,
                                  _sz, _vp]),
    "ccq_moe_fp8row_ffn_shared": (_int, [_vp, _vp, _vp, _vp, ctypes.c_float, _vp, _int, _i64, _i64,
                                         ctypes.POINTER(ccq_fp8row_experts), _vp, _sz, _vp]),
    "ccq_f32_gemm_workspace_size": (_sz, [_i64, _i64, _i64]),
    "ccq_f32_gemm": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "ccq_expert_ffn_f32_workspace_size": (_sz, [_i64, _i64]),
    "ccq_expert_ffn_f32": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "ccq_moe_f32_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "ccq_moe_f32_ffn": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _int, _i64, _i64, _i64,
                               _i64, _i64, _vp, _sz, _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Open the library once (thread-safe) and bind every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise CcqLibraryError(
                f"{LIB_PATH} not found: build it with `python -m ccut._build` (from costcut-infer_amd/) "
                "or __graft_entry__.build(); the quantized path has no CPU fallback")
        try:
            handle = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:  # pragma: no cover - depends on the host
            raise CcqLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
        return handle


def last_error() -> str:
    return lib().ccq_last_error().decode("utf-8", "replace")


def check(rc: int, what: str) -> None:
    """Raise the reference's exception types: ValueError for argument errors
    (``quant/method.py:42,98,131``), RuntimeError for launch failures."""
    if rc == 0:
        return
    msg = last_error()
    if rc < 0:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)

"""AWQ int4 weights on the GPU: packing helpers, the load-time re-pack into the
gfx950 tile layout, and the fused dequant-GEMM.

Format (public AutoAWQ GEMM packing): ``qweight`` int32 ``[K, N/8]`` with
column ``8c + j`` of word ``[k, c]`` at bit ``4 * [0,4,1,5,2,6,3,7][j]``;
``qzeros`` int32 ``[K/G, N/8]`` packed the same way; ``scales`` fp16 (or
bf16) ``[K/G, N]``; ``W[k, n] = (q - z) * s`` and ``y = x @ W``.  The
reference registers group-quantized layers under the names ``.scales`` /
``.zero_points`` (``python/ccut/quant/compressed_tensors.py:209-211``) but
has no arithmetic for them; this module supplies it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ccut import _dev
from ccut._lib import call, lib

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def pack_awq(q: torch.Tensor) -> torch.Tensor:
    """``q [R, N]`` integers 0..15 -> int32 ``[R, N/8]`` in AWQ order (runs
    wherever ``q`` lives)."""
    if q.shape[-1] % 8:
        raise ValueError(f"pack_awq: N={q.shape[-1]} is not a multiple of 8")
    q8 = q.to(torch.int64).reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    word = torch.zeros(q8.shape[:-1], dtype=torch.int64, device=q.device)
    for i, col in enumerate(AWQ_ORDER):
        word |= (q8[..., col] & 0xF) << (4 * i)
    return torch.where(word >= 2 ** 31, word - 2 ** 32, word).to(torch.int32)


def unpack_awq(packed: torch.Tensor) -> torch.Tensor:
    """int32 ``[R, N/8]`` -> uint8 ``[R, N]`` (inverse of :func:`pack_awq`)."""
    w = packed.to(torch.int64) & 0xFFFFFFFF
    cols = [((w >> (4 * AWQ_REVERSE_ORDER[j])) & 0xF) for j in range(8)]
    return torch.stack(cols, dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 8).to(torch.uint8)


@dataclass
class AwqWeights:
    """One AWQ linear resident in HBM, re-packed once for the GPU kernels.

    ``w_tiled`` has the bytes of ``qweight`` in the tile layout of
    ``ccq_awq_repack``; ``sz`` holds one 32-bit word per (column, group) with
    the scale bits and the zero point (``ccq_awq_pack_sz``)."""

    w_tiled: torch.Tensor
    sz: torch.Tensor
    scale_dtype: torch.dtype
    K: int
    N: int
    group_size: int

    @property
    def nbytes(self) -> int:
        """Bytes resident in HBM."""
        return self.w_tiled.numel() * self.w_tiled.element_size() + self.sz.numel() * self.sz.element_size()

    @property
    def format_bytes(self) -> int:
        """Bytes of the AWQ format itself (int4 weights, 16-bit scales, int4
        zeros): the algorithmic traffic of one pass over the weight."""
        groups = self.K // self.group_size
        return self.K * self.N // 2 + groups * self.N * 2 + groups * self.N // 2


def _scale_code(scales) -> int:
    dt = scales if isinstance(scales, torch.dtype) else scales.dtype
    if dt == torch.float16:
        return 1
    if dt == torch.bfloat16:
        return 2
    raise ValueError(f"AWQ scales must be float16 or bfloat16, got {dt}")


def repack(qweight, K: int, N: int) -> torch.Tensor:
    """AWQ ``qweight`` -> tile layout (device tensor of the same byte count)."""
    qw = _dev.to_device(qweight).view(torch.int32).reshape(K, N // 8)
    out = torch.empty_like(qw)
    call("ccq_awq_repack", qw.data_ptr(), out.data_ptr(), K, N, _dev.stream_ptr())
    return out


def unpack_tiled(w_tiled: torch.Tensor, K: int, N: int) -> torch.Tensor:
    out = torch.empty((K, N // 8), dtype=torch.int32, device=w_tiled.device)
    call("ccq_awq_unpack_tiled", w_tiled.data_ptr(), out.data_ptr(), K, N, _dev.stream_ptr())
    return out


def pack_sz(qzeros, scales, K: int, N: int, group_size: int) -> torch.Tensor:
    """``qzeros [K/G, N/8]`` + ``scales [K/G, N]`` -> ``sz [N, words]`` uint32
    (stored as int32) with ``words = ccq_awq_sz_words(K, G)``."""
    qz = _dev.to_device(qzeros).view(torch.int32).contiguous()
    sc = _dev.to_device(scales).contiguous()
    words = lib().ccq_awq_sz_words(K, group_size)
    out = torch.empty((N, words), dtype=torch.int32, device=qz.device)
    call("ccq_awq_pack_sz", qz.data_ptr(), sc.data_ptr(), _scale_code(sc), out.data_ptr(), K, N, group_size,
         _dev.stream_ptr())
    return out


def prepare(qweight, qzeros, scales, group_size: int = 128) -> AwqWeights:
    """Upload (if needed) and re-pack one AWQ linear.  Validates shapes with
    the reference's error type (``ValueError``, ``quant/method.py:42``)."""
    qz = _dev.to_device(qzeros).view(torch.int32)
    sc = _dev.to_device(scales)
    if sc.dtype not in (torch.float16, torch.bfloat16):
        sc = sc.to(torch.float16)
    if sc.dim() != 2:
        raise ValueError(f"AWQ scales must be 2-D [K/G, N], got {tuple(sc.shape)}")
    if group_size not in (32, 64, 128):
        raise ValueError(f"AWQ group size {group_size} not in (32, 64, 128)")
    groups, N = sc.shape
    K = groups * group_size
    qw = _dev.to_device(qweight).view(torch.int32)
    if qw.numel() != K * N // 8:
        raise ValueError(f"AWQ qweight has {qw.numel()} words, expected K*N/8 = {K * N // 8}")
    if qz.numel() != groups * N // 8:
        raise ValueError(f"AWQ qzeros has {qz.numel()} words, expected {groups * N // 8}")
    if K % 128 or N % 16:
        raise ValueError(f"AWQ GPU path needs K % 128 == 0 and N % 16 == 0 (K={K}, N={N})")
    return AwqWeights(repack(qw, K, N), pack_sz(qz.reshape(groups, N // 8), sc, K, N, group_size), sc.dtype, K, N,
                      group_size)


def dequant(qweight, qzeros, scales, group_size: int = 128) -> torch.Tensor:
    """Bit-exact ``W [K, N] float32 = (q - z) * s`` on the device."""
    qz = _dev.to_device(qzeros).view(torch.int32)
    sc = _dev.to_device(scales)
    groups, N = sc.shape
    K = groups * group_size
    qw = _dev.to_device(qweight).view(torch.int32)
    out = torch.empty((K, N), dtype=torch.float32, device=qw.device)
    call("ccq_awq_dequant", qw.data_ptr(), qz.data_ptr(), sc.data_ptr(), _scale_code(sc), out.data_ptr(),
         K, N, group_size, _dev.stream_ptr())
    return out


def gemm(x: torch.Tensor, w: AwqWeights, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``y = x @ dequant(W)`` with fp32 accumulation; x fp16/bf16 ``[M, K]``."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"AWQ GEMM activations must be float16 or bfloat16, got {x.dtype}")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    M, K = x2.shape
    if K != w.K:
        raise ValueError(f"AWQ GEMM: x has {K} features, weight expects {w.K}")
    out_dtype = out_dtype or x.dtype
    y = torch.empty((M, w.N), dtype=out_dtype, device=x.device)
    nbytes = lib().ccq_w4_gemm_workspace_size(M, K, w.N, w.group_size)
    ws = _dev.workspace("w4_gemm", nbytes, x.device) if nbytes else None
    call("ccq_w4_gemm", x2.data_ptr(), _dev.DTYPE_CODE[x.dtype], w.w_tiled.data_ptr(), w.sz.data_ptr(),
         _scale_code(w.scale_dtype), y.data_ptr(), _dev.DTYPE_CODE[out_dtype], M, K, w.N, w.group_size,
         ws.data_ptr() if ws is not None else None, nbytes, _dev.stream_ptr(x.device))
    return y.reshape(*x.shape[:-1], w.N)

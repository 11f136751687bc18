"""Oracle: FP8 e4m3 with 128x128 block weight scales and per-token-per-128
dynamic activation quantization.

Test infrastructure only (see ``oracle/__init__.py``).

The reference implements FP8 with one scale per output row only
(``python/ccut/quant/kernels.py:150-171``) and its "w8a8" path does not
quantize activations (``quant/method.py:133-140``).  The block-scaled scheme
restated here is the public DeepSeek-V3 style FP8 format:

* weights ``w [N, K]`` e4m3fn bytes, ``s_w [N/128, K/128]`` float32,
  ``W[n, k] = fp8(w[n, k]) * s_w[n//128, k//128]`` (one float32 rounding);
* activations ``x [T, K]``: ``amax = max|x|`` over each 128-channel block of a
  token, ``s_a = max(amax, 1e-12) / 448`` (float32), ``q = RNE(clip(x / s_a,
  -448, 448))`` to e4m3fn;
* ``y = (fp8(q) * s_a) @ W.T`` in float32 (dequantize-then-matmul);
* the MoE expert: ``expert_ffn`` of the reference on these dequantized
  weights, the intermediate in float32.

Parity against the reference is unpinned (the scheme is absent there).  RNE
encoding is pinned against ``torch.Tensor.to(torch.float8_e4m3fn)``.
"""

from __future__ import annotations

import numpy as np

from oracle.ref_quant import FP8_TABLE, silu_mul_fused

BLOCK = 128
AMAX_FLOOR = np.float32(1e-12)
FP8_MAX = np.float32(448.0)

_POS = FP8_TABLE[:0x7F].astype(np.float64)  # codes 0x00..0x7E, increasing
# two codes at once: entry b0 | b1 << 8 holds the float32 bits of
# (FP8_TABLE[b0], FP8_TABLE[b1]) (a byte-pair lookup is much faster in numpy
# than a per-byte one)
_T32 = FP8_TABLE.astype(np.float32).view(np.uint32).astype(np.uint64)
_PAIR = ((_T32[:, None] << np.uint64(32)) | _T32[None, :]).reshape(-1)


def decode(w: np.ndarray) -> np.ndarray:
    """e4m3fn bytes -> float32 values (``FP8_TABLE[w]``)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    if w.ndim == 0 or w.shape[-1] % 2:
        return FP8_TABLE[w].astype(np.float32)
    return _PAIR[w.view(np.uint16)].view(np.float32).reshape(w.shape)


def float32_to_fp8_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn, round-to-nearest-even, saturating to +-448,
    NaN -> 0x7F.  Brute-force nearest search over the 127 finite magnitudes."""
    v = np.asarray(x, dtype=np.float32).reshape(-1).astype(np.float64)
    a = np.minimum(np.abs(v), 448.0)
    hi = np.searchsorted(_POS, a, side="left")  # first code with value >= a
    hi = np.clip(hi, 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    dlo = a - _POS[lo]
    dhi = _POS[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(_POS[hi] == a, hi, code)
    sign = np.where(np.signbit(v), 0x80, 0)
    out = (code | sign).astype(np.uint8)
    out[np.isnan(v)] = 0x7F
    return out


def act_quant(x: np.ndarray, block: int = BLOCK) -> tuple[np.ndarray, np.ndarray]:
    """Per-token-per-``block`` dynamic quantization -> ``(q u8 [T,K],
    s_a f32 [T, K/block])``."""
    x = np.asarray(x, dtype=np.float32)
    T, K = x.shape
    assert K % block == 0
    xb = x.reshape(T, K // block, block)
    amax = np.abs(xb).max(axis=2).astype(np.float32)
    s = (np.maximum(amax, AMAX_FLOOR) / FP8_MAX).astype(np.float32)
    scaled = (xb / s[:, :, None]).astype(np.float32)
    scaled = np.clip(scaled, -FP8_MAX, FP8_MAX)
    q = float32_to_fp8_rne(scaled).reshape(T, K)
    return q, s


def act_dequant(q: np.ndarray, s: np.ndarray, block: int = BLOCK) -> np.ndarray:
    T, K = q.shape
    dec = FP8_TABLE[q].astype(np.float64).reshape(T, K // block, block)
    return (dec * np.asarray(s, dtype=np.float64)[:, :, None]).astype(np.float32).reshape(T, K)


def block_dequant(w: np.ndarray, s_w: np.ndarray, block: int = BLOCK) -> np.ndarray:
    """``W [N, K] f32 = fp8(w) * s_w[n//128, k//128]``.  The decoded code has
    at most 4 significant bits, so the float32 product is the correctly
    rounded exact product (one rounding, as in float64 then a cast)."""
    w = np.asarray(w, dtype=np.uint8)
    N, K = w.shape
    s = np.asarray(s_w, dtype=np.float32)
    nb, kb = -(-N // block), -(-K // block)
    dec = np.zeros((nb * block, kb * block), dtype=np.float32)
    dec[:N, :K] = decode(w)
    out = dec.reshape(nb, block, kb, block) * s[:nb, None, :kb, None]
    return out.reshape(nb * block, kb * block)[:N, :K]


def linear(x: np.ndarray, w: np.ndarray, s_w: np.ndarray) -> np.ndarray:
    """Quantize x per token per 128, dequantize both sides, float32 matmul."""
    q, s = act_quant(x)
    return act_dequant(q, s) @ block_dequant(w, s_w).T


def to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), back to float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def expert_ffn(x, wg, sg, wu, su, wd, sd) -> np.ndarray:
    """One FP8-block expert as the reference's ``expert_ffn`` computes it on
    dequantized weights (``blocks/moe.py:122-141``): ``down(silu(x Wg^T) *
    (x Wu^T))`` in float32, with x quantized per token per 128 (the block
    scheme's dynamic activation quantization) before gate and up, and the
    SiLU intermediate kept in float32 (no rounding or re-quantization
    before the down projection).

    ``wg, wu [I, H]``, ``wd [H, I]`` e4m3 bytes (row = output channel) with
    block scales ``[N/128, K/128]``."""
    gate = linear(x, wg, sg)
    up = linear(x, wu, su)
    h = silu_mul_fused(gate, up)
    return h @ block_dequant(wd, sd).T

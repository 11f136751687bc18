"""Oracle: restatement of the reference's quant kernels and Linear methods.

Test infrastructure only (see ``oracle/__init__.py``).  numpy, float64 where
the reference's numba code computes in float64 and stores float32, so each
stored value is the single rounding of the same exact product.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# FP8 e4m3fn  (reference python/ccut/quant/kernels.py:52-123)
# ---------------------------------------------------------------------------


def fp8_e4m3_to_float32(code: np.ndarray) -> np.ndarray:
    """e4m3fn byte -> float32.  Follows ``kernels.py:52-74``.

    exp == 0: ``mant/8 * 2^-6``; exp == 15 and mant == 7: NaN; otherwise
    ``(1 + mant/8) * 2^(exp-7)``; bit 7 is the sign.  All values are exact in
    float32.
    """
    b = np.asarray(code, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    exp = (b >> 3) & 0x0F
    mant = b & 0x07
    val = np.where(exp == 0, mant * 0.125 * 2.0 ** -6, (1.0 + mant * 0.125) * np.exp2(exp - 7.0))
    val = np.where((exp == 15) & (mant == 7), np.nan, val)
    return (sign * val).astype(np.float32)


FP8_TABLE = fp8_e4m3_to_float32(np.arange(256, dtype=np.uint8))


def float32_to_fp8_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn byte with the reference's rounding.  Follows
    ``kernels.py:77-123``.

    Round-half-UP on the magnitude (``int(m*8 + 0.5)``, not RNE); ``|v| >= 464``
    saturates to 0x7E (448); NaN -> 0x7F; ``-0.0`` -> 0x00 (the sign test is
    ``v < 0``); subnormal branch below 2^-6 rounds ``v*512`` half-up and carries
    into 0x08.  ``e = floor(log2 v)`` is taken from the float32 exponent field,
    which equals the reference's float64 ``np.floor(np.log2(v))`` for every
    normal float32 input.
    """
    v = np.asarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(v.shape[0], dtype=np.uint8)
    vd = v.astype(np.float64)
    nan = np.isnan(vd)
    sign = np.where(vd < 0, 0x80, 0x00).astype(np.int64)
    a = np.abs(vd)
    res = np.zeros(v.shape[0], dtype=np.int64)
    sat = a >= 464.0
    zero = a == 0.0
    sub = (a < 0.015625) & ~zero
    norm = ~(sat | zero | sub | nan)
    # subnormal: mant = int(v*512 + 0.5), carry to the smallest normal
    t = a[sub] * 512.0
    ms = np.floor(t + 0.5).astype(np.int64)
    res[sub] = np.where(ms >= 8, 0x08, ms)
    # normal: v in [2^-6, 464)
    an = a[norm]
    e = np.floor(np.log2(an)).astype(np.int64)
    m = an * np.exp2(-e.astype(np.float64)) - 1.0
    mant = np.floor(m * 8.0 + 0.5).astype(np.int64)
    ec = e + 7
    carry = mant >= 8
    mant = np.where(carry, 0, mant)
    ec = np.where(carry, ec + 1, ec)
    mant = np.where((ec >= 15) & (mant > 6), 6, mant)
    res[norm] = ((ec & 0xF) << 3) | mant
    res[sat] = 0x7E
    res = res | sign
    res[zero] = sign[zero]
    res[nan] = 0x7F
    out[:] = res.astype(np.uint8)
    return out


def fp8_dequant_mat(w: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Per-output-row FP8 dequant ``out[i,j] = fp8(w[i,j]) * scale[i]``.

    Follows ``kernels.py:150-171`` (and the identical ``fp8_dequant_row``
    ``kernels.py:126-147``): the product of the exact decoded value and the
    float32 scale is formed in float64 and stored to float32 (one rounding).
    """
    w = np.asarray(w, dtype=np.uint8)
    s = np.asarray(scale, dtype=np.float32).reshape(-1).astype(np.float64)
    dec = FP8_TABLE[w].astype(np.float64)
    return (dec * s[:, None]).astype(np.float32)


def int4_dequant_row(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Reference int4: signed two's-complement nibbles, low nibble first, one
    float32 scale per INPUT column.  Follows ``kernels.py:276-295``.

    ``packed [rows, cols/2] u8``, ``scale [cols] f32`` -> ``[rows, cols] f32``
    with ``out[r, 2j] = lo * scale[2j]`` and ``out[r, 2j+1] = hi * scale[2j+1]``
    (float64 product, float32 store).
    """
    p = np.asarray(packed, dtype=np.uint8)
    s = np.asarray(scale, dtype=np.float32).reshape(-1)
    cols = s.shape[0]
    p = p[:, : cols // 2].astype(np.int64)
    lo = p & 0x0F
    hi = (p >> 4) & 0x0F
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty((p.shape[0], cols), dtype=np.float32)
    sd = s.astype(np.float64)
    out[:, 0::2] = (lo.astype(np.float64) * sd[0::2]).astype(np.float32)
    out[:, 1::2] = (hi.astype(np.float64) * sd[1::2]).astype(np.float32)
    return out


def silu_mul_fused(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``out = g / (1 + exp(-g)) * u`` in float64, stored float32.
    Follows ``kernels.py:219-231``."""
    g = np.asarray(gate, dtype=np.float32).astype(np.float64)
    u = np.asarray(up, dtype=np.float32).astype(np.float64)
    return ((g / (1.0 + np.exp(-g))) * u).astype(np.float32)


def group_broadcast_scale(scale_groups: np.ndarray, group_size: int) -> np.ndarray:
    """``out[i*G + j] = s[i]``.  Follows ``kernels.py:258-268``."""
    return np.repeat(np.asarray(scale_groups, dtype=np.float32), group_size)


# ---------------------------------------------------------------------------
# Linear methods  (reference quant/weight_only.py, quant/method.py)
# ---------------------------------------------------------------------------


def _raw_u8(weight_bytes) -> np.ndarray:
    if isinstance(weight_bytes, (bytes, bytearray, memoryview)):
        return np.frombuffer(weight_bytes, dtype=np.uint8)
    return np.asarray(weight_bytes).reshape(-1).view(np.uint8)


def weight_only_apply(weight_bytes, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``WeightOnlyMethod.apply`` for int4: reshape the raw bytes to
    ``[out, in/2]``, dequantize, ``x @ W.T`` in float32.
    Follows ``weight_only.py:37-54`` (file lines 37-54 of the reference)."""
    x = np.asarray(x, dtype=np.float32)
    in_features = x.shape[1]
    packed = _raw_u8(weight_bytes).reshape(-1, in_features // 2)
    w = int4_dequant_row(packed, scale)
    return x @ w.T


def fp8_linear_apply(weight_bytes, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``LinearMethod.apply`` on the ``w8a16`` path (also used for ``w8a8``,
    which does not quantize x): ``x @ (fp8(w) * s[:,None]).T`` in float32.
    Follows ``method.py:100-111`` and ``method.py:120-125,133-140``."""
    x = np.asarray(x, dtype=np.float32)
    in_features = x.shape[1]
    w_q = _raw_u8(weight_bytes).reshape(-1, in_features)
    w = fp8_dequant_mat(w_q, scale)
    return x @ w.T


def bf16_bits_to_float32(u16: np.ndarray) -> np.ndarray:
    """BF16 bits -> float32 by a 16-bit left shift.  Follows
    ``io_/safetensors_io.py:53-57``."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


NF4_TABLE = np.array([-1.0, -0.6961928, -0.39238566, -0.08857854, 0.21522858, 0.51903564, 0.8228427, 1.1266499],
                     dtype=np.float32)


def nf4_dequant_row(packed: np.ndarray, scale: np.ndarray, table: np.ndarray = NF4_TABLE) -> np.ndarray:
    """nf4_dequant_row (reference python/ccut/quant/kernels.py:299-322): the
    int4 layout, out[r, 2j] = table[lo] * scale[2j], out[r, 2j+1] =
    table[hi] * scale[2j+1].  The reference indexes its 8-entry table with
    the 4-bit code unchecked; codes past the table give NaN here."""
    p = np.asarray(packed, np.uint8)
    s = np.asarray(scale, np.float32)
    cols = s.shape[0]
    t = np.full(16, np.nan, np.float32)
    t[: len(table)] = np.asarray(table, np.float32)
    out = np.empty((p.shape[0], cols), np.float32)
    out[:, 0::2] = t[p[:, : cols // 2] & 0x0F] * s[0::2]
    out[:, 1::2] = t[(p[:, : cols // 2] >> 4) & 0x0F] * s[1::2]
    return out

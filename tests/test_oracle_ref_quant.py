"""Pin the oracle's restatement of the reference quant kernels
(reference python/ccut/quant/kernels.py, weight_only.py, method.py)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ref_quant as rq


def test_fp8_decode_table_matches_torch_e4m3fn():
    """All 256 codes vs torch.float8_e4m3fn (the OCP e4m3fn library decode)."""
    codes = np.arange(256, dtype=np.uint8)
    ours = rq.fp8_e4m3_to_float32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert set(np.nonzero(nan)[0].tolist()) == {0x7F, 0xFF}
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # incl. -0.0 at 0x80
    # closed-form spot values of the format
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6 and ours[0x38] == 1.0


def test_reference_fp8_round_trip_test_rehosted():
    """reference python/tests/test_quant.py:30-41 on the oracle."""
    torch.manual_seed(0)
    x = (torch.randn(64, 32) * 3).numpy()
    scale = np.abs(x).max(axis=0) / 448.0
    q = np.clip(x / scale[None, :], -448, 448)
    codes = rq.float32_to_fp8_e4m3(q.ravel())
    dec = rq.fp8_e4m3_to_float32(codes).reshape(x.shape) * scale[None, :]
    tr = torch.from_numpy(q).to(torch.float8_e4m3fn).float().numpy() * scale[None, :]
    mask = np.abs(tr) > 1e-3
    rel = np.abs(dec[mask] - tr[mask]) / np.abs(tr[mask])
    assert float(rel.max()) < 0.05


def _halfup_bruteforce(v: float) -> int:
    """Nearest finite e4m3fn magnitude, ties toward the larger magnitude,
    saturating (>= 464 -> 448): the rounding rule of kernels.py:85."""
    if math.isnan(v):
        return 0x7F
    sign = 0x80 if v < 0 else 0
    a = abs(v)
    if a == 0:
        return sign
    if a >= 464.0:
        return sign | 0x7E
    table = rq.FP8_TABLE[:0x7F].astype(np.float64)
    best, bd = 0, None
    for c in range(0x7F):
        d = abs(table[c] - a)
        if bd is None or d < bd or (d == bd and table[c] > table[best]):
            best, bd = c, d
    return sign | best


def test_float32_to_fp8_halfup_matches_bruteforce():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * 50,
        rng.standard_normal(1000).astype(np.float32) * 0.01,
        (rng.standard_normal(500) * 1e-3).astype(np.float32),
        # exact midpoints between neighbouring codes (the half-up ties)
        ((rq.FP8_TABLE[1:0x7E].astype(np.float64) + rq.FP8_TABLE[2:0x7F]) / 2).astype(np.float32),
        np.array([0.0, -0.0, 448.0, 455.9, 463.99, 464.0, 1e9, -1e9, np.inf, -np.inf, np.nan,
                  2.0 ** -10, 2.0 ** -11, -(2.0 ** -10), 1.5e-45], dtype=np.float32),
    ])
    got = rq.float32_to_fp8_e4m3(vals)
    want = np.array([_halfup_bruteforce(float(v)) for v in vals], dtype=np.uint8)
    # -0.0: v < 0 is False in the reference, so the code is 0x00
    assert np.array_equal(got, want)


def test_fp8_dequant_mat_closed_form():
    rng = np.random.default_rng(2)
    w = rng.integers(0, 256, size=(7, 33), dtype=np.uint8)
    s = rng.random(7).astype(np.float32) + 0.1
    out = rq.fp8_dequant_mat(w, s)
    for i in range(7):
        for j in range(33):
            v = float(rq.FP8_TABLE[w[i, j]]) * float(s[i])
            if math.isnan(v):
                assert math.isnan(out[i, j])
            else:
                assert out[i, j] == np.float32(v)


def test_reference_w4a16_test_rehosted():
    """reference python/tests/test_quant.py:115-150: same seed, same explicit
    per-byte loop, on the oracle's weight_only_apply."""
    torch.manual_seed(13)
    w4 = torch.randint(0, 255, (10, 16), dtype=torch.uint8).numpy()
    s4 = (torch.rand(32) + 0.1).numpy()
    x = torch.randn(4, 32).numpy()
    y = rq.weight_only_apply(w4.tobytes(), s4, x)
    lo = np.empty(w4.shape, dtype=np.int8)
    hi = np.empty(w4.shape, dtype=np.int8)
    for i in range(w4.shape[0]):
        for j in range(w4.shape[1]):
            b = int(w4[i, j])
            l, h = b & 0x0F, (b >> 4) & 0x0F
            lo[i, j] = l - 16 if l >= 8 else l
            hi[i, j] = h - 16 if h >= 8 else h
    W = np.empty((10, 32), dtype=np.float32)
    W[:, 0::2] = lo.astype(np.float32) * s4[0::2]
    W[:, 1::2] = hi.astype(np.float32) * s4[1::2]
    assert np.allclose(y, x @ W.T, atol=1e-5)
    # and the dequantized matrix itself is bit-exact
    assert np.array_equal(rq.int4_dequant_row(w4, s4), W)


def test_int4_dequant_sign_extension():
    packed = np.array([[0x0F, 0x80, 0x78]], dtype=np.uint8)
    s = np.ones(6, dtype=np.float32)
    assert rq.int4_dequant_row(packed, s).tolist() == [[-1.0, 0.0, 0.0, -8.0, -8.0, 7.0]]


def test_silu_mul_closed_form():
    rng = np.random.default_rng(3)
    g = rng.standard_normal(1000).astype(np.float32) * 4
    u = rng.standard_normal(1000).astype(np.float32)
    ref = (torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).float().numpy()
    got = rq.silu_mul_fused(g, u)
    assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_fp8_linear_apply_matches_float64():
    rng = np.random.default_rng(4)
    w = rng.integers(0, 0x7E, size=(12, 40), dtype=np.uint8)  # finite codes
    s = rng.random(12).astype(np.float32)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    y = rq.fp8_linear_apply(w.tobytes(), s, x)
    ref = x.astype(np.float64) @ (rq.FP8_TABLE[w].astype(np.float64) * s[:, None].astype(np.float64)).T
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-4)


def test_bf16_bits():
    x = np.array([1.0, -2.5, 3.140625], dtype=np.float32)
    u16 = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(rq.bf16_bits_to_float32(u16), x)


def test_nf4_dequant_table_and_layout():
    """Each code's value is the table entry times its column scale (low
    nibble = even column); codes past the 8-entry table are NaN."""
    from oracle.ref_quant import NF4_TABLE, nf4_dequant_row

    packed = np.array([[0x10, 0x32, 0x54, 0x76, 0x98]], np.uint8)
    scale = np.array([1, 2, 4, 8, 0.5, 0.25, 1, 1, 1, 1], np.float32)
    out = nf4_dequant_row(packed, scale)
    codes = [0, 1, 2, 3, 4, 5, 6, 7, 8, 9]
    for c, code in enumerate(codes[:8]):
        assert out[0, c] == np.float32(NF4_TABLE[code] * scale[c])
    assert np.isnan(out[0, 8]) and np.isnan(out[0, 9])
    # a 16-entry table makes every code valid
    t16 = np.linspace(-1, 1, 16).astype(np.float32)
    out16 = nf4_dequant_row(packed, scale, t16)
    assert out16[0, 9] == np.float32(t16[9] * scale[9])


def test_group_broadcast_scale_loop():
    """out[i*G + j] == s[i] element by element (a tile instead of a repeat,
    or a wrong group size, fails), for G = 1, 3 and 128."""
    from oracle.ref_quant import group_broadcast_scale

    rng = np.random.default_rng(4)
    for groups, G in ((5, 1), (7, 3), (16, 128)):
        s = rng.standard_normal(groups).astype(np.float32)
        out = group_broadcast_scale(s, G)
        assert out.dtype == np.float32 and out.shape == (groups * G,)
        for i in range(groups):
            for j in range(G):
                assert out[i * G + j] == s[i]

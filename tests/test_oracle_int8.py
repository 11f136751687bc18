"""The INT8 oracle (oracle/int8.py) pinned by the reference's own test
(python/tests/test_quant.py:44-59, rebuilt here from its seeded torch
inputs), closed forms and brute force."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int8 as oi8


def test_matches_reference_test_int8_w8a8():
    """python/tests/test_quant.py:44-59: W8A8 against the torch restatement
    of the same quantization (sc = amax/127, factor 127/sc, round, clamp),
    weights given [K, N]."""
    torch.manual_seed(1)
    xa = torch.randn(4, 16)
    wb = torch.randint(-127, 127, (16, 8)).float()
    scale_t = torch.rand(8) + 0.1
    sc = xa.abs().max(dim=1).values / 127
    xq = torch.clamp(torch.round(xa * (127 / sc)[:, None]), -127, 127).to(torch.int8)
    acc = xq.long() @ wb.to(torch.int8).long()
    y_ref = acc.float() * sc[:, None] * scale_t[None, :]
    y = oi8.w8a8(wb.to(torch.int8).numpy().T.copy(), scale_t.numpy(), xa.numpy())
    assert np.allclose(y, y_ref.numpy(), atol=1e-3)
    # and the quantized activations and scales agree exactly with that restatement
    xq2, xs2 = oi8.quantize_per_token(xa.numpy())
    assert np.array_equal(xq2, xq.numpy())
    assert np.array_equal(xs2, sc.numpy())


def test_quantize_per_token_closed_forms():
    # amax = 16129/128 -> x_scale = 127/128 and factor = 128 exactly: x * 128 is
    # exact and round() is half to even
    amax = np.float32(16129 / 128)
    row = np.array([amax, 2.5 / 128, 3.5 / 128, -2.5 / 128, 0.4 / 128, -126.6 / 128, 200 / 128, 0.0],
                   dtype=np.float32)
    xq, xs = oi8.quantize_per_token(row[None, :])
    assert xs[0] == np.float32(127 / 128)
    assert xq[0].tolist() == [127, 2, 4, -2, 0, -127, 127, 0]
    # the factor is 127 / (amax / 127) = 16129 / amax: every |x| above about
    # amax / 127 saturates (the reference's formula, kept as is)
    xq, xs = oi8.quantize_per_token(np.array([[1.0, 0.5, 0.1, 1.0 / 127, 0.5 / 127]], np.float32))
    assert xq[0].tolist() == [127, 127, 127, 127, 64]
    # zero row: amax 1, x_scale = float32(1 / 127), codes 0
    xq, xs = oi8.quantize_per_token(np.zeros((2, 5), np.float32))
    assert np.all(xq == 0) and np.all(xs == np.float32(1.0) / np.float32(127.0))
    # NaN row: amax NaN fails "> 0" -> 1; NaN codes cast to 0
    xq, xs = oi8.quantize_per_token(np.array([[np.nan, 1.0 / 16129, -3.0 / 16129]], np.float32))
    assert xs[0] == np.float32(1.0) / np.float32(127.0)
    assert xq[0].tolist() == [0, 1, -3]
    # inf row: x_scale inf, factor 0, every code 0 (inf * 0 is NaN -> 0)
    xq, xs = oi8.quantize_per_token(np.array([[np.inf, 5.0, -1.0]], np.float32))
    assert np.isinf(xs[0]) and xq[0].tolist() == [0, 0, 0]
    with pytest.raises(ValueError):
        oi8.quantize_per_token(np.zeros((3, 0), np.float32))  # numpy's max over an empty axis


def test_int8_matmul_brute_force_and_range():
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, (3, 7)).astype(np.int8)
    b = rng.integers(-127, 128, (7, 5)).astype(np.int8)
    got = oi8.int8_matmul(a, b)
    for i in range(3):
        for j in range(5):
            assert got[i, j] == sum(int(a[i, t]) * int(b[t, j]) for t in range(7))
    # the largest sum the GPU path accepts (K < 131072) stays inside int32
    assert 127 * 127 * ((1 << 17) - 1) < 2**31 - 1


def test_w8a8_epilogue_order_and_dequant():
    """y = (float32(acc) * x_scale) * w_scale, left to right in float32; a
    case where the other association rounds differently pins the order."""
    # one element 0.3: x_scale = float32(0.3) / 127, code 127 (saturated), acc = 127
    x = np.array([[0.3]], np.float32)
    w = np.array([[1]], np.int8)
    ws = np.float32(0.13)
    xq, x_scale = oi8.quantize_per_token(x)
    assert xq[0, 0] == 127 and x_scale[0] == np.float32(0.3) / np.float32(127)
    acc = np.float32(127)
    assert (acc * x_scale[0]) * ws != acc * (x_scale[0] * ws)
    y = oi8.w8a8(w, np.array([ws], np.float32), x)
    assert y[0, 0] == (acc * x_scale[0]) * ws
    # dequant: one float32 rounding of the exact product
    w = np.array([[-127, 3, 0], [5, -1, 127]], np.int8)
    s = np.array([0.1, 2.0 ** -3], np.float32)
    d = oi8.dequant_row(w, s)
    assert d[1].tolist() == [5 / 8, -1 / 8, 127 / 8]
    assert d[0, 0] == np.float32(-127 * np.float64(np.float32(0.1)))


def test_quantize_cols_closed_forms():
    # amax 127: inv = 1, so q = round-half-even(x) exactly
    x = np.array([[0.5, 1.5, 2.5, -0.5, -2.5, 200.0, -1e9, 3.49]], np.float32)
    q = oi8.quantize_cols(x, np.full(8, 127.0, np.float32))
    assert q[0].tolist() == [0, 2, 2, 0, -2, 127, -127, 3]
    # amax not > 0 -> inv 0 -> codes 0; amax 254 -> inv 0.5
    q = oi8.quantize_cols(np.array([[5.0, 3.0, 5.0]], np.float32), np.array([0.0, -1.0, 254.0], np.float32))
    assert q[0].tolist() == [0, 0, 2]  # 5 * 0.5 = 2.5 -> 2 (half to even)
    # brute force against a per-element float64 loop
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((4, 9)) * 3).astype(np.float32)
    a = np.abs(x).max(axis=0).astype(np.float32)
    q = oi8.quantize_cols(x, a)
    for r in range(4):
        for c in range(9):
            v = round(float(x[r, c]) * (127.0 / float(a[c])))  # Python round: half to even
            assert q[r, c] == max(-127, min(127, v))

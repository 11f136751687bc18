"""The MX oracle (oracle/mx.py) pinned by closed forms: E8M0 against
ldexp and its two special bytes, the 4-bit table against the reference's
stated code meaning (python/ccut/quant/mx.py:77-82), group broadcast against
a per-element loop (partial last group included)."""

from __future__ import annotations

import numpy as np

from oracle import mx as omx
from oracle.ref_quant import fp8_e4m3_to_float32


def test_e8m0_closed_forms():
    e = np.arange(256, dtype=np.uint8)
    v = omx.e8m0_to_float(e)
    assert v[0] == 0.0 and np.isnan(v[255])
    assert v[127] == 1.0 and v[128] == 2.0 and v[126] == 0.5
    assert np.array_equal(v[1:255], np.ldexp(np.float32(1), np.arange(1, 255) - 127).astype(np.float32))
    assert v[1] == np.finfo(np.float32).tiny  # 2^-126, the smallest normal


def test_fp4_table_and_nibble_order():
    # codes 0..3 -> 0, .5, 1, 1.5; bit 2 negates; bit 3 is ignored
    expect = [0.0, 0.5, 1.0, 1.5, -0.0, -0.5, -1.0, -1.5]
    packed = np.array([[(hi << 4) | lo for lo, hi in zip(range(0, 16, 2), range(1, 16, 2))]], np.uint8)
    w = omx.dequant_mxfp4(packed, None, 32)
    assert w.shape == (1, 16)
    assert w[0].tolist() == expect + expect
    assert np.signbit(w[0, 4]) and not np.signbit(w[0, 0])


def test_group_scales_per_element_loop():
    rng = np.random.default_rng(2)
    rows, cols, G = 3, 70, 32  # 3 groups per row, the last one 6 wide
    codes = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    codes[codes & 0x7F == 0x7F] = 0x10  # no NaN codes
    sc = rng.integers(100, 140, rows * 3).astype(np.uint8)
    w = omx.dequant_mxfp8(codes, sc, G)
    vals = fp8_e4m3_to_float32(codes.reshape(-1)).reshape(rows, cols)
    for r in range(rows):
        for c in range(cols):
            assert w[r, c] == np.float32(vals[r, c] * np.float32(2.0 ** (int(sc[r * 3 + c // G]) - 127)))
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    w4 = omx.dequant_mxfp4(packed, sc, G, scale2=0.75)
    for r in range(rows):
        for c in range(cols):
            code = (packed[r, c // 2] >> (4 * (c % 2))) & 15
            base = [0.0, 0.5, 1.0, 1.5][code & 3] * (-1.0 if code & 4 else 1.0)
            expect = np.float32(np.float32(base * 2.0 ** (int(sc[r * 3 + c // G]) - 127)) * np.float32(0.75))
            assert w4[r, c] == expect


def test_special_scales_propagate():
    codes = np.full((1, 64), 0x38, np.uint8)  # 1.0
    w = omx.dequant_mxfp8(codes, np.array([0, 255], np.uint8), 32)
    assert np.all(w[0, :32] == 0.0) and np.all(np.isnan(w[0, 32:]))

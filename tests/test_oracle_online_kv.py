"""The oracle's load-time and KV FP8 quantizers pinned by closed forms:
rows built from e4m3 values times an exact power-of-two scale come back
code for code, zero / NaN / invalid-scale rows, and round-trip bounds."""

from __future__ import annotations

import numpy as np

from oracle import online_kv as ok
from oracle.ref_quant import fp8_e4m3_to_float32

FINITE = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)


def _bf16_bytes(x: np.ndarray) -> bytes:
    u = np.asarray(x, np.float32).view(np.uint32)
    assert np.all(u & 0xFFFF == 0), "values must be exact in bf16"
    return (u >> 16).astype(np.uint16).tobytes()


def test_exact_rows_round_trip_code_for_code():
    rng = np.random.default_rng(0)
    codes = rng.choice(FINITE, size=(6, 64))
    codes[:, 0] = 0x7E  # 448: the row's amax, so amax / 448 = the chosen scale
    scale = 2.0 ** rng.integers(-6, 3, size=6)
    w = fp8_e4m3_to_float32(codes) * scale[:, None].astype(np.float32)
    got = ok.quantize_buffer(_bf16_bytes(w), None, 64)
    dec = lambda c: fp8_e4m3_to_float32(c).view(np.uint32)  # noqa: E731  (+0 and -0 codes differ only in sign)
    assert np.array_equal(got, codes) or np.array_equal(dec(got) & 0x7fffffff, dec(codes) & 0x7fffffff)
    kc, ks = ok.kv_quant(w[None])
    assert np.array_equal(fp8_e4m3_to_float32(ks[0]), scale.astype(np.float32))
    assert np.array_equal(np.abs(fp8_e4m3_to_float32(kc[0])), np.abs(fp8_e4m3_to_float32(codes)))


def test_special_rows():
    w = np.array([[0.0] * 4, [1.0, -2.0, np.nan, 4.0], [1.0, 2.0, 3.0, 500.0]], dtype=np.float32)
    got = ok.quantize_buffer(_bf16_bytes(np.nan_to_num(w, nan=0.0)), np.array([0.0, -1.0, np.nan]), 4)
    # scales 0, -1, NaN are all replaced by 1: plain clip + encode
    assert got[0].tolist() == [0, 0, 0, 0] and got[2, 3] == 0x7E
    nan_row = np.frombuffer(_bf16_bytes(np.array([1.0, -2.0, 0.0, 4.0], np.float32)), dtype=np.uint16).copy()
    nan_row[2] = 0x7FC0  # a bf16 NaN: amax is NaN, the scale falls back to 1, the NaN codes 0x7F
    row = ok.quantize_buffer(nan_row.tobytes(), None, 4)[0]
    assert row[2] == 0x7F and fp8_e4m3_to_float32(row[[0, 1, 3]]).tolist() == [1.0, -2.0, 4.0]
    kc, ks = ok.kv_quant(np.zeros((2, 1, 3, 8), np.float32))
    assert not kc.any() and not ks.any()
    assert (ok.kv_dequant(kc, ks) == 0).all()
    kc, ks = ok.kv_quant(np.array([[[[1.0, np.nan]]]], np.float32))
    assert kc.reshape(-1).tolist() == [0x7F, 0x7F] and ks.reshape(-1).tolist() == [0x7F]


def test_round_trip_bounds():
    rng = np.random.default_rng(1)
    kv = (rng.standard_normal((2, 3, 5, 128)) * 3).astype(np.float32)
    codes, scales = ok.kv_quant(kv)
    back = ok.kv_dequant(codes, scales)
    amax = np.abs(kv).max(axis=-1, keepdims=True)
    # e4m3: 3 mantissa bits for the value and for the scale byte
    assert np.all(np.abs(back - kv) <= amax * (2.0 ** -3))
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    w = ((w.view(np.uint32) >> 16) << 16).view(np.float32)
    codes = ok.quantize_buffer(_bf16_bytes(w), None, 256)
    s = (np.abs(w).max(axis=1) / 448.0).astype(np.float32)[:, None]
    assert np.all(np.abs(fp8_e4m3_to_float32(codes) * s - w) <= np.abs(w) * 2.0 ** -4 + s * 2.0 ** -9)

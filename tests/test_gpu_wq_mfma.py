"""GPU parity of the decoded-weight MFMA linear (``ccq_wq_mfma_linear_f32``),
the batched form of the reference's dequantize-then-matmul layers for FP8 /
INT8 per-row weights (python/ccut/quant/fp8.py:35-42,
quant/method.py:100-140) and the MX formats (quant/mx.py:37-94).

Against the oracle: outputs within 1e-5 of max|y| of a float64 product of
the oracle's dequantized weights (x is split into bf16 hi + lo, so each
term carries at most 2^-18 relative error before float32 summation);
one-hot activations give every weight exactly, bit for bit, for all
finite codes and their scales."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int8 as oint8
from oracle import mx as omx
from oracle import ref_quant as orq

pytestmark = pytest.mark.gpu

FP8_ROW, INT8_ROW, MXFP8, MXFP4 = 0, 1, 2, 3


def _same(a, b):
    """Equal values, NaN where NaN (a -0 weight sums to +0 with the zero
    terms, as in any float product x @ W.T)."""
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb])


def _case(fmt, K, N, G, rng, finite=True):
    """(raw weight bytes, scale array or None, scale2, dequantized W)."""
    s2 = 1.0
    if fmt in (FP8_ROW, MXFP8):
        codes = rng.integers(0, 256, (N, K)).astype(np.uint8)
        if finite:
            codes[(codes & 0x7F) == 0x7F] = 0x38
        if fmt == FP8_ROW:
            sc = (np.abs(rng.standard_normal(N)) * 0.05 + 1e-3).astype(np.float32)
            return codes, sc, s2, orq.fp8_dequant_mat(codes, sc)
        sc = rng.integers(112, 140, N * (K // G)).astype(np.uint8)
        return codes, sc, s2, omx.dequant_mxfp8(codes, sc, G)
    if fmt == INT8_ROW:
        w = rng.integers(-128, 128, (N, K)).astype(np.int8)
        sc = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float32)
        return w.view(np.uint8), sc, s2, oint8.dequant_row(w, sc)
    packed = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    if G == 0:  # MXFP4 without scales
        return packed, None, s2, omx.dequant_mxfp4(packed, None, 32, None)
    sc = rng.integers(112, 140, N * (K // G)).astype(np.uint8)
    s2 = 0.375 if G == 16 else 1.0
    return packed, sc, s2, omx.dequant_mxfp4(packed, sc, G, np.float32(s2) if G == 16 else None)


def _run(gpu, fmt, x, raw, sc, s2, N, G):
    from ccut import _dev
    from ccut._lib import call

    M, K = x.shape
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    rd = torch.from_numpy(np.ascontiguousarray(raw)).to(gpu)
    sd = None if sc is None else torch.from_numpy(np.ascontiguousarray(sc)).to(gpu)
    y = torch.full((M, N), float("nan"), device=gpu)
    call("ccq_wq_mfma_linear_f32", xd.data_ptr(), rd.data_ptr(), None if sd is None else sd.data_ptr(), y.data_ptr(),
         M, K, N, fmt, G, float(s2), _dev.stream_ptr())
    torch.cuda.synchronize()
    return y.cpu().numpy()


FORMATS = [(FP8_ROW, 0), (INT8_ROW, 0), (MXFP8, 32), (MXFP8, 16), (MXFP4, 32), (MXFP4, 16), (MXFP4, 0)]


@pytest.mark.parametrize("fmt,G", FORMATS)
@pytest.mark.parametrize("M,K,N", [(1, 256, 64), (8, 512, 70), (16, 1024, 192), (17, 256, 130), (33, 768, 96),
                                   (70, 512, 200), (130, 256, 64)])
def test_wq_matches_oracle(gpu, fmt, G, M, K, N):
    rng = np.random.default_rng(1000 * fmt + 10 * G + M + K + N)
    raw, sc, s2, w = _case(fmt, K, N, G, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = _run(gpu, fmt, x, raw, sc, s2, N, G)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.all(np.isfinite(y))
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)), (fmt, G, M, K, N)


@pytest.mark.parametrize("fmt,G", FORMATS)
def test_wq_one_hot_is_exact(gpu, fmt, G):
    """x = identity: y[b, r] = W[r, b] bit for bit, so every code's decode
    and its scale (row or group) are checked through the MFMA path."""
    K, N = 256, 72
    rng = np.random.default_rng(7 + fmt * 10 + G)
    raw, sc, s2, w = _case(fmt, K, N, G, rng)
    if fmt in (FP8_ROW, MXFP8):  # all finite e4m3 codes across the rows
        codes = (np.arange(N * K, dtype=np.int64).reshape(N, K) * 5) % 256
        raw = np.where((codes & 0x7F) == 0x7F, 0x11, codes).astype(np.uint8)
        w = orq.fp8_dequant_mat(raw, sc) if fmt == FP8_ROW else omx.dequant_mxfp8(raw, sc, G)
    x = np.eye(K, dtype=np.float32)
    y = _run(gpu, fmt, x, raw, sc, s2, N, G)
    assert _same(y, np.ascontiguousarray(w.T))


def test_wq_row_of_nan_code(gpu):
    """A NaN code (0x7F) makes its output column NaN for every batch row, as
    the float32 product of the dequantized weights does; other columns stay
    finite and within tolerance."""
    rng = np.random.default_rng(3)
    K, N, M = 256, 64, 12
    raw, sc, s2, w = _case(FP8_ROW, K, N, 0, rng)
    raw[5, 17] = 0x7F
    w = orq.fp8_dequant_mat(raw, sc)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = _run(gpu, FP8_ROW, x, raw, sc, s2, N, 0)
    assert np.all(np.isnan(y[:, 5]))
    keep = np.arange(N) != 5
    ref = x.astype(np.float64) @ w[keep].astype(np.float64).T
    assert np.max(np.abs(y[:, keep] - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("batch", [8, 24, 64])
def test_dispatch_through_layer_entries(gpu, batch):
    """ccq_fp8_linear_f32, ccq_int8_linear_f32 and ccq_mx_linear_f32 run the
    MFMA kernel at 8 rows and more (in_features % 256 == 0) and agree with
    it bit for bit."""
    from ccut import _dev
    from ccut._lib import call

    K, N = 512, 96
    rng = np.random.default_rng(batch)
    x = rng.standard_normal((batch, K)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    for fmt, G, entry in [(FP8_ROW, 0, "ccq_fp8_linear_f32"), (INT8_ROW, 0, "ccq_int8_linear_f32"),
                          (MXFP8, 32, "ccq_mx_linear_f32"), (MXFP4, 16, "ccq_mx_linear_f32")]:
        raw, sc, s2, w = _case(fmt, K, N, G, rng)
        rd = torch.from_numpy(np.ascontiguousarray(raw)).to(gpu)
        sd = torch.from_numpy(np.ascontiguousarray(sc)).to(gpu)
        y = torch.empty((batch, N), device=gpu)
        if entry == "ccq_mx_linear_f32":
            call(entry, xd.data_ptr(), rd.data_ptr(), sd.data_ptr(), y.data_ptr(), batch, K, N, fmt - 2, G, float(s2),
                 _dev.stream_ptr())
        else:
            call(entry, xd.data_ptr(), rd.data_ptr(), sd.data_ptr(), y.data_ptr(), batch, K, N, _dev.stream_ptr())
        torch.cuda.synchronize()
        direct = _run(gpu, fmt, x, raw, sc, s2, N, G)
        assert np.array_equal(y.cpu().numpy(), direct), entry
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.max(np.abs(direct - ref)) <= 1e-5 * np.max(np.abs(ref))

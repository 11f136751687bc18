"""GPU parity of the load-time and KV-cache FP8 quantizers (reference
python/ccut/quant/online.py:37-64, kv.py:70-101) with the oracle: codes,
scale bytes and read-back bit-exact, special rows included."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import online_kv as ok

pytestmark = pytest.mark.gpu


def _bf16_rows(rng, rows, cols):
    w = (rng.standard_normal((rows, cols)) * 0.03).astype(np.float32)
    u = (w.view(np.uint32) >> 16).astype(np.uint16)
    u[1] = 0  # a zero row
    u[2, 5] = 0x7FC0  # NaN
    u[3, 7] = 0x7F80  # +inf
    u[4, :] = (np.float32(-3.0).view(np.uint32) >> 16)  # constant row (ties at the clip)
    return u


@pytest.mark.parametrize("cols", [64, 300, 2048, 4096, 8192])
def test_quantize_buffer_bitexact(gpu, cols):
    from ccut.quant.online import quantize_buffer_inplace

    rng = np.random.default_rng(cols)
    u = _bf16_rows(rng, 9, cols)
    for scale in (None, np.array([1e-3, 0.0, -1.0, np.nan, 2e-4, 5e-5, 1.0, 3e-3, 1e-5], np.float32)):
        out = np.empty((9, cols), np.uint8)
        quantize_buffer_inplace(u.tobytes(), scale, out)
        assert np.array_equal(out, ok.quantize_buffer(u.tobytes(), scale, cols))
    dev_out = torch.empty((9, cols), dtype=torch.uint8, device=gpu)
    quantize_buffer_inplace(torch.from_numpy(u.view(np.int16)).to(gpu), None, dev_out)
    assert np.array_equal(dev_out.cpu().numpy(), ok.quantize_buffer(u.tobytes(), None, cols))


@pytest.mark.parametrize("dim", [8, 64, 128, 256, 320])
def test_kv_quant_dequant_bitexact(gpu, dim):
    from ccut.quant.kv import dequantize_kv_token, quantize_kv_token

    rng = np.random.default_rng(dim)
    kv = (rng.standard_normal((2, 4, 7, dim)) * 2).astype(np.float32)
    kv[0, 1, 2] = 0.0
    kv[1, 3, 0, 3] = np.nan
    kv[1, 0, 5, 1] = -np.inf
    codes = np.empty(kv.shape, np.uint8)
    scales = np.empty(kv.shape[:-1], np.uint8)
    quantize_kv_token(kv, codes, scales)
    c0, s0 = ok.kv_quant(kv)
    assert np.array_equal(codes, c0) and np.array_equal(scales, s0)
    back = np.empty(kv.shape, np.float32)
    dequantize_kv_token(codes, scales, back)
    assert np.array_equal(back.view(np.uint32), ok.kv_dequant(c0, s0).view(np.uint32))
    # device tensors in and out
    kd = torch.from_numpy(kv).to(gpu)
    cd = torch.empty(kv.shape, dtype=torch.uint8, device=gpu)
    sd = torch.empty(kv.shape[:-1], dtype=torch.uint8, device=gpu)
    quantize_kv_token(kd, cd, sd)
    assert np.array_equal(cd.cpu().numpy(), c0) and np.array_equal(sd.cpu().numpy(), s0)

"""GPU parity of NF4 weight-only (reference python/ccut/quant/kernels.py:
299-322, weight_only.py:37-54) and the per-column int8 quantizer
(kernels.py:192-211) with the oracle: dequantized weights and codes
bit-exact, the NF4 layer within 1e-5 of max|y| of a float64 product."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import int8 as oi8
from oracle import ref_quant as orq

pytestmark = pytest.mark.gpu


def _same(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                                           b[~nb].view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(3, 16), (17, 300), (64, 4096)])
def test_nf4_dequant_bitexact(gpu, rows, cols):
    from ccut.quant import kernels

    rng = np.random.default_rng(rows + cols)
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    scale = (rng.random(cols) * 0.1 + 1e-3).astype(np.float32)
    out = np.empty((rows, cols), np.float32)
    kernels.nf4_dequant_row(packed, scale, orq.NF4_TABLE, out)
    assert _same(out, orq.nf4_dequant_row(packed, scale))
    t16 = np.linspace(-1, 1, 16).astype(np.float32)
    kernels.nf4_dequant_row(packed, scale, t16, out)
    assert _same(out, orq.nf4_dequant_row(packed, scale, t16))


def test_nf4_weight_only_layer(gpu):
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.spec import GroupShape, LayerQuantSpec, QuantDType, QuantKey, ScaleDesc, ScaleStrategy

    rng = np.random.default_rng(7)
    K, N, B = 512, 96, 5
    key = QuantKey(QuantDType.NF4, ScaleStrategy.PER_CHANNEL, QuantDType.FP32, ScaleStrategy.NO_SCALE, True,
                   GroupShape())
    spec = LayerQuantSpec(layer_name="mlp.down_proj", weight_key=key,
                          scales=(ScaleDesc(name="weight_scale", dtype="F32", shape=(K,)),))
    m = make_method_for_spec(spec)
    packed = (rng.integers(0, 8, (N, K)) | (rng.integers(0, 8, (N, K)) << 4)).astype(np.uint8)[:, : K // 2]
    scale = (rng.random(K) * 0.1 + 1e-3).astype(np.float32)
    x = rng.standard_normal((B, K)).astype(np.float32)
    y = m.apply(packed.tobytes(), {"weight_scale": scale}, x)
    w = orq.nf4_dequant_row(packed, scale)
    ref = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("rows,cols", [(1, 7), (33, 300), (128, 2048)])
def test_int8_quantize_row_bitexact(gpu, rows, cols):
    from ccut.quant import kernels

    rng = np.random.default_rng(rows * cols)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    amax = np.abs(x).max(axis=0).astype(np.float32)
    amax[0] = 0.0
    if cols > 2:
        amax[1] = -1.0
        amax[2] = amax[2] * 0.5  # saturates
    x[0, -1] = np.nan
    out = np.empty((rows, cols), np.int8)
    kernels.int8_quantize_row(x, amax, out)
    assert np.array_equal(out, oi8.quantize_cols(x, amax))

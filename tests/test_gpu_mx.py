"""GPU parity of the MX formats (reference python/ccut/quant/mx.py:21-94,
kernels.py:240-256) with the oracle: E8M0 decode and dequantized weights
bit-exact, the float32 layer within 1e-5 of max|y| of a float64 product."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mx as omx

pytestmark = pytest.mark.gpu


def _same(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                                           b[~nb].view(np.uint32))


def test_e8m0_all_bytes(gpu):
    from ccut.quant import kernels

    e = np.arange(256, dtype=np.uint8)
    assert _same(kernels.mx_e8m0_to_float(e), omx.e8m0_to_float(e))


@pytest.mark.parametrize("rows,cols,G", [(5, 64, 32), (7, 70, 32), (33, 4096, 32), (4, 48, 16), (6, 64, 16), (3, 96, 16)])
def test_mx_dequant_bitexact(gpu, rows, cols, G):
    from ccut.quant.mx import mx_dequant

    rng = np.random.default_rng(rows * cols + G)
    gpr = (cols + G - 1) // G
    sc = rng.integers(110, 140, rows * gpr).astype(np.uint8)
    sc[0] = 0
    sc[-1] = 255
    codes = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    w = mx_dequant(codes.tobytes(), sc, cols, "mxfp8", G)
    assert _same(w, omx.dequant_mxfp8(codes, sc, G))
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    for s2 in (None, np.float32(0.3)):
        for scale in (sc, None):
            w4 = mx_dequant(packed.tobytes(), scale, cols, "nvfp4" if s2 is not None else "mxfp4", G, s2)
            assert _same(w4, omx.dequant_mxfp4(packed, scale, G, s2))


def _spec(dtype_key, n_scales=1):
    from ccut.quant.spec import LayerQuantSpec, ScaleDesc, get_quant_key

    scales = (ScaleDesc(name="weight_scale", dtype="U8", shape=(1,)),)
    if n_scales == 2:
        scales += (ScaleDesc(name="weight_global_scale", dtype="F32", shape=(1,)),)
    return LayerQuantSpec(layer_name="mlp.experts.0.up_proj", weight_key=get_quant_key(dtype_key), scales=scales)


@pytest.mark.parametrize("key,batch,K,N", [("mxfp8_dynamic", 1, 4096, 512), ("mxfp8_dynamic", 9, 320, 70),
                                           ("mxfp4_dynamic", 3, 2048, 256), ("nvfp4_dynamic", 16, 512, 96)])
def test_mx_method_apply(gpu, key, batch, K, N):
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.mx import MxLinearMethod

    rng = np.random.default_rng(K + N + batch)
    nv = key.startswith("nvfp4")
    m = make_method_for_spec(_spec(key, 2 if nv else 1))
    assert isinstance(m, MxLinearMethod)
    G = m.group_size
    assert G == (16 if nv else 32)
    gpr = (K + G - 1) // G
    sc = rng.integers(118, 134, N * gpr).astype(np.uint8)
    x = rng.standard_normal((batch, K)).astype(np.float32)
    if key.startswith("mxfp8"):
        codes = rng.integers(0, 256, (N, K)).astype(np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0x30  # finite weights
        w = omx.dequant_mxfp8(codes, sc, G)
        raw = codes.tobytes()
        scales = {"weight_scale": sc}
    else:
        packed = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
        s2 = np.array([0.5, 0.25], np.float32) if nv else None
        w = omx.dequant_mxfp4(packed, sc, G, None if s2 is None else np.float32(s2).mean())
        raw = packed.tobytes()
        scales = {"weight_scale": sc}
        if nv:
            scales["weight_global_scale"] = s2
    y = m.apply(raw, scales, x)
    ref = omx.apply(w, x)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    # device tensors in, device tensor out; scales given as float exponents
    yd = m.apply(torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(gpu),
                 {k: torch.from_numpy(np.asarray(v, np.float32)).to(gpu) for k, v in scales.items()},
                 torch.from_numpy(x).to(gpu))
    assert yd.is_cuda and np.array_equal(yd.cpu().numpy(), y)


def test_mxfp8_requires_scales(gpu):
    from ccut.quant.method import make_method_for_spec

    m = make_method_for_spec(_spec("mxfp8_dynamic"))
    with pytest.raises(ValueError):
        m.apply(np.zeros((4, 64), np.uint8).tobytes(), {}, np.zeros((1, 64), np.float32))


@pytest.mark.parametrize("fmt,G", [(0, 32), (0, 16), (1, 32), (1, 16)])
def test_mx_linear_one_hot_is_exact(gpu, fmt, G):
    """x = one-hot rows: every output is one weight exactly (the other terms
    are zeros), so each code's decode and its group scale are checked bit
    for bit through the fused kernel (all 256 e4m3fn codes but the NaNs, all
    16 FP4 codes)."""
    from ccut import _dev
    from ccut._lib import call

    K, N = 64, 8
    rng = np.random.default_rng(fmt * 10 + G)
    sc = rng.integers(100, 150, N * (K // G)).astype(np.uint8)
    if fmt == 0:
        codes = np.arange(N * K, dtype=np.int64).reshape(N, K) % 256
        codes = np.where((codes & 0x7F) == 0x7F, 0x11, codes).astype(np.uint8)
        w = omx.dequant_mxfp8(codes, sc, G)
        raw = codes
        s2 = 1.0
    else:
        nib = (np.arange(N * K).reshape(N, K) * 7) % 16
        raw = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
        s2 = 0.75
        w = omx.dequant_mxfp4(raw, sc, G, np.float32(s2))
    x = np.eye(K, dtype=np.float32)
    xd = torch.from_numpy(x).to(gpu)
    rd = torch.from_numpy(np.ascontiguousarray(raw)).to(gpu)
    sd = torch.from_numpy(sc).to(gpu)
    y = torch.empty((K, N), device=gpu)
    call("ccq_mx_linear_f32", xd.data_ptr(), rd.data_ptr(), sd.data_ptr(), y.data_ptr(), K, K, N, fmt, G, s2,
         _dev.stream_ptr())
    assert np.array_equal(y.cpu().numpy(), w.T)


def test_mx_linear_scale_edges_documented(gpu):
    """The fused MX linear applies the E8M0 scale to each group's partial
    sum and NVFP4's scale2 to the row sum, where the reference multiplies
    every weight.  A non-power-of-two scale2 stays within float32
    summation tolerance of the per-weight product.  At E8M0 byte 254 the
    reference's per-weight W = lut * 2^127 is still finite (1.5 * 2^127 is
    below the float32 maximum), so zero activations give 0 on both sides."""
    from ccut.quant.mx import mx_linear

    rng = np.random.default_rng(21)
    rows, cols, G = 8, 256, 16
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    sc = rng.integers(118, 136, rows * cols // G).astype(np.uint8)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    s2 = np.float32(0.7371)  # not a power of two
    y = mx_linear(torch.from_numpy(packed).to(gpu), torch.from_numpy(sc).to(gpu), torch.from_numpy(x).to(gpu),
                  "nvfp4", G, s2).cpu().numpy()
    w = omx.dequant_mxfp4(packed, sc, G, s2).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    hi = np.full(rows * cols // G, 254, dtype=np.uint8)
    yz = mx_linear(torch.from_numpy(packed).to(gpu), torch.from_numpy(hi).to(gpu),
                   torch.zeros((2, cols), device=gpu), "mxfp4", G).cpu().numpy()
    assert np.all(yz == 0.0)

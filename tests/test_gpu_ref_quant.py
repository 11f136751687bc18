"""GPU parity of the reference-format kernels against the oracle
(bit-exact codecs / dequant; float32 Linear within summation order)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_quant as rq

pytestmark = pytest.mark.gpu


def test_fp8_decode_all_codes(gpu):
    from ccut.quant import kernels

    codes = np.arange(256, dtype=np.uint8)
    got = kernels.fp8_e4m3_to_float32(codes)
    want = rq.fp8_e4m3_to_float32(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _edge_values() -> np.ndarray:
    rng = np.random.default_rng(11)
    t = rq.FP8_TABLE[:0x7F].astype(np.float64)
    mids = ((t[1:-1] + t[2:]) / 2).astype(np.float32)
    return np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 60,
        rng.standard_normal(50000).astype(np.float32) * 0.01,
        (rng.standard_normal(50000) * 1e-4).astype(np.float32),
        mids, -mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
        np.array([0.0, -0.0, 448.0, 463.99997, 464.0, 1e9, -1e9, np.inf, -np.inf, np.nan, 2.0 ** -10,
                  -(2.0 ** -10), 1.5e-45, -1.5e-45, 1e-40], dtype=np.float32),
    ])


def test_f32_to_fp8_halfup_bitexact(gpu):
    from ccut.quant import kernels

    v = _edge_values()
    assert np.array_equal(kernels.float32_to_fp8_e4m3(v), rq.float32_to_fp8_e4m3(v))


def test_fp8_dequant_mat_bitexact(gpu):
    from ccut.quant import kernels

    rng = np.random.default_rng(1)
    w = rng.integers(0, 256, size=(67, 301), dtype=np.uint8)
    s = (rng.standard_normal(67) * 3).astype(np.float32)
    out = np.empty((67, 301), dtype=np.float32)
    kernels.fp8_dequant_mat(w, s, out)
    ref = rq.fp8_dequant_mat(w, s)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_int4_dequant_bitexact(gpu):
    from ccut.quant import kernels

    rng = np.random.default_rng(2)
    p = rng.integers(0, 256, size=(33, 50), dtype=np.uint8)
    s = (rng.standard_normal(100) * 0.7).astype(np.float32)
    out = np.empty((33, 100), dtype=np.float32)
    kernels.int4_dequant_row(p, s, out)
    assert np.array_equal(out.view(np.uint32), rq.int4_dequant_row(p, s).view(np.uint32))


def test_silu_mul_within_one_ulp(gpu):
    from ccut.quant import kernels

    rng = np.random.default_rng(3)
    g = (rng.standard_normal((64, 97)) * 5).astype(np.float32)
    u = rng.standard_normal((64, 97)).astype(np.float32)
    out = np.empty_like(g)
    kernels.silu_mul_fused(g, u, out)
    ref = rq.silu_mul_fused(g, u)
    ulp = np.abs(out.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1


def test_reference_w4a16_test_on_gpu(gpu):
    """reference python/tests/test_quant.py:115-150 against this API."""
    from ccut.quant.spec import LayerQuantSpec, ScaleDesc, get_quant_key
    from ccut.quant.weight_only import WeightOnlyMethod

    torch.manual_seed(13)
    w4 = torch.randint(0, 255, (10, 16), dtype=torch.uint8).numpy()
    s4 = (torch.rand(32) + 0.1).numpy()
    m = WeightOnlyMethod(LayerQuantSpec("t.int4", get_quant_key("int4_w4a16_sym"),
                                        scales=(ScaleDesc(name="t.int4.weight_scale", dtype="F32", shape=()),)))
    x = torch.randn(4, 32).numpy()
    y = m.apply(w4.tobytes(), {"t.int4.weight_scale": s4}, x)
    assert isinstance(y, np.ndarray) and y.dtype == np.float32
    assert np.allclose(y, rq.weight_only_apply(w4.tobytes(), s4, x), atol=1e-5)


def test_reference_fp8_round_trip_on_gpu(gpu):
    """reference python/tests/test_quant.py:30-41 against this API."""
    from ccut.quant import kernels

    torch.manual_seed(0)
    x = (torch.randn(64, 32) * 3).numpy()
    scale = np.abs(x).max(axis=0) / 448.0
    q = np.clip(x / scale[None, :], -448, 448)
    codes = kernels.float32_to_fp8_e4m3(q.ravel().astype(np.float32))
    dec = kernels.fp8_e4m3_to_float32(codes).reshape(x.shape) * scale[None, :]
    tr = torch.from_numpy(q).to(torch.float8_e4m3fn).float().numpy() * scale[None, :]
    mask = np.abs(tr) > 1e-3
    assert float((np.abs(dec[mask] - tr[mask]) / np.abs(tr[mask])).max()) < 0.05


@pytest.mark.parametrize("batch", [1, 3, 8, 9, 20])
def test_int4_linear_f32_parity(gpu, batch):
    from ccut.quant.weight_only import int4_linear_f32

    rng = np.random.default_rng(batch)
    out_f, in_f = 37, 96
    p = rng.integers(0, 256, size=(out_f, in_f // 2), dtype=np.uint8)
    s = (rng.random(in_f) + 0.1).astype(np.float32)
    x = rng.standard_normal((batch, in_f)).astype(np.float32)
    y = int4_linear_f32(p.tobytes(), s, x)
    ref = rq.weight_only_apply(p.tobytes(), s, x)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("batch", [1, 5, 16])
def test_fp8_linear_method_parity(gpu, batch):
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.spec import LayerQuantSpec, ScaleDesc, get_quant_key

    rng = np.random.default_rng(100 + batch)
    out_f, in_f = 48, 200
    w = rng.integers(0, 0x7E, size=(out_f, in_f), dtype=np.uint8)
    w[rng.random(w.shape) < 0.5] |= 0x80  # negative codes too
    s = (rng.random(out_f) * 0.1).astype(np.float32)
    x = rng.standard_normal((batch, in_f)).astype(np.float32)
    spec = LayerQuantSpec("l.fp8", get_quant_key("fp8_static_channel_sym"),
                          scales=(ScaleDesc(name="l.fp8.weight_scale", dtype="F32", shape=()),))
    m = make_method_for_spec(spec)
    m.create_weights(spec)
    assert m.compute_path == "w8a16"
    y = m.apply(w.tobytes(), {"l.fp8.weight_scale": s}, x)
    ref = rq.fp8_linear_apply(w.tobytes(), s, x)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("groups,G", [(16, 128), (11, 128), (7, 3), (1, 1)])
def test_group_broadcast_scale_bitexact(gpu, groups, G):
    """ccq_group_broadcast_scale against the oracle, numpy and device forms;
    an ``out`` longer than groups * G keeps its tail (the reference writes
    only the leading elements)."""
    from ccut.quant import kernels as qk
    from oracle.ref_quant import group_broadcast_scale as ref_gbs

    rng = np.random.default_rng(groups * G)
    s = rng.standard_normal(groups).astype(np.float32)
    ref = ref_gbs(s, G)
    out = np.full(groups * G + 5, 7.0, dtype=np.float32)
    got = qk.group_broadcast_scale(s, G, out)
    assert got is out
    assert np.array_equal(out[: groups * G].view(np.uint32), ref.view(np.uint32))
    assert np.all(out[groups * G:] == 7.0)
    dev = torch.full((groups * G + 3,), -1.0, device=gpu)
    qk.group_broadcast_scale(torch.from_numpy(s).to(gpu), G, dev)
    d = dev.cpu().numpy()
    assert np.array_equal(d[: groups * G].view(np.uint32), ref.view(np.uint32)) and np.all(d[groups * G:] == -1.0)
    assert np.array_equal(qk.group_broadcast_scale(s, G, None), ref)


# ---- the streaming float32 Linear (16-byte weight pieces, x staged in LDS):
# rows whose bytes are whole 16-byte pieces; batches 1..17 cover the 1-, 2-
# and 4-row passes and their remainders, out_features not a multiple of the
# 16 rows of a workgroup.  The bound is the float32 summation error scale
# |x| @ |W|.T (the order of the sum differs from the oracle's); a wrong
# element, row or scale is off by the size of y itself.
def _err_ok(y, ref, x, w_f32):
    bound = np.abs(x).astype(np.float64) @ np.abs(w_f32).astype(np.float64).T
    return bool(np.all(np.abs(y.astype(np.float64) - ref.astype(np.float64)) <= 1e-5 * bound + 1e-30))


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 9, 17])
@pytest.mark.parametrize("out_f,in_f", [(37, 512), (300, 2048)])
def test_fp8_linear_f32_streaming(gpu, batch, out_f, in_f):
    from ccut.quant.method import fp8_linear_f32

    rng = np.random.default_rng(1000 * batch + out_f)
    w = rng.integers(0, 0x7F, size=(out_f, in_f), dtype=np.uint8)  # no NaN codes
    w[rng.random(w.shape) < 0.5] |= 0x80
    s = (rng.random(out_f) * 0.1 + 1e-3).astype(np.float32)
    x = rng.standard_normal((batch, in_f)).astype(np.float32)
    y = fp8_linear_f32(w.tobytes(), s, x)
    ref = rq.fp8_linear_apply(w.tobytes(), s, x)
    assert y.shape == ref.shape
    assert _err_ok(y, ref, x, rq.fp8_dequant_mat(w, s))


def test_fp8_linear_f32_streaming_all_codes_exact(gpu):
    """One-hot x: y[0, r] = fp8(code r) * s[r] with one rounding, as the
    reference forms W; every code, NaN codes included (rows of zeros
    elsewhere, so 0 * NaN never enters a sum)."""
    from ccut.quant.method import fp8_linear_f32

    in_f, c0 = 64, 37
    w = np.zeros((256, in_f), dtype=np.uint8)
    w[:, c0] = np.arange(256, dtype=np.uint8)
    s = np.linspace(0.5, 3.0, 256).astype(np.float32)
    x = np.zeros((1, in_f), dtype=np.float32)
    x[0, c0] = 1.0
    y = fp8_linear_f32(w.tobytes(), s, x)[0] + np.float32(0)  # -0 -> +0, as the sum over the row gives
    want = rq.fp8_dequant_mat(w, s)[:, c0] + np.float32(0)
    nan = np.isnan(want)
    assert nan.sum() == 2 and np.array_equal(np.isnan(y), nan)
    assert np.array_equal(y[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("batch", [1, 4, 6])
@pytest.mark.parametrize("out_f,in_f", [(19, 256), (130, 4096)])
def test_int8_linear_f32_streaming(gpu, batch, out_f, in_f):
    from ccut.quant.int8 import w8a16_linear
    from oracle import int8 as oi8

    rng = np.random.default_rng(7 * batch + in_f)
    w = rng.integers(-128, 128, size=(out_f, in_f), dtype=np.int8)
    s = (rng.random(out_f) * 0.02 + 1e-3).astype(np.float32)
    x = rng.standard_normal((batch, in_f)).astype(np.float32)
    y = w8a16_linear(w.tobytes(), s, x)
    y = y.cpu().numpy() if isinstance(y, torch.Tensor) else y
    ref = oi8.w8a16(w, s, x)
    assert _err_ok(y, ref, x, oi8.dequant_row(w, s))


@pytest.mark.parametrize("batch", [1, 2, 8])
@pytest.mark.parametrize("out_f,in_f", [(21, 64), (260, 2048)])
def test_int4_linear_f32_streaming(gpu, batch, out_f, in_f):
    from ccut.quant.weight_only import int4_linear_f32

    rng = np.random.default_rng(3 * batch + out_f)
    p = rng.integers(0, 256, size=(out_f, in_f // 2), dtype=np.uint8)
    s = (rng.random(in_f) + 0.1).astype(np.float32)
    x = rng.standard_normal((batch, in_f)).astype(np.float32)
    y = int4_linear_f32(p.tobytes(), s, x)
    ref = rq.weight_only_apply(p.tobytes(), s, x)
    assert _err_ok(y, ref, x, rq.int4_dequant_row(p, s))

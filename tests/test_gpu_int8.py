"""GPU parity of the INT8 linear layer (reference python/ccut/quant/int8.py:
20-100, kernels.py:180-189) with the oracle: per-token activation codes and
scales, the W8A8 output and the dequantized weights bit-exact; the W8A16
float32 product within 1e-5 of max|y|."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int8 as oi8

pytestmark = pytest.mark.gpu


def _same(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit-identical float32 arrays, any NaN matching any NaN (0 * inf gives
    0xFFC00000 on x86 and 0x7FC00000 on the GPU)."""
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                                           b[~nb].view(np.uint32))


def _acts(rng, M, K):
    x = (rng.standard_normal((M, K)) * 0.7).astype(np.float32)
    if M > 4 and K > 8:
        x[1] = 0.0                 # zero row
        x[2, 3] = np.nan           # NaN row
        x[3, 5] = np.inf           # inf row
        x[4] = np.float32(16129 / 128) * np.sign(x[4])  # ties at the clip
        x[4, :4] = np.array([2.5, 3.5, -2.5, 0.5], np.float32) / 128  # exact halves
    return x


@pytest.mark.parametrize("M,K", [(1, 16), (7, 100), (64, 4096), (300, 7168), (5, 1)])
def test_act_quant_bitexact(gpu, M, K):
    from ccut.quant.int8 import quantize_per_token

    rng = np.random.default_rng(M * 7 + K)
    x = _acts(rng, M, K)
    xq, xs = quantize_per_token(x)
    rq, rs = oi8.quantize_per_token(x)
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), rs.view(np.uint32))


# decode (K split over workgroups), prefill (one split), ragged tiles, K % 16 != 0
@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (16, 7168, 2048), (3, 2048, 70), (130, 1024, 520),
                                   (256, 4096, 1024), (65, 48, 1), (7, 100, 33), (2, 8, 3), (4, 7168, 2048),
                                   (4, 16384, 64), (2, 4096, 14336), (5, 4096, 300), (40, 4096, 256),
                                   (200, 2048, 130), (33, 64, 129)])
def test_w8a8_linear_bitexact(gpu, M, K, N):
    from ccut.quant.int8 import w8a8_linear

    rng = np.random.default_rng(M + K + N)
    x = _acts(rng, M, K)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = (rng.random(N) * 0.02 + 1e-4).astype(np.float32)
    y = w8a8_linear(w.tobytes(), s, x)
    ref = oi8.w8a8(w, s, x)
    assert _same(y, ref)


def test_w8a8_largest_k_no_overflow(gpu):
    """K = 131056 (the largest multiple of 16 below the limit): every product
    +-127 * 127, sums at the int32 edge."""
    from ccut.quant.int8 import int8_linear

    K = 131056
    xq = torch.full((2, K), 127, dtype=torch.int8, device=gpu)
    xq[1, ::2] = -127
    w = torch.full((3, K), 127, dtype=torch.int8, device=gpu)
    w[2] = -127
    xs = torch.ones(2, device=gpu)
    ws = torch.ones(3, device=gpu)
    y = int8_linear(xq, xs, w, ws).cpu().numpy()
    ref = (xq.cpu().numpy().astype(np.int64) @ w.cpu().numpy().astype(np.int64).T).astype(np.float32)
    assert np.array_equal(y, ref)
    assert y[0, 0] == np.float32(16129 * K)


def test_int8_method_dispatch_and_paths(gpu):
    from ccut.quant.int8 import Int8LinearMethod
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.spec import K_INT8_STATIC_CHANNEL_SYM, LayerQuantSpec, ScaleDesc, get_quant_key

    rng = np.random.default_rng(11)
    M, K, N = 9, 512, 96
    x = _acts(rng, M, K)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = (rng.random(N) * 0.02 + 1e-4).astype(np.float32)
    spec = LayerQuantSpec(layer_name="mlp.down_proj", weight_key=get_quant_key(K_INT8_STATIC_CHANNEL_SYM),
                          scales=(ScaleDesc(name="weight_scale", dtype="F32", shape=(N,)),))
    m = make_method_for_spec(spec)
    assert isinstance(m, Int8LinearMethod) and m.compute_path == "w8a16"
    y16 = m.apply(w.tobytes(), {"weight_scale": s}, x)
    r16 = oi8.w8a16(w, s, x)
    fin = np.isfinite(r16).all(axis=1)
    assert np.all(np.abs(y16[fin] - r16[fin]) <= 1e-5 * np.abs(r16[fin]).max())
    m8 = Int8LinearMethod(spec, compute_mode="w8a8")
    assert m8.compute_path == "w8a8"
    y8 = m8.apply(w.tobytes(), {"weight_scale": s}, x)
    assert _same(y8, oi8.w8a8(w, s, x))
    # device tensors in, device tensor out
    yd = m8.apply(torch.from_numpy(w).to(gpu), {"weight_scale": torch.from_numpy(s).to(gpu)},
                  torch.from_numpy(x).to(gpu))
    assert yd.is_cuda and _same(yd.cpu().numpy(), y8)


def test_int8_dequant_row_bitexact(gpu):
    from ccut.quant import kernels

    rng = np.random.default_rng(5)
    w = rng.integers(-128, 128, (37, 301)).astype(np.int8)
    s = (rng.standard_normal(37) * 0.1).astype(np.float32)
    out = np.empty((37, 301), np.float32)
    kernels.int8_dequant_row(w, s, out)
    assert np.array_equal(out.view(np.uint32), oi8.dequant_row(w, s).view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(1, 4096, 14336), (4, 7168, 2048), (3, 1024, 96), (4, 16384, 256)])
def test_w8a8_fused_matches_two_kernels(gpu, M, K, N):
    """ccq_int8_w8a8_linear (activation quantization inside the GEMM up to 4
    rows) against ccq_int8_act_quant + ccq_int8_linear: scales and outputs
    bit-identical, twice in a row on the shared workspace."""
    from ccut import _dev
    from ccut._lib import call, lib
    from ccut.quant.int8 import int8_linear, quantize_per_token

    rng = np.random.default_rng(M * 31 + K + N)
    w = torch.from_numpy(rng.integers(-127, 128, (N, K)).astype(np.int8)).to(gpu)
    s = torch.from_numpy((rng.random(N) * 0.02 + 1e-4).astype(np.float32)).to(gpu)
    for rows in (M, max(1, M - 2)):
        x = torch.from_numpy(_acts(rng, rows, K)).to(gpu)
        xs = torch.empty(rows, device=gpu)
        y = torch.empty((rows, N), device=gpu)
        nb = int(lib().ccq_int8_w8a8_workspace_size(rows, K, N))
        ws = _dev.workspace("int8_w8a8", nb, gpu) if nb else None
        call("ccq_int8_w8a8_linear", x.data_ptr(), xs.data_ptr(), w.data_ptr(), s.data_ptr(), y.data_ptr(), rows, K,
             N, ws.data_ptr() if ws is not None else None, nb, _dev.stream_ptr())
        xq2, xs2 = quantize_per_token(x)
        y2 = int8_linear(xq2, xs2, w, s)
        assert np.array_equal(xs.cpu().numpy().view(np.uint32), xs2.cpu().numpy().view(np.uint32))
        assert _same(y.cpu().numpy(), y2.cpu().numpy())

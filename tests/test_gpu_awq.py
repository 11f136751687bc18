"""GPU parity of the AWQ int4 path: re-pack round trip and dequant bit-exact,
fused dequant-GEMM within max|dy| <= 2e-2 * max|y_ref| of the oracle's
dequantize-then-matmul (fp32 accumulate; fp16/bf16 out)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import awq as oawq

pytestmark = pytest.mark.gpu

TOL = 2e-2          # the path's stated tolerance (relative to max|y_ref|)
# Regression bounds of the benchmark configurations: about 3x the error
# measured on MI355X, below the 2e-2 contract, so that a several-fold loss of
# accuracy fails even while the contract still holds
REGRESS_C1 = 8e-4
REGRESS_C2 = 1.2e-3
TIGHT = 2e-3        # float32 outputs: only accumulation order differs


def _make(K, N, G, seed, scale_dtype=np.float16):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((K // G, N))) * 0.01 + 1e-3).astype(np.float32)
    return oawq.pack(q), oawq.pack(z), s.astype(scale_dtype) if scale_dtype is np.float16 else s


def test_pack_matches_oracle(gpu):
    from ccut.quant.awq import pack_awq, unpack_awq

    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(64, 96), dtype=np.uint8)
    qt = torch.from_numpy(q).to(gpu)
    assert np.array_equal(pack_awq(qt).cpu().numpy(), oawq.pack(q))
    assert np.array_equal(unpack_awq(torch.from_numpy(oawq.pack(q)).to(gpu)).cpu().numpy(), q)


@pytest.mark.parametrize("K,N", [(128, 16), (256, 64), (1408, 2048), (2048, 1408)])
def test_repack_round_trip(gpu, K, N):
    from ccut.quant import awq

    rng = np.random.default_rng(K + N)
    words = rng.integers(0, 2 ** 32, size=(K, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qw = torch.from_numpy(words).to(gpu)
    tiled = awq.repack(qw, K, N)
    assert tiled.numel() == qw.numel()
    assert not torch.equal(tiled, qw)  # really re-ordered
    back = awq.unpack_tiled(tiled, K, N)
    assert torch.equal(back, qw)


@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("sdt", ["f16", "bf16"])
def test_dequant_bitexact(gpu, G, sdt):
    from ccut.quant import awq

    K, N = 512, 96
    qw, qz, s = _make(K, N, G, seed=G)
    st = torch.from_numpy(s.astype(np.float32)).to(gpu).to(torch.float16 if sdt == "f16" else torch.bfloat16)
    W = awq.dequant(torch.from_numpy(qw).to(gpu), torch.from_numpy(qz).to(gpu), st, G).cpu().numpy()
    ref = oawq.dequant(qw, qz, st.float().cpu().numpy(), G)
    assert np.array_equal(W.view(np.uint32), ref.view(np.uint32))


def _gemm_case(gpu, M, K, N, G, xdt, ydt, seed):
    from ccut.quant import awq

    qw, qz, s = _make(K, N, G, seed)
    w = awq.prepare(torch.from_numpy(qw).to(gpu), torch.from_numpy(qz).to(gpu), torch.from_numpy(s).to(gpu), G)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g).to(xdt)
    y = awq.gemm(x.to(gpu), w, out_dtype=ydt).float().cpu().numpy()
    ref = oawq.linear(x.float().numpy(), qw, qz, s, G)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    return err


@pytest.mark.parametrize("M", [1, 2, 4, 5, 16, 17, 33])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_gemm_parity_m_sweep(gpu, M, xdt):
    assert _gemm_case(gpu, M, 512, 256, 128, xdt, torch.float32, seed=M) <= TIGHT
    assert _gemm_case(gpu, M, 512, 256, 128, xdt, xdt, seed=M) <= TOL


@pytest.mark.parametrize("M", [65, 128, 200, 513])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_gemm_prefill_grouped_kernel(gpu, M, xdt):
    """M > 64 with group 128 and N % 128 == 0 runs the tiled prefill kernel
    (64/128-row tiles, activations staged in LDS)."""
    assert _gemm_case(gpu, M, 768, 384, 128, xdt, torch.float32, seed=M) <= TIGHT
    assert _gemm_case(gpu, M, 768, 384, 128, xdt, xdt, seed=M + 1) <= TOL


@pytest.mark.parametrize("M,K,N", [(200, 384, 512), (130, 256, 256), (300, 640, 384), (97, 1024, 768)])
def test_gemm_prefill_grouped_shapes(gpu, M, K, N):
    """Grouped kernel with 256-column blocks (N % 256 == 0) and 128-column
    blocks, odd and even numbers of k-tiles."""
    assert _gemm_case(gpu, M, K, N, 128, torch.bfloat16, torch.float32, seed=M + K) <= TIGHT
    assert _gemm_case(gpu, M, K, N, 128, torch.float16, torch.float32, seed=M + N) <= TIGHT


@pytest.mark.parametrize("G", [32, 64])
def test_gemm_parity_groups(gpu, G):
    assert _gemm_case(gpu, 3, 384, 160, G, torch.float16, torch.float32, seed=G) <= TIGHT


def test_gemm_config_single_linear_k2048_n5632(gpu):
    """x fp16 [1, 2048], W int4 2048 -> 5632, group 128, fp16 out."""
    err = _gemm_case(gpu, 1, 2048, 5632, 128, torch.float16, torch.float16, seed=1)
    print(f"[C1] awq gemv K=2048 N=5632: rel err {err:.3e}")
    assert err <= TOL
    assert err <= REGRESS_C1  # measured 2.65e-4 (fp16 output rounding dominates)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemm_config_skinny_k4096_n14336(gpu, M):
    """K=4096 N=14336 group 128, M in {1, 4, 16}, fp16 in/out."""
    err = _gemm_case(gpu, M, 4096, 14336, 128, torch.float16, torch.float16, seed=10 + M)
    print(f"[C2] awq gemm K=4096 N=14336 M={M}: rel err {err:.3e}")
    assert err <= TOL
    assert err <= REGRESS_C2  # measured 3.2e-4 .. 4.0e-4 for M = 16, 4, 1


def test_weight_only_method_awq(gpu):
    """AWQ behind the reference's apply(weight_bytes, scales, x) boundary:
    numpy float32 in, numpy float32 out."""
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.spec import LayerQuantSpec, ScaleDesc, get_quant_key

    K, N, G = 256, 128, 128
    qw, qz, s = _make(K, N, G, seed=5)
    spec = LayerQuantSpec("mlp.experts.0.gate_proj", get_quant_key("int4_awq_w4a16"),
                          scales=(ScaleDesc("mlp.experts.0.gate_proj.scales", "F16", (K // G, N)),
                                  ScaleDesc("mlp.experts.0.gate_proj.zero_points", "I32", (K // G, N // 8))))
    m = make_method_for_spec(spec)
    m.create_weights(spec)
    assert m.compute_path == "w4a16"
    x = np.random.default_rng(5).standard_normal((3, K)).astype(np.float32)
    scales = {"mlp.experts.0.gate_proj.scales": s, "mlp.experts.0.gate_proj.zero_points": qz}
    y = m.apply(qw, scales, x)
    assert isinstance(y, np.ndarray) and y.shape == (3, N) and y.dtype == np.float32
    ref = oawq.linear(x, qw, qz, s, G)
    # x enters the MFMA as fp16 (|x| < 65504: one rounding to 11 significant
    # bits of the float32 input)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"awq apply float32 x (fp16 MFMA inputs): rel err {err:.3e}")
    assert err <= 1e-3
    y2 = m.apply(qw, scales, x)  # second call reuses the prepared weights
    assert np.array_equal(y, y2)
    # activations past the float16 range go as bf16 (float32's range) and stay finite
    xb = x * np.float32(1e6)
    yb = m.apply(qw, scales, xb)
    refb = oawq.linear(xb, qw, qz, s, G)
    assert np.isfinite(yb).all() and np.abs(yb - refb).max() <= TOL * np.abs(refb).max()

"""GPU parity of the block-scaled FP8 path (128x128 weight blocks,
per-token-per-128 activations) against the oracle (``oracle/fp8_block.py``):
activation quantization and the weight re-pack bit-exact; the linear and
the MoE expert FFN within max|dy| <= 2e-2 * max|y_ref| (tighter for float32
outputs of the linear, where only the accumulation order differs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8_block as ofb

pytestmark = pytest.mark.gpu

TOL = 2e-2
TIGHT = 2e-3


def _fp8_weights(rng, E, N, K):
    v = np.clip(rng.standard_normal((E, N, K)) * 0.02, -448, 448).astype(np.float32)
    w = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    s = (np.abs(rng.standard_normal((E, N // 128, K // 128))) * 0.01 + 1e-3).astype(np.float32)
    return w, s


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,K", [(5, 256), (33, 896), (2, 7168)])
def test_act_quant_bitexact(gpu, xdt, rows, K):
    from ccut.quant import fp8_block

    g = torch.Generator().manual_seed(rows * 7 + K)
    x = (torch.randn((rows, K), generator=g) * torch.rand((rows, 1), generator=g) * 30).to(xdt)
    x[0, :128] = 0.0                       # all-zero block: scale floor
    if rows > 1:
        x[1, 5] = 1e4 if xdt != torch.float16 else 6e4   # one dominant value
        x[1, 200 % K] = 3e-5               # subnormal e4m3 after scaling
    q, s = fp8_block.act_quant(x.to(gpu))
    rq, rs = ofb.act_quant(x.float().numpy())
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), rq)


def test_repack_round_trip(gpu):
    from ccut.quant import fp8_block

    rng = np.random.default_rng(3)
    w = rng.integers(0, 256, size=(256, 384), dtype=np.uint8)
    s = np.ones((2, 3), dtype=np.float32)
    pw = fp8_block.prepare(w, s)
    assert not torch.equal(pw.w_tiled.cpu(), torch.from_numpy(w))
    assert np.array_equal(fp8_block.unpack(pw).cpu().numpy(), w)


@pytest.mark.parametrize("M", [1, 7, 64, 130])
def test_block_linear_parity(gpu, M):
    from ccut.quant import fp8_block

    rng = np.random.default_rng(M)
    w, s = _fp8_weights(rng, 1, 384, 512)
    x = rng.standard_normal((M, 512)).astype(np.float32)
    y = fp8_block.linear(w[0], s[0], x)             # numpy in -> numpy float32 out
    assert isinstance(y, np.ndarray) and y.dtype == np.float32 and y.shape == (M, 384)
    ref = ofb.linear(x, w[0], s[0])
    assert np.abs(y - ref).max() <= TIGHT * np.abs(ref).max()


def test_block_linear_bf16_device(gpu):
    from ccut.quant import fp8_block

    rng = np.random.default_rng(9)
    w, s = _fp8_weights(rng, 1, 256, 1024)
    pw = fp8_block.prepare(torch.from_numpy(w[0]).to(gpu), torch.from_numpy(s[0]).to(gpu))
    x = torch.from_numpy(rng.standard_normal((20, 1024)).astype(np.float32)).to(torch.bfloat16)
    y = fp8_block.linear(pw, None, x.to(gpu))
    assert y.is_cuda and y.dtype == torch.bfloat16
    ref = ofb.linear(x.float().numpy(), w[0], s[0])
    assert np.abs(y.float().cpu().numpy() - ref).max() <= TOL * np.abs(ref).max()


def test_fp8_block_method_boundary(gpu):
    """Block FP8 behind the reference's apply(weight_bytes, scales, x)."""
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.spec import LayerQuantSpec, ScaleDesc, get_quant_key

    rng = np.random.default_rng(11)
    w, s = _fp8_weights(rng, 1, 256, 384)
    spec = LayerQuantSpec("mlp.experts.3.down_proj", get_quant_key("fp8_block128_dynamic_group"),
                          scales=(ScaleDesc("mlp.experts.3.down_proj.weight_scale_inv", "F32", (2, 3)),))
    m = make_method_for_spec(spec)
    m.create_weights(spec)
    x = rng.standard_normal((4, 384)).astype(np.float32)
    y = m.apply(w[0].tobytes(), {"mlp.experts.3.down_proj.weight_scale_inv": s[0]}, x)
    ref = ofb.linear(x, w[0], s[0])
    assert y.shape == (4, 256) and np.abs(y - ref).max() <= TIGHT * np.abs(ref).max()
    with pytest.raises(ValueError):
        m.apply(w[0].tobytes(), {}, x)


def _moe_ref(x, ids, wts, wg, sg, wu, su, wd, sd):
    """Per token: sum over its slots (in slot order) of w * FP8 block expert
    FFN (oracle); tokens of one expert go through the oracle together."""
    T, k = ids.shape
    y = np.zeros((T, x.shape[1]), dtype=np.float32)
    rows = {}
    for e in np.unique(ids):
        t_idx = np.nonzero((ids == e).any(axis=1))[0]
        out = ofb.expert_ffn(x[t_idx], wg[e], sg[e], wu[e], su[e], wd[e], sd[e])
        for j, t in enumerate(t_idx):
            rows[(t, e)] = out[j]
    for t in range(T):
        for sl in range(k):
            y[t] += wts[t, sl] * rows[(t, ids[t, sl])]
    return y


# the last three run the stages with the weights streamed into registers
# (K blocks >= 6 and a multiple of 4): 150 rows per expert (a full and a
# ragged tile), a few rows per expert with empty experts, and gate/up only
@pytest.mark.parametrize("T,k,E,H,I", [(1, 2, 8, 256, 256), (20, 2, 8, 256, 384), (70, 4, 6, 384, 256),
                                       (300, 4, 8, 1024, 1024), (40, 2, 24, 1536, 1024), (96, 2, 4, 2048, 512)])
def test_moe_fp8_parity(gpu, T, k, E, H, I):
    from ccut.blocks import moe

    rng = np.random.default_rng(T + E)
    wg, sg = _fp8_weights(rng, E, I, H)
    wu, su = _fp8_weights(rng, E, I, H)
    wd, sd = _fp8_weights(rng, E, H, I)
    dev = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    ex = moe.Fp8Experts.from_block((dev(wg), dev(sg)), (dev(wu), dev(su)), (dev(wd), dev(sd)))
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    y = moe.moe_forward_fp8(x.to(gpu), torch.from_numpy(lg).to(gpu), ex, top_k=k,
                            out_dtype=torch.float32).cpu().numpy()
    from oracle import moe as omoe

    w0, ids0 = omoe.topk_softmax(lg, k)
    ref = _moe_ref(x.float().numpy(), ids0, w0, wg, sg, wu, su, wd, sd)
    assert np.abs(y - ref).max() <= TOL * np.abs(ref).max()

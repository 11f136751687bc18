"""The float32 products on the fp32 matrix cores (costcut-infer_amd/csrc/
ccq_f32.hip): the router x @ gate_w.T (reference
python/ccut/experts/pipeline.py:145), expert_ffn on float32 weights
(blocks/moe.py:122-141) and moe_combine over float32 experts
(blocks/moe.py:144-174), against float64 products of the same float32
operands on the CPU.

Bounds: the products are float32 and only the float32 accumulation rounds,
so max|dy| <= 1e-5 * max|y_64| for the router and the linear products;
expert_ffn adds the rounding of the intermediate (1e-5 as well)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe

pytestmark = pytest.mark.gpu


def _unused_for_dropped(ids, E):
    """ids with each negative entry replaced by an expert that row does not
    use, for the oracle's combine with a zero weight there (it finds a
    token's slot of an expert by the first match, so a repeated id would
    take the wrong slot's weight)."""
    out = ids.copy()
    for t in range(ids.shape[0]):
        for s in range(ids.shape[1]):
            if out[t, s] < 0:
                out[t, s] = min(set(range(E)) - set(out[t].tolist()))
    return out


def _rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("T,E,H", [(16, 64, 2048), (1, 256, 2048), (2048, 256, 7168), (5, 7, 33), (70, 130, 260),
                                   (3, 200, 132), (16, 256, 7168)])
def test_router_logits_vs_float64(gpu, T, E, H):
    """x @ gate_w.T with gate_w as stored [E, H]; the top-k ids of those
    logits are the oracle's bit for bit (routing on the same logits)."""
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    rng = np.random.default_rng(T * 7 + E)
    x = rng.standard_normal((T, H)).astype(np.float32)
    gw = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    lg = ExpertPipeline.router_logits(x, gw)
    ref = x.astype(np.float64) @ gw.astype(np.float64).T
    err = _rel(lg.cpu().numpy(), ref)
    print(f"router T={T} E={E} H={H}: rel err {err:.2e}")
    assert lg.shape == (T, E) and err <= 1e-5
    k = min(8, E)
    w, ids = moe.topk_softmax(lg, k, True)
    w0, ids0 = omoe.topk_softmax(lg.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ids0)
    assert np.abs(w.cpu().numpy() - w0).max() <= 1e-6


@pytest.mark.parametrize("M,K,N", [(1, 2048, 512), (37, 512, 2048), (64, 256, 64), (3, 30, 10), (130, 100, 66),
                                   (200, 3000, 72)])
def test_f32_gemm_nn_vs_float64(gpu, M, K, N):
    """x @ w for w [K, N] (expert_ffn's orientation), 16-byte and
    per-element load paths, ragged tiles."""
    from ccut._lib import call, lib

    rng = np.random.default_rng(M + K + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((K, N)).astype(np.float32)
    xd, wd = torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu)
    y = torch.empty((M, N), dtype=torch.float32, device=gpu)
    call("ccq_f32_gemm", xd.data_ptr(), wd.data_ptr(), y.data_ptr(), M, K, N, 0, None, 0, None)
    ref = x.astype(np.float64) @ w.astype(np.float64)
    assert _rel(y.cpu().numpy(), ref) <= 1e-5
    nbytes = lib().ccq_f32_gemm_workspace_size(M, K, N)
    if nbytes:  # K split over workgroups, partial sums added in split order
        ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
        y2 = torch.empty((M, N), dtype=torch.float32, device=gpu)
        call("ccq_f32_gemm", xd.data_ptr(), wd.data_ptr(), y2.data_ptr(), M, K, N, 0, ws.data_ptr(), nbytes, None)
        assert _rel(y2.cpu().numpy(), ref) <= 1e-5


def test_expert_ffn_f32_ornith_shapes(gpu):
    """expert_ffn(x, Wg, Wu, Wd) at hidden 2048, inter 512 against the
    oracle's restatement (numpy float32) and a float64 recomputation."""
    from ccut.blocks import moe

    rng = np.random.default_rng(11)
    H, I = 2048, 512
    x = rng.standard_normal((24, H)).astype(np.float32)
    wg, wu = ((rng.standard_normal((H, I)) * 0.03).astype(np.float32) for _ in range(2))
    wd = (rng.standard_normal((I, H)) * 0.03).astype(np.float32)
    y = moe.expert_ffn(x, wg, wu, wd)
    assert isinstance(y, np.ndarray) and y.shape == (24, H)
    g, u = x.astype(np.float64) @ wg, x.astype(np.float64) @ wu
    ref64 = (g / (1.0 + np.exp(-g)) * u) @ wd.astype(np.float64)
    err = _rel(y, ref64)
    print(f"expert_ffn f32: rel err vs float64 {err:.2e}")
    assert err <= 1e-5
    assert _rel(y, omoe.expert_ffn(x, wg, wu, wd).astype(np.float64)) <= 1e-5
    yd = moe.expert_ffn(torch.from_numpy(x).to(gpu), wg, wu, wd)  # device in, device out
    assert yd.is_cuda and np.array_equal(yd.cpu().numpy(), y)


def test_moe_combine_f32_grouped(gpu):
    """moe_combine with float32 experts from w_lookup: one grouped call, the
    oracle's per-expert loop as reference; an id outside the routed set and
    a shared expert's add."""
    from ccut.blocks import moe

    rng = np.random.default_rng(12)
    T, E, H, I, k = 40, 12, 256, 128, 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    W = {e: ((rng.standard_normal((H, I)) * 0.05).astype(np.float32),
             (rng.standard_normal((H, I)) * 0.05).astype(np.float32),
             (rng.standard_normal((I, H)) * 0.05).astype(np.float32)) for e in range(E)}
    w, ids = omoe.topk_softmax(rng.standard_normal((T, E)).astype(np.float32), k)
    y = moe.moe_combine(x, ids, w, w_lookup=W.__getitem__)
    ref = omoe.moe_combine(x, ids, w, W.__getitem__)
    assert _rel(y, ref.astype(np.float64)) <= 1e-5
    ids2 = ids.copy()
    ids2[::5, 0] = -1
    sh = rng.standard_normal((T, H)).astype(np.float32)
    y2 = moe.moe_combine(torch.from_numpy(x).to(gpu), torch.from_numpy(ids2).to(gpu), torch.from_numpy(w).to(gpu),
                         w_lookup=W.__getitem__, shared=torch.from_numpy(sh).to(gpu), shared_gate=0.5).cpu().numpy()
    w2 = np.where(ids2 >= 0, w, 0).astype(np.float32)
    ref2 = omoe.moe_combine(x, _unused_for_dropped(ids2, E), w2, W.__getitem__) + np.float32(0.5) * sh
    assert _rel(y2, ref2.astype(np.float64)) <= 1e-5

"""GPU parity of ExpertPipeline.step (reference python/ccut/experts/
pipeline.py:123-204) against the oracle: router, topk_softmax, expert FFN,
weighted combine, shared expert; the per-expert reader path (float32
weights, timeouts drop an expert) and the fused int4 layer path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import awq as oawq
from oracle import moe as omoe

pytestmark = pytest.mark.gpu


class _Reader:
    """Per-expert float32 weights, as the reference's ExpertReader.get."""

    def __init__(self, W, slow=()):
        self.W, self.slow = W, set(slow)
        self.prefetched, self.gets = [], []

    def prefetch(self, layer, ids):
        self.prefetched.append(list(ids))
        return len(ids)

    def get(self, layer, eid, timeout=30.0):
        self.gets.append(eid)
        if eid in self.slow:
            raise TimeoutError(f"expert {eid}")
        return self.W[eid]

    def stats(self):
        return {"hits": 7, "misses": 2}


class _Proj:
    def __init__(self, w):
        self.w = w

    def apply(self, x):
        if isinstance(x, torch.Tensor):  # device activations stay on the device
            return x.float() @ torch.from_numpy(self.w).to(x.device).T
        return (np.asarray(x, np.float32) @ self.w.T).astype(np.float32)


def _case(seed, T=8, E=16, H=64, I=32):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    gate_w = (rng.standard_normal((E, H)) * 0.2).astype(np.float32)
    W = {e: tuple((rng.standard_normal(s) * 0.1).astype(np.float32) for s in ((H, I), (H, I), (I, H)))
         for e in range(E)}
    return x, gate_w, W


def _logits(gpu, x, gate_w):
    # the step's own router, same operands on the same device
    from ccut.experts import ExpertPipeline

    return ExpertPipeline.router_logits(x, gate_w).cpu().numpy()


def test_step_per_expert_reader_matches_oracle(gpu):
    from ccut.experts import ExpertPipeline

    x, gate_w, W = _case(1)
    r = _Reader(W)
    pipe = ExpertPipeline(r, num_workers=1, speculative_window=4, prefetch_steps_ahead=2)
    y = pipe.step(3, x, gate_w, top_k=4, norm_topk_prob=True)
    w0, ids0 = omoe.topk_softmax(_logits(gpu, x, gate_w), 4)
    ref = omoe.moe_combine(x, ids0, w0, W.__getitem__)
    assert isinstance(y, np.ndarray) and y.dtype == np.float32 and y.shape == x.shape
    assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max()
    assert sorted(r.gets) == sorted(set(ids0.reshape(-1).tolist()))
    assert r.prefetched[-1] == ids0.reshape(-1).tolist()
    # second step: the speculative prefetch from the route history, metrics
    y2 = pipe.step(3, x, gate_w, top_k=4, norm_topk_prob=False)
    w1, ids1 = omoe.topk_softmax(_logits(gpu, x, gate_w), 4, False)
    ref2 = omoe.moe_combine(x, ids1, w1, W.__getitem__)
    assert np.abs(y2 - ref2).max() <= 1e-4 * np.abs(ref2).max()
    m = pipe.metrics
    assert m.steps == 2 and m.speculative_total == 1 and m.speculative_correct == 1
    assert m.compute_ns > 0 and (m.ring_hits, m.ring_misses) == (7, 2)
    # prefetches: step 1's experts, then step 2's speculative guess (token 0's
    # experts of step 1) and step 2's experts
    assert len(r.prefetched) == 3 and set(r.prefetched[1]) == set(ids0[0].tolist())


def test_step_timeout_policies(gpu):
    """A timed-out expert: "renormalize" (default) rescales each affected
    token's surviving weights to the token's original weight sum, "drop"
    leaves them as they are (the reference's code), "raise" re-raises; the
    metrics count the timeouts and the assignments left out."""
    from ccut.experts import ExpertPipeline

    x, gate_w, W = _case(2)
    w0, ids0 = omoe.topk_softmax(_logits(gpu, x, gate_w), 4)
    slow = int(ids0[0, 0])
    zero = tuple(np.zeros_like(a) for a in W[slow])
    lookup = lambda e: zero if e == slow else W[e]  # noqa: E731
    hit = ids0 == slow
    # drop: the slow expert contributes nothing, other weights unchanged
    pipe = ExpertPipeline(_Reader(W, slow=[slow]), metrics_enabled=False, on_expert_timeout="drop")
    y = pipe.step(0, x, gate_w, top_k=4)
    ref = omoe.moe_combine(x, ids0, w0, lookup)
    assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max()
    assert pipe.metrics is None
    # renormalize: surviving weights of affected tokens scaled by sum / kept sum
    pipe = ExpertPipeline(_Reader(W, slow=[slow]))
    y = pipe.step(0, x, gate_w, top_k=4)
    kept = np.where(hit, 0.0, w0).astype(np.float32)
    scale = (w0.sum(axis=1, keepdims=True) / kept.sum(axis=1, keepdims=True)).astype(np.float32)
    ref = omoe.moe_combine(x, ids0, (kept * scale).astype(np.float32), lookup)
    assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max()
    assert pipe.metrics.expert_timeouts == 1 and pipe.metrics.dropped_assignments == int(hit.sum())
    assert pipe.metrics.to_dict()["expert_timeouts"] == 1
    # a token whose only routed expert timed out keeps zeros (one slot)
    w1, ids1 = omoe.topk_softmax(_logits(gpu, x, gate_w), 1)
    pipe = ExpertPipeline(_Reader(W, slow=[int(ids1[0, 0])]))
    y1 = pipe.step(0, x, gate_w, top_k=1)
    assert np.all(y1[ids1[:, 0] == ids1[0, 0]] == 0.0) and np.isfinite(y1).all()
    # raise
    pipe = ExpertPipeline(_Reader(W, slow=[slow]), on_expert_timeout="raise")
    with pytest.raises(TimeoutError):
        pipe.step(0, x, gate_w, top_k=4)
    with pytest.raises(ValueError):
        ExpertPipeline(_Reader(W), on_expert_timeout="ignore")


def test_step_rejects_wrongly_oriented_weights(gpu):
    """Weights handed over [out, in] (the reference reader's slot layout) are
    refused rather than multiplied the wrong way round."""
    from ccut.experts import ExpertPipeline

    x, gate_w, W = _case(4)
    Wt = {e: tuple(a.T.copy() for a in w) for e, w in W.items()}
    with pytest.raises(ValueError, match="expected gate/up"):
        ExpertPipeline(_Reader(Wt)).step(0, x, gate_w, top_k=2)


def test_step_shared_expert_device_io(gpu):
    from ccut.experts import ExpertPipeline

    x, gate_w, W = _case(3)
    rng = np.random.default_rng(30)
    H, S = x.shape[1], 48
    sp = {"gate_proj": _Proj((rng.standard_normal((S, H)) * 0.1).astype(np.float32)),
          "up_proj": _Proj((rng.standard_normal((S, H)) * 0.1).astype(np.float32)),
          "down_proj": _Proj((rng.standard_normal((H, S)) * 0.1).astype(np.float32))}
    pipe = ExpertPipeline(_Reader(W))
    y = pipe.step(1, torch.from_numpy(x).to(gpu), gate_w, top_k=2, shared_projs=sp, shared_gate=0.5)
    assert isinstance(y, torch.Tensor) and y.is_cuda
    w0, ids0 = omoe.topk_softmax(_logits(gpu, x, gate_w), 2)
    ref = omoe.moe_combine(x, ids0, w0, W.__getitem__)
    s, su = sp["gate_proj"].apply(x), sp["up_proj"].apply(x)
    inter = (s / (1.0 + np.exp(-s.astype(np.float64))) * su).astype(np.float32)
    ref = ref + np.float32(0.5) * sp["down_proj"].apply(inter)
    yh = y.cpu().numpy()
    assert np.abs(yh - ref).max() <= 1e-4 * np.abs(ref).max()


def test_step_fused_int4_layer(gpu):
    """reader.experts(layer) hands the whole layer over in device format: one
    fused call, bfloat16 activations, max|dy| <= 2e-2 max|y_ref|."""
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    E, H, I, G, T, k = 16, 256, 128, 128, 8, 4
    rng = np.random.default_rng(4)

    def one(K, N):
        q = rng.integers(0, 16, size=(E, K, N), dtype=np.uint8)
        z = rng.integers(0, 16, size=(E, K // G, N), dtype=np.uint8)
        s = (np.abs(rng.standard_normal((E, K // G, N))) * 0.01 + 1e-3).astype(np.float16)
        return (np.stack([oawq.pack(q[e]) for e in range(E)]), np.stack([oawq.pack(z[e]) for e in range(E)]), s)

    gate, up, down = one(H, I), one(H, I), one(I, H)
    dev = lambda t: tuple(torch.from_numpy(a).to(gpu) for a in t)  # noqa: E731
    ex = moe.W4Experts.from_awq(dev(gate), dev(up), dev(down), group_size=G)

    class _LayerReader:
        def experts(self, layer):
            return ex

    x = rng.standard_normal((T, H)).astype(np.float32)
    gate_w = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    y = ExpertPipeline(_LayerReader()).step(0, x, gate_w, top_k=k)
    w0, ids0 = omoe.topk_softmax(_logits(gpu, x, gate_w), k)
    lookup = lambda e: tuple(oawq.dequant(t[0][e], t[1][e], t[2][e], G) for t in (gate, up, down))  # noqa: E731
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    ref = omoe.moe_combine(xb, ids0, w0, lookup)
    assert np.abs(y - ref).max() <= 2e-2 * np.abs(ref).max()


def test_step_fused_fp8_layer(gpu):
    """reader.experts(layer) returning FP8 128x128 block experts: one fused
    call (float32 activations quantized per token per 128 channels inside)."""
    from test_gpu_fp8_block import TOL as FP8_TOL, _fp8_weights, _moe_ref

    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    E, H, I, T, k = 8, 256, 256, 12, 2
    rng = np.random.default_rng(5)
    wg, sg = _fp8_weights(rng, E, I, H)
    wu, su = _fp8_weights(rng, E, I, H)
    wd, sd = _fp8_weights(rng, E, H, I)
    dev = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    ex = moe.Fp8Experts.from_block((dev(wg), dev(sg)), (dev(wu), dev(su)), (dev(wd), dev(sd)))

    class _LayerReader:
        def experts(self, layer):
            return ex

    x = rng.standard_normal((T, H)).astype(np.float32)
    gate_w = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    y = ExpertPipeline(_LayerReader()).step(2, x, gate_w, top_k=k)
    w0, ids0 = omoe.topk_softmax(_logits(gpu, x, gate_w), k)
    ref = _moe_ref(x, ids0, w0, wg, sg, wu, su, wd, sd)
    assert np.abs(y - ref).max() <= FP8_TOL * np.abs(ref).max()

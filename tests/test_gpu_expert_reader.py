"""ExpertReader (reference python/ccut/experts/reader.py:86-340) on the GPU:
slots bit-identical to the oracle's dequant of the checkpoint segments (in
expert_ffn's [in, out] orientation), ring reuse, prefetch and timeouts;
ExpertPipeline over a reader, per-expert (FP8 per-row) and fused (AWQ
layer) paths, against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _ckpt import PATTERN, write_awq, write_fp8
from oracle import awq as oawq
from oracle import moe as omoe
from oracle import ref_quant as orq

pytestmark = pytest.mark.gpu


def _reader(path, L, E, **kw):
    from ccut.experts import ExpertReader, build_expert_index

    idx = build_expert_index(path, PATTERN, num_layers=L, num_experts=E)
    return ExpertReader(idx, path, num_layers=L, **kw)


def test_fp8_slots_bitexact_and_ring(gpu, tmp_path):
    ref = write_fp8(tmp_path, L=2, E=3)
    r = _reader(tmp_path, 2, 3, ring_slots=2, num_workers=2)
    try:
        for e in range(3):
            g, u, d = r.get(1, e, timeout=30.0)
            for proj, got in (("gate", g), ("up", u), ("down", d)):
                codes, scale = ref[(1, e, proj)]  # [out, in] as the checkpoint stores it
                assert got.is_cuda and got.dtype == torch.float32
                assert np.array_equal(got.cpu().numpy().view(np.uint32),
                                      orq.fp8_dequant_mat(codes, scale).T.view(np.uint32))
        # two slots: expert 0 of layer 1 was refilled away, 1 and 2 are ready
        assert r.rings[1].find(0) is None and r.rings[1].find(2) is not None
        st = r.stats()
        assert st["reads"] == 3 and st["misses"] == 3
        assert r.prefetch(1, [2, 0]) == 1  # 2 is ready, 0 is queued
        r.get(1, 0)
        assert r.stats()["hits"] >= 1 and r.rings[1].find(0) is not None
        with pytest.raises(TimeoutError, match="not in the expert index"):
            r.get(0, 7, timeout=0.3)
    finally:
        r.close()


def test_unreadable_segment_times_out(gpu, tmp_path):
    write_fp8(tmp_path, L=1, E=2)
    r = _reader(tmp_path, 1, 2, ring_slots=1, num_workers=2)
    try:
        e = r.index.entries[(0, 1)]
        segs = dict(e.segments)
        segs["gate.weight"] = (segs["gate.weight"][0], segs["gate.weight"][1], segs["gate.weight"][2], "I64")
        r.index.entries[(0, 1)] = type(e)(e.shard, segs, e.shapes)
        with pytest.raises(TimeoutError, match="not supported"):
            r.get(0, 1, timeout=1.0)
        assert r.get(0, 0)[0].shape == (64, 32)  # gate [hidden, inter]
    finally:
        r.close()


class _PerExpertOnly:
    """A reader that offers no whole-layer form, so the pipeline takes the
    reference's per-expert path (reader.get + expert_ffn + combine)."""

    def __init__(self, r):
        self._r = r

    def __getattr__(self, name):
        if name == "experts":
            raise AttributeError(name)
        return getattr(self._r, name)


@pytest.mark.parametrize("H,I,per_expert", [(2048, 512, False), (2048, 512, True), (64, 64, False)])
def test_pipeline_over_fp8_reader(gpu, tmp_path, H, I, per_expert):
    """An FP8 per-row checkpoint with the Ornith shapes (hidden 2048, expert
    intermediate 512: gate/up stored [512, 2048], down [2048, 512]) -- the
    layer handed over whole (Fp8RowExperts, fused kernels) or read per
    expert -- and with hidden == inter, where a missing transpose would go
    unnoticed by the shapes (per expert: not a multiple of 256): y = sum_e w
    * down(silu(x Wg^T) * (x Wu^T)) with W as stored, i.e. x @ W.T."""
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    ref = write_fp8(tmp_path, L=1, E=4, H=H, I=I)
    r = _reader(tmp_path, 1, 4)
    fused = not per_expert and H % 256 == 0 and I % 256 == 0
    pipe = ExpertPipeline(_PerExpertOnly(r) if per_expert else r)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((6, H)) * 0.05).astype(np.float32)
    gate_w = (rng.standard_normal((4, H)) * 0.2).astype(np.float32)
    try:
        y = pipe.step(0, x, gate_w, top_k=2)
    finally:
        pipe.close()
    logits = ExpertPipeline.router_logits(x, gate_w).cpu().numpy()  # the step's own router
    w0, ids0 = omoe.topk_softmax(logits, 2)
    W = {e: tuple(orq.fp8_dequant_mat(*ref[(0, e, p)]) for p in ("gate", "up", "down")) for e in range(4)}
    yr = np.zeros_like(x)
    for t in range(x.shape[0]):
        for s_ in range(2):
            wg, wu, wd = W[int(ids0[t, s_])]       # [out, in] as stored
            g, u = x[t] @ wg.T, x[t] @ wu.T
            yr[t] += w0[t, s_] * ((g / (1.0 + np.exp(-g.astype(np.float64))) * u).astype(np.float32) @ wd.T)
    assert y.shape == (6, H)
    assert np.abs(y - yr).max() <= 1e-4 * np.abs(yr).max()
    assert pipe.metrics.steps == 1
    if fused:
        assert isinstance(r.experts(0), moe.Fp8RowExperts) and pipe.metrics.ring_misses == 0
    else:
        assert pipe.metrics.ring_misses >= 1


def test_awq_reader_slots_and_fused_layer(gpu, tmp_path):
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    E, H, I, G = 4, 256, 128, 128
    ref = write_awq(tmp_path, L=1, E=E, H=H, I=I, G=G)
    r = _reader(tmp_path, 1, E)
    try:
        g, u, d = r.get(0, 2)
        for proj, got in (("gate", g), ("up", u), ("down", d)):
            assert np.array_equal(got.cpu().numpy(), oawq.dequant(*ref[(0, 2, proj)], G))
        ex = r.experts(0)
        assert isinstance(ex, moe.W4Experts) and r.experts(0) is ex
        rng = np.random.default_rng(4)
        x = rng.standard_normal((8, H)).astype(np.float32)
        gate_w = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
        y = ExpertPipeline(r).step(0, x, gate_w, top_k=2)
    finally:
        r.close()
    logits = ExpertPipeline.router_logits(x, gate_w).cpu().numpy()  # the step's own router
    w0, ids0 = omoe.topk_softmax(logits, 2)
    lookup = lambda e: tuple(oawq.dequant(*ref[(0, e, p)], G) for p in ("gate", "up", "down"))  # noqa: E731
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    yr = omoe.moe_combine(xb, ids0, w0, lookup)
    assert np.abs(y - yr).max() <= 2e-2 * np.abs(yr).max()


def test_get_survives_eviction_by_prefetch(gpu, tmp_path):
    """Prefetches that refill a slot between a fill and the waiting get()
    (more experts queued than slots) do not starve the get."""
    write_fp8(tmp_path, L=1, E=4, H=64, I=64)
    r = _reader(tmp_path, 1, 4, ring_slots=2, num_workers=2)
    try:
        for _ in range(3):
            r.prefetch(0, [2, 0, 1, 3, 2, 1])
            for e in range(4):
                assert r.get(0, e, timeout=10.0)[0].shape == (64, 64)
    finally:
        r.close()

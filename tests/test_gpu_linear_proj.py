"""LinearProj over a weight reader (reference python/ccut/models/generic.py:
48-91 WeightReader / FakeWeightReader, :99-176 LinearProj, :220-231
build_linear_projs) on the GPU: the projection's bytes uploaded once and
applied through the quantized kernels; dequant_weight bit-exact with the
oracle; apply within 1e-5 of a float64 product of the oracle's weight; and
the projections as the shared expert of ExpertPipeline.step (reference
experts/pipeline.py:181-190)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import ref_quant as orq

pytestmark = pytest.mark.gpu

FP8_CHANNEL = {"num_bits": 8, "type": "float", "strategy": "channel", "dynamic": False, "symmetric": True}
FP8_TOKEN = {"num_bits": 8, "type": "float", "strategy": "token", "dynamic": True, "symmetric": True}


def _ct_config():
    from ccut.quant.compressed_tensors import CompressedTensorsConfig

    return CompressedTensorsConfig.from_config({"quant_method": "compressed-tensors", "config_groups": {
        "group_0": {"targets": ["Linear"], "weights": FP8_CHANNEL, "input_activations": FP8_TOKEN}},
        "ignore": []})


class _Counting:
    """Counts segment reads of a reader."""

    def __init__(self, r):
        self.r, self.reads = r, 0

    def segment(self, layer, key):
        self.reads += 1
        return self.r.segment(layer, key)

    def shape(self, layer, key):
        return self.r.shape(layer, key)

    def scales(self, layer, key):
        return self.r.scales(layer, key)


def _fp8_table(rng, layer, names):
    """e4m3 [out, in] codes + F32 per-row scales for each (name, out, in)."""
    table, shapes, ref = {}, {}, {}
    for name, o, i in names:
        codes = (rng.integers(0, 256, size=(o, i), dtype=np.uint8) & np.uint8(0xBF)).astype(np.uint8)
        scale = (np.abs(rng.standard_normal(o)) * 0.02 + 1e-3).astype(np.float32)
        table[(layer, name)] = codes.tobytes()
        table[(layer, name + ".weight_scale")] = scale.tobytes()
        shapes[(layer, name)] = (o, i, "F8_E4M3")
        ref[name] = orq.fp8_dequant_mat(codes, scale)
    return table, shapes, ref


def test_linear_proj_fp8_per_channel(gpu):
    from ccut.quant.linear import FakeWeightReader, LinearProj

    rng = np.random.default_rng(1)
    name = "model.layers.3.mlp.shared_expert.gate_proj"
    table, shapes, ref = _fp8_table(rng, 3, [(name, 512, 2048)])
    reader = _Counting(FakeWeightReader(table, shapes))
    proj = LinearProj(3, name, 512, 2048, reader, _ct_config())
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    y = proj.apply(x)
    W = ref[name]
    ref64 = x.astype(np.float64) @ W.astype(np.float64).T
    assert isinstance(y, np.ndarray) and y.shape == (3, 512)
    assert np.abs(y - ref64).max() <= 1e-5 * np.abs(ref64).max()
    y2 = proj.apply(torch.from_numpy(x).to(gpu))
    assert y2.is_cuda and np.array_equal(y2.cpu().numpy(), y)
    assert reader.reads == 1  # bytes uploaded once per projection
    wd = proj.dequant_weight()
    assert wd.is_cuda and np.array_equal(wd.cpu().numpy().view(np.uint32), W.view(np.uint32))


def test_linear_proj_unquantized_bf16(gpu):
    from ccut.quant.linear import FakeWeightReader, build_linear_projs

    rng = np.random.default_rng(2)
    w = torch.from_numpy(rng.standard_normal((96, 160)).astype(np.float32)).to(torch.bfloat16)
    table = {(0, "lm.up_proj"): w.view(torch.uint16).numpy().tobytes()}
    projs = build_linear_projs(0, FakeWeightReader(table, {(0, "lm.up_proj"): (96, 160, "BF16")}), None, "lm.",
                               {"up_proj": (96, 160)})
    x = rng.standard_normal((5, 160)).astype(np.float32)
    y = projs["up_proj"].apply(x)
    W = w.float().numpy().astype(np.float64)
    ref = x.astype(np.float64) @ W.T
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    assert np.array_equal(projs["up_proj"].dequant_weight().cpu().numpy(), w.float().numpy())


def test_linear_proj_missing_scale_raises(gpu):
    from ccut.quant.linear import FakeWeightReader, LinearProj

    rng = np.random.default_rng(3)
    name = "model.layers.0.mlp.shared_expert.up_proj"
    table, shapes, _ = _fp8_table(rng, 0, [(name, 256, 256)])
    del table[(0, name + ".weight_scale")]
    with pytest.raises(ValueError, match="scale"):
        LinearProj(0, name, 256, 256, FakeWeightReader(table, shapes), _ct_config()).apply(np.zeros((1, 256), np.float32))


def test_linear_projs_as_shared_expert_in_step(gpu):
    """ExpertPipeline.step with a per-row FP8 expert layer (fused) and the
    shared expert's gate/up/down as LinearProj objects: y = routed sum +
    shared_gate * down(silu(x Wg^T) * (x Wu^T))."""
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline
    from ccut.quant.linear import FakeWeightReader, build_linear_projs

    rng = np.random.default_rng(4)
    E, H, I, T, k = 16, 512, 256, 6, 4
    pre = "model.layers.2.mlp.shared_expert."
    table, shapes, ref = _fp8_table(rng, 2, [(pre + "gate_proj", I, H), (pre + "up_proj", I, H),
                                            (pre + "down_proj", H, I)])
    projs = build_linear_projs(2, FakeWeightReader(table, shapes), _ct_config(), pre,
                               {"gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)})
    lay = {p: ((rng.integers(0, 256, size=(E, o, i), dtype=np.uint8) & np.uint8(0xBF)).astype(np.uint8),
               (np.abs(rng.standard_normal((E, o))) * 0.02 + 1e-3).astype(np.float32))
           for p, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    ex = moe.Fp8RowExperts.from_rows(*((torch.from_numpy(lay[p][0]).to(gpu), torch.from_numpy(lay[p][1]).to(gpu))
                                       for p in ("gate", "up", "down")))

    class Layer:
        def experts(self, layer):
            return ex

    x = rng.standard_normal((T, H)).astype(np.float32)
    gate_w = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    pipe = ExpertPipeline(Layer())
    y = pipe.step(2, x, gate_w, top_k=k, shared_projs=projs, shared_gate=0.75)
    w0, ids0 = omoe.topk_softmax(pipe.router_logits(x, gate_w).cpu().numpy(), k)
    lookup = lambda e: tuple(orq.fp8_dequant_mat(lay[p][0][e], lay[p][1][e]).T.copy()  # noqa: E731
                             for p in ("gate", "up", "down"))
    routed = omoe.moe_combine(x, ids0, w0, lookup)
    shared = omoe.expert_ffn(x, ref[pre + "gate_proj"].T, ref[pre + "up_proj"].T, ref[pre + "down_proj"].T)
    yr = routed + np.float32(0.75) * shared
    err = np.abs(y - yr).max() / np.abs(yr).max()
    print(f"step with LinearProj shared expert: rel err {err:.3e}")
    assert err <= 1e-4

"""Checkpoint formats on the load path and behind the operator API, on the
GPU against the oracle: block-FP8 expert segments (e4m3 [out, in] +
weight_scale_inv [out/128, in/128], the reference's reader only knows
per-row scales, experts/reader.py:142-251) and int4 group experts under
compressed-tensors' group tensor names (compressed_tensors.py:209-211) --
ExpertReader slots bit-exact, the whole layer through experts(layer) into
the fused kernels, and config.json -> resolve_checkpoint_quant ->
get_layer_spec -> make_method_for_spec -> apply."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from _ckpt import PATTERN, write_ct_int4, write_fp8_block
from oracle import awq as oawq
from oracle import fp8_block as ofb
from oracle import moe as omoe

pytestmark = pytest.mark.gpu


def _reader(path, L, E):
    from ccut.experts import ExpertReader, build_expert_index

    return ExpertReader(build_expert_index(path, PATTERN, num_layers=L, num_experts=E), path, num_layers=L)


@pytest.mark.parametrize("scale_name", ["weight_scale_inv", "weight_scale"])
def test_fp8_block_slots_and_fused_layer(gpu, tmp_path, scale_name):
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    E, H, I = 4, 384, 256
    ref = write_fp8_block(tmp_path, E=E, H=H, I=I, scale_name=scale_name)
    r = _reader(tmp_path, 1, E)
    try:
        g, u, d = r.get(0, 1)
        for proj, got in (("gate", g), ("up", u), ("down", d)):
            w, s = ref[(0, 1, proj)]
            assert np.array_equal(got.cpu().numpy().view(np.uint32), ofb.block_dequant(w, s).T.view(np.uint32))
        ex = r.experts(0)
        assert isinstance(ex, moe.Fp8Experts) and (ex.hidden, ex.inter, ex.num_experts) == (H, I, E)
        rng = np.random.default_rng(2)
        x = rng.standard_normal((10, H)).astype(np.float32)
        gate_w = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
        y = ExpertPipeline(r).step(0, x, gate_w, top_k=2)
    finally:
        r.close()
    logits = ExpertPipeline.router_logits(x, gate_w).cpu().numpy()  # the step's own router
    w0, ids0 = omoe.topk_softmax(logits, 2)
    yr = np.zeros_like(x)
    for e in range(E):
        rows = np.nonzero((ids0 == e).any(axis=1))[0]
        if rows.size == 0:
            continue
        out = ofb.expert_ffn(x[rows], *ref[(0, e, "gate")], *ref[(0, e, "up")], *ref[(0, e, "down")])
        for j, t in enumerate(rows):
            yr[t] += w0[t, list(ids0[t]).index(e)] * out[j]
    assert np.abs(y - yr).max() <= 2e-2 * np.abs(yr).max()


def test_fp8_block_small_shapes_stay_per_expert(gpu, tmp_path):
    """Shapes the fused kernels do not take (inter 200) still load per expert,
    with the partial last 128-block of the scales."""
    write_fp8_block(tmp_path, E=2, H=256, I=200)
    r = _reader(tmp_path, 1, 2)
    try:
        assert r.experts(0) is None
        g, u, d = r.get(0, 0)
        assert g.shape == (256, 200) and d.shape == (200, 256)
    finally:
        r.close()


def test_compressed_tensors_int4_slots_and_fused_layer(gpu, tmp_path):
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline

    E, H, I, G = 4, 256, 128, 128
    ref = write_ct_int4(tmp_path, E=E, H=H, I=I, G=G)
    r = _reader(tmp_path, 1, E)
    try:
        g, u, d = r.get(0, 3)
        for proj, got in (("gate", g), ("up", u), ("down", d)):
            assert np.array_equal(got.cpu().numpy(), oawq.dequant(*ref[(0, 3, proj)], G))
        ex = r.experts(0)
        assert isinstance(ex, moe.W4Experts)
        rng = np.random.default_rng(5)
        x = rng.standard_normal((6, H)).astype(np.float32)
        gate_w = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
        y = ExpertPipeline(r).step(0, x, gate_w, top_k=2)
    finally:
        r.close()
    logits = ExpertPipeline.router_logits(x, gate_w).cpu().numpy()  # the step's own router
    w0, ids0 = omoe.topk_softmax(logits, 2)
    lookup = lambda e: tuple(oawq.dequant(*ref[(0, e, p)], G) for p in ("gate", "up", "down"))  # noqa: E731
    yr = omoe.moe_combine(torch.from_numpy(x).to(torch.bfloat16).float().numpy(), ids0, w0, lookup)
    assert np.abs(y - yr).max() <= 2e-2 * np.abs(yr).max()


def _config(d, quant_cfg):
    (d / "config.json").write_text(json.dumps({"architectures": ["X"], "quantization_config": quant_cfg}))


def test_registry_to_method_apply(gpu, tmp_path):
    """A layer spec resolved from config.json runs behind apply(weight_bytes,
    scales, x) on the GPU: compressed-tensors int4 group (AWQ packing) and
    fp8 128x128 blocks."""
    from ccut.quant.method import make_method_for_spec
    from ccut.quant.registry import resolve_checkpoint_quant

    ref = write_ct_int4(tmp_path / "ct", E=1, H=256, I=128, G=128)
    _config(tmp_path / "ct", {"quant_method": "compressed-tensors", "ignore": ["re:.*mlp\\.gate$"],
                              "config_groups": {"g": {"targets": ["Linear"], "weights": {
                                  "num_bits": 4, "type": "int", "strategy": "group", "group_size": 128,
                                  "symmetric": False}}}})
    name = "model.layers.0.mlp.experts.0.down_proj"
    spec = resolve_checkpoint_quant(tmp_path / "ct").get_layer_spec(name)
    m = make_method_for_spec(spec)
    m.create_weights(spec)
    qw, qz, s = ref[(0, 0, "down")]
    x = np.random.default_rng(1).standard_normal((3, qw.shape[0])).astype(np.float32)
    y = m.apply(qw, {name + ".scales": s, name + ".zero_points": qz}, x)
    yr = oawq.linear(x, qw, qz, s, 128)
    assert isinstance(y, np.ndarray) and np.abs(y - yr).max() <= 2e-2 * np.abs(yr).max()

    refb = write_fp8_block(tmp_path / "fp8", E=1, H=256, I=384)
    _config(tmp_path / "fp8", {"quant_method": "fp8", "fmt": "e4m3", "activation_scheme": "dynamic",
                               "weight_block_size": [128, 128]})
    name = "model.layers.0.mlp.experts.0.gate_proj"
    spec = resolve_checkpoint_quant(tmp_path / "fp8").get_layer_spec(name)
    m = make_method_for_spec(spec)
    w, sw = refb[(0, 0, "gate")]
    x = np.random.default_rng(2).standard_normal((5, w.shape[1])).astype(np.float32)
    y = m.apply(w.tobytes(), {name + ".weight_scale_inv": sw}, x)
    yr = ofb.linear(x, w, sw)
    assert y.shape == (5, w.shape[0]) and np.abs(y - yr).max() <= 2e-3 * np.abs(yr).max()

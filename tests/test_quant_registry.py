"""Checkpoint format registration (reference python/ccut/quant/registry.py,
compressed_tensors.py): config.json -> QuantizationConfig -> per-layer
LayerQuantSpec -> make_method_for_spec, on synthetic config.json files (the
reference's own tests, python/tests/test_quant.py:62-112, read the Ornith
checkpoint's config, which is not available here; they are re-hosted on an
equivalent config).  Host logic only, no GPU."""

from __future__ import annotations

import json

import pytest

from ccut.quant.method import make_method_for_spec
from ccut.quant.registry import (
    QUANTIZATION_METHODS,
    AwqConfig,
    Fp8BlockConfig,
    UnquantizedConfig,
    list_supported_quant,
    resolve_checkpoint_quant,
)
from ccut.quant.spec import K_AWQ_W4A16, K_FP8_BLOCK128, QuantDType, ScaleStrategy

# the 7 ignore regexes of a compressed-tensors MoE checkpoint: lm_head,
# embeddings, router, shared-expert gate, linear attention, vision tower
ORNITH_IGNORE = ["re:.*lm_head$", "re:.*embed_tokens$", "re:.*mlp\\.gate$", "re:.*shared_expert_gate$",
                 "re:.*linear_attn.*", "re:.*visual.*", "re:.*mtp.*"]


def _write(d, quant_cfg, nested=True):
    cfg = {"architectures": ["X"], "text_config": {"quantization_config": quant_cfg}} if nested else \
        {"architectures": ["X"], "quantization_config": quant_cfg}
    (d / "config.json").write_text(json.dumps(cfg))
    return d


def _ct(weights, acts=None, ignore=ORNITH_IGNORE, targets=("Linear",)):
    grp = {"targets": list(targets), "weights": weights}
    if acts is not None:
        grp["input_activations"] = acts
    return {"quant_method": "compressed-tensors", "quantization_status": "compressed",
            "config_groups": {"group_0": grp}, "ignore": ignore}


FP8_CHANNEL = {"num_bits": 8, "type": "float", "strategy": "channel", "dynamic": False, "symmetric": True}
FP8_TOKEN = {"num_bits": 8, "type": "float", "strategy": "token", "dynamic": True, "symmetric": True}


def test_compressed_tensors_ignore_rules(tmp_path):
    """Reference python/tests/test_quant.py:62-71 on an equivalent config."""
    cfg = resolve_checkpoint_quant(_write(tmp_path, _ct(FP8_CHANNEL, FP8_TOKEN)))
    assert cfg.name == "compressed-tensors"
    assert cfg.is_layer_skipped("lm_head")
    assert cfg.is_layer_skipped("model.language_model.embed_tokens")
    assert cfg.is_layer_skipped("model.language_model.layers.0.mlp.gate")
    assert cfg.is_layer_skipped("model.language_model.layers.0.linear_attn.in_proj_qkv")
    assert not cfg.is_layer_skipped("model.language_model.layers.3.self_attn.q_proj")
    assert not cfg.is_layer_skipped("model.language_model.layers.3.mlp.experts.0.gate_proj")


def test_method_dispatch_for_compressed_tensors_layer(tmp_path):
    """Reference python/tests/test_quant.py:107-112: per-channel FP8 experts
    take the w8a16 path; an ignored layer is a skipped BF16 passthrough."""
    cfg = resolve_checkpoint_quant(_write(tmp_path, _ct(FP8_CHANNEL, FP8_TOKEN)))
    spec = cfg.get_layer_spec("model.language_model.layers.0.mlp.experts.0.gate_proj")
    assert spec.weight_key.weight_dtype == QuantDType.FP8_E4M3
    assert spec.weight_key.weight_scale == ScaleStrategy.PER_CHANNEL
    assert [s.name for s in spec.scales] == ["model.language_model.layers.0.mlp.experts.0.gate_proj.weight_scale"]
    assert make_method_for_spec(spec).compute_path == "w8a16"
    router = cfg.get_layer_spec("model.language_model.layers.0.mlp.gate")
    assert router.skipped and make_method_for_spec(router).compute_path == "bf16"
    assert cfg.get_layer_spec("model.norm").skipped  # no group targets it


def test_online_quant_rules(tmp_path):
    """Reference python/tests/test_quant.py:74-86: checkpoint and online
    quantization exclude each other; unknown shorthands are rejected."""
    with pytest.raises(ValueError):
        resolve_checkpoint_quant(_write(tmp_path, _ct(FP8_CHANNEL)), online_quantization="fp8_per_token")
    plain = tmp_path / "plain"
    plain.mkdir()
    (plain / "config.json").write_text(json.dumps({"architectures": ["LlamaForCausalLM"]}))
    with pytest.raises(ValueError):
        resolve_checkpoint_quant(plain, online_quantization="NOPE")
    assert isinstance(resolve_checkpoint_quant(plain), UnquantizedConfig)
    on = resolve_checkpoint_quant(plain, online_quantization="fp8_per_token", quant_ignore=["lm_head"])
    assert on.name == "online" and on.get_layer_spec("lm_head").skipped
    s = on.get_layer_spec("model.layers.0.mlp.down_proj")
    assert s.weight_key.weight_dtype == QuantDType.FP8_E4M3 and not s.skipped
    with pytest.raises(FileNotFoundError):
        resolve_checkpoint_quant(tmp_path / "missing")


def test_supported_and_unregistered(tmp_path):
    names = list_supported_quant()
    assert {"compressed-tensors", "awq", "fp8"} <= set(names)
    assert QUANTIZATION_METHODS["awq"] is AwqConfig and QUANTIZATION_METHODS["fp8"] is Fp8BlockConfig
    with pytest.raises(ValueError, match="not registered"):
        resolve_checkpoint_quant(_write(tmp_path, {"quant_method": "gptq", "bits": 4}))


def test_compressed_tensors_int4_group_is_awq(tmp_path):
    """int4 strategy=group weights -> K_AWQ_W4A16 with the group size along
    the input dimension, scales / zero points under the group tensor names,
    dispatched to the AWQ weight-only method."""
    w = {"num_bits": 4, "type": "int", "strategy": "group", "group_size": 64, "symmetric": False}
    cfg = resolve_checkpoint_quant(_write(tmp_path, _ct(w), nested=False))
    name = "model.layers.5.mlp.experts.17.down_proj"
    spec = cfg.get_layer_spec(name)
    assert spec.weight_key.name == K_AWQ_W4A16 and spec.weight_key.is_awq()
    assert spec.weight_key.group_shape.group_size == 64
    assert [s.name for s in spec.scales] == [name + ".scales", name + ".zero_points"]
    m = make_method_for_spec(spec)
    assert m.compute_path == "w4a16" and m.is_awq and m.group_size == 64
    sym = dict(w, symmetric=True)
    with pytest.raises(ValueError):
        resolve_checkpoint_quant(_write(tmp_path, _ct(sym))).get_layer_spec(name)


@pytest.mark.parametrize("strategy", ["channel", "tensor"])
def test_compressed_tensors_int4_not_group_raises(tmp_path, strategy):
    """int4 weights with a per-channel or per-tensor scale have no kernel
    here: they must raise, not resolve to the INT8 keys (whose kernels would
    read packed nibbles as int8 codes)."""
    w = {"num_bits": 4, "type": "int", "strategy": strategy, "symmetric": True}
    cfg = resolve_checkpoint_quant(_write(tmp_path, _ct(w)))
    with pytest.raises(ValueError, match="int4"):
        cfg.get_layer_spec("model.layers.0.mlp.experts.0.up_proj")


def test_compressed_tensors_pack_quantized_int4_raises(tmp_path):
    """The compressed-tensors pack-quantized layout (weight_packed [out, in/8])
    is not the AWQ-packed layout the int4 kernels read: such a config raises
    instead of loading nibbles in the wrong order."""
    w = {"num_bits": 4, "type": "int", "strategy": "group", "group_size": 128, "symmetric": False}
    qc = dict(_ct(w), format="pack-quantized")
    cfg = resolve_checkpoint_quant(_write(tmp_path, qc))
    with pytest.raises(NotImplementedError, match="pack-quantized"):
        cfg.get_layer_spec("model.layers.0.mlp.experts.0.up_proj")
    # FP8 channel groups under the same format key still resolve
    qf = dict(_ct(FP8_CHANNEL, FP8_TOKEN), format="pack-quantized")
    spec = resolve_checkpoint_quant(_write(tmp_path, qf)).get_layer_spec("model.layers.0.mlp.experts.0.up_proj")
    assert spec.weight_key.weight_dtype == QuantDType.FP8_E4M3


def test_compressed_tensors_fp8_block(tmp_path):
    """FP8 strategy=block [128, 128] with per-token-group activations ->
    K_FP8_BLOCK128, dispatched to the block FP8 method."""
    w = {"num_bits": 8, "type": "float", "strategy": "block", "block_structure": [128, 128], "symmetric": True}
    a = {"num_bits": 8, "type": "float", "strategy": "group", "group_size": 128, "dynamic": True}
    cfg = resolve_checkpoint_quant(_write(tmp_path, _ct(w, a)))
    name = "model.layers.1.mlp.experts.3.up_proj"
    spec = cfg.get_layer_spec(name)
    assert spec.weight_key.name == K_FP8_BLOCK128 and spec.effective_key().is_fp8_block()
    assert spec.effective_key().act_scale == ScaleStrategy.PER_GROUP
    assert [s.name for s in spec.scales] == [name + ".weight_scale"]
    m = make_method_for_spec(spec)
    assert m.is_block and m.compute_path == "w8a8"
    bad = dict(w, block_structure=[64, 64])
    with pytest.raises(ValueError):
        resolve_checkpoint_quant(_write(tmp_path, _ct(bad))).get_layer_spec(name)


def test_awq_checkpoint_config(tmp_path):
    q = {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True, "version": "gemm",
         "modules_to_not_convert": ["visual"]}
    cfg = resolve_checkpoint_quant(_write(tmp_path, q))
    assert isinstance(cfg, AwqConfig)
    name = "model.layers.0.mlp.experts.2.gate_proj"
    spec = cfg.get_layer_spec(name)
    assert spec.weight_key.is_awq() and [s.name for s in spec.scales] == [name + ".scales", name + ".qzeros"]
    assert make_method_for_spec(spec).is_awq
    assert cfg.get_layer_spec("model.visual.blocks.0.attn.qkv_proj").skipped
    assert cfg.get_layer_spec("lm_head").skipped and cfg.get_layer_spec("model.layers.0.mlp.gate").skipped
    for bad in ({"bits": 8}, {"group_size": 96}, {"version": "gemv"}, {"zero_point": False}):
        with pytest.raises(ValueError):
            resolve_checkpoint_quant(_write(tmp_path, dict(q, **bad)))


def test_fp8_block_checkpoint_config(tmp_path):
    q = {"quant_method": "fp8", "fmt": "e4m3", "activation_scheme": "dynamic", "weight_block_size": [128, 128]}
    cfg = resolve_checkpoint_quant(_write(tmp_path, q))
    name = "model.layers.3.mlp.experts.9.down_proj"
    spec = cfg.get_layer_spec(name)
    assert spec.weight_key.is_fp8_block() and spec.scales[0].name == name + ".weight_scale_inv"
    assert make_method_for_spec(spec).is_block
    with pytest.raises(NotImplementedError):  # per-tensor FP8: the reference's Fp8Config raises too
        resolve_checkpoint_quant(_write(tmp_path, {"quant_method": "fp8", "activation_scheme": "dynamic"}))
    with pytest.raises(ValueError):
        resolve_checkpoint_quant(_write(tmp_path, dict(q, activation_scheme="static")))

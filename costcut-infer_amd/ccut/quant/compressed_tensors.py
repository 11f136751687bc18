"""compressed-tensors checkpoints (reference
``python/ccut/quant/compressed_tensors.py:44-233``): ``config_groups`` and
the ``ignore`` regexes of ``quantization_config`` -> one ``LayerQuantSpec``
per layer.

Weight strategies: ``channel`` / ``tensor`` (FP8 or INT8, as the
reference; int4 raises), ``group`` (FP8 as the reference; **int4** ->
``K_AWQ_W4A16`` with the group size along the input dimension) and
``block`` (FP8 with ``block_structure [128, 128]`` -> ``K_FP8_BLOCK128``,
scales ``<layer>.weight_scale`` [out/128, in/128]).

The int4 group layout read here is this package's own: the AWQ GEMM packing
(``qweight`` [in, out/8] int32, 4-bit zero points packed the same way, fp16
scales [in/G, out]) stored under ``<layer>.weight`` / ``.zero_points`` /
``.scales``.  It is not the compressed-tensors ``pack-quantized`` layout
(``weight_packed`` [out, in/8], ``weight_scale``, ``weight_zero_point``,
symmetric by default); a config whose ``format`` names that layout raises
``NotImplementedError`` for its int4 groups, as the reference raises for
every integer group.  Activation strategies:
``token`` / ``tensor`` / ``channel`` / ``dynamic`` / ``row`` as the
reference, and ``group`` (per token per group, the activation side of block
FP8).

The element type of a group comes from its ``dtype`` entry when present
(the reference's spelling, e.g. ``"fp8"``), else from the standard
``type`` + ``num_bits`` pair (``float``/8 -> fp8, ``int``/8 -> int8,
``int``/4 -> int4).  Layers matching an ``ignore`` regex (``re:`` prefix,
``search`` semantics) pass through in BF16; so do layers no group targets.
"""

from __future__ import annotations

import re
from pathlib import Path

from ccut.quant.registry import QuantizationConfig, _compile_ignore, _register
from ccut.quant.spec import (
    K_AWQ_W4A16,
    K_BF16,
    K_FP8_BLOCK128,
    K_FP8_DYNAMIC_TOKEN_SYM,
    K_FP8_STATIC_CHANNEL_SYM,
    K_FP8_STATIC_TENSOR_SYM,
    K_INT8_STATIC_CHANNEL_SYM,
    GroupShape,
    LayerQuantSpec,
    QuantDType,
    QuantKey,
    ScaleDesc,
    ScaleStrategy,
    get_quant_key,
)

__all__ = ["CompressedTensorsConfig", "registered_classes"]


def _elem_type(cfg: dict) -> str:
    """``fp8`` / ``int8`` / ``int4`` (or the group's own ``dtype`` string)."""
    if "dtype" in cfg:
        return str(cfg["dtype"]).casefold()
    kind = str(cfg.get("type", "float")).casefold()
    bits = int(cfg.get("num_bits", 8))
    if kind == "float":
        if bits != 8:
            raise ValueError(f"compressed-tensors: {bits}-bit float weights are not supported")
        return "fp8"
    if kind == "int" and bits in (4, 8):
        return f"int{bits}"
    raise ValueError(f"compressed-tensors: type={kind!r} num_bits={bits} is not supported")


def _with_scale(base: QuantKey, weight_scale: str, group_shape: GroupShape | None = None) -> QuantKey:
    return QuantKey(weight_dtype=base.weight_dtype, weight_scale=weight_scale, act_dtype=base.act_dtype,
                    act_scale=base.act_scale, symmetric=base.symmetric,
                    group_shape=group_shape if group_shape is not None else base.group_shape, name=base.name)


def _weight_key(w_cfg: dict) -> QuantKey:
    """``weights`` of a config group -> weight ``QuantKey`` (reference
    ``compressed_tensors.py:44-71`` for channel / tensor / FP8 group)."""
    strategy = str(w_cfg.get("strategy", "tensor")).casefold()
    dt = _elem_type(w_cfg)
    fp8 = "fp8" in dt or "float" in dt
    if dt == "int4" and strategy != "group":
        raise ValueError(f"compressed-tensors int4 weights with strategy {strategy!r}: only group-wise int4 "
                         "(strategy 'group') is supported")
    if strategy == "channel":
        return _with_scale(get_quant_key(K_FP8_STATIC_CHANNEL_SYM if fp8 else K_INT8_STATIC_CHANNEL_SYM),
                           ScaleStrategy.PER_CHANNEL)
    if strategy == "tensor":
        return _with_scale(get_quant_key(K_FP8_STATIC_TENSOR_SYM if fp8 else K_INT8_STATIC_CHANNEL_SYM),
                           ScaleStrategy.PER_TENSOR)
    if strategy == "group":
        gs = int(w_cfg.get("group_size") or 128)
        if fp8:
            return _with_scale(get_quant_key(K_FP8_DYNAMIC_TOKEN_SYM), ScaleStrategy.PER_GROUP, GroupShape(rows=gs))
        if dt == "int4":
            if gs not in (32, 64, 128):
                raise ValueError(f"compressed-tensors int4 group_size={gs} not in (32, 64, 128)")
            if w_cfg.get("symmetric", False):
                raise ValueError("compressed-tensors int4 groups: symmetric (zero-point-free) weights are not "
                                 "supported; the int4 kernels take 4-bit zero points")
            return _with_scale(get_quant_key(K_AWQ_W4A16), ScaleStrategy.PER_GROUP, GroupShape(rows=gs))
        raise ValueError(f"compressed-tensors {dt} group strategy is not supported (group_size={gs})")
    if strategy == "block":
        block = list(w_cfg.get("block_structure") or [128, 128])
        if not fp8 or block != [128, 128]:
            raise ValueError(f"compressed-tensors block strategy: {dt} with block_structure {block} "
                             "(FP8 128x128 only)")
        return get_quant_key(K_FP8_BLOCK128)
    raise ValueError(f"unknown weights.strategy {strategy!r}")


def _act_key(a_cfg: dict) -> QuantKey:
    """``input_activations`` of a config group -> activation ``QuantKey``
    (reference ``compressed_tensors.py:74-100``, plus ``group``)."""
    strategy = str(a_cfg.get("strategy", "dynamic")).casefold()
    dt = _elem_type(a_cfg)
    fp8 = "fp8" in dt or "float" in dt
    if strategy in ("dynamic", "row"):
        strategy = "token"
    if strategy == "token":
        base = get_quant_key(K_FP8_DYNAMIC_TOKEN_SYM if fp8 else K_INT8_STATIC_CHANNEL_SYM)
        return QuantKey(weight_dtype=base.act_dtype, weight_scale=ScaleStrategy.PER_TOKEN, symmetric=True,
                        name=f"act_{base.name}")
    if strategy == "tensor":
        base = get_quant_key(K_FP8_STATIC_TENSOR_SYM if fp8 else K_INT8_STATIC_CHANNEL_SYM)
        return QuantKey(weight_dtype=base.act_dtype, weight_scale=ScaleStrategy.PER_TENSOR, symmetric=True,
                        name=f"act_{base.name}")
    if strategy == "channel":
        base = get_quant_key(K_INT8_STATIC_CHANNEL_SYM)
        return QuantKey(weight_dtype=base.act_dtype, weight_scale=ScaleStrategy.PER_CHANNEL, symmetric=True,
                        name=f"act_{base.name}")
    if strategy == "group":
        gs = int(a_cfg.get("group_size") or 128)
        if not fp8:
            raise ValueError(f"compressed-tensors {dt} activation groups are not supported")
        return QuantKey(weight_dtype=QuantDType.FP8_E4M3, weight_scale=ScaleStrategy.PER_GROUP, symmetric=True,
                        group_shape=GroupShape(rows=gs), name="act_fp8_dynamic_group")
    raise ValueError(f"unknown input_activations.strategy {strategy!r}")


def _linear_name(layer_name: str) -> bool:
    return ("_proj" in layer_name or ".fc" in layer_name or layer_name.endswith(".gate")
            or "shared_expert" in layer_name)


def _targets(group: dict, layer_name: str) -> bool:
    """Whether a config group's ``targets`` select the layer (reference
    ``compressed_tensors.py:103-141``): ``Linear`` = any linear projection
    name; ``re:<regex>`` (fullmatch or search); ``*`` wildcards; a literal
    name or suffix.  A group without targets selects every layer."""
    targets = group.get("targets")
    if not targets:
        return True
    if isinstance(targets, str):
        targets = [t for t in targets.split(",") if t.strip()]
    for t in (t.strip() for t in targets):
        if not t:
            continue
        if t.startswith("Linear"):
            if _linear_name(layer_name):
                return True
        elif t.startswith("re:"):
            if re.fullmatch(t[3:], layer_name) or re.search(t[3:], layer_name):
                return True
        elif "*" in t:
            if re.fullmatch(t.replace("*", ".*"), layer_name):
                return True
        elif layer_name == t or layer_name.endswith(t):
            return True
    return False


@_register("compressed-tensors")
class CompressedTensorsConfig(QuantizationConfig):
    """``quant_method = "compressed-tensors"`` (reference
    ``compressed_tensors.py:144-233``)."""

    def __init__(self, quant_cfg: dict, ignore_patterns: list[str], groups: list[dict],
                 model_dir: Path | None = None):
        self.quant_cfg = quant_cfg
        self.ignore_patterns = _compile_ignore(ignore_patterns)
        self.groups = groups
        self.model_dir = model_dir
        self._specs: dict[str, LayerQuantSpec] = {}

    @classmethod
    def from_config(cls, quant_cfg: dict, model_dir: str | Path | None = None) -> "CompressedTensorsConfig":
        raw = quant_cfg.get("config_groups", [])
        if isinstance(raw, dict):
            groups = list(raw.values())
        elif isinstance(raw, list):
            groups = list(raw)
        else:
            raise ValueError(f"config_groups of type {type(raw).__name__}")
        if not groups:
            raise ValueError("compressed-tensors quantization_config has no config_groups")
        return cls(quant_cfg, list(quant_cfg.get("ignore", [])), groups, Path(model_dir) if model_dir else None)

    def is_layer_skipped(self, layer_name: str) -> bool:
        """A layer matching an ``ignore`` regex passes through in BF16."""
        return any(rx.search(layer_name) for rx in self.ignore_patterns)

    def get_layer_spec(self, layer_name: str) -> LayerQuantSpec:
        spec = self._specs.get(layer_name)
        if spec is not None:
            return spec
        skipped = self.is_layer_skipped(layer_name)
        for group in self.groups:
            if not _targets(group, layer_name):
                continue
            w_cfg = group["weights"]
            a_cfg = group.get("input_activations") or {}
            w_key = _weight_key(w_cfg)
            fmt = str(group.get("format") or self.quant_cfg.get("format") or "").casefold()
            if w_key.is_awq() and fmt == "pack-quantized":
                raise NotImplementedError(
                    f"{layer_name}: compressed-tensors pack-quantized int4 (weight_packed [out, in/8]) is not "
                    "read; int4 groups must be stored in the AWQ GEMM packing under .weight/.zero_points/.scales")
            a_key = _act_key(a_cfg) if a_cfg else None
            strategy = str(w_cfg.get("strategy", "tensor")).casefold()
            if strategy == "group":
                names = ((f"{layer_name}.scales", "F16" if w_key.is_awq() else "F32"),
                         (f"{layer_name}.zero_points", "I32" if w_key.is_awq() else "F32"))
            else:
                names = ((f"{layer_name}.weight_scale", "F32"),)
            spec = LayerQuantSpec(layer_name=layer_name, weight_key=w_key, activation_key=a_key,
                                  scales=tuple(ScaleDesc(n, d, ()) for n, d in names), skipped=skipped,
                                  quant_method=self.name)
            self._specs[layer_name] = spec
            return spec
        spec = LayerQuantSpec(layer_name, get_quant_key(K_BF16), skipped=True, quant_method=self.name)
        self._specs[layer_name] = spec
        return spec

    def resolve_scale_names(self, layer_name: str, actual_weights: set[str]) -> tuple[str, ...]:
        """The scale tensors a layer actually has among ``actual_weights``
        (reference ``compressed_tensors.py:214-222``)."""
        found = tuple(layer_name + s for s in (".weight_scale", ".scales", ".weight_scale_2")
                      if layer_name + s in actual_weights)
        return found or (layer_name + ".weight_scale",)

    def validate(self) -> None:
        for name, spec in self._specs.items():
            if not spec.skipped and not spec.scales:
                raise ValueError(f"quantized layer {name} has no scale tensor")


def registered_classes() -> list[type[QuantizationConfig]]:
    """Every config class this package registers (reference
    ``compressed_tensors.py:236-237``)."""
    from ccut.quant.registry import AwqConfig, Fp8BlockConfig

    return [CompressedTensorsConfig, AwqConfig, Fp8BlockConfig]

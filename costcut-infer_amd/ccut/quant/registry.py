"""Checkpoint quantization formats: the ``QUANTIZATION_METHODS`` table and
``resolve_checkpoint_quant`` (reference ``python/ccut/quant/registry.py:28-154``).

A checkpoint's ``config.json`` names its format in
``quantization_config.quant_method``; the registered ``QuantizationConfig``
class parses it (``from_config``) and hands out one ``LayerQuantSpec`` per
layer name (``get_layer_spec``), which ``make_method_for_spec`` turns into
the method that runs the layer on the GPU.  Registered here:

* ``compressed-tensors`` (``ccut.quant.compressed_tensors``): the
  reference's format, plus int4 ``strategy=group`` weights -> ``K_AWQ_W4A16``
  and FP8 ``strategy=block`` 128x128 weights -> ``K_FP8_BLOCK128``;
* ``awq``: AutoAWQ GEMM checkpoints (``qweight`` / ``qzeros`` / ``scales``)
  -> ``K_AWQ_W4A16``;
* ``fp8``: FP8 checkpoints with ``weight_block_size = [128, 128]``
  (``weight_scale_inv`` per block) -> ``K_FP8_BLOCK128``; other bare FP8
  configs raise ``NotImplementedError``, as the reference's ``Fp8Config``
  does (``quant/fp8.py:37-51``).

An unregistered ``quant_method`` raises ``ValueError`` listing the
registered ones, as the reference does.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

from ccut.quant.spec import (
    GroupShape,
    K_AWQ_W4A16,
    K_BF16,
    K_FP8_BLOCK128,
    LayerQuantSpec,
    QuantDType,
    QuantKey,
    ScaleDesc,
    get_quant_key,
)

__all__ = [
    "QUANTIZATION_METHODS",
    "ONLINE_SHORTHANDS",
    "QuantizationConfig",
    "UnquantizedConfig",
    "AwqConfig",
    "Fp8BlockConfig",
    "resolve_checkpoint_quant",
    "list_supported_quant",
]


class QuantizationConfig:
    """One checkpoint format (reference ``registry.py:28-49``): ``from_config``
    parses ``quantization_config``; ``get_layer_spec`` gives a layer's
    ``LayerQuantSpec``; ``validate`` checks the parsed layers after loading."""

    name: str = "base"

    @classmethod
    def from_config(cls, quant_cfg: dict, model_dir: str | Path | None = None) -> "QuantizationConfig":
        raise NotImplementedError

    def get_layer_spec(self, layer_name: str) -> LayerQuantSpec:
        raise NotImplementedError

    def validate(self) -> None:
        return None


#: quant_method -> config class (filled on first use, see _register_all)
QUANTIZATION_METHODS: dict[str, type[QuantizationConfig]] = {}


def _register(name: str):
    """Class decorator: ``QUANTIZATION_METHODS[name] = cls`` (reference
    ``registry.py:52-60``)."""

    def wrap(cls: type[QuantizationConfig]) -> type[QuantizationConfig]:
        cls.name = name
        QUANTIZATION_METHODS[name] = cls
        return cls

    return wrap


def _register_all() -> None:
    """Import the modules whose classes register themselves (lazily, so the
    format modules may import this one)."""
    from ccut.quant import compressed_tensors  # noqa: F401  (registers itself)


#: online quantization shorthands (reference ``registry.py:75-82``)
ONLINE_SHORTHANDS: dict[str, dict] = {
    "fp8_per_token": {"weight": "fp8_static_channel_sym", "act": "fp8_dynamic_token_sym", "compute": "w8a16"},
    "int8_per_token": {"weight": "int8_static_channel_sym", "act": "int8_dynamic_token_sym", "compute": "w8a16"},
    "int8_per_channel_weight_only": {"weight": "int8_static_channel_sym", "act": None, "compute": "w8a16"},
    "mxfp8": {"weight": "mxfp8_dynamic", "act": None, "compute": "w8a16"},
    "nvfp4_per_token": {"weight": "nvfp4_dynamic", "act": None, "compute": "w4a16"},
}


def list_supported_quant() -> list[str]:
    _register_all()
    return sorted(QUANTIZATION_METHODS)


def _compile_ignore(patterns) -> list[re.Pattern]:
    """``re:``-prefixed regexes (compressed-tensors convention) or plain
    regexes; matched with ``search``."""
    return [re.compile(p[3:] if p.startswith("re:") else p) for p in (patterns or [])]


class UnquantizedConfig(QuantizationConfig):
    """No ``quantization_config``: every layer passes through in BF16/FP16
    (reference ``registry.py:89-104``)."""

    name = "none"

    def __init__(self, weight_dtype: str = "bf16"):
        self.weight_dtype = weight_dtype

    @classmethod
    def from_config(cls, quant_cfg: dict, model_dir: str | Path | None = None) -> "UnquantizedConfig":
        return cls()

    def get_layer_spec(self, layer_name: str) -> LayerQuantSpec:
        key = QuantKey(QuantDType.BF16 if self.weight_dtype == "bf16" else QuantDType.FP16, name="unquant")
        return LayerQuantSpec(layer_name, key, skipped=True, quant_method="none")


def _skipped_spec(layer_name: str, method: str) -> LayerQuantSpec:
    return LayerQuantSpec(layer_name, get_quant_key(K_BF16), skipped=True, quant_method=method)


@_register("awq")
class AwqConfig(QuantizationConfig):
    """AutoAWQ GEMM checkpoints: ``{"quant_method": "awq", "bits": 4,
    "group_size": G, "zero_point": true, "version": "gemm",
    "modules_to_not_convert": [...]}``.  Linear layers (``*_proj``, ``.fc*``)
    get ``K_AWQ_W4A16`` with group G along the input dimension and the
    tensors ``<layer>.qweight`` (int32 [in, out/8]), ``<layer>.qzeros``
    (int32 [in/G, out/8]) and ``<layer>.scales`` (fp16 [in/G, out]); a layer
    whose name contains an entry of ``modules_to_not_convert`` (and the
    router ``mlp.gate``, embeddings, lm_head) passes through."""

    def __init__(self, group_size: int, not_convert: list[str], scale_dtype: str = "F16"):
        self.group_size = int(group_size)
        self.not_convert = list(not_convert)
        self.scale_dtype = scale_dtype
        self._specs: dict[str, LayerQuantSpec] = {}

    @classmethod
    def from_config(cls, quant_cfg: dict, model_dir: str | Path | None = None) -> "AwqConfig":
        bits = int(quant_cfg.get("bits", quant_cfg.get("w_bit", 4)))
        if bits != 4:
            raise ValueError(f"awq: {bits}-bit weights are not supported (4-bit only)")
        G = int(quant_cfg.get("group_size", quant_cfg.get("q_group_size", 128)))
        if G not in (32, 64, 128):
            raise ValueError(f"awq: group_size={G} not in (32, 64, 128)")
        if not quant_cfg.get("zero_point", True):
            raise ValueError("awq: symmetric (no zero point) checkpoints are not supported")
        version = str(quant_cfg.get("version", "gemm")).casefold()
        if version != "gemm":
            raise ValueError(f"awq: packing version {version!r} is not supported (GEMM packing only)")
        return cls(G, quant_cfg.get("modules_to_not_convert") or [])

    def is_layer_skipped(self, layer_name: str) -> bool:
        if any(m and m in layer_name for m in self.not_convert):
            return True
        tail = layer_name.rsplit(".", 1)[-1]
        return tail in ("lm_head", "embed_tokens", "gate") or not (tail.endswith("_proj") or tail.startswith("fc"))

    def get_layer_spec(self, layer_name: str) -> LayerQuantSpec:
        spec = self._specs.get(layer_name)
        if spec is not None:
            return spec
        if self.is_layer_skipped(layer_name):
            spec = _skipped_spec(layer_name, self.name)
        else:
            base = get_quant_key(K_AWQ_W4A16)
            key = QuantKey(base.weight_dtype, base.weight_scale, base.act_dtype, base.act_scale, base.symmetric,
                           GroupShape(rows=self.group_size), name=base.name)
            spec = LayerQuantSpec(layer_name, key,
                                  scales=(ScaleDesc(f"{layer_name}.scales", self.scale_dtype, ()),
                                          ScaleDesc(f"{layer_name}.qzeros", "I32", ())),
                                  quant_method=self.name)
        self._specs[layer_name] = spec
        return spec

    def validate(self) -> None:
        for name, spec in self._specs.items():
            if not spec.skipped and len(spec.scales) < 2:
                raise ValueError(f"awq layer {name} has no scales / zero points")


@_register("fp8")
class Fp8BlockConfig(QuantizationConfig):
    """FP8 checkpoints with 128x128 weight blocks: ``{"quant_method": "fp8",
    "fmt": "e4m3", "activation_scheme": "dynamic", "weight_block_size":
    [128, 128], "modules_to_not_convert": [...]}``.  Linear layers get
    ``K_FP8_BLOCK128`` with ``<layer>.weight`` (e4m3 [out, in]) and
    ``<layer>.weight_scale_inv`` (float32 [out/128, in/128]); activations are
    quantized per token per 128 at run time.  Without ``weight_block_size``
    (per-tensor FP8) the config raises ``NotImplementedError``, as the
    reference's ``Fp8Config.from_config`` does (``quant/fp8.py:37-51``)."""

    def __init__(self, not_convert: list[str]):
        self.not_convert = list(not_convert)
        self._specs: dict[str, LayerQuantSpec] = {}

    @classmethod
    def from_config(cls, quant_cfg: dict, model_dir: str | Path | None = None) -> "Fp8BlockConfig":
        block = quant_cfg.get("weight_block_size")
        if block is None:
            raise NotImplementedError("fp8 checkpoints without weight_block_size (per-tensor FP8) are not parsed; "
                                      "use compressed-tensors or 128x128 block FP8")
        if list(block) != [128, 128]:
            raise ValueError(f"fp8: weight_block_size={list(block)} (128x128 blocks only)")
        fmt = str(quant_cfg.get("fmt", "e4m3")).casefold()
        if fmt != "e4m3":
            raise ValueError(f"fp8: fmt={fmt!r} (e4m3 only)")
        if str(quant_cfg.get("activation_scheme", "dynamic")).casefold() != "dynamic":
            raise ValueError("fp8: static activation scales are not supported (dynamic per-token-per-128 only)")
        return cls(quant_cfg.get("modules_to_not_convert") or quant_cfg.get("ignored_layers") or [])

    def is_layer_skipped(self, layer_name: str) -> bool:
        if any(m and m in layer_name for m in self.not_convert):
            return True
        tail = layer_name.rsplit(".", 1)[-1]
        return tail in ("lm_head", "embed_tokens", "gate") or not (tail.endswith("_proj") or tail.startswith("fc"))

    def get_layer_spec(self, layer_name: str) -> LayerQuantSpec:
        spec = self._specs.get(layer_name)
        if spec is None:
            spec = (_skipped_spec(layer_name, self.name) if self.is_layer_skipped(layer_name) else
                    LayerQuantSpec(layer_name, get_quant_key(K_FP8_BLOCK128),
                                   scales=(ScaleDesc(f"{layer_name}.weight_scale_inv", "F32", ()),),
                                   quant_method=self.name))
            self._specs[layer_name] = spec
        return spec


def resolve_checkpoint_quant(model_dir: str | Path, online_quantization: str | None = None,
                             quant_ignore: list[str] | None = None) -> QuantizationConfig:
    """A checkpoint's ``QuantizationConfig`` (reference ``registry.py:108-154``):

    * no ``quantization_config`` (top level or under ``text_config``) and no
      online shorthand -> :class:`UnquantizedConfig`;
    * a ``quantization_config`` -> the registered class of its
      ``quant_method``; unregistered -> ``ValueError`` naming the supported
      ones;
    * ``online_quantization`` (a key of ``ONLINE_SHORTHANDS``; "auto",
      "none" and "" mean none) -> ``OnlineQuantConfig``; together with a
      checkpoint ``quantization_config`` -> ``ValueError`` (they exclude
      each other); an unknown shorthand -> ``ValueError``.
    ``FileNotFoundError`` when ``config.json`` is missing."""
    model_dir = Path(model_dir)
    cfg_path = model_dir / "config.json"
    if not cfg_path.exists():
        raise FileNotFoundError(f"{cfg_path}: no config.json")
    cfg = json.loads(cfg_path.read_bytes())
    text_cfg = cfg.get("text_config", cfg)
    quant_cfg = text_cfg.get("quantization_config") or cfg.get("quantization_config")

    online = (online_quantization or "auto").casefold()
    if online in ("auto", "none", ""):
        online = None
    if online is not None:
        if online not in ONLINE_SHORTHANDS:
            raise ValueError(f"unknown online quantization shorthand {online!r}; choices: "
                             f"{sorted(ONLINE_SHORTHANDS)}")
        if quant_cfg:
            raise ValueError(f"online quantization ({online}) and the checkpoint's own quantization "
                             f"({quant_cfg.get('quant_method')}) exclude each other; set only one")
        from ccut.quant.online import OnlineQuantConfig

        return OnlineQuantConfig.from_config(ONLINE_SHORTHANDS[online], model_dir, ignore_patterns=quant_ignore)
    if not quant_cfg:
        return UnquantizedConfig()
    _register_all()
    method = quant_cfg.get("quant_method", "")
    cls = QUANTIZATION_METHODS.get(method)
    if cls is None:
        raise ValueError(f"checkpoint quantization format {method!r} is not registered; supported: "
                         f"{list_supported_quant()}")
    return cls.from_config(quant_cfg, model_dir)


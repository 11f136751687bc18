"""Declarative quantization specs (same names, fields and semantics as the
reference's ``python/ccut/quant/spec.py:29-194``).

A layer's weight layout is described by data -- ``QuantKey`` (dtype, scale
strategy, symmetry, group shape) inside a ``LayerQuantSpec`` -- and the
method layer dispatches on it.  Two keys are added for the formats the GPU
path serves: AWQ int4 with zero points and 128-row groups, and FP8 e4m3 with
128x128 block scales and per-token-per-128 dynamic activations.
"""

from __future__ import annotations

from dataclasses import dataclass, field

__all__ = [
    "QuantDType",
    "ScaleStrategy",
    "GroupShape",
    "QuantKey",
    "ScaleDesc",
    "LayerQuantSpec",
    "get_quant_key",
    "K_BF16",
    "K_FP8_DYNAMIC_TOKEN_SYM",
    "K_FP8_STATIC_CHANNEL_SYM",
    "K_FP8_STATIC_TENSOR_SYM",
    "K_INT8_STATIC_CHANNEL_SYM",
    "K_INT8_DYNAMIC_TOKEN_SYM",
    "K_INT8_W4A16_SYM",
    "K_NF4_W4A16",
    "K_MXFP8_DYNAMIC",
    "K_MXFP4_DYNAMIC",
    "K_NVFP4_DYNAMIC",
    "K_AWQ_W4A16",
    "K_FP8_BLOCK128",
]


class QuantDType:
    """Stored element type (reference ``spec.py:29-44``)."""

    BF16 = "bf16"
    FP16 = "fp16"
    FP32 = "fp32"
    INT8 = "int8"
    FP8_E4M3 = "fp8_e4m3"
    FP8_E5M2 = "fp8_e5m2"
    INT4 = "int4"
    NF4 = "nf4"
    MXFP8 = "mxfp8"
    MXFP4 = "mxfp4"
    NVFP4 = "nvfp4"

    ALL = (BF16, FP16, FP32, INT8, FP8_E4M3, FP8_E5M2, INT4, NF4, MXFP8, MXFP4, NVFP4)


class ScaleStrategy:
    """Scale granularity (reference ``spec.py:47-54``)."""

    PER_TENSOR = "tensor"
    PER_CHANNEL = "channel"
    PER_TOKEN = "token"
    PER_GROUP = "group"
    NO_SCALE = "none"


@dataclass(frozen=True)
class GroupShape:
    """Group size along the input dim (``rows``) and, for block scales, along
    the output dim (``cols``).  Reference ``spec.py:57-69``."""

    rows: int | None = None
    cols: int | None = None

    def is_grouped(self) -> bool:
        return bool(self.rows) and self.rows > 0

    @property
    def group_size(self) -> int:
        return self.rows or 0

    def is_block(self) -> bool:
        return self.is_grouped() and bool(self.cols) and self.cols > 0


K_FP8_DYNAMIC_TOKEN_SYM = "fp8_dynamic_token_sym"
K_FP8_STATIC_CHANNEL_SYM = "fp8_static_channel_sym"
K_FP8_STATIC_TENSOR_SYM = "fp8_static_tensor_sym"
K_INT8_STATIC_CHANNEL_SYM = "int8_static_channel_sym"
K_INT8_DYNAMIC_TOKEN_SYM = "int8_dynamic_token_sym"
K_INT8_W4A16_SYM = "int4_w4a16_sym"
K_NF4_W4A16 = "nf4_w4a16"
K_MXFP8_DYNAMIC = "mxfp8_dynamic"
K_MXFP4_DYNAMIC = "mxfp4_dynamic"
K_NVFP4_DYNAMIC = "nvfp4_dynamic"
K_BF16 = "bf16"
K_AWQ_W4A16 = "int4_awq_w4a16"
K_FP8_BLOCK128 = "fp8_block128_dynamic_group"


@dataclass(frozen=True)
class QuantKey:
    """Weight/activation quantization of one layer (reference ``spec.py:101-136``)."""

    weight_dtype: str = QuantDType.BF16
    weight_scale: str = ScaleStrategy.NO_SCALE
    act_dtype: str = QuantDType.BF16
    act_scale: str = ScaleStrategy.NO_SCALE
    symmetric: bool = True
    group_shape: GroupShape = field(default_factory=GroupShape)
    name: str = ""

    def is_quantized(self) -> bool:
        return self.weight_scale != ScaleStrategy.NO_SCALE

    def is_weight_only(self) -> bool:
        return self.is_quantized() and self.act_scale == ScaleStrategy.NO_SCALE

    def is_w8a8(self) -> bool:
        return self.is_quantized() and self.act_scale != ScaleStrategy.NO_SCALE

    def compute_path(self) -> str:
        """``bf16`` / ``w8a16`` / ``w8a8`` / ``w4a16`` (reference ``spec.py:130-136``)."""
        if not self.is_quantized():
            return "bf16"
        if self.is_weight_only():
            return "w4a16" if self.weight_dtype in (QuantDType.INT4, QuantDType.NF4) else "w8a16"
        return "w8a8"

    # formats served by the GPU kernels ------------------------------------
    def is_awq(self) -> bool:
        """int4 with 4-bit zero points and groups along K (AWQ GEMM packing)."""
        return (self.weight_dtype == QuantDType.INT4 and self.weight_scale == ScaleStrategy.PER_GROUP
                and not self.symmetric and self.group_shape.is_grouped())

    def is_fp8_block(self) -> bool:
        """FP8 e4m3 weights with 2-D block scales."""
        return self.weight_dtype == QuantDType.FP8_E4M3 and self.group_shape.is_block()


_KEY_REGISTRY: dict[str, QuantKey] = {}


def _reg(name: str, key: QuantKey) -> QuantKey:
    _KEY_REGISTRY[name] = key
    return key


def get_quant_key(name: str) -> QuantKey:
    """Predefined key by name, case-insensitive; ``KeyError`` when unknown
    (reference ``spec.py:93-98``)."""
    key = _KEY_REGISTRY.get(name.casefold())
    if key is None:
        raise KeyError(f"unknown QuantKey {name!r}; registered: {sorted(_KEY_REGISTRY)}")
    return key


_D, _S = QuantDType, ScaleStrategy
_reg(K_BF16, QuantKey(_D.BF16, _S.NO_SCALE, _D.BF16, _S.NO_SCALE, True))
_reg(K_FP8_DYNAMIC_TOKEN_SYM, QuantKey(_D.FP8_E4M3, _S.PER_CHANNEL, _D.FP32, _S.PER_TOKEN, True))
_reg(K_FP8_STATIC_CHANNEL_SYM, QuantKey(_D.FP8_E4M3, _S.PER_CHANNEL, _D.FP32, _S.PER_TOKEN, True))
_reg(K_FP8_STATIC_TENSOR_SYM, QuantKey(_D.FP8_E4M3, _S.PER_TENSOR, _D.FP32, _S.PER_TOKEN, True))
_reg(K_INT8_STATIC_CHANNEL_SYM, QuantKey(_D.INT8, _S.PER_CHANNEL, _D.FP32, _S.PER_TOKEN, True))
_reg(K_INT8_DYNAMIC_TOKEN_SYM, QuantKey(_D.INT8, _S.PER_CHANNEL, _D.FP32, _S.PER_TOKEN, True))
_reg(K_INT8_W4A16_SYM, QuantKey(_D.INT4, _S.PER_CHANNEL, _D.FP32, _S.NO_SCALE, True))
_reg(K_NF4_W4A16, QuantKey(_D.NF4, _S.PER_CHANNEL, _D.FP16, _S.NO_SCALE, True))
_reg(K_MXFP8_DYNAMIC, QuantKey(_D.MXFP8, _S.PER_GROUP, _D.BF16, _S.PER_TOKEN, False, GroupShape(rows=32)))
_reg(K_MXFP4_DYNAMIC, QuantKey(_D.MXFP4, _S.PER_GROUP, _D.BF16, _S.PER_TOKEN, False, GroupShape(rows=32)))
_reg(K_NVFP4_DYNAMIC, QuantKey(_D.NVFP4, _S.PER_GROUP, _D.BF16, _S.PER_TOKEN, False, GroupShape(rows=16)))
_reg(K_AWQ_W4A16, QuantKey(_D.INT4, _S.PER_GROUP, _D.FP16, _S.NO_SCALE, False, GroupShape(rows=128),
                           name=K_AWQ_W4A16))
_reg(K_FP8_BLOCK128, QuantKey(_D.FP8_E4M3, _S.PER_GROUP, _D.FP8_E4M3, _S.PER_GROUP, True,
                              GroupShape(rows=128, cols=128), name=K_FP8_BLOCK128))


@dataclass(frozen=True)
class ScaleDesc:
    """Layout of one scale tensor (reference ``spec.py:152-164``)."""

    name: str
    dtype: str
    shape: tuple[int, ...]
    offset: int = 0
    length: int = 0

    def is_e8m0(self) -> bool:
        return self.dtype.upper() in ("U8", "F8_E8M0")


@dataclass(frozen=True)
class LayerQuantSpec:
    """Full quantization spec of one layer (reference ``spec.py:167-194``)."""

    layer_name: str
    weight_key: QuantKey
    activation_key: QuantKey | None = None
    scales: tuple[ScaleDesc, ...] = ()
    skipped: bool = False
    quant_method: str = ""

    def effective_key(self) -> QuantKey:
        """The activation key overrides the act side of the weight key."""
        if self.skipped or self.activation_key is None:
            return self.weight_key
        return QuantKey(
            weight_dtype=self.weight_key.weight_dtype,
            weight_scale=self.weight_key.weight_scale,
            act_dtype=self.activation_key.weight_dtype,
            act_scale=self.activation_key.weight_scale,
            symmetric=self.weight_key.symmetric,
            group_shape=self.weight_key.group_shape,
            name=self.weight_key.name,
        )

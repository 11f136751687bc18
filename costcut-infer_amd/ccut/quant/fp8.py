"""FP8 Linear method (reference ``python/ccut/quant/fp8.py:19-51``).

Per-channel FP8 (the reference's format: ``[out, in]`` e4m3fn bytes, one
scale per output row) runs the W8A16 float32 path; 128x128 block-scaled FP8
(``QuantKey.is_fp8_block()``) runs the FP8 MFMA path with per-token-per-128
dynamic activation quantization (``ccut.quant.fp8_block``).
"""

from __future__ import annotations

from ccut.quant.method import LinearMethod, QuantizeMethodBase
from ccut.quant.spec import LayerQuantSpec

__all__ = ["Fp8LinearMethod", "Fp8Config"]


class Fp8LinearMethod(QuantizeMethodBase):
    """Reads FP8 bytes + scales, multiplies on the GPU."""

    def __init__(self, spec: LayerQuantSpec, compute_mode: str = "w8a16"):
        self.spec = spec
        self.compute_mode = compute_mode.casefold()
        key = spec.effective_key()
        self.is_block = key.is_fp8_block()
        if self.is_block:
            self.compute_path = "w8a8"
        else:
            self.compute_path = "w8a8" if self.compute_mode == "w8a8" else "w8a16"
        self.scale_name = spec.scales[0].name if spec.scales else None
        self._inner = LinearMethod(key, scale_name=self.scale_name, compute_mode=self.compute_mode)

    def create_weights(self, spec: LayerQuantSpec) -> None:
        super().create_weights(spec)

    def apply(self, weight_bytes, scales: dict, x):
        if self.is_block:
            from ccut.quant import fp8_block

            scale = scales.get(self.scale_name) if self.scale_name else None
            if scale is None:
                raise ValueError(f"FP8 block layer is missing its scale tensor ({self.scale_name})")
            return fp8_block.linear(weight_bytes, scale, x)
        return self._inner.apply(weight_bytes, scales, x)


class Fp8Config:
    """Bare ``quant_method="fp8"`` checkpoints (reference ``fp8.py:37-51``):
    the 128x128 block form is parsed by ``ccut.quant.registry.Fp8BlockConfig``
    (registered as "fp8"); any other form raises, as the reference's does."""

    name = "fp8"

    @classmethod
    def from_config(cls, quant_cfg: dict, model_dir=None):
        from ccut.quant.registry import Fp8BlockConfig

        return Fp8BlockConfig.from_config(quant_cfg, model_dir)

    def get_layer_spec(self, layer_name: str):
        raise NotImplementedError

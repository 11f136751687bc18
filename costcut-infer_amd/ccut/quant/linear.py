"""Model-side linear projections over a weight reader: ``WeightReader`` /
``FakeWeightReader`` (reference ``python/ccut/models/generic.py:48-91``),
``LinearProj`` (``:99-176``) and ``build_linear_projs`` (``:220-231``).

A ``LinearProj`` is one projection (layer, tensor name, ``[out, in]``) whose
bytes come from a reader; ``apply(x [batch, in]) -> [batch, out]`` computes
``x @ W.T`` with ``W`` the dequantized weight.  The reference dequantizes
``W`` to float32 on first use and caches that matrix per (layer, proj).
Here the first use uploads the projection's bytes and scales to HBM once and
keeps them quantized; ``apply`` runs the layer's quantized method on them
(``make_method_for_spec``: e4m3 per row -> ``ccq_fp8_linear_f32`` / the
decoded-weight MFMA kernel, int8 -> ``ccq_int8_linear_f32``, AWQ ->
``ccq_w4_gemm``, block FP8, MX), so a call reads the weight's own bytes
instead of 4 bytes per weight.  Unquantized (BF16 / F16 / F32) projections
are widened to float32 once and multiplied on ``ccq_f32_gemm``.
``dequant_weight()`` returns the float32 ``[out, in]`` matrix (a device
tensor, cached), as the reference's does.

Differences from the reference, on purpose: it keys the scales it reads by
the last component of the spec's scale names and then picks one by its
length (``generic.py:146-151,207-217``); here the scale tensors a spec names
are handed to the method under those names (a reader's ``scales`` may return
one array -- the weight scale -- or a dict of named arrays, for formats with
several, such as AWQ's scales and zero points).
"""

from __future__ import annotations

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call
from ccut.quant.method import _f32_input, _return, _unpack_weight, f32_linear, make_method_for_spec
from ccut.quant.spec import LayerQuantSpec, QuantDType

__all__ = ["WeightReader", "FakeWeightReader", "LinearProj", "build_linear_projs"]

_FLOAT_DTYPES = {"BF16": QuantDType.BF16, "F16": QuantDType.FP16, "F32": QuantDType.FP32,
                 QuantDType.BF16: QuantDType.BF16, QuantDType.FP16: QuantDType.FP16, QuantDType.FP32: QuantDType.FP32}


class WeightReader:
    """Source of projection bytes (reference ``generic.py:48-72``):
    ``segment(layer, key) -> bytes`` (the raw tensor in its stored dtype),
    ``shape(layer, key) -> (rows, cols, dtype)``, ``scales(layer, key)`` ->
    the scale array (or a dict of named arrays), None when unquantized."""

    def segment(self, layer: int, tensor_key: str) -> bytes:
        raise NotImplementedError

    def shape(self, layer: int, tensor_key: str) -> tuple[int, int, str]:
        raise NotImplementedError

    def scales(self, layer: int, tensor_key: str):
        return None


class FakeWeightReader(WeightReader):
    """Resident tables (reference ``generic.py:75-91``): ``table[(layer,
    key)]`` bytes, ``shapes[(layer, key)]``; a projection's scale is the F32
    bytes under ``key + ".weight_scale"``."""

    def __init__(self, table: dict, shapes: dict):
        self._table = table
        self._shapes = shapes

    def segment(self, layer: int, tensor_key: str) -> bytes:
        return self._table[(layer, tensor_key)]

    def shape(self, layer: int, tensor_key: str) -> tuple[int, int, str]:
        return self._shapes[(layer, tensor_key)]

    def scales(self, layer: int, tensor_key: str):
        raw = self._table.get((layer, tensor_key + ".weight_scale"))
        return None if raw is None else np.frombuffer(raw, dtype=np.float32)


class LinearProj:
    """One projection of a layer: ``apply(x) = x @ W.T`` on the GPU."""

    def __init__(self, layer: int, name: str, out_dim: int, in_dim: int, reader: WeightReader, quant_cfg):
        self.layer = layer
        self.name = name
        self.out_dim = out_dim
        self.in_dim = in_dim
        self.reader = reader
        self.quant_cfg = quant_cfg
        self._loaded = False
        self._spec: LayerQuantSpec | None = None
        self._method = None
        self._raw: torch.Tensor | None = None
        self._scales: dict = {}
        self._w32: torch.Tensor | None = None  # float32 [out, in]: unquantized weights, or dequant_weight()

    # ---- one upload per projection ----
    def _load(self) -> None:
        if self._loaded:
            return
        spec = self.quant_cfg.get_layer_spec(self.name) if self.quant_cfg is not None else None
        raw = _dev.raw_u8(self.reader.segment(self.layer, self.name))
        if spec is None or spec.skipped:
            dtype = self._stored_float_dtype(spec)
            w = _unpack_weight(raw, dtype)
            if w.numel() != self.out_dim * self.in_dim:
                raise ValueError(f"{self.name}: {w.numel()} weights for [{self.out_dim}, {self.in_dim}]")
            self._w32 = w.reshape(self.out_dim, self.in_dim).contiguous()
        else:
            method = make_method_for_spec(spec)
            method.create_weights(spec)
            got = self.reader.scales(self.layer, self.name)
            if isinstance(got, dict):
                by_suffix = {k.rsplit(".", 1)[-1]: v for k, v in got.items()}
                scales = {}
                for sd in spec.scales:
                    v = got.get(sd.name, by_suffix.get(sd.name.rsplit(".", 1)[-1]))
                    if v is not None:
                        scales[sd.name] = v
            elif got is not None and spec.scales:
                scales = {spec.scales[0].name: got}
            else:
                scales = {}
            if spec.scales and spec.scales[0].name not in scales:
                raise ValueError(f"{self.name}: quantized projection without its scale tensor "
                                 f"({spec.scales[0].name})")
            self._scales = {k: _dev.to_device(v) if not isinstance(v, torch.Tensor) else v.to(raw.device)
                            for k, v in scales.items()}
            self._raw = raw
            self._method = method
            self._spec = spec
        self._loaded = True

    def _stored_float_dtype(self, spec) -> str:
        try:
            dt = self.reader.shape(self.layer, self.name)[2]
        except (NotImplementedError, KeyError):
            dt = None
        if dt is None and spec is not None:
            dt = spec.effective_key().weight_dtype
        return _FLOAT_DTYPES.get(dt, QuantDType.BF16)

    # ---- reference API ----
    def dequant_weight(self) -> torch.Tensor:
        """``W`` as float32 ``[out, in]`` on the device (cached)."""
        self._load()
        if self._w32 is not None:
            return self._w32
        key = self._spec.effective_key()
        wd = key.weight_dtype
        scale = self._scales.get(self._spec.scales[0].name) if self._spec.scales else None
        if wd == QuantDType.FP8_E4M3 and not key.is_fp8_block():
            s = scale.float().reshape(-1).contiguous()
            w = torch.empty((self.out_dim, self.in_dim), dtype=torch.float32, device=self._raw.device)
            call("ccq_fp8_dequant", self._raw.data_ptr(), s.data_ptr(), w.data_ptr(), self.out_dim, self.in_dim,
                 _dev.stream_ptr(self._raw.device))
        elif wd == QuantDType.FP8_E4M3:
            from ccut.quant import fp8_block

            w = fp8_block.dequant(self._raw.reshape(self.out_dim, self.in_dim), scale.float())
        elif wd == QuantDType.INT8:
            from ccut.quant import kernels as qk

            w = torch.empty((self.out_dim, self.in_dim), dtype=torch.float32, device=self._raw.device)
            qk.int8_dequant_row(self._raw.view(torch.int8).reshape(self.out_dim, self.in_dim),
                                scale.float().reshape(-1), w)
        elif key.is_awq():
            from ccut.quant import awq

            zeros = self._scales.get(self._spec.scales[1].name) if len(self._spec.scales) > 1 else None
            w = awq.dequant(self._raw.view(torch.int32).reshape(self.in_dim, self.out_dim // 8), zeros, scale,
                            self.in_dim // scale.shape[0]).float().T.contiguous()
        else:
            raise NotImplementedError(f"{self.name}: dequant_weight for {wd}")
        self._w32 = w
        return w

    def apply(self, x):
        """``x [batch, in] @ W.T -> [batch, out]`` float32 (numpy in, numpy
        out; a device tensor in, a device tensor out)."""
        self._load()
        if self._method is None:
            return _return(f32_linear(_f32_input(x), self._w32), x)
        return self._method.apply(self._raw, self._scales, x)


def build_linear_projs(layer: int, reader: WeightReader, quant_cfg, prefix: str,
                       names: dict[str, tuple[int, int]]) -> dict[str, LinearProj]:
    """``names = {"gate_proj": (out, in), ...}`` -> ``LinearProj`` per tensor
    ``{prefix}{name}`` (reference ``generic.py:220-231``)."""
    return {n: LinearProj(layer, f"{prefix}{n}", o, i, reader, quant_cfg) for n, (o, i) in names.items()}

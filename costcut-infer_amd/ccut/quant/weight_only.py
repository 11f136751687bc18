"""W4 weight-only methods on the GPU (reference ``python/ccut/quant/
weight_only.py:24-54``).

Two int4 layouts sit behind the same ``apply(weight_bytes, scales, x)``:

* the reference's own int4 (``QuantKey`` ``int4_w4a16_sym``): signed nibbles,
  low nibble first, one float32 scale per input column, ``[out, in/2]`` bytes
  -- float32 in and out, the reference's numbers;
* AWQ (``QuantKey.is_awq()``): ``weight_bytes`` is ``qweight`` int32
  ``[K, N/8]`` (or an :class:`~ccut.quant.awq.AwqWeights` already prepared),
  ``scales`` holds the per-group scales and the packed zero points under the
  spec's scale names (``<layer>.scales``, ``<layer>.zero_points`` as named by
  ``quant/compressed_tensors.py:209-211``; ``qzeros``/``scales`` accepted too).
"""

from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call
from ccut.quant import awq
from ccut.quant.method import QuantizeMethodBase, _f32_input, _return
from ccut.quant.spec import LayerQuantSpec, QuantDType

__all__ = ["WeightOnlyMethod", "int4_linear_f32", "nf4_linear_f32", "NF4_LUT"]

# The reference's NF4 table (weight_only.py:18-21, kernels.py:299-302): eight
# values, indexed by the 4-bit code; codes 8..15 fall past it (NaN here).
NF4_LUT = np.array([-1.0, -0.6961928, -0.39238566, -0.08857854, 0.21522858, 0.51903564, 0.8228427, 1.1266499],
                   dtype=np.float32)


def nf4_linear_f32(weight_bytes, scale, x, table=NF4_LUT):
    """``x @ nf4_dequant(W).T`` in float32 (reference ``weight_only.py:47-54``,
    the NF4 branch): the int4 layout with the code looked up in ``table``."""
    xd = _f32_input(x)
    batch, in_f = xd.shape
    if in_f % 2:
        raise ValueError(f"nf4 weight-only needs an even in_features, got {in_f}")
    raw = _dev.raw_u8(weight_bytes)
    if raw.numel() % (in_f // 2):
        raise ValueError(f"nf4 weight of {raw.numel()} bytes is not a multiple of in_features/2={in_f // 2}")
    out_f = raw.numel() // (in_f // 2)
    s = _dev.to_device(np.asarray(scale, dtype=np.float32) if not isinstance(scale, torch.Tensor) else scale,
                       torch.float32).reshape(-1)
    if s.numel() != in_f:
        raise ValueError(f"nf4 scale has {s.numel()} entries, expected one per input column ({in_f})")
    tb = _dev.to_device(np.asarray(table, np.float32)).reshape(-1)
    if tb.numel() > 16:
        raise ValueError(f"NF4 table has {tb.numel()} entries (at most 16)")
    y = torch.empty((batch, out_f), dtype=torch.float32, device=xd.device)
    call("ccq_nf4_linear_f32", xd.data_ptr(), raw.data_ptr(), s.data_ptr(), tb.data_ptr(), tb.numel(), y.data_ptr(),
         batch, in_f, out_f, _dev.stream_ptr())
    return _return(y, x)


def int4_linear_f32(weight_bytes, scale, x):
    """``x @ int4_dequant(W).T`` in float32 (reference ``weight_only.py:47-54``)."""
    xd = _f32_input(x)
    batch, in_f = xd.shape
    if in_f % 2:
        raise ValueError(f"int4 weight-only needs an even in_features, got {in_f}")
    raw = _dev.raw_u8(weight_bytes)
    if raw.numel() % (in_f // 2):
        raise ValueError(f"int4 weight of {raw.numel()} bytes is not a multiple of in_features/2={in_f // 2}")
    out_f = raw.numel() // (in_f // 2)
    s = _dev.to_device(np.asarray(scale, dtype=np.float32) if not isinstance(scale, torch.Tensor) else scale,
                       torch.float32).reshape(-1)
    if s.numel() != in_f:
        raise ValueError(f"int4 scale has {s.numel()} entries, expected one per input column ({in_f})")
    y = torch.empty((batch, out_f), dtype=torch.float32, device=xd.device)
    call("ccq_int4_linear_f32", xd.data_ptr(), raw.data_ptr(), s.data_ptr(), y.data_ptr(), batch, in_f, out_f,
         _dev.stream_ptr())
    return _return(y, x)


def _lookup(scales: dict, names: tuple[str, ...]):
    for n in names:
        if n in scales and scales[n] is not None:
            return scales[n]
    return None


class WeightOnlyMethod(QuantizeMethodBase):
    """W4A16: dequant fused into the GPU GEMM."""

    compute_path = "w4a16"
    _CACHE_SIZE = 16

    def __init__(self, spec: LayerQuantSpec):
        self.spec = spec
        key = spec.effective_key()
        self.weight_dtype = key.weight_dtype
        self.is_awq = key.is_awq()
        self.group_size = key.group_shape.group_size or 128
        self.scale_name = spec.scales[0].name if spec.scales else None
        self.zero_name = spec.scales[1].name if len(spec.scales) > 1 else None
        self._prepared: OrderedDict = OrderedDict()

    def create_weights(self, spec: LayerQuantSpec) -> None:
        QuantizeMethodBase.create_weights(self, spec)

    # AWQ ---------------------------------------------------------------
    def prepare(self, weight_bytes, scales: dict) -> awq.AwqWeights:
        """Upload + re-pack once (the load-time step the reference's
        ``process_weights_after_loading`` hook stands for)."""
        if isinstance(weight_bytes, awq.AwqWeights):
            return weight_bytes
        key = (id(weight_bytes), id(scales.get(self.scale_name)) if self.scale_name else None)
        hit = self._prepared.get(key)
        if hit is not None and hit[0] is weight_bytes:
            self._prepared.move_to_end(key)
            return hit[1]
        s = _lookup(scales, (self.scale_name, "scales") if self.scale_name else ("scales",))
        z = _lookup(scales, (self.zero_name, "zero_points", "qzeros") if self.zero_name else ("zero_points", "qzeros"))
        if s is None or z is None:
            raise ValueError(f"AWQ layer needs scales and zero points (got keys {sorted(scales)})")
        w = awq.prepare(weight_bytes, z, s, self.group_size)
        self._prepared[key] = (weight_bytes, w)
        while len(self._prepared) > self._CACHE_SIZE:
            self._prepared.popitem(last=False)
        return w

    def apply(self, weight_bytes, scales: dict, x):
        if self.is_awq:
            w = self.prepare(weight_bytes, scales)
            if isinstance(x, torch.Tensor) and x.is_cuda and x.dtype in (torch.float16, torch.bfloat16):
                return awq.gemm(x, w)
            # float32 / host activations, float32 out: the MFMA takes them
            # as float16 (11 significant bits) when every |x| fits its
            # range, else as bfloat16 (8 bits, float32's range); the sums
            # and the output stay float32, so nothing else can overflow
            xd = _dev.to_device(x, torch.float32)
            xdt = _dev.half_for_mfma(xd, x if _dev.is_host(x) else None)
            y = awq.gemm(xd.to(xdt), w, out_dtype=torch.float32)
            return _return(y, x)
        if self.weight_dtype == QuantDType.INT4:
            scale = scales.get(self.scale_name) if self.scale_name else None
            if scale is None:
                raise ValueError(f"W4 layer is missing its scale tensor ({self.scale_name})")
            return int4_linear_f32(weight_bytes, scale, x)
        if self.weight_dtype == QuantDType.NF4:
            scale = scales.get(self.scale_name) if self.scale_name else None
            if scale is None:
                raise ValueError(f"W4 layer is missing its scale tensor ({self.scale_name})")
            return nf4_linear_f32(weight_bytes, scale, x)
        raise ValueError(f"weight-only does not support {self.weight_dtype}")

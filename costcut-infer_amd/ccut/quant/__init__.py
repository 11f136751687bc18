"""Quantized Linear operator API on the GPU (mirrors the reference's
``ccut.quant``: spec, method, weight_only, fp8, kernels, registry) plus the
AWQ and FP8-block formats."""

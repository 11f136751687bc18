"""ccut -- MI355X (gfx950) implementation of CostCut-Infer's quantized
expert-matmul path behind the reference's operator API
(``ccut.quant.*`` methods, ``ccut.blocks.moe``).

The compute runs in ``libccq_hip.so`` (hand-written HIP for CDNA4, C ABI in
``include/ccq.h``); torch provides device memory and streams.
"""

__version__ = "0.1.0"

"""MoE routing / expert FFN blocks on the GPU (mirrors ``ccut.blocks.moe``)."""

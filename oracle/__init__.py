"""CPU oracle for the quantized expert-matmul path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithms of CostCut-Infer's quantized
Linear / MoE expert path (reference ``python/ccut/quant/kernels.py``,
``quant/weight_only.py``, ``quant/method.py``, ``blocks/moe.py``) and of the two
public formats the reference does not implement (AWQ int4 GEMM packing, FP8
e4m3 with 128x128 block scales).  Every function cites the reference file:line
(or the public format) it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(``costcut-infer_amd/ccut``) never imports it: the product runs on the GPU
through ``libccq_hip.so`` and raises when that library is missing.

Pinning (what makes each function trustworthy, see ``tests/test_oracle_*.py``):

* ``ref_quant.fp8_e4m3_to_float32``  exhaustive 256-code table vs
  ``torch.float8_e4m3fn`` + the reference's own round-trip test
  (reference ``python/tests/test_quant.py:30``).
* ``ref_quant.float32_to_fp8_e4m3``  brute force against the nearest-value
  search over the 256-code table with the reference's half-up tie rule;
  saturation / NaN / subnormal special cases.
* ``ref_quant.int4_dequant_row`` / ``weight_only_apply``  re-hosts the
  reference's known-answer test ``python/tests/test_quant.py:115`` with the same
  torch seed and its explicit per-byte loop.
* ``ref_quant.fp8_dequant_mat``  closed form vs the exhaustive table.
* ``ref_quant.silu_mul_fused``  closed form vs ``torch.nn.functional.silu``.
* ``moe.topk``  brute force (``np.argsort(kind="stable")``) + the
  reference's invariants ``python/tests/test_blocks.py:127``.
* ``moe.topk_softmax``  numpy float32 semantics of ``blocks/moe.py:71-89``
  (the same library the reference runs), invariants of test_blocks.py:127.
* ``moe.moe_combine`` / ``moe.expert_order``  brute-force dict restatement of
  ``blocks/moe.py:163-173`` on tiny inputs.
* ``awq.*``  parity unpinned by the reference (AWQ is absent there); pinned by
  the public AutoAWQ GEMM packing definition: pack/unpack round trip over
  random words, per-nibble brute force, exactness of (q-z)*s in fp32.
* ``fp8_block.*``  parity unpinned by the reference (128x128 block FP8 is
  absent there); pinned by torch's RNE ``.to(torch.float8_e4m3fn)`` as the
  library routine and the |q| <= 448 / dequant round-trip invariants.
"""

"""The C ABI (include/ccq.h): the library loads, exports every declared
symbol, binds every signature, and rejects bad arguments on the host before
touching a GPU (no device is needed for any call in this file)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ccq.h"


def declared() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(ccq_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_path():
    names = declared()
    for must in ("ccq_w4_gemm", "ccq_awq_repack", "ccq_awq_pack_sz", "ccq_awq_dequant", "ccq_topk_softmax", "ccq_moe_align",
                 "ccq_moe_w4_ffn", "ccq_int4_linear_f32", "ccq_fp8_linear_f32", "ccq_f32_to_fp8"):
        assert must in names


def test_library_exports_every_declared_symbol(built_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(built_lib)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (ccq_\w+)", out))
    missing = declared() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_ctypes_binding_covers_header(built_lib):
    from ccut import _lib

    assert set(_lib.SIGNATURES) == declared()
    lib = _lib.lib()
    assert lib.ccq_version() >= 100
    assert isinstance(_lib.last_error(), str)


@pytest.fixture(scope="module")
def lib(built_lib):
    from ccut import _lib

    return _lib.lib()


def test_w4_gemm_rejects_bad_shapes(lib):
    from ccut._lib import CCQ_BF16, CCQ_EINVAL, CCQ_F16, last_error

    p = ctypes.c_void_p(16)  # never dereferenced: validation comes first
    rc = lib.ccq_w4_gemm(p, CCQ_F16, p, p, CCQ_F16, p, CCQ_F16, 1, 100, 64, 128, None, 0, None)
    assert rc == CCQ_EINVAL and "K % 128" in last_error()
    rc = lib.ccq_w4_gemm(p, CCQ_F16, p, p, CCQ_F16, p, CCQ_F16, 1, 256, 64, 96, None, 0, None)
    assert rc == CCQ_EINVAL and "group_size" in last_error()
    rc = lib.ccq_w4_gemm(p, 7, p, p, CCQ_F16, p, CCQ_F16, 1, 256, 64, 128, None, 0, None)
    assert rc == CCQ_EINVAL and "x_dtype" in last_error()
    rc = lib.ccq_w4_gemm(None, CCQ_BF16, p, p, CCQ_F16, p, CCQ_F16, 1, 256, 64, 128, None, 0, None)
    assert rc == CCQ_EINVAL and "null" in last_error()
    rc = lib.ccq_w4_gemm(ctypes.c_void_p(18), CCQ_BF16, p, p, CCQ_F16, p, CCQ_F16, 1, 256, 64, 128, None, 0, None)
    assert rc == CCQ_EINVAL and "aligned" in last_error()
    # M == 0 is an empty product: success without a launch
    assert lib.ccq_w4_gemm(p, CCQ_F16, p, p, CCQ_F16, p, CCQ_F16, 0, 256, 64, 128, None, 0, None) == 0
    # prefill-sized M needs the group-sum workspace
    assert lib.ccq_w4_gemm_workspace_size(64, 256, 128, 128) == 0
    assert lib.ccq_w4_gemm_workspace_size(65, 256, 128, 128) == 768 + 512  # group sums + row ids
    assert lib.ccq_w4_gemm_workspace_size(200, 256, 128, 64) == 0
    rc = lib.ccq_w4_gemm(p, CCQ_F16, p, p, CCQ_F16, p, CCQ_F16, 65, 256, 128, 128, None, 0, None)
    assert rc == CCQ_EINVAL and "workspace" in last_error()


def test_routing_rejects_bad_args(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    p = ctypes.c_void_p(256)
    assert lib.ccq_topk_softmax(p, p, p, 4, 2000, 4, 1, None) == CCQ_EINVAL and "E=" in last_error()
    assert lib.ccq_topk_softmax(p, p, p, 4, 64, 17, 1, None) == CCQ_EINVAL
    assert lib.ccq_topk_softmax(p, p, p, 4, 64, 8, 9, None) == CCQ_EINVAL and "mode" in last_error()
    assert lib.ccq_topk_softmax(p, p, p, 0, 64, 8, 1, None) == 0
    assert lib.ccq_moe_align(p, 10, 8, 0, p, p, p, p, None) == CCQ_EINVAL
    assert lib.ccq_moe_align(p, 70000, 8, 16, p, p, p, p, None) == CCQ_EINVAL
    assert lib.ccq_moe_align_max_tiles(96, 64, 16) == 6 + 64
    assert lib.ccq_moe_align_max_tiles(6, 64, 16) == 1 + 6
    assert lib.ccq_moe_combine(p, p, p, 9, 2, 2, 8, None) == CCQ_EINVAL


def test_reference_format_rejects(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    p = ctypes.c_void_p(256)
    assert lib.ccq_int4_dequant(p, p, p, 3, 7, None) == CCQ_EINVAL and "even" in last_error()
    assert lib.ccq_int4_linear_f32(p, p, p, p, 2, 7, 4, None) == CCQ_EINVAL
    assert lib.ccq_fp8_dequant(p, p, p, -1, 4, None) == CCQ_EINVAL
    assert lib.ccq_awq_repack(p, p, 128, 24, None) == CCQ_EINVAL
    assert lib.ccq_awq_repack(p, p, 128, 32, None) == CCQ_EINVAL and "in-place" in last_error()
    assert lib.ccq_awq_dequant(p, p, p, 1, p, 130, 64, 128, None) == CCQ_EINVAL
    assert lib.ccq_awq_pack_sz(p, p, 1, p, 256, 24, 128, None) == CCQ_EINVAL
    assert lib.ccq_awq_pack_sz(p, p, 1, p, 256, 32, 96, None) == CCQ_EINVAL and "group_size" in last_error()
    assert lib.ccq_awq_pack_sz(p, p, 3, p, 256, 32, 128, None) == CCQ_EINVAL and "scale_dtype" in last_error()


def test_sz_words_padding(lib):
    """Scale/zero words per column: K/G groups rounded up to whole chunks of
    4 k-tiles (512 rows)."""
    assert lib.ccq_awq_sz_words(2048, 128) == 16
    assert lib.ccq_awq_sz_words(1408, 128) == 12   # 11 k-tiles -> 12
    assert lib.ccq_awq_sz_words(1408, 64) == 24
    assert lib.ccq_awq_sz_words(128, 32) == 16     # 1 k-tile -> 4, 4 groups each
    assert lib.ccq_awq_sz_words(4096, 128) == 32
    assert lib.ccq_awq_sz_words(100, 128) == 0
    assert lib.ccq_awq_sz_words(256, 96) == 0


def test_moe_w4_descriptor_validation(lib):
    from ccut._lib import CCQ_EINVAL, ccq_w4_experts, last_error

    ex = ccq_w4_experts(*([256] * 6), 1, 64, 2048, 1400, 128)  # inter not a multiple of 128
    p = ctypes.c_void_p(256)
    assert lib.ccq_moe_w4_ffn(p, 2, p, p, p, 2, 1, 6, ctypes.byref(ex), p, 1 << 30, None) == CCQ_EINVAL
    assert "multiples of 128" in last_error()
    ex.inter = 1408
    assert lib.ccq_moe_w4_workspace_size(16, 6, ctypes.byref(ex)) > 0
    # the layer from logits: routing mode and k are checked before any launch
    assert lib.ccq_moe_w4_forward(p, 2, p, 16, 6, 5, None, None, p, 2, ctypes.byref(ex), p, 1 << 30,
                                  None) == CCQ_EINVAL
    assert "mode" in last_error()
    assert lib.ccq_moe_w4_forward(p, 2, p, 16, 17, 1, None, None, p, 2, ctypes.byref(ex), p, 1 << 30,
                                  None) == CCQ_EINVAL


def test_fp8_block_rejects_bad_args(lib):
    from ccut._lib import CCQ_BF16, CCQ_EINVAL, ccq_fp8_experts, last_error

    p = ctypes.c_void_p(256)
    assert lib.ccq_fp8_act_quant(p, CCQ_BF16, 4, 100, p, p, None) == CCQ_EINVAL and "128" in last_error()
    assert lib.ccq_fp8_act_quant(p, 9, 4, 128, p, p, None) == CCQ_EINVAL and "x_dtype" in last_error()
    assert lib.ccq_fp8_act_quant(p, CCQ_BF16, 0, 128, p, p, None) == 0
    assert lib.ccq_fp8_block_repack(p, p, 24, 128, None) == CCQ_EINVAL
    assert lib.ccq_fp8_block_repack(p, p, 64, 128, None) == CCQ_EINVAL and "N % 128" in last_error()
    assert lib.ccq_fp8_block_repack(p, p, 128, 128, None) == CCQ_EINVAL and "in-place" in last_error()
    assert lib.ccq_fp8_block_linear_workspace_size(4, 100) == 0
    need = lib.ccq_fp8_block_linear_workspace_size(4, 256)
    assert need > 0 and need % 256 == 0
    rc = lib.ccq_fp8_block_linear(p, CCQ_BF16, p, p, p, CCQ_BF16, 4, 256, 200, p, need, None)
    assert rc == CCQ_EINVAL and "N %" in last_error()
    rc = lib.ccq_fp8_block_linear(p, CCQ_BF16, p, p, p, CCQ_BF16, 4, 256, 256, p, need - 1, None)
    assert rc == CCQ_EINVAL and "workspace" in last_error()
    ex = ccq_fp8_experts(*([256] * 6), 8, 7168, 2000)
    assert lib.ccq_moe_fp8_workspace_size(16, 8, ctypes.byref(ex)) == 0
    assert lib.ccq_moe_fp8_ffn(p, CCQ_BF16, p, p, p, CCQ_BF16, 16, 8, ctypes.byref(ex), p, 1 << 40, None) == CCQ_EINVAL
    assert "multiples of 128" in last_error()
    ex.inter = 2048
    assert lib.ccq_moe_fp8_workspace_size(16, 8, ctypes.byref(ex)) > 16 * 7168
    assert lib.ccq_moe_fp8_ffn(p, CCQ_BF16, p, p, p, CCQ_BF16, 16, 9, ctypes.byref(ex), p, 1 << 40, None) == CCQ_EINVAL


def test_int8_rejects_bad_args(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    p = ctypes.c_void_p(256)
    assert lib.ccq_int8_linear(p, p, p, p, p, -1, 64, 64, None, 0, None) == CCQ_EINVAL
    assert lib.ccq_int8_linear(p, p, p, p, p, 1, 1 << 17, 64, None, 0, None) == CCQ_EINVAL
    assert "overflow" in last_error()
    assert lib.ccq_int8_linear(None, p, p, p, p, 1, 64, 64, None, 0, None) == CCQ_EINVAL
    assert lib.ccq_int8_linear(p, p, p, p, p, 0, 64, 64, None, 0, None) == 0  # empty: no launch
    # decode shapes split K over workgroups and need the partial-sum workspace
    need = lib.ccq_int8_linear_workspace_size(1, 4096, 4096)
    assert need == 4 * 4096 * 4  # 128 strips of 32 columns x 4 waves x 4 splits = 2048 waves
    assert lib.ccq_int8_linear_workspace_size(4096, 4096, 4096) == 0
    assert lib.ccq_int8_linear_workspace_size(1, 100, 4096) == 0  # K % 16 != 0: no split
    rc = lib.ccq_int8_linear(p, p, p, p, p, 1, 4096, 4096, None, 0, None)
    assert rc == CCQ_EINVAL and "workspace" in last_error()
    rc = lib.ccq_int8_linear(p, p, p, p, p, 1, 4096, 4096, p, need - 1, None)
    assert rc == CCQ_EINVAL and "workspace" in last_error()
    assert lib.ccq_int8_act_quant(p, p, p, -1, 8, None) == CCQ_EINVAL
    assert lib.ccq_int8_act_quant(p, p, p, 0, 8, None) == 0
    assert lib.ccq_int8_dequant(p, p, p, 3, -1, None) == CCQ_EINVAL
    assert lib.ccq_int8_linear_f32(p, p, p, p, -2, 7, 4, None) == CCQ_EINVAL
    # the whole layer: fused up to 4 rows (workspace only for the K split),
    # else the quantized rows (256-byte aligned) ahead of the split partials
    assert lib.ccq_int8_w8a8_workspace_size(1, 4096, 14336) == 0
    assert lib.ccq_int8_w8a8_workspace_size(1, 4096, 4096) == 4 * 4096 * 4
    assert lib.ccq_int8_w8a8_workspace_size(16, 4096, 14336) == 16 * 4096
    assert lib.ccq_int8_w8a8_workspace_size(5, 100, 7) == 512
    assert lib.ccq_int8_w8a8_linear(p, p, p, p, p, 2, 0, 8, None, 0, None) == CCQ_EINVAL and "K=0" in last_error()
    rc = lib.ccq_int8_w8a8_linear(p, p, p, p, p, 16, 4096, 14336, None, 0, None)
    assert rc == CCQ_EINVAL and "workspace" in last_error()


def test_mx_rejects_bad_args(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    p = ctypes.c_void_p(256)
    assert lib.ccq_mx_dequant(p, p, p, 2, 64, 2, 32, 1.0, None) == CCQ_EINVAL and "fmt" in last_error()
    assert lib.ccq_mx_dequant(p, None, p, 2, 64, 0, 32, 1.0, None) == CCQ_EINVAL and "scales" in last_error()
    assert lib.ccq_mx_dequant(p, p, p, 2, 63, 1, 32, 1.0, None) == CCQ_EINVAL and "even" in last_error()
    assert lib.ccq_mx_linear_f32(p, p, p, p, 1, 64, 8, 0, 0, 1.0, None) == CCQ_EINVAL and "group_size" in last_error()
    assert lib.ccq_mx_linear_f32(p, p, None, p, 0, 64, 8, 1, 32, 1.0, None) == 0  # empty batch, no scales: ok
    assert lib.ccq_e8m0_to_f32(p, p, -1, None) == CCQ_EINVAL


def test_wq_mfma_rejects_bad_args(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    p = ctypes.c_void_p(256)
    f = lib.ccq_wq_mfma_linear_f32
    assert f(p, p, p, p, 4, 256, 8, 4, 32, 1.0, None) == CCQ_EINVAL and "fmt" in last_error()
    assert f(p, p, p, p, 4, 320, 8, 0, 0, 1.0, None) == CCQ_EINVAL and "multiple of 256" in last_error()
    assert f(p, p, p, p, -1, 256, 8, 0, 0, 1.0, None) == CCQ_EINVAL and "negative" in last_error()
    assert f(p, p, None, p, 4, 256, 8, 0, 0, 1.0, None) == CCQ_EINVAL and "scales" in last_error()
    assert f(p, p, p, p, 4, 256, 8, 2, 8, 1.0, None) == CCQ_EINVAL and "group_size" in last_error()
    assert f(ctypes.c_void_p(260), p, p, p, 4, 256, 8, 0, 0, 1.0, None) == CCQ_EINVAL and "aligned" in last_error()
    assert f(p, p, None, p, 0, 256, 8, 3, 32, 1.0, None) == 0  # empty batch: nothing to do


def test_fp8row_moe_rejects_bad_args(lib):
    from ccut._lib import CCQ_EINVAL, ccq_fp8row_experts, last_error

    p = ctypes.c_void_p(256)
    ex = ccq_fp8row_experts(256, 256, 256, 256, 256, 256, 8, 2048, 512)
    f = lib.ccq_moe_fp8row_ffn
    assert f(p, p, p, p, 0, 4, 2, None, p, 1 << 20, None) == CCQ_EINVAL and "null experts" in last_error()
    bad = ccq_fp8row_experts(256, 256, 256, 256, 256, 256, 8, 2000, 512)
    assert f(p, p, p, p, 0, 4, 2, ctypes.byref(bad), p, 1 << 20, None) == CCQ_EINVAL and "multiples of 256" in last_error()
    unaligned = ccq_fp8row_experts(264, 256, 256, 256, 256, 256, 8, 2048, 512)
    assert f(p, p, p, p, 0, 4, 2, ctypes.byref(unaligned), p, 1 << 20, None) == CCQ_EINVAL and "aligned" in last_error()
    assert f(p, p, p, p, 0, 4, 9, ctypes.byref(ex), p, 1 << 20, None) == CCQ_EINVAL  # k > E
    assert f(p, p, p, p, 0, 30000, 8, ctypes.byref(ex), p, 1 << 20, None) == CCQ_EINVAL and "65536" in last_error()
    assert f(p, p, p, p, 7, 4, 2, ctypes.byref(ex), p, 1 << 20, None) == CCQ_EINVAL and "y_dtype" in last_error()
    assert f(ctypes.c_void_p(260), p, p, p, 0, 4, 2, ctypes.byref(ex), p, 1 << 20, None) == CCQ_EINVAL
    assert f(p, p, p, p, 0, 4, 2, ctypes.byref(ex), p, 64, None) == CCQ_EINVAL and "workspace" in last_error()
    assert f(p, p, p, p, 0, 0, 2, ctypes.byref(ex), None, 0, None) == 0  # no tokens: nothing to do
    assert lib.ccq_moe_fp8row_workspace_size(16, 8, ctypes.byref(ex)) > 16 * 8 * (2048 + 512) * 4
    assert lib.ccq_moe_fp8row_workspace_size(16, 8, ctypes.byref(bad)) == 0
    assert lib.ccq_moe_fp8row_ffn_shared(p, p, p, None, 1.0, p, 0, 4, 2, ctypes.byref(ex), p, 1 << 20,
                                         None) == CCQ_EINVAL and "shared" in last_error()


def test_f32_gemm_rejects_bad_args(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    p = ctypes.c_void_p(256)
    assert lib.ccq_f32_gemm(p, p, p, 4, 64, 8, 2, None, 0, None) == CCQ_EINVAL and "trans_w" in last_error()
    assert lib.ccq_f32_gemm(p, p, p, -1, 64, 8, 0, None, 0, None) == CCQ_EINVAL and "negative" in last_error()
    assert lib.ccq_f32_gemm(p, None, p, 4, 64, 8, 0, None, 0, None) == CCQ_EINVAL and "null" in last_error()
    assert lib.ccq_f32_gemm(p, p, p, 0, 64, 8, 1, None, 0, None) == 0  # no rows
    assert lib.ccq_f32_gemm_workspace_size(4, 64, 8) == 0  # too shallow to split
    assert lib.ccq_expert_ffn_f32(p, p, p, p, p, 4, 64, 32, p, 16, None) == CCQ_EINVAL and "workspace" in last_error()
    assert lib.ccq_expert_ffn_f32(p, p, p, p, p, 4, 0, 32, p, 1 << 20, None) == CCQ_EINVAL
    assert lib.ccq_expert_ffn_f32_workspace_size(4, 32) == 4 * 32 * 4
    f = lib.ccq_moe_f32_ffn
    assert f(p, p, p, p, p, p, None, 0.0, p, 0, 4, 2, 2000, 64, 32, p, 1 << 20, None) == CCQ_EINVAL  # E > 1024
    assert f(p, p, p, None, p, p, None, 0.0, p, 0, 4, 2, 8, 64, 32, p, 1 << 20, None) == CCQ_EINVAL and "null" in last_error()
    assert f(p, p, p, p, p, p, None, 0.0, p, 0, 4, 2, 8, 64, 32, p, 64, None) == CCQ_EINVAL and "workspace" in last_error()
    assert lib.ccq_moe_f32_workspace_size(4, 2, 8, 64, 32) > 0


def test_launch_timer_arguments(lib):
    from ccut._lib import CCQ_EINVAL, last_error

    assert lib.ccq_launch_timer(ctypes.c_void_p(256), None) == CCQ_EINVAL and "both" in last_error()
    assert lib.ccq_launch_timer(None, None) == 0  # clears

"""Build-time check of the kernels that stream data into registers with
inline-assembly loads (the register-streamed FP8 MoE kernels and the
decoded-weight MFMA linear): on the register allocator's output, no
instruction reads, copies or spills a register whose load is still in
flight, and no instance spills (costcut-infer_amd/csrc/check_inflight.py).
Needs hipcc, not a GPU."""

from __future__ import annotations

import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CHECK = ROOT / "costcut-infer_amd" / "csrc" / "check_inflight.py"


@pytest.mark.skipif(not (shutil.which("hipcc") or Path("/opt/rocm/bin/hipcc").exists()), reason="needs hipcc")
def test_no_inflight_register_use():
    r = subprocess.run([sys.executable, str(CHECK)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "wq_mfma_kernel" in r.stdout and "fp8_moe_rb_kernel" in r.stdout and "wq_moe_kernel" in r.stdout

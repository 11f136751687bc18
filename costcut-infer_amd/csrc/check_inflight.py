"""Build-time check of the kernels that stream data into registers with
inline-assembly loads: the register-streamed FP8 MoE kernels
(``fp8_moe_rb_kernel`` in ccq_fp8.hip) and the decoded-weight MFMA linear
(``wq_mfma_kernel`` in ccq_wmfma.hip).

Their loads are inline-assembly ``global_load_*`` whose destination
registers are handed to the compiler only by a later inline assembly that
takes them as tied (``"+v"``) operands, after an ``s_waitcnt``.  Between the
load and that hand-over the data has not arrived, so the compiler must
neither read, copy nor spill those registers.  This script compiles each
source for gfx950, dumps each kernel's machine code after greedy register
allocation (virtual registers, with every copy and spill the allocator
inserted), and runs a dataflow over the control-flow graph: a (virtual
register, sub-register) defined by such a load is in flight until an inline
assembly takes it as a tied operand; any other instruction that names it
while in flight is reported.

    python costcut-infer_amd/csrc/check_inflight.py      # exit 1 on a finding

It also reports each kernel's VGPR and spill counts (from the assembly).
"""

from __future__ import annotations

import concurrent.futures as cf
import re
import subprocess
import sys
import tempfile
from pathlib import Path

CSRC = Path(__file__).resolve().parent
INCLUDE = CSRC.parent.parent / "include"
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", f"-I{INCLUDE}", "--cuda-device-only"]
# source -> pattern of the kernels to check (every instance in the build)
TARGETS = {"ccq_fp8.hip": r"_ZN3ccq17fp8_moe_rb_kernel\w+",
           "ccq_wmfma.hip": r"_ZN3ccq(?:14wq_mfma_kernel|13wq_moe_kernel)\w+"}


def _overlap(a, b):
    if a[0] != b[0]:
        return False
    if not a[1] or not b[1] or a[1] == b[1]:
        return True
    return bool(set(a[1].split("_")) & set(b[1].split("_")))


def check_mir(text: str) -> list[str]:
    """Dataflow over one function's MIR dump; returns the offending lines."""
    blocks, order, cur = {}, [], None
    for line in text.split("\n"):
        mb = re.match(r"^(\d+B\s+)?bb\.(\d+)", line)
        if mb:
            cur = int(mb.group(2))
            blocks[cur] = {"ins": [], "succ": []}
            order.append(cur)
            continue
        if cur is None:
            continue
        if "successors:" in line:
            blocks[cur]["succ"] = [int(x) for x in re.findall(r"%bb\.(\d+)", line)]
            continue
        mi = re.match(r"\s*\d+B\s+(.*)", line)
        if mi:
            blocks[cur]["ins"].append(mi.group(1))
    if not order:
        return ["no machine code found"]
    state = {b: None for b in order}
    state[order[0]] = frozenset()
    work, found = [order[0]], {}
    while work:
        b = work.pop()
        live = set(state[b])
        for ins in blocks[b]["ins"]:
            if "INLINEASM" in ins and "global_load" in ins and "global_load_lds" not in ins:  # (LDS DMA: no register)
                d = re.search(r"def (?:undef |dead |early-clobber )*%(\d+)(?:\.(\w+))?", ins)
                if d is None:  # a load whose destination is not a virtual register
                    found.setdefault("unparsed load: " + ins[:160], b)
                    continue
                key = (d.group(1), d.group(2) or "")
                live = {x for x in live if not _overlap(x, key)}
                live.add(key)
                continue
            if "INLINEASM" in ins and "tiedto" in ins:
                for v, sub in re.findall(r"reguse tiedto:\$\d+\], %(\d+)(?:\.(\w+))?", ins):
                    live = {x for x in live if not _overlap(x, (v, sub))}
                continue
            for v, sub in re.findall(r"%(\d+)(?:\.(\w+))?", ins):
                if any(_overlap(x, (v, sub)) for x in live):
                    found.setdefault(ins[:160], b)
        out = frozenset(live)
        for s in blocks[b]["succ"]:
            if state.get(s) is None:
                state[s] = out
                work.append(s)
            elif not out <= state[s]:
                state[s] = state[s] | out
                work.append(s)
    return [f"bb.{b}: {ins}" for ins, b in found.items()]


def _check_kernel(src: Path, text: str, k: str) -> tuple[str, int]:
    m = re.search(r"\.name:\s+" + re.escape(k) + r"\b(.*?)\.vgpr_count:\s+(\d+)", text, re.S)
    sp = re.search(r"\.vgpr_spill_count:\s+(\d+)", text[m.end():m.end() + 400]) if m else None
    vg, spills = (m.group(2) if m else "?"), (sp.group(1) if sp else "?")
    r = subprocess.run([HIPCC, *FLAGS, "-S", str(src), "-o", "/dev/null", "-mllvm", "-print-after=greedy",
                        "-mllvm", f"-filter-print-funcs={k}"], capture_output=True, text=True)
    dump = r.stdout + r.stderr
    mir = next((f for f in dump.split("# *** IR Dump After") if "# Machine code for function " + k in f), "")
    issues = check_mir(mir)
    lines = [f"{k}: {vg} VGPRs, {spills} spills, {len(issues)} in-flight register uses"]
    lines += ["    " + line for line in issues[:10]]
    return "\n".join(lines), len(issues) + (0 if spills == "0" else 1)


def main(jobs: int = 8) -> int:
    bad = 0
    with tempfile.TemporaryDirectory() as td, cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for name, pattern in TARGETS.items():
            src = CSRC / name
            asm = Path(td) / (src.stem + ".s")
            subprocess.run([HIPCC, *FLAGS, "-S", str(src), "-o", str(asm)], check=True, capture_output=True)
            text = asm.read_text()
            kernels = sorted(set(re.findall(r"\.name:\s+(" + pattern + r")\b", text)))
            if not kernels:
                print(f"{name}: no kernel matches {pattern}")
                bad += 1
            for report, n in ex.map(lambda k: _check_kernel(src, text, k), kernels):
                print(report)
                bad += n
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())

#!/usr/bin/env python
"""Benchmark of the quantized expert-matmul path on one MI355X.

Headline workload: int4 (AWQ, group 128) MoE expert FFN decode -- 64 experts,
top-6 routing from softmax of N(0,1) router logits over [T, 64], hidden 2048,
expert intermediate 1408, bf16 activations, T = 16 tokens.  One step is one
MoE layer from router logits (ccq_moe_w4_forward): the gate/up + SiLU kernel
that routes the batch inside its workgroups, the down kernel, the weighted
combine, replayed from a HIP graph.  Steps rotate over 4 distinct layer
weight sets (1.15 GB) so the 256 MiB Infinity Cache cannot serve repeated
weights.  ``value`` is algorithmic bytes (weights of the experts actually
routed + activations) per second of wall time for whole steps, with inputs
resident in HBM.

``roofline`` is the dominant kernel of the step, that same routed gate/up
launch (ccq_moe_w4_route_gate_up runs exactly it): algorithmic bytes per
launch / its average duration.  That duration comes from :func:`kernel_time`:
HIP events that each launch's own dispatch records at the kernel's start and
end (ccq_launch_timer), the interval rocprofv3's kernel trace reports; the
average over back-to-back launches bracketed by one pair of events (which
adds the gap between launches) is reported beside it.  Other device times
come from :func:`device_time`: a spin kernel holds the stream while the host
enqueues all launches, so they run back to back and the HIP events on that
stream bracket device time only.

Also reported (``extra``): the same layer at T=1 (20 rotating layers, > 512
MiB of routed weights), the T=16 layer with a shared expert run in the same
kernels (65 experts), the AWQ skinny GEMM at K=4096 N=14336 M in {1,4,16}
and the single AWQ GEMV K=2048 N=5632 (kernel GB/s); the reference-format
FP8 per-row and the MX linears (MXFP4 / MXFP8, up to 64 rows on the
decoded-weight MFMA kernel), INT8 W8A8, the FP8 quantizers; the prefill workloads
as TFLOP/s against the matching dense MFMA peak: int4 MoE prefill (128
experts, skewed top-8, hidden 2048, inter 768, T = 512 and 4096, bf16 MFMA,
4 rotating weight sets) and FP8 block MoE prefill (256 experts, top-8,
T = 2048, hidden 7168, inter 2048, FP8 MFMA); the MoE layer on the
reference checkpoint's own expert format (e4m3 [out, in] with per-row
scales, 256 experts, top-8, hidden 2048, inter 512, float32 activations)
at T = 1, 16 and 512 (GB/s of the routed experts' bytes).  ``cpu_baseline`` times the
reference's algorithm (the CPU oracle: dequant to float32, BLAS matmuls,
per-expert grouping) on the host, per workload, in two variants: dequant on
every call, and matmuls on cached float32 weights.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "costcut-infer_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
PEAK_BF16 = 2.5166e15      # dense bf16 MFMA FLOP/s
PEAK_FP8 = 5.0332e15       # dense fp8 MFMA FLOP/s
PEAK_INT8 = 5.0332e15      # dense int8 MFMA OP/s

E, TOPK, HID, INTER, GROUP = 64, 6, 2048, 1408, 128
# HBM bytes / algorithmic bytes of the routed decode gate/up launch, from
# rocprofv3 FETCH_SIZE and WRITE_SIZE runs of the same kernel on the
# torch-free driver (costcut-infer_amd/drivers/moe_driver.cpp, mode w4f,
# T=16), each scaled by the counter's reading for a 64 MiB streaming copy
# (profiles/moe_decode_int4_kernel_stats.md holds the table and commands);
# counters cannot be taken inside this process, so the bench scales its own
# algorithmic bytes by the measured ratio
GATE_UP_TRAFFIC_RATIO = 1.029
LAYERS = 4
LAYERS_T1 = 20  # T=1 routes 6 experts (27 MB) per layer: 20 layers touch > 512 MiB
METRIC = "int4 MoE decode GB/s (% HBM peak) + FP8/int4 prefill TFLOP/s (% MFMA peak)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary workloads")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------- timing --
_SLEEP_CYCLES_PER_MS: float | None = None


def _sleep_calibration() -> float:
    """Cycles of ``torch.cuda._sleep`` per millisecond on this device."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        import torch

        n = 1_000_000
        torch.cuda._sleep(n)  # warm
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        torch.cuda._sleep(n)
        b.record()
        b.synchronize()
        _SLEEP_CYCLES_PER_MS = n / max(a.elapsed_time(b), 1e-3)
    return _SLEEP_CYCLES_PER_MS


def device_time(launches, reps: int = 1) -> float:
    """Average device seconds per launch of ``launches`` (callables that each
    enqueue one kernel on the current stream), run back to back ``reps``
    times.  The stream is held by a spin kernel while the host enqueues, and
    the hold is lengthened until it outlasts the host's enqueue time."""
    import torch

    n = len(launches) * reps
    hold_ms = 5.0
    for _ in range(6):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        torch.cuda._sleep(int(_sleep_calibration() * hold_ms))
        a.record()
        for _r in range(reps):
            for f in launches:
                f()
        b.record()
        host_ms = (time.perf_counter() - t0) * 1e3
        b.synchronize()
        if host_ms < 0.8 * hold_ms:
            return a.elapsed_time(b) * 1e-3 / n
        hold_ms = 2.0 * host_ms + 5.0
    raise RuntimeError("device_time: host enqueue never finished inside the stream hold")


def kernel_time(launches, reps: int = 1) -> float:
    """Average duration in seconds of the one kernel each of ``launches``
    enqueues (a ccq entry point that launches exactly one kernel), from a
    pair of HIP events per launch that the kernel's own dispatch records
    (``ccq_launch_timer`` -> hipExtLaunchKernel): the interval from the
    kernel's start to its end, which is what rocprofv3's kernel trace
    reports, without the gap between back-to-back launches that events
    bracketing the whole run include.  The launches run back to back behind
    a stream hold as in :func:`device_time`."""
    import torch

    from ccut import _lib

    lib = _lib.lib()
    n = len(launches) * reps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in evs:  # creates the HIP events, so that cuda_event is a handle
        a.record()
        b.record()
    torch.cuda.synchronize()
    torch.cuda._sleep(int(_sleep_calibration() * (5.0 + 0.05 * n)))
    i = 0
    for _r in range(reps):
        for f in launches:
            a, b = evs[i]
            _lib.check(lib.ccq_launch_timer(ctypes.c_void_p(a.cuda_event), ctypes.c_void_p(b.cuda_event)),
                       "ccq_launch_timer")
            f()
            lib.ccq_launch_timer(None, None)  # a call that launched nothing leaves no armed timer behind
            i += 1
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) * 1e-3 / n


# -------------------------------------------------------------- workloads --
class Layer:
    def __init__(self, idx: int, T: int, dev):
        import torch

        from ccut import workloads as wl
        from ccut.blocks import moe

        self.experts = moe.W4Experts.from_awq(
            wl.awq_experts(E, HID, INTER, GROUP, seed=1000 + 3 * idx, device=dev),
            wl.awq_experts(E, HID, INTER, GROUP, seed=1001 + 3 * idx, device=dev),
            wl.awq_experts(E, INTER, HID, GROUP, seed=1002 + 3 * idx, device=dev),
            GROUP)
        self.logits = wl.router_logits(T, E, seed=77 + idx, device=dev)
        torch.cuda.synchronize()


def moe_step_bytes(layer, x, T: int) -> tuple[int, int]:
    """(algorithmic bytes of one layer step, distinct experts routed):
    weights of every routed expert once, activations in and out, router
    logits, routing ids and weights."""
    import torch

    from ccut.blocks import moe

    _, ids = moe.topk_softmax(layer.logits, TOPK, True)
    uniq = int(torch.unique(ids).numel())
    act = x.numel() * x.element_size() * 2 + layer.logits.numel() * 4 + T * TOPK * (8 + 4)
    return uniq * layer.experts.bytes_per_expert + act, uniq


def bench_moe(T: int, steps: int, warmup: int, dev, n_layers: int = LAYERS):
    """Whole MoE layer steps replayed from a HIP graph (wall time) over
    ``n_layers`` distinct layers, plus the device time of the step's routed
    gate/up kernel."""
    import torch

    from ccut import workloads as wl
    from ccut.blocks import moe

    layers = [Layer(i, T, dev) for i in range(n_layers)]
    x = wl.activations(T, HID, seed=5, device=dev, dtype=torch.bfloat16)
    ys = [torch.empty((T, HID), dtype=torch.bfloat16, device=dev) for _ in range(n_layers)]
    per = [moe_step_bytes(l, x, T) for l in layers]

    def step(i):
        l = layers[i % n_layers]
        moe.moe_forward_w4(x, l.logits, l.experts, TOPK, True, out=ys[i % n_layers])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n_layers):
            step(i)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_layers):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // n_layers)
    n_steps = reps * n_layers
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        graph.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    total_bytes = sum(per[i % n_layers][0] for i in range(n_steps))
    return {
        "T": T, "steps": n_steps, "layers": n_layers, "ms_per_step": dt / n_steps * 1e3,
        "GBps": total_bytes / dt / 1e9, "unique_experts": [p[1] for p in per],
        "bytes_per_step": [p[0] for p in per], "distinct_bytes": sum(p[0] for p in per),
        "gate_up": time_gate_up(layers, x, T, dev),
    }


def bench_moe_shared(T: int, dev, n_layers: int = LAYERS):
    """The decode layer with a shared expert in the same kernels
    (``ccq_moe_w4_forward_shared``: 64 routed experts + the shared one last,
    top-6, every token's seventh slot the shared expert with gate 0.5);
    device time per layer over ``n_layers`` distinct weight sets.
    Algorithmic bytes: the routed experts' and the shared expert's weights
    once, activations, logits, routing."""
    import dataclasses

    import torch

    from ccut import workloads as wl
    from ccut.blocks import moe

    layers = []
    for i in range(n_layers):
        ex = moe.W4Experts.from_awq(
            wl.awq_experts(E + 1, HID, INTER, GROUP, seed=2000 + 3 * i, device=dev),
            wl.awq_experts(E + 1, HID, INTER, GROUP, seed=2001 + 3 * i, device=dev),
            wl.awq_experts(E + 1, INTER, HID, GROUP, seed=2002 + 3 * i, device=dev), GROUP)
        layers.append((dataclasses.replace(ex, shared_expert=True), wl.router_logits(T, E, seed=90 + i, device=dev)))
    x = wl.activations(T, HID, seed=5, device=dev, dtype=torch.bfloat16)
    y = torch.empty((T, HID), dtype=torch.bfloat16, device=dev)
    nb = []
    for ex, lg in layers:
        _, ids = moe.topk_softmax(lg, TOPK, True)
        uniq = int(torch.unique(ids).numel()) + 1
        nb.append(uniq * ex.bytes_per_expert + x.numel() * 2 * 2 + lg.numel() * 4 + T * (TOPK + 1) * 12)
    launches = [lambda ex=ex, lg=lg: moe.moe_forward_w4(x, lg, ex, TOPK, True, out=y, shared_gate=0.5)
                for ex, lg in layers]
    launches[0]()
    torch.cuda.synchronize()
    avg = device_time(launches, reps=8)
    b = sum(nb) / len(nb)
    return {"T": T, "avg_us": avg * 1e6, "bytes": b, "GBps": b / avg / 1e9, "frac_hbm": b / avg / PEAK_HBM,
            "layers": n_layers}


def time_gate_up(layers, x, T: int, dev):
    """Device time of the step's gate/up + SiLU kernel with the routing
    inside its workgroups (ccq_moe_w4_route_gate_up: the first launch of
    ccq_moe_w4_forward), rotating over the layers.  Algorithmic bytes per
    launch: gate and up weights (int4 + fp16 scales + int4 zeros) of the
    routed experts, the router logits and activations read, the routing and
    the intermediate written."""
    import torch

    from ccut import _dev, _lib
    from ccut.blocks import moe

    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    launches, gu_bytes, keep = [], [], []
    for l in layers:
        _, ids = moe.topk_softmax(l.logits, TOPK, True)
        desc = l.experts.descriptor()
        nbytes = lib.ccq_moe_w4_workspace_size(T, TOPK, ctypes.byref(desc))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        keep.append((desc, ws))
        uniq = int(torch.unique(ids).numel())
        gu_bytes.append(uniq * l.experts.gate_up_bytes_per_expert + x.numel() * 2 + l.logits.numel() * 4
                        + T * TOPK * (8 + 4) + T * TOPK * INTER * 2)
        args = (ctypes.c_void_p(x.data_ptr()), _dev.DTYPE_CODE[x.dtype], ctypes.c_void_p(l.logits.data_ptr()), T,
                TOPK, 1, None, None, ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), nbytes,
                ctypes.c_void_p(stream))
        launches.append(lambda a=args: lib.ccq_moe_w4_route_gate_up(*a))
    for f in launches:
        _lib.check(f(), "ccq_moe_w4_route_gate_up")
    torch.cuda.synchronize()
    reps = max(1, 100 // len(launches))
    avg = kernel_time(launches, reps=reps)
    b2b = device_time(launches, reps=reps)
    avg_bytes = sum(gu_bytes) / len(gu_bytes)
    return {"avg_us": avg * 1e6, "bytes": avg_bytes, "GBps": avg_bytes / avg / 1e9,
            "back_to_back_us": b2b * 1e6}


def bench_gemm(M: int, K: int, N: int, dev, copies: int):
    """Device time of ccq_w4_gemm rotating over distinct weight copies
    (> 512 MiB in total, so the Infinity Cache cannot serve repeats)."""
    import torch

    from ccut import _lib
    from ccut import workloads as wl
    from ccut.quant import awq

    lib = _lib.lib()
    ws = []
    for c in range(copies):
        qw, qz, s = wl.awq_linear(K, N, GROUP, seed=500 + c, device=dev)
        ws.append(awq.prepare(qw, qz, s, GROUP))
    x = wl.activations(M, K, seed=9, device=dev, dtype=torch.float16)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    ref = awq.gemm(x, ws[0])  # through the Python API once
    stream = torch.cuda.current_stream().cuda_stream
    nws = lib.ccq_w4_gemm_workspace_size(M, K, N, GROUP)
    wsb = torch.empty(max(nws, 256), dtype=torch.uint8, device=dev)
    launches = []
    for w in ws:
        args = (ctypes.c_void_p(x.data_ptr()), 1, ctypes.c_void_p(w.w_tiled.data_ptr()),
                ctypes.c_void_p(w.sz.data_ptr()), 1, ctypes.c_void_p(y.data_ptr()), 1, M, K, N, GROUP,
                ctypes.c_void_p(wsb.data_ptr()), nws, ctypes.c_void_p(stream))
        launches.append(lambda a=args: lib.ccq_w4_gemm(*a))
    _lib.check(launches[0](), "ccq_w4_gemm")
    torch.cuda.synchronize()
    if not torch.equal(y, ref):
        raise RuntimeError("bench_gemm: raw launch and API disagree")
    avg = device_time(launches, reps=4)
    nbytes = ws[0].format_bytes + M * K * 2 + M * N * 2
    return {"M": M, "K": K, "N": N, "avg_us": avg * 1e6, "bytes": nbytes, "GBps": nbytes / avg / 1e9,
            "frac_hbm": nbytes / avg / PEAK_HBM, "TFLOPs": 2.0 * M * K * N / avg / 1e12}


def bench_quantizers(dev):
    """Load-time FP8 quantization of a BF16 weight [7168, 2048] and per-token
    FP8 KV quantization / read-back of [2, 8, 4096, 128] float32, each over
    distinct buffers (> 512 MiB in total).  Algorithmic bytes: 2 + 1 B per
    weight element; 4 + 1 B per KV element (+ 1 B per row)."""
    import torch

    from ccut import _lib

    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = ctypes.c_void_p
    g = torch.Generator(device=dev).manual_seed(3)
    out = {}
    R, C, copies = 7168, 2048, 20
    ws = [(torch.randn((R, C), generator=g, device=dev) * 0.02).to(torch.bfloat16) for _ in range(copies)]
    q = torch.empty((R, C), dtype=torch.uint8, device=dev)
    launches = [lambda w=w: lib.ccq_quantize_rows_fp8(vp(w.data_ptr()), None, vp(q.data_ptr()), R, C, stream)
                for w in ws]
    _lib.check(launches[0](), "ccq_quantize_rows_fp8")
    avg = device_time(launches, reps=2)
    nb = R * C * 3
    out["online_fp8_quant_7168x2048"] = {"avg_us": avg * 1e6, "bytes": nb, "GBps": nb / avg / 1e9,
                                         "frac_hbm": nb / avg / PEAK_HBM}
    del ws
    rows, dim, copies = 2 * 8 * 4096, 128, 16
    kvs = [torch.randn((rows, dim), generator=g, device=dev) for _ in range(copies)]
    codes = [torch.empty((rows, dim), dtype=torch.uint8, device=dev) for _ in range(copies)]
    scales = [torch.empty(rows, dtype=torch.uint8, device=dev) for _ in range(copies)]
    back = torch.empty((rows, dim), dtype=torch.float32, device=dev)
    lq = [lambda i=i: lib.ccq_kv_quant_fp8(vp(kvs[i].data_ptr()), vp(codes[i].data_ptr()), vp(scales[i].data_ptr()),
                                           rows, dim, stream) for i in range(copies)]
    ld = [lambda i=i: lib.ccq_kv_dequant_fp8(vp(codes[i].data_ptr()), vp(scales[i].data_ptr()), vp(back.data_ptr()),
                                             rows, dim, stream) for i in range(copies)]
    _lib.check(lq[0](), "ccq_kv_quant_fp8")
    for name, launches in (("kv_fp8_quant_2x8x4096x128", lq), ("kv_fp8_dequant_2x8x4096x128", ld)):
        avg = device_time(launches, reps=2)
        nb = rows * dim * 5 + rows
        out[name] = {"avg_us": avg * 1e6, "bytes": nb, "GBps": nb / avg / 1e9, "frac_hbm": nb / avg / PEAK_HBM}
    return out


def bench_int8(M: int, K: int, N: int, dev, copies: int = 1):
    """INT8 W8A8 linear y = x @ W.T through ``ccq_int8_w8a8_linear``:
    per-token activation quantization of x [M, K] float32 (inside the GEMM up
    to 4 rows), the int8 MFMA GEMM with its float32 epilogue (plus the
    split-K reduction where K is split), device time per layer over
    ``copies`` distinct weight matrices.  Algorithmic bytes: N*K weight bytes
    + 4*M*K (x) + 4*M*N (y) + 4*N (scales); ops 2*M*N*K."""
    import torch

    from ccut import _lib

    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = ctypes.c_void_p
    g = torch.Generator(device=dev).manual_seed(13)
    ws = [torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8) for _ in range(copies)]
    sc = torch.rand(N, generator=g, device=dev) * 0.01
    x = torch.randn((M, K), generator=g, device=dev)
    xs = torch.empty(M, device=dev)
    y = torch.empty((M, N), device=dev)
    nws = int(lib.ccq_int8_w8a8_workspace_size(M, K, N))
    wsp = torch.empty(max(nws, 256), dtype=torch.uint8, device=dev)

    def layer(w):
        _lib.check(lib.ccq_int8_w8a8_linear(vp(x.data_ptr()), vp(xs.data_ptr()), vp(w.data_ptr()),
                                            vp(sc.data_ptr()), vp(y.data_ptr()), M, K, N, vp(wsp.data_ptr()), nws,
                                            stream), "ccq_int8_w8a8_linear")

    launches = [lambda w=w: layer(w) for w in ws]
    launches[0]()
    torch.cuda.synchronize()
    avg = device_time(launches, reps=max(1, 24 // copies))
    nb = N * K + 4 * M * K + 4 * M * N + 4 * N
    ops = 2.0 * M * N * K
    return {"avg_us": avg * 1e6, "bytes": nb, "GBps": nb / avg / 1e9, "frac_hbm": nb / avg / PEAK_HBM,
            "TOPs": ops / avg / 1e12, "frac_int8_peak": ops / avg / PEAK_INT8, "workspace_bytes": nws}


def bench_ref_fp8_linear(M: int, K: int, N: int, dev, copies: int = 12):
    """The reference's own FP8 format (e4m3fn ``[N, K]``, one float32 scale
    per output row, the checkpoints' per-channel FP8) through
    ``ccq_fp8_linear_f32``: y = x @ (fp8(W) * s).T in float32 for float32 x
    [M, K]; device time per call over ``copies`` distinct weight matrices.
    Algorithmic bytes: N*K + 4*N + 4*M*K + 4*M*N."""
    import torch

    from ccut import _lib

    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = ctypes.c_void_p
    g = torch.Generator(device=dev).manual_seed(17)
    ws = [torch.randint(0, 0x7F, (N, K), generator=g, device=dev, dtype=torch.uint8) for _ in range(copies)]
    sc = torch.rand(N, generator=g, device=dev) * 0.01
    x = torch.randn((M, K), generator=g, device=dev)
    y = torch.empty((M, N), device=dev)

    def call(w):
        _lib.check(lib.ccq_fp8_linear_f32(vp(x.data_ptr()), vp(w.data_ptr()), vp(sc.data_ptr()), vp(y.data_ptr()),
                                          M, K, N, stream), "ccq_fp8_linear_f32")

    launches = [lambda w=w: call(w) for w in ws]
    launches[0]()
    torch.cuda.synchronize()
    avg = device_time(launches, reps=max(1, 24 // copies))
    nb = N * K + 4 * N + 4 * M * K + 4 * M * N
    return {"avg_us": avg * 1e6, "bytes": nb, "GBps": nb / avg / 1e9, "frac_hbm": nb / avg / PEAK_HBM,
            "weight_sets": copies}


def bench_mx(fmt: str, M: int, K: int, N: int, dev, copies: int = 6):
    """MX linear y = x @ W.T through ``ccut.quant.mx.mx_linear`` (the
    decoded-weight MFMA kernel, W formed in registers, bf16 hi/lo products),
    ``copies`` distinct weights.  Algorithmic bytes: weight codes + E8M0
    scales (one per 32 columns) + 4*M*K (x) + 4*M*N (y)."""
    import torch

    from ccut.quant.mx import mx_linear

    g = torch.Generator(device=dev).manual_seed(17)
    row_bytes = K if fmt == "mxfp8" else K // 2
    ws = [torch.randint(0, 255, (N, row_bytes), generator=g, device=dev, dtype=torch.uint8) for _ in range(copies)]
    sc = torch.randint(120, 130, (N * K // 32,), generator=g, device=dev, dtype=torch.uint8)
    x = torch.randn((M, K), generator=g, device=dev)
    launches = [lambda w=w: mx_linear(w, sc, x, fmt, 32) for w in ws]
    launches[0]()
    torch.cuda.synchronize()
    avg = device_time(launches, reps=max(1, 24 // copies))
    nb = N * row_bytes + N * K // 32 + 4 * M * K + 4 * M * N
    return {"avg_us": avg * 1e6, "bytes": nb, "GBps": nb / avg / 1e9, "frac_hbm": nb / avg / PEAK_HBM}


def bench_int4_prefill(T: int, dev, sets: int = 4):
    """int4 (AWQ g128) MoE prefill layer: 128 experts, top-8 of a skewed
    router (logits N(0,1) + per-expert bias N(0,2)), hidden 2048, inter 768,
    bf16 activations; device time of whole ccq_moe_w4_ffn calls (align,
    grouped gate/up + SiLU, grouped down, combine) after routing, rotating
    over ``sets`` distinct weight sets (each routed set is 157-189 MB, so 4
    sets exceed the 256 MiB Infinity Cache)."""
    import torch

    from ccut import workloads as wl
    from ccut.blocks import moe

    Ep, Hp, Ip, k = 128, 2048, 768, 8
    exs = [moe.W4Experts.from_awq(wl.awq_experts(Ep, Hp, Ip, GROUP, seed=71 + 10 * i, device=dev),
                                  wl.awq_experts(Ep, Hp, Ip, GROUP, seed=72 + 10 * i, device=dev),
                                  wl.awq_experts(Ep, Ip, Hp, GROUP, seed=73 + 10 * i, device=dev), GROUP)
           for i in range(sets)]
    x = wl.activations(T, Hp, seed=74, device=dev)
    lg = wl.router_logits(T, Ep, seed=75, device=dev, skew_std=2.0)
    w, ids = moe.topk_softmax(lg, k, True)
    for ex in exs:
        moe.moe_ffn_w4(x, ids, w, ex)
    torch.cuda.synchronize()
    t = device_time([lambda ex=ex: moe.moe_ffn_w4(x, ids, w, ex) for ex in exs], reps=max(1, 12 // sets))
    uniq = int(torch.unique(ids).numel())
    flops = 2.0 * T * k * 3 * Hp * Ip
    nbytes = uniq * exs[0].bytes_per_expert + T * Hp * 2 * 2
    counts = torch.bincount(ids.reshape(-1), minlength=Ep)
    res = {"T": T, "us": t * 1e6, "TFLOPs": flops / t / 1e12, "frac_bf16_peak": flops / t / PEAK_BF16,
           "GBps": nbytes / t / 1e9, "frac_hbm": nbytes / t / PEAK_HBM, "experts_routed": uniq,
           "max_expert_rows": int(counts.max()), "min_expert_rows": int(counts.min()), "weight_sets": sets,
           "distinct_routed_bytes": sets * uniq * exs[0].bytes_per_expert}
    del exs
    torch.cuda.empty_cache()
    return res


def bench_fp8row_moe(T: int, dev):
    """MoE layer on experts in the reference checkpoint's own format (the
    Ornith layout: e4m3 [out, in] with one BF16 scale per output row):
    256 experts, top-8 (logits N(0,1)), hidden 2048, expert intermediate 512,
    float32 activations; device time of whole ccq_moe_fp8row_ffn calls after
    routing (align, gate/up + SiLU, down, combine).  One layer is 768 MiB;
    the calls rotate over routings of distinct random logits so that the
    experts read per rotation exceed 512 MiB (the 256 MiB Infinity Cache
    cannot serve repeats).  Algorithmic bytes: the routed experts' codes and
    BF16 row scales, x and y in float32."""
    import torch

    from ccut import workloads as wl
    from ccut.blocks import moe

    Ep, Hp, Ip, k = 256, 2048, 512, 8
    ex = moe.Fp8RowExperts.from_rows(wl.fp8_row_weights(Ep, Ip, Hp, seed=91, device=dev),
                                     wl.fp8_row_weights(Ep, Ip, Hp, seed=92, device=dev),
                                     wl.fp8_row_weights(Ep, Hp, Ip, seed=93, device=dev))
    x = wl.activations(T, Hp, seed=94, device=dev, dtype=torch.float32)
    rot = max(2, min(32, (512 << 20) // max(1, min(T * k, Ep) * ex.bytes_per_expert) + 1))
    routes, nb, seen = [], [], set()
    for i in range(rot):
        w, ids = moe.topk_softmax(wl.router_logits(T, Ep, seed=950 + i, device=dev), k, True)
        u = torch.unique(ids)
        seen.update(u.tolist())
        routes.append((w, ids))
        nb.append(int(u.numel()) * ex.bytes_per_expert + T * Hp * 4 * 2 + T * k * 12)
    for w, ids in routes:
        moe.moe_ffn_fp8row(x, ids, w, ex)
    torch.cuda.synchronize()
    t = device_time([lambda w=w, ids=ids: moe.moe_ffn_fp8row(x, ids, w, ex) for w, ids in routes],
                    reps=max(1, 32 // rot))
    b = sum(nb) / len(nb)
    res = {"T": T, "us": t * 1e6, "bytes": b, "GBps": b / t / 1e9, "frac_hbm": b / t / PEAK_HBM,
           "routings": rot, "distinct_bytes": len(seen) * ex.bytes_per_expert,
           "TFLOPs": 2.0 * T * k * 3 * Hp * Ip / t / 1e12}
    del ex
    torch.cuda.empty_cache()
    return res


def bench_fp8_prefill(dev, T: int = 2048):
    """FP8 e4m3 block-scaled (128x128 weight blocks, per-token-per-128
    activations) MoE prefill layer: 256 experts, top-8 (logits N(0,1)),
    hidden 7168, inter 2048, bf16 activations; device time of whole
    ccq_moe_fp8_ffn calls after routing.  HBM-bound: 11.3 GB of weights for
    1.44 TFLOP (arithmetic intensity ~128 FLOP/B < the FP8 ridge ~629)."""
    import torch

    from ccut import workloads as wl
    from ccut.blocks import moe

    Ep, Hp, Ip, k = 256, 7168, 2048, 8
    ex = moe.Fp8Experts.from_block(wl.fp8_block_weights(Ep, Ip, Hp, seed=81, device=dev),
                                   wl.fp8_block_weights(Ep, Ip, Hp, seed=82, device=dev),
                                   wl.fp8_block_weights(Ep, Hp, Ip, seed=83, device=dev))
    torch.cuda.empty_cache()
    x = wl.activations(T, Hp, seed=84, device=dev)
    lg = wl.router_logits(T, Ep, seed=85, device=dev)
    w, ids = moe.topk_softmax(lg, k, True)
    moe.moe_ffn_fp8(x, ids, w, ex)
    torch.cuda.synchronize()
    t = device_time([lambda: moe.moe_ffn_fp8(x, ids, w, ex)], reps=5)
    uniq = int(torch.unique(ids).numel())
    flops = 2.0 * T * k * 3 * Hp * Ip
    nbytes = uniq * ex.bytes_per_expert + T * Hp * 2 * 2
    roof = min(PEAK_FP8, flops / nbytes * PEAK_HBM)
    res = {"T": T, "us": t * 1e6, "TFLOPs": flops / t / 1e12, "frac_fp8_peak": flops / t / PEAK_FP8,
           "frac_roofline": flops / t / roof, "roofline_TFLOPs": roof / 1e12, "GBps": nbytes / t / 1e9,
           "frac_hbm": nbytes / t / PEAK_HBM, "experts_routed": uniq}
    del ex
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------- CPU baseline --
def _median_s(fn, runs: int = 5) -> float:
    """Median wall seconds of ``runs`` calls after one warmup call."""
    import statistics

    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _combine_subset(omoe, x, ids, w, lookup):
    """moe_combine over the assignments with an expert id >= 0 (the oracle's
    grouping and float32 weighted sum; -1 marks an assignment left out)."""
    import numpy as np

    out = np.zeros_like(x)
    for eid, toks in omoe.expert_order(ids).items():
        if eid < 0:
            continue
        wg, wu, wd = lookup(eid)
        y = omoe.expert_ffn(x[np.array(toks, dtype=np.int64)], wg, wu, wd)
        for i, t in enumerate(toks):
            out[t] += w[t, list(ids[t]).index(eid)] * y[i]
    return out


def cpu_baselines(runs: int = 5) -> dict:
    """The reference's algorithm on the host for every workload, in two
    variants: (i) ``dequant`` -- every call dequantizes the weights it uses to
    float32 and multiplies (WeightOnlyMethod.apply / expert_ffn on freshly
    dequantized experts, quant/weight_only.py:37-54, blocks/moe.py:122-174);
    (ii) ``cached`` -- float32 weights dequantized once, matmuls only (the
    LinearProj cache, models/generic.py:137-161).  The oracle's numpy
    restatement (kind "port"), BLAS and the per-expert dequants on all
    threads of this process's CPU affinity; median of ``runs`` after one
    warmup.  Expert weights come from a small pool of distinct experts reused
    by id (the work per call does not depend on which expert it is).  The
    FP8 layer is timed on its first 4 routed experts and extrapolated by
    assignment count (labelled), so is the int4 layer at T=4096 (its first
    8192 assignments)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    from oracle import awq as oawq
    from oracle import fp8_block as ofb
    from oracle import moe as omoe
    from oracle.ref_quant import silu_mul_fused

    cores = len(os.sched_getaffinity(0))
    os.environ["OMP_NUM_THREADS"] = str(cores)
    torch.set_num_threads(cores)
    rng = np.random.default_rng(3)
    out = {}
    pool = ThreadPoolExecutor(max_workers=cores)

    def awq_mat(K, N):
        q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
        z = rng.integers(0, 16, size=(K // GROUP, N), dtype=np.uint8)
        s = (np.abs(rng.standard_normal((K // GROUP, N))) * 0.01 + 1e-3).astype(np.float16)
        return oawq.pack(q), oawq.pack(z), s

    def entry(name, nbytes, flops, t_dequant, t_cached, sample, extrapolated=False):
        out[name] = {"dequant": {"s": t_dequant, "GBps": nbytes / t_dequant / 1e9, "TFLOPs": flops / t_dequant / 1e12},
                     "cached": {"s": t_cached, "GBps": nbytes / t_cached / 1e9, "TFLOPs": flops / t_cached / 1e12},
                     "bytes": nbytes, "flops": flops, "cores": cores, "kind": "port", "sample": sample,
                     "extrapolated": extrapolated}

    with threadpool_limits(cores):
        # single AWQ linears: GEMV K=2048 N=5632 and the skinny GEMM K=4096 N=14336
        for (M, K, N, name) in ((1, 2048, 5632, "awq_gemv_k2048_n5632"), (1, 4096, 14336, "awq_gemm_k4096_n14336_m1"),
                                (4, 4096, 14336, "awq_gemm_k4096_n14336_m4"),
                                (16, 4096, 14336, "awq_gemm_k4096_n14336_m16")):
            qw, qz, s = awq_mat(K, N)
            x = rng.standard_normal((M, K)).astype(np.float32)
            W = oawq.dequant(qw, qz, s, GROUP)
            chunks = [(r, min(K, r + 8 * GROUP)) for r in range(0, K, 8 * GROUP)]

            def dequant_par():  # row blocks of 8 groups on the worker threads
                parts = pool.map(lambda rc: oawq.dequant(qw[rc[0]:rc[1]], qz[rc[0] // GROUP:rc[1] // GROUP],
                                                         s[rc[0] // GROUP:rc[1] // GROUP], GROUP), chunks)
                return np.concatenate(list(parts), axis=0)

            td = _median_s(lambda: x @ dequant_par(), runs)
            tc = _median_s(lambda: x @ W, runs)
            nb = K * N // 2 + (K // GROUP) * N * 2 + (K // GROUP) * N // 2 + M * (K + N) * 2
            entry(name, nb, 2.0 * M * K * N, td, tc, f"x [{M}, {K}] @ W [{K}, {N}], one full call")
        # int4 MoE layers (decode T=1, 16; prefill T=512, 4096): the routed
        # experts in first-appearance order, up to max_a assignments of them
        # (the rest extrapolated by assignment count)
        for (T, Ep, Hp, Ip, k, skew, max_a, name) in ((16, E, HID, INTER, TOPK, 0.0, None, "moe_decode_T16"),
                                                      (1, E, HID, INTER, TOPK, 0.0, None, "moe_decode_T1"),
                                                      (512, 128, 2048, 768, 8, 2.0, None, "int4_moe_prefill_T512"),
                                                      (4096, 128, 2048, 768, 8, 2.0, 8192,
                                                       "int4_moe_prefill_T4096")):
            P = 4
            experts = [(awq_mat(Hp, Ip), awq_mat(Hp, Ip), awq_mat(Ip, Hp)) for _ in range(P)]
            cached = {e: tuple(oawq.dequant(*m, GROUP) for m in experts[e]) for e in range(P)}
            x = rng.standard_normal((T, Hp)).astype(np.float32)
            lg = rng.standard_normal((T, Ep)).astype(np.float32)
            if skew:
                lg = lg + rng.standard_normal((1, Ep)).astype(np.float32) * skew
            w, ids = omoe.topk_softmax(lg, k)
            order = omoe.expert_order(ids)
            routed, n_sub = [], 0
            for e, toks in order.items():
                if max_a is not None and n_sub >= max_a:
                    break
                routed.append(e)
                n_sub += len(toks)
            keep = np.isin(ids, routed)
            ids_s = np.where(keep, ids, -1)  # assignments outside the subset: no expert (contribute nothing)

            def lookup_of(mats):
                return lambda e: mats[e]

            def per_call():
                mats = dict(zip(routed, pool.map(lambda e: tuple(oawq.dequant(*m, GROUP) for m in experts[e % P]),
                                                 routed)))
                return _combine_subset(omoe, x, ids_s, w, lookup_of(mats))

            td = _median_s(per_call, runs)
            tc = _median_s(lambda: _combine_subset(omoe, x, ids_s, w, lambda e: cached[e % P]), runs)
            scale = T * k / n_sub
            per_expert = 2 * (Hp * Ip // 2 + (Hp // GROUP) * Ip * 2 + (Hp // GROUP) * Ip // 2) + \
                (Ip * Hp // 2 + (Ip // GROUP) * Hp * 2 + (Ip // GROUP) * Hp // 2)
            nb = len(order) * per_expert + T * Hp * 2 * 2
            sample = f"top-{k} of {Ep} experts, {len(order)} routed, T={T}, H={Hp}, I={Ip}: "
            sample += "the whole layer" if scale == 1 else \
                f"{len(routed)} experts ({n_sub} of {T * k} assignments) timed, x {scale:.2f} by assignment count"
            entry(name, nb, 2.0 * T * k * 3 * Hp * Ip, td * scale, tc * scale, sample, extrapolated=scale != 1)
        # FP8 block MoE prefill: 4 routed experts timed, extrapolated by assignments
        Ep, Hp, Ip, T, k = 256, 7168, 2048, 2048, 8
        lg = rng.standard_normal((T, Ep)).astype(np.float32)
        w, ids = omoe.topk_softmax(lg, k)
        order = omoe.expert_order(ids)
        sub = list(order)[:4]
        n_sub = sum(len(order[e]) for e in sub)
        x = rng.standard_normal((T, Hp)).astype(np.float32)
        P = 4

        def fp8_mat(N, K):
            return (rng.integers(0, 0x7E, size=(N, K), dtype=np.uint8),
                    (np.abs(rng.standard_normal((N // 128, K // 128))) * 0.01 + 1e-3).astype(np.float32))

        fexp = [(fp8_mat(Ip, Hp), fp8_mat(Ip, Hp), fp8_mat(Hp, Ip)) for _ in range(P)]
        fcached = {e: tuple(ofb.block_dequant(*m) for m in fexp[e]) for e in range(P)}

        def fp8_layer(deq):
            mats = dict(zip(sub, pool.map(lambda e: deq(e % P), sub)))
            for e in sub:
                rows = np.asarray(order[e])
                xq = ofb.act_dequant(*ofb.act_quant(x[rows]))
                g, u, d = mats[e]
                silu_mul_fused(xq @ g.T, xq @ u.T) @ d.T

        td = _median_s(lambda: fp8_layer(lambda i: tuple(ofb.block_dequant(*m) for m in fexp[i])), runs)
        tc = _median_s(lambda: fp8_layer(lambda i: fcached[i]), runs)
        scale = T * k / n_sub
        nb = len(order) * (3 * Hp * Ip + 3 * (Hp // 128) * (Ip // 128) * 4) + T * Hp * 2 * 2
        entry("fp8_moe_prefill_T2048", nb, 2.0 * T * k * 3 * Hp * Ip, td * scale, tc * scale,
              f"4 of {len(order)} routed experts ({n_sub} of {T * k} assignments) timed, x {scale:.1f} by "
              "assignment count", extrapolated=True)
    pool.shutdown()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path runs on a single MI355X); --gpus {args.gpus} is not "
              "supported", file=sys.stderr)
        sys.exit(2)
    import torch

    from ccut import _lib

    _lib.lib()
    dev = torch.device("cuda", 0)
    log(f"device {torch.cuda.get_device_name(0)}; MoE decode T={args.tokens}")
    head = bench_moe(args.tokens, args.steps, args.warmup, dev)
    gu = head["gate_up"]
    log(f"moe decode T={args.tokens}: {head['GBps']:.1f} GB/s, {head['ms_per_step'] * 1e3:.1f} us/step; "
        f"gate/up kernel {gu['avg_us']:.2f} us = {gu['GBps']:.1f} GB/s ({gu['back_to_back_us']:.2f} us per "
        "launch back to back)")
    extra = {}
    if not args.no_extra:
        t1 = bench_moe(1, args.steps, args.warmup, dev, n_layers=LAYERS_T1)
        extra["moe_decode_T1"] = t1
        log(f"moe decode T=1: {t1['GBps']:.1f} GB/s, {t1['ms_per_step'] * 1e3:.1f} us/step; gate/up kernel "
            f"{t1['gate_up']['avg_us']:.2f} us = {t1['gate_up']['GBps']:.1f} GB/s")
        for M in (1, 4, 16):
            r = bench_gemm(M, 4096, 14336, dev=dev, copies=24)
            extra[f"awq_gemm_k4096_n14336_m{M}"] = r
            log(f"awq gemm K=4096 N=14336 M={M}: {r['GBps']:.1f} GB/s ({r['avg_us']:.2f} us)")
        r = bench_moe_shared(16, dev)
        extra["moe_decode_T16_shared_expert"] = r
        log(f"MoE decode T=16 + shared expert in-kernel: {r['avg_us']:.2f} us, {r['GBps']:.1f} GB/s "
            f"({r['frac_hbm']:.3f} of HBM peak)")
        r = bench_gemm(1, 2048, 5632, dev=dev, copies=96)
        extra["awq_gemv_k2048_n5632"] = r
        log(f"awq gemv K=2048 N=5632: {r['GBps']:.1f} GB/s ({r['avg_us']:.2f} us)")
        for Tp in (512, 4096):
            r = bench_int4_prefill(Tp, dev)
            extra[f"int4_moe_prefill_T{Tp}"] = r
            log(f"int4 MoE prefill T={Tp}: {r['us']:.1f} us, {r['TFLOPs']:.1f} TFLOP/s "
                f"({r['frac_bf16_peak']:.3f} of bf16 peak), {r['GBps']:.0f} GB/s")
        for name, r in bench_quantizers(dev).items():
            extra[name] = r
            log(f"{name}: {r['GBps']:.0f} GB/s = {r['frac_hbm']:.3f} of HBM peak ({r['avg_us']:.2f} us)")
        for M, copies in ((1, 6), (16, 6), (4096, 1)):
            r = bench_int8(M, 4096, 14336, dev, copies=copies)
            extra[f"int8_w8a8_k4096_n14336_m{M}"] = r
            log(f"int8 w8a8 K=4096 N=14336 M={M}: {r['avg_us']:.2f} us, {r['GBps']:.0f} GB/s "
                f"({r['frac_hbm']:.3f} of HBM peak), {r['TOPs']:.1f} TOP/s ({r['frac_int8_peak']:.3f} of int8 peak)")
        for M in (1, 4, 16):
            r = bench_ref_fp8_linear(M, 4096, 14336, dev)
            extra[f"ref_fp8_rowscale_linear_k4096_n14336_m{M}"] = r
            log(f"reference FP8 per-row linear K=4096 N=14336 M={M}: {r['avg_us']:.2f} us, {r['GBps']:.0f} GB/s "
                f"({r['frac_hbm']:.3f} of HBM peak)")
        for fmt, M in (("mxfp4", 1), ("mxfp8", 1), ("mxfp4", 16), ("mxfp8", 16), ("mxfp4", 64)):
            r = bench_mx(fmt, M, 4096, 14336, dev)
            extra[f"{fmt}_linear_k4096_n14336_m{M}"] = r
            log(f"{fmt} linear K=4096 N=14336 M={M}: {r['avg_us']:.2f} us, {r['GBps']:.0f} GB/s "
                f"({r['frac_hbm']:.3f} of HBM peak)")
        for Tr in (1, 16, 512):
            r = bench_fp8row_moe(Tr, dev)
            extra[f"fp8row_moe_ornith_T{Tr}"] = r
            log(f"fp8 per-row (checkpoint format) MoE layer T={Tr}: {r['us']:.1f} us, {r['GBps']:.0f} GB/s "
                f"({r['frac_hbm']:.3f} of HBM peak)")
        r = bench_fp8_prefill(dev)
        extra["fp8_moe_prefill_T2048"] = r
        log(f"fp8 block MoE prefill T=2048: {r['us']:.1f} us, {r['TFLOPs']:.1f} TFLOP/s ({r['frac_fp8_peak']:.3f} "
            f"of fp8 peak, {r['frac_roofline']:.3f} of its HBM roofline), {r['GBps']:.0f} GB/s")
    cpu = None
    if not args.no_cpu:
        log("cpu baselines (the reference algorithm on the host)")
        cpus = cpu_baselines()
        extra["cpu_baselines"] = cpus
        hd = cpus[f"moe_decode_T{args.tokens}"] if f"moe_decode_T{args.tokens}" in cpus else cpus["moe_decode_T16"]
        cpu = {"value": round(hd["dequant"]["GBps"], 4), "unit": "GB/s", "cores": hd["cores"], "kind": "port",
               "sample": "the MoE decode layer (64 experts, top-6, H=2048, I=1408, AWQ g128, T=16): numpy oracle, "
                         "per-call dequant of every routed expert to float32 (parallel over experts) + BLAS "
                         f"matmuls + per-expert grouping, median of 5 after a warmup, {hd['cores']} threads",
               "cached_fp32_value": round(hd["cached"]["GBps"], 4)}
        for name, r in cpus.items():
            log(f"cpu {name}: dequant {r['dequant']['s'] * 1e3:.1f} ms, cached {r['cached']['s'] * 1e3:.1f} ms"
                + (" (extrapolated)" if r["extrapolated"] else ""))
    out = {
        "metric": METRIC,
        "value": round(head["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights (AWQ g128), bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded; no checkpoints offline)",
        "config": {"workload": f"int4 MoE expert FFN decode: 64 experts top-6, hidden 2048, inter 1408, "
                               f"AWQ group 128, T={args.tokens}, 4 rotating layer weight sets",
                   "tokens": args.tokens, "experts": E, "top_k": TOPK, "hidden": HID, "inter": INTER,
                   "group": GROUP, "hip_graph": True},
        "frac_hbm_peak": round(head["GBps"] * 1e9 / PEAK_HBM, 4),
        "roofline": {"bound": "hbm",
                     "kernel": "w4_stream_kernel<bf16,f16,SiLU,MT=2,NQ=2,ROUTE=1> (MoE gate/up, routed in-kernel)",
                     "achieved": round(gu["GBps"], 2), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(gu["GBps"] * 1e9 / PEAK_HBM, 4), "avg_us": round(gu["avg_us"], 3),
                     "algorithmic_bytes": round(gu["bytes"]),
                     "traffic": round(gu["bytes"] * GATE_UP_TRAFFIC_RATIO)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

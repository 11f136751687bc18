"""One MoE step as the reference's ``ExpertPipeline.step`` (reference
``python/ccut/experts/pipeline.py:34-204``), same names, arguments and
metrics, on the GPU operators of this package.

A step: speculative prefetch from the route history, the router
``x @ gate_w.T`` (``ccq_f32_gemm``), ``topk_softmax``, prefetch of the
routed experts, the experts' FFN with the weighted combine, the shared expert
and the metrics.  The expert weights come from ``reader`` in one of two ways:

* ``reader.experts(layer)`` returning a whole layer in device format
  (``W4Experts``, ``Fp8Experts`` or ``Fp8RowExperts``): one fused call
  (``moe_ffn_w4`` / ``moe_ffn_fp8`` / ``moe_ffn_fp8row``); activations go
  to the int4 kernels as bfloat16, to the per-row FP8 kernels (the
  reference checkpoint's own format) as float32.
* otherwise ``reader.get(layer, eid, timeout)`` per routed expert returning
  float32 ``(w_gate [hidden, inter], w_up [hidden, inter], w_down [inter,
  hidden])``, the orientation ``expert_ffn`` takes, then ``expert_ffn``
  and the weighted add over all of them in one grouped call
  (``moe_combine`` -> ``ccq_moe_f32_ffn``; reference
  ``pipeline.py:155-179`` loops over the experts).  Weights
  of any other shape raise ``ValueError`` (the reference's reader hands over
  ``[out, in]`` slots here, ``pipeline.py:160-170``; this package's
  ``ExpertReader`` returns ``[in, out]``).

An expert whose read raises ``TimeoutError`` is handled by
``on_expert_timeout``: ``"renormalize"`` (default) leaves it out and
rescales each affected token's surviving routing weights so they keep the
token's original weight sum -- the redistribution the reference's comment
at ``pipeline.py:161`` describes, where its code only skips the expert;
``"drop"`` leaves it out with the other weights unchanged (what the
reference's code does); ``"raise"`` re-raises.  Timed-out experts and the
assignments left out are counted in ``metrics.expert_timeouts`` /
``metrics.dropped_assignments``.

``reader.prefetch(layer, ids)``, ``reader.stats()`` and ``reader.close()``
are called when the reader has them.
"""

from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass
from typing import Iterable

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call, lib
from ccut.blocks import moe

__all__ = ["PipelineMetrics", "ExpertPipeline", "RouteHistory"]


@dataclass
class PipelineMetrics:
    """Timings of the step's stages (reference ``pipeline.py:34-63``)."""

    compute_ns: int = 0
    prefetch_ns: int = 0
    overlap_ns: int = 0
    steps: int = 0
    speculative_correct: int = 0
    speculative_total: int = 0
    ring_hits: int = 0
    ring_misses: int = 0
    ring_evicted: int = 0
    expert_timeouts: int = 0
    dropped_assignments: int = 0

    def overlap_ratio(self) -> float:
        return self.overlap_ns / self.compute_ns if self.compute_ns > 0 else 0.0

    def speculative_accept_rate(self) -> float:
        return self.speculative_correct / self.speculative_total if self.speculative_total > 0 else 0.0

    def to_dict(self) -> dict:
        return {
            "compute_ns": self.compute_ns,
            "prefetch_ns": self.prefetch_ns,
            "overlap_ns": self.overlap_ns,
            "overlap_ratio": round(self.overlap_ratio(), 4),
            "steps": self.steps,
            "spec_accept_rate": round(self.speculative_accept_rate(), 4),
            "ring_hits": self.ring_hits,
            "ring_misses": self.ring_misses,
            "expert_timeouts": self.expert_timeouts,
            "dropped_assignments": self.dropped_assignments,
        }


class RouteHistory:
    """Sliding window of routing decisions (reference ``pipeline.py:66-84``):
    ``predict`` returns the experts seen most often in the window, most
    frequent first (ties in first-seen order)."""

    def __init__(self, window: int = 4):
        self.window = window
        self._hist: deque[set[int]] = deque(maxlen=window)

    def record(self, topk_ids: Iterable[int]) -> None:
        self._hist.append(set(int(x) for x in topk_ids))

    def predict(self, top_k: int) -> list[int]:
        if not self._hist:
            return []
        counts: dict[int, int] = {}
        for step in self._hist:
            for e in step:
                counts[e] = counts.get(e, 0) + 1
        return [e for e, _ in sorted(counts.items(), key=lambda kv: -kv[1])[:top_k]]


class ExpertPipeline:
    """Routing + expert FFN + combine + shared expert per step (reference
    ``pipeline.py:87-208``)."""

    def __init__(self, reader, num_workers: int = 2, speculative_window: int = 4, prefetch_steps_ahead: int = 2,
                 metrics_enabled: bool = True, on_expert_timeout: str = "renormalize"):
        if on_expert_timeout not in ("renormalize", "drop", "raise"):
            raise ValueError(f"on_expert_timeout={on_expert_timeout!r}: expected 'renormalize', 'drop' or 'raise'")
        self.on_expert_timeout = on_expert_timeout
        self.reader = reader
        self.num_workers = num_workers
        self.prefetch_steps_ahead = prefetch_steps_ahead
        self.metrics = PipelineMetrics() if metrics_enabled else None
        self.history = RouteHistory(window=speculative_window)

    def _prefetch(self, layer: int, ids: list[int]):
        fn = getattr(self.reader, "prefetch", None)
        return fn(layer, ids) if fn is not None else 0

    @staticmethod
    def router_logits(x, gate_w) -> torch.Tensor:
        """The router ``x @ gate_w.T`` in float32 (reference
        ``pipeline.py:145``) as a device tensor [T, E]: ``ccq_f32_gemm`` with
        ``gate_w`` as stored ([E, H]), float32 products on the fp32 matrix
        cores."""
        xd = _dev.to_device(x, torch.float32).contiguous()
        gw = _dev.to_device(gate_w, torch.float32).contiguous()
        if xd.dim() != 2 or gw.dim() != 2 or xd.shape[1] != gw.shape[1]:
            raise ValueError(f"router: x {tuple(xd.shape)} and gate_w {tuple(gw.shape)} must be [T, H] and [E, H]")
        T, H = xd.shape
        E = gw.shape[0]
        logits = torch.empty((T, E), dtype=torch.float32, device=xd.device)
        nbytes = lib().ccq_f32_gemm_workspace_size(T, H, E)
        ws = _dev.workspace("f32_gemm", nbytes, xd.device) if nbytes else None
        call("ccq_f32_gemm", xd.data_ptr(), gw.data_ptr(), logits.data_ptr(), T, H, E, 1,
             ws.data_ptr() if ws is not None else None, nbytes, _dev.stream_ptr(xd.device))
        return logits

    def step(self, layer: int, x, gate_w, top_k: int = 8, norm_topk_prob: bool = True,
             shared_projs: dict | None = None, shared_gate: float = 1.0):
        """``y [T, hidden]`` float32 for ``x [T, hidden]``: numpy in, numpy
        out; a device tensor in, a device tensor out."""
        t0 = time.monotonic_ns()
        if self.metrics and self.prefetch_steps_ahead > 0:  # speculative prefetch
            pred = self.history.predict(top_k)
            if pred:
                self.metrics.speculative_total += 1
                if self._prefetch(layer, pred):
                    self.metrics.speculative_correct += 1
        xd = _dev.to_device(x, torch.float32)
        if xd.dim() != 2:
            raise ValueError(f"x must be [T, hidden], got {tuple(xd.shape)}")
        logits = self.router_logits(xd, gate_w)
        weights, ids = moe.topk_softmax(logits, top_k, norm_topk_prob)
        ids_h = ids.cpu().numpy()
        self.history.record(ids_h[0])  # the first token's experts, as the reference records
        flat_ids = ids_h.reshape(-1).tolist()
        t_pf0 = time.monotonic_ns()
        self._prefetch(layer, flat_ids)
        # the shared expert first, so that its add rides in the combine's
        # epilogue; its time counts as prefetch time, as in the reference
        s_out, shared_ns = None, 0
        if shared_projs is not None and "gate_proj" in shared_projs:
            ts0 = time.monotonic_ns()
            s = shared_projs["gate_proj"].apply(x)
            su = shared_projs["up_proj"].apply(x)
            from ccut.quant import kernels as qk

            inter = qk.silu_mul_fused(s, su, None)
            s_out = _dev.to_device(shared_projs["down_proj"].apply(inter), torch.float32).contiguous()
            shared_ns = time.monotonic_ns() - ts0
        t_c0 = time.monotonic_ns()
        layer_experts = getattr(self.reader, "experts", None)
        ex = layer_experts(layer) if layer_experts is not None else None
        shared_done = False
        if isinstance(ex, moe.W4Experts):
            out = moe.moe_ffn_w4(xd.to(torch.bfloat16), ids, weights, ex, out_dtype=torch.float32,
                                 shared=s_out, shared_gate=shared_gate)
            shared_done = True
        elif isinstance(ex, moe.Fp8Experts):
            out = moe.moe_ffn_fp8(xd, ids, weights, ex, out_dtype=torch.float32, shared=s_out,
                                  shared_gate=shared_gate)
            shared_done = True
        elif isinstance(ex, moe.Fp8RowExperts):
            out = moe.moe_ffn_fp8row(xd, ids, weights, ex, out_dtype=torch.float32, shared=s_out,
                                     shared_gate=shared_gate)
            shared_done = True
        elif ex is not None:
            raise TypeError(f"reader.experts({layer}) returned {type(ex).__name__}, "
                            "expected W4Experts, Fp8Experts or Fp8RowExperts")
        else:
            out, shared_done = self._per_expert(layer, xd, ids, weights, flat_ids, s_out, shared_gate)
        if s_out is not None and not shared_done:
            moe.shared_expert_add(out, s_out, shared_gate)
        torch.cuda.synchronize(xd.device)
        t_c1 = time.monotonic_ns()
        t1 = time.monotonic_ns()
        if self.metrics is not None:
            compute = t_c1 - t_c0
            prefetch = t_pf0 - t0 + (t1 - t_c1) + shared_ns
            self.metrics.compute_ns += compute
            self.metrics.prefetch_ns += prefetch
            self.metrics.overlap_ns += min(compute, prefetch)
            self.metrics.steps += 1
            stats = getattr(self.reader, "stats", None)
            if stats is not None:
                st = stats()
                self.metrics.ring_hits = st.get("hits", 0)
                self.metrics.ring_misses = st.get("misses", 0)
        return _dev.to_host(out) if _dev.is_host(x) else out

    def _per_expert(self, layer: int, xd: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                    flat_ids: list[int], s_out, shared_gate: float):
        """The reference's per-expert path (``pipeline.py:155-179``): each
        routed expert's float32 weights from ``reader.get``, then
        ``expert_ffn`` + the weighted add for all of them in one grouped
        ``moe_combine`` call; timeouts as ``on_expert_timeout`` says."""
        H = xd.shape[1]
        resolved: dict[int, tuple] = {}
        for eid in sorted(set(e for e in flat_ids if e >= 0)):
            try:
                wg, wu, wd = self.reader.get(layer, int(eid), timeout=30.0)
            except TimeoutError:
                if self.on_expert_timeout == "raise":
                    raise
                if self.metrics is not None:
                    self.metrics.expert_timeouts += 1
                continue
            I = wg.shape[1] if wg.ndim == 2 else -1
            if tuple(wg.shape) != (H, I) or tuple(wu.shape) != (H, I) or tuple(wd.shape) != (I, H):
                raise ValueError(f"reader.get({layer}, {eid}): expert weights gate {tuple(wg.shape)}, up "
                                 f"{tuple(wu.shape)}, down {tuple(wd.shape)}; expected gate/up [hidden={H}, inter] "
                                 f"and down [inter, hidden={H}]")
            resolved[eid] = (wg, wu, wd)
        missing = set(e for e in flat_ids if e >= 0) - set(resolved)
        ids_used, w_used = ids, weights
        if missing:
            ids_used = ids.clone()
            for eid in missing:
                ids_used[ids_used == eid] = -1
            kept = ids_used >= 0
            if self.metrics is not None:
                self.metrics.dropped_assignments += int((~kept & (ids >= 0)).sum().item())
            if self.on_expert_timeout == "renormalize":
                w_kept = torch.where(kept, weights, torch.zeros_like(weights))
                total = torch.where(ids >= 0, weights, torch.zeros_like(weights)).sum(dim=1, keepdim=True)
                left = w_kept.sum(dim=1, keepdim=True)
                scale = torch.where(left != 0, total / torch.where(left != 0, left, torch.ones_like(left)),
                                    torch.zeros_like(left))
                w_used = (w_kept * scale).contiguous()
        if resolved:
            out = moe.moe_combine(xd, ids_used, w_used, w_lookup=resolved.__getitem__, shared=s_out,
                                  shared_gate=shared_gate)
            return out, True
        return torch.zeros_like(xd), False

    def close(self) -> None:
        close = getattr(self.reader, "close", None)
        if close is not None:
            close()

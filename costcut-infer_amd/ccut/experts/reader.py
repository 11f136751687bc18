"""Expert weight reader over an expert index (reference
``python/ccut/experts/reader.py:38-340``): per-layer rings of ready experts,
background workers that fill them on ``prefetch``, ``get`` that waits for a
fill and raises ``TimeoutError`` rather than returning stale weights.

A slot holds one expert's ``(gate, up, down)`` as float32 device tensors,
dequantized on the GPU from the checkpoint segments:

* ``F8_E4M3`` / ``F8_E5M2`` weight ``[out, in]`` with an optional per-row
  scale (``weight_scale`` / ``_scale``, ``[out]`` or ``[out, 1]``, BF16 /
  F16 / F32): ``fp8_dequant_mat`` (``ccq_fp8_dequant``); E5M2 is decoded by
  torch;
* ``F8_E4M3`` weight ``[out, in]`` with 128x128 block scales
  (``weight_scale_inv`` or ``weight_scale`` of shape ``[ceil(out/128),
  ceil(in/128)]``, F32 / BF16): ``ccq_fp8_block_dequant``;
* ``BF16`` / ``F16`` / ``F32`` weight: converted to float32;
* AWQ ``qweight`` / ``qzeros`` / ``scales`` (int32 ``[K, N/8]``, int32
  ``[K/G, N/8]``, F16/BF16 ``[K/G, N]``), or the same packing under the
  compressed-tensors group names ``weight`` (I32) / ``zero_points`` /
  ``scales``: ``ccq_awq_dequant`` to ``[K, N]``.

Every slot is in ``expert_ffn``'s orientation, ``[in, out]``: gate/up
``[hidden, inter]``, down ``[inter, hidden]`` (reference
``blocks/moe.py:122-141``).  FP8 and float checkpoints store ``[out, in]``
and are transposed once when the slot is filled; AWQ is ``[in, out]``
already.  (The reference's reader keeps the checkpoint's ``[out, in]`` and
its pipeline hands those slots to ``expert_ffn`` untransposed,
``experts/pipeline.py:170``: a shape error, or ``x @ W`` in place of
``x @ W.T`` when hidden == inter.)

``experts(layer)`` additionally hands over a whole layer in a fused
kernels' device format, built once per layer, which ``ExpertPipeline``
uses instead of per-expert reads: an AWQ layer as ``W4Experts``, a
block-FP8 layer as ``Fp8Experts`` (hidden and inter multiples of 128), and
the reference checkpoint's own format -- e4m3 ``[out, in]`` with per-row
scales, hidden and inter multiples of 256 -- as ``Fp8RowExperts`` (the
codes in place, scales widened to float32).
"""

from __future__ import annotations

import os
import threading
import time
from pathlib import Path

import numpy as np
import torch

from ccut import _dev
from ccut.experts.index import ExpertEntry, ExpertIndex, read_header

__all__ = ["ExpertReader", "ExpertRing", "RingFullError"]


class RingFullError(RuntimeError):
    """No slot can take another expert (reference ``reader.py:38-40``)."""


class _Slot:
    __slots__ = ("expert_id", "layer", "gate", "up", "down", "ready", "seq", "filling")

    def __init__(self, layer: int):
        self.expert_id, self.layer = -1, layer
        self.gate = self.up = self.down = None
        self.ready, self.seq, self.filling = False, 0, False


class ExpertRing:
    """Fixed slots of one layer, refilled round robin (reference ``reader.py:55-83``)."""

    def __init__(self, layer: int, slots: int):
        if slots < 1:
            raise ValueError(f"ring needs at least one slot, got {slots}")
        self.layer = layer
        self.slots = [_Slot(layer) for _ in range(slots)]
        self._next = 0

    def find(self, expert_id: int) -> _Slot | None:
        for s in self.slots:
            if s.ready and s.expert_id == expert_id:
                return s
        return None

    def take_slot(self) -> _Slot | None:
        """The next slot in round-robin order that no worker is filling (None
        when every slot is being filled)."""
        for _ in range(len(self.slots)):
            s = self.slots[self._next]
            self._next = (self._next + 1) % len(self.slots)
            if not s.filling:
                return s
        return None

    def invalidate(self, expert_id: int) -> None:
        for s in self.slots:
            if s.expert_id == expert_id:
                s.ready, s.expert_id = False, -1


_FLOAT_DTYPES = {"BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32}


class ExpertReader:
    def __init__(self, index: ExpertIndex, model_dir: str | Path, num_layers: int, ring_slots: int = 2,
                 verify_crc: bool = False, num_workers: int = 2, device: torch.device | None = None):
        self.index = index
        self.model_dir = Path(model_dir)
        self.device = device if device is not None else _dev.require_gpu()
        self.rings = {l: ExpertRing(l, ring_slots) for l in range(num_layers)}
        self._verify_crc = verify_crc  # accepted for signature parity; safetensors carries no checksums
        self._fds: dict[str, tuple[int, int]] = {}  # shard -> (fd, data start)
        self._cv = threading.Condition()
        self._queue: list[tuple[int, int]] = []
        self._pending: set[tuple[int, int]] = set()
        self._failed: dict[tuple[int, int], str] = {}
        self._seq = 0
        self._stop = False
        self._layers: dict[int, object] = {}
        self._stats = {"reads": 0, "hits": 0, "misses": 0, "prefetches": 0, "stale": 0}
        self._workers = [threading.Thread(target=self._worker, name=f"expert-prefetch-{w}", daemon=True)
                         for w in range(max(1, num_workers))]
        for t in self._workers:
            t.start()

    # ---- segment IO ----
    def _shard_fd(self, shard: str) -> tuple[int, int]:
        with self._cv:
            got = self._fds.get(shard)
            if got is None:
                path = self.model_dir / shard
                start, _ = read_header(path)
                got = (os.open(path, os.O_RDONLY), start)
                self._fds[shard] = got
            return got

    def _read(self, entry: ExpertEntry, key: str) -> tuple[np.ndarray, str, tuple[int, ...]]:
        off, length, _, dtype = entry.segments[key]
        fd, start = self._shard_fd(entry.shard)
        raw = os.pread(fd, length, start + off)
        if len(raw) != length:
            raise OSError(f"{entry.shard}: short read of {key} ({len(raw)} of {length} bytes)")
        return np.frombuffer(raw, dtype=np.uint8), dtype, tuple(entry.shapes.get(key, ()))

    @staticmethod
    def _pick(segs: dict, proj: str, suffixes: tuple[str, ...]) -> str | None:
        for base in (f"{proj}_proj", proj):
            for suf in suffixes:
                if base + suf in segs:
                    return base + suf
        return None

    def _awq_keys(self, segs: dict, proj: str) -> tuple[str, str, str] | None:
        """(weight, zeros, scales) segment keys of an AWQ-packed projection:
        AutoAWQ names, or the compressed-tensors group names."""
        qkey = self._pick(segs, proj, (".qweight",))
        if qkey is not None:
            base = qkey[: -len(".qweight")]
            return qkey, base + ".qzeros", base + ".scales"
        zkey = self._pick(segs, proj, (".zero_points",))
        if zkey is not None:
            base = zkey[: -len(".zero_points")]
            wkey = base + ".weight" if base + ".weight" in segs else base
            if wkey in segs and segs[wkey][3] in ("I32", "U32") and base + ".scales" in segs:
                return wkey, zkey, base + ".scales"
        return None

    def _fp8_scale(self, entry: ExpertEntry, proj: str, rows: int, cols: int):
        """("row", [rows] f32) or ("block", [ceil(rows/128), ceil(cols/128)]
        f32) or ("row", ones) when the projection has no scale tensor."""
        skey = self._pick(entry.segments, proj, (".weight_scale_inv", ".weight_scale", "_scale"))
        if skey is None:
            return "row", torch.ones(rows, dtype=torch.float32, device=self.device)
        sc = self._device_tensor(entry, skey).float()
        shape = tuple(sc.shape)
        if sc.numel() == rows and (len(shape) <= 1 or shape[-1] == 1):
            return "row", sc.reshape(-1)
        blocks = (-(-rows // 128), -(-cols // 128))
        if shape == blocks:
            return "block", sc.contiguous()
        raise ValueError(f"{proj}: scale {skey} of shape {shape} for a [{rows}, {cols}] weight (expected "
                         f"[{rows}] / [{rows}, 1] per row or {list(blocks)} per 128x128 block)")

    def _dequant(self, entry: ExpertEntry, proj: str) -> torch.Tensor:
        """One projection as float32 ``[in, out]`` on the device."""
        segs = entry.segments
        keys = self._awq_keys(segs, proj)
        if keys is not None:
            from ccut.quant import awq

            qw, qz, sc = (self._device_tensor(entry, k) for k in keys)
            K = qw.shape[0]
            return awq.dequant(qw, qz, sc, K // sc.shape[0]).float()
        wkey = self._pick(segs, proj, (".weight", ""))
        if wkey is None:
            raise KeyError(f"no {proj} weight segment among {sorted(segs)}")
        raw, dtype, shape = self._read(entry, wkey)
        rows, cols = _shape_2d(int(entry.segments[wkey][2]), shape)
        if dtype in ("F8_E4M3", "F8_E5M2"):
            kind, scale = self._fp8_scale(entry, proj, rows, cols)
            w = torch.from_numpy(raw.copy()).to(self.device).reshape(rows, cols)
            if kind == "block":
                if dtype != "F8_E4M3":
                    raise NotImplementedError(f"{proj}: block scales with {dtype} weights")
                from ccut.quant import fp8_block

                return fp8_block.dequant(w, scale).T.contiguous()
            if dtype == "F8_E4M3":
                from ccut.quant import kernels as qk

                out = torch.empty((rows, cols), dtype=torch.float32, device=self.device)
                return qk.fp8_dequant_mat(w, scale, out).T.contiguous()
            return (w.view(torch.float8_e5m2).float() * scale[:, None]).T.contiguous()
        if dtype in _FLOAT_DTYPES:
            t = torch.from_numpy(raw.copy()).view(_FLOAT_DTYPES[dtype]).reshape(rows, cols)
            return t.to(self.device).float().T.contiguous()
        raise NotImplementedError(f"expert segment dtype {dtype} is not supported")

    def _device_tensor(self, entry: ExpertEntry, key: str) -> torch.Tensor:
        raw, dtype, shape = self._read(entry, key)
        tdt = {"I32": torch.int32, "U32": torch.int32, **_FLOAT_DTYPES}.get(dtype)
        if tdt is None:
            raise NotImplementedError(f"segment {key} of dtype {dtype}")
        return torch.from_numpy(raw.copy()).view(tdt).reshape(shape or (-1,)).to(self.device)

    # ---- slots ----
    def _fill(self, layer: int, expert_id: int, slot: _Slot) -> None:
        entry = self.index.entries[(layer, expert_id)]
        g, u, d = (self._dequant(entry, p) for p in ("gate", "up", "down"))
        torch.cuda.synchronize(self.device)
        with self._cv:
            self._seq += 1
            slot.expert_id, slot.layer = expert_id, layer
            slot.gate, slot.up, slot.down = g, u, d
            slot.ready, slot.seq = True, self._seq
            self._stats["reads"] += 1

    def _worker(self) -> None:
        while True:
            with self._cv:
                while not self._queue and not self._stop:
                    self._cv.wait()
                if self._stop:
                    return
                layer, eid = self._queue.pop(0)
                ring = self.rings[layer]
                if ring.find(eid) is not None:
                    self._pending.discard((layer, eid))
                    self._cv.notify_all()
                    continue
                slot = ring.take_slot()
                if slot is None:  # every slot of the layer is being filled: wait for one
                    self._queue.insert(0, (layer, eid))
                    self._cv.wait(timeout=0.5)
                    continue
                slot.ready, slot.filling = False, True  # never handed out half written
            try:
                self._fill(layer, eid, slot)
            except Exception as exc:  # the waiting get() times out; the reason is kept
                with self._cv:
                    slot.expert_id = -1
                    self._failed[(layer, eid)] = repr(exc)
            with self._cv:
                slot.filling = False
                self._pending.discard((layer, eid))
                self._cv.notify_all()

    def _enqueue(self, layer: int, eid: int) -> bool:
        key = (layer, eid)
        if key in self._pending or self._stop:
            return False
        if (layer, eid) not in self.index.entries:
            self._failed[key] = "not in the expert index"
            return False
        self._queue.append(key)
        self._pending.add(key)
        self._stats["prefetches"] += 1
        self._cv.notify_all()
        return True

    def prefetch(self, layer: int, expert_ids) -> int:
        """Queue the experts that are neither ready nor queued; returns how many were queued."""
        n = 0
        with self._cv:
            ring = self.rings[layer]
            for eid in expert_ids:
                if ring.find(int(eid)) is not None:
                    self._stats["hits"] += 1
                elif self._enqueue(layer, int(eid)):
                    n += 1
        return n

    def get(self, layer: int, expert_id: int, timeout: float = 30.0):
        """``(gate [hidden, inter], up [hidden, inter], down [inter, hidden])``
        float32 device tensors of a ready expert, waiting for its fill;
        ``TimeoutError`` when it is not ready in time."""
        deadline = time.monotonic() + timeout
        with self._cv:
            ring = self.rings[layer]
            s = ring.find(expert_id)
            if s is not None:
                self._stats["hits"] += 1
                return s.gate, s.up, s.down
            self._stats["misses"] += 1
            self._failed.pop((layer, expert_id), None)
            self._enqueue(layer, expert_id)
            while True:
                s = ring.find(expert_id)
                if s is not None:
                    return s.gate, s.up, s.down
                if (layer, expert_id) not in self._pending and (layer, expert_id) not in self._failed:
                    # filled and already refilled for another expert before
                    # this thread woke: queue it again
                    self._enqueue(layer, expert_id)
                left = deadline - time.monotonic()
                if left <= 0:
                    why = self._failed.get((layer, expert_id))
                    raise TimeoutError(f"expert (layer={layer}, expert={expert_id}) not ready after {timeout}s"
                                       + (f": {why}" if why else ""))
                self._cv.wait(timeout=min(left, 0.5))

    def experts(self, layer: int):
        """The whole layer as ``W4Experts`` (AWQ segments), ``Fp8Experts``
        (e4m3 segments with 128x128 block scales, hidden and inter multiples
        of 128) or ``Fp8RowExperts`` (e4m3 with per-row scales, multiples of
        256), built once; None when the layer is in another format
        (per-expert reads)."""
        if layer in self._layers:
            return self._layers[layer]
        e0 = self.index.get(layer, 0)
        ex = None
        if e0 is not None and self._awq_keys(e0.segments, "gate") is not None:
            from ccut.blocks import moe

            def stack(proj):
                parts = []
                for eid in range(self.index.num_experts):
                    entry = self.index.entries[(layer, eid)]
                    parts.append([self._device_tensor(entry, k) for k in self._awq_keys(entry.segments, proj)])
                return tuple(torch.stack([p[i] for p in parts]) for i in range(3))

            gate, up, down = stack("gate"), stack("up"), stack("down")
            K = gate[0].shape[1]
            ex = moe.W4Experts.from_awq(gate, up, down, group_size=K // gate[2].shape[1])
        elif e0 is not None and self._is_fp8_block(e0):
            from ccut.blocks import moe

            def stack_fp8(proj):
                ws, ss = [], []
                for eid in range(self.index.num_experts):
                    entry = self.index.entries[(layer, eid)]
                    wkey = self._pick(entry.segments, proj, (".weight", ""))
                    raw, _, shape = self._read(entry, wkey)
                    rows, cols = _shape_2d(int(entry.segments[wkey][2]), shape)
                    kind, sc = self._fp8_scale(entry, proj, rows, cols)
                    if kind != "block":
                        raise ValueError(f"layer {layer} expert {eid} {proj}: per-row scales in a block-FP8 layer")
                    ws.append(torch.from_numpy(raw.copy()).to(self.device).reshape(rows, cols))
                    ss.append(sc)
                return torch.stack(ws), torch.stack(ss)

            ex = moe.Fp8Experts.from_block(stack_fp8("gate"), stack_fp8("up"), stack_fp8("down"))
        elif e0 is not None and self._is_fp8_row(e0):
            from ccut.blocks import moe

            def stack_rows(proj):
                ws, ss = [], []
                for eid in range(self.index.num_experts):
                    entry = self.index.entries[(layer, eid)]
                    wkey = self._pick(entry.segments, proj, (".weight", ""))
                    raw, dtype, shape = self._read(entry, wkey)
                    if dtype != "F8_E4M3":
                        raise ValueError(f"layer {layer} expert {eid} {proj}: {dtype} weight in an F8_E4M3 layer")
                    rows, cols = _shape_2d(int(entry.segments[wkey][2]), shape)
                    kind, sc = self._fp8_scale(entry, proj, rows, cols)
                    if kind != "row":
                        raise ValueError(f"layer {layer} expert {eid} {proj}: block scales in a per-row FP8 layer")
                    ws.append(torch.from_numpy(raw.copy()).to(self.device).reshape(rows, cols))
                    ss.append(sc)
                return torch.stack(ws), torch.stack(ss)

            ex = moe.Fp8RowExperts.from_rows(stack_rows("gate"), stack_rows("up"), stack_rows("down"))
        self._layers[layer] = ex
        return ex

    def _is_fp8_row(self, entry: ExpertEntry) -> bool:
        """e4m3 gate/up/down weights with one scale per output row (or none),
        in shapes the fused per-row kernels take (hidden and inter multiples
        of 256): the reference checkpoint's own expert format."""
        for proj in ("gate", "up", "down"):
            wkey = self._pick(entry.segments, proj, (".weight", ""))
            if wkey is None or entry.segments[wkey][3] != "F8_E4M3":
                return False
            shape = tuple(entry.shapes.get(wkey, ()))
            if len(shape) != 2 or shape[0] % 256 or shape[1] % 256:
                return False
            try:
                kind, _ = self._fp8_scale(entry, proj, shape[0], shape[1])
            except ValueError:
                return False
            if kind != "row":
                return False
        return True

    def _is_fp8_block(self, entry: ExpertEntry) -> bool:
        """e4m3 gate weight with 128x128 block scales, shapes the fused FP8
        kernels take (both dimensions multiples of 128, at least 256)."""
        wkey = self._pick(entry.segments, "gate", (".weight", ""))
        if wkey is None or entry.segments[wkey][3] != "F8_E4M3":
            return False
        shape = tuple(entry.shapes.get(wkey, ()))
        if len(shape) != 2 or shape[0] % 128 or shape[1] % 128 or min(shape) < 256:
            return False
        try:
            kind, _ = self._fp8_scale(entry, "gate", shape[0], shape[1])
        except ValueError:
            return False
        return kind == "block"

    def stats(self) -> dict:
        return dict(self._stats)

    def close(self) -> None:
        with self._cv:
            self._stop = True
            self._cv.notify_all()
        for t in self._workers:
            t.join(timeout=2.0)
        for fd, _ in self._fds.values():
            os.close(fd)
        self._fds.clear()


def _shape_2d(numel: int, shape: tuple[int, ...]) -> tuple[int, int]:
    if len(shape) >= 2:
        rows = 1
        for s in shape[:-1]:
            rows *= s
        return rows, shape[-1]
    raise ValueError(f"segment of {numel} elements has no 2-D shape {shape}")

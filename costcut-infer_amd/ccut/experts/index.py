"""Expert tensor index of a safetensors checkpoint (reference
``python/ccut/experts/index.py:40-276``): which shard and byte range holds
each segment of each (layer, expert), found by parsing shard headers only.

The tensor names are matched by a pattern with ``{layer}``, ``{expert}`` and
``{proj}`` placeholders (plain text, or a regex when it contains a
backslash), anchored at the start; what follows the match (``.weight``,
``.weight_scale``, ``.qweight``, ``.scales`` ...) is the segment key's
suffix: key = ``proj + suffix`` (``.weight`` when nothing follows).
Offsets are relative to the shard's data area (after the 8-byte length and
the JSON header), as in the safetensors format.
"""

from __future__ import annotations

import hashlib
import json
import re
import struct
import time
from dataclasses import dataclass, field
from pathlib import Path

__all__ = ["ExpertEntry", "ExpertIndex", "build_expert_index", "load_expert_index", "parse_expert_pattern",
           "read_header", "list_shards"]

CACHE_VERSION = 1


def parse_expert_pattern(pattern: str) -> re.Pattern[str]:
    """Regex of an expert tensor name pattern (reference ``index.py:40-61``):
    ``{layer}`` / ``{expert}`` capture digits, ``{proj}`` lowercase letters and
    underscores; plain text is escaped first; anchored at the start only."""
    rx = pattern if "\\" in pattern else re.escape(pattern)
    for ph, grp in (("layer", r"(?P<layer>\d+)"), ("expert", r"(?P<expert>\d+)"), ("proj", r"(?P<proj>[a-z_]+)")):
        rx = rx.replace("\\{" + ph + "\\}", grp).replace("{" + ph + "}", grp)
    return re.compile("^" + rx)


def read_header(path: str | Path) -> tuple[int, dict[str, tuple[str, tuple[int, ...], int, int]]]:
    """``(data_start, {name: (dtype, shape, begin, end)})`` of a safetensors
    file; begin/end are offsets into the data area."""
    with open(path, "rb") as fh:
        head = fh.read(8)
        if len(head) < 8:
            raise ValueError(f"{path}: shorter than a safetensors header")
        (n,) = struct.unpack("<Q", head)
        if n > 64 * 1024 * 1024:
            raise ValueError(f"{path}: header of {n} bytes, not a safetensors file")
        meta = json.loads(fh.read(n).decode("utf-8"))
    meta.pop("__metadata__", None)
    out = {}
    for name, info in meta.items():
        b, e = (int(v) for v in info["data_offsets"])
        if e < b:
            raise ValueError(f"{path}: tensor {name} has data_offsets {b}..{e}")
        out[name] = (info["dtype"], tuple(int(d) for d in info["shape"]), b, e)
    return 8 + n, out


def list_shards(model_dir: str | Path) -> tuple[list[str], int]:
    """Shard file names in manifest order (``model.safetensors.index.json``
    weight map, else every ``*.safetensors`` sorted) and the manifest's
    tensor count (0 without a manifest)."""
    model_dir = Path(model_dir)
    idx = model_dir / "model.safetensors.index.json"
    if idx.exists():
        wm = json.loads(idx.read_text()).get("weight_map", {})
        shards = list(dict.fromkeys(wm.values()))
        return [s for s in shards if (model_dir / s).exists()], len(wm)
    return sorted(p.name for p in model_dir.glob("*.safetensors")), 0


def _manifest_hash(model_dir: Path, shards: list[str]) -> str:
    h = hashlib.sha256()
    idx = model_dir / "model.safetensors.index.json"
    if idx.exists():
        h.update(idx.read_bytes())
    for s in shards:
        h.update(f"{s}:{(model_dir / s).stat().st_size};".encode())
    return h.hexdigest()


@dataclass(frozen=True)
class ExpertEntry:
    """Segments of one expert: key -> (offset, length, numel, dtype) in its shard."""

    shard: str
    segments: dict[str, tuple[int, int, int, str]]
    shapes: dict[str, tuple[int, ...]] = field(default_factory=dict)

    def bytes_total(self) -> int:
        return sum(s[1] for s in self.segments.values())


@dataclass
class ExpertIndex:
    model_path: str
    pattern: str
    num_layers: int
    num_experts: int
    top_k: int
    entries: dict[tuple[int, int], ExpertEntry] = field(default_factory=dict)
    tensors_total: int = 0
    build_ms: float = 0.0
    manifest_hash: str = ""

    def get(self, layer: int, expert: int) -> ExpertEntry | None:
        return self.entries.get((layer, expert))

    def coverage(self) -> tuple[int, int]:
        return len(self.entries), self.num_layers * self.num_experts

    def verify(self) -> None:
        have, want = self.coverage()
        if have != want:
            raise ValueError(f"expert index covers {have} of {want} (layers={self.num_layers} x "
                             f"experts={self.num_experts})")

    def to_dict(self) -> dict:
        return {
            "version": CACHE_VERSION,
            "model_path": self.model_path,
            "pattern": self.pattern,
            "num_layers": self.num_layers,
            "num_experts": self.num_experts,
            "top_k": self.top_k,
            "tensors_total": self.tensors_total,
            "manifest_hash": self.manifest_hash,
            "entries": {f"{l}:{e}": {"shard": v.shard, "segments": {k: list(s) for k, s in v.segments.items()},
                                     "shapes": {k: list(s) for k, s in v.shapes.items()}}
                        for (l, e), v in self.entries.items()},
        }

    @classmethod
    def from_dict(cls, d: dict) -> "ExpertIndex":
        entries = {}
        for key, v in d["entries"].items():
            l, e = (int(x) for x in key.split(":"))
            entries[(l, e)] = ExpertEntry(v["shard"], {k: tuple(s) for k, s in v["segments"].items()},
                                          {k: tuple(s) for k, s in v.get("shapes", {}).items()})
        return cls(d["model_path"], d["pattern"], d["num_layers"], d["num_experts"], d.get("top_k", 8), entries,
                   d.get("tensors_total", 0), 0.0, d.get("manifest_hash", ""))


_NUMEL_BYTES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "U64": 8, "I32": 4, "U32": 4, "I16": 2,
                "U16": 2, "I8": 1, "U8": 1, "BOOL": 1, "F8_E4M3": 1, "F8_E5M2": 1}


def build_expert_index(model_dir: str | Path, pattern: str, num_layers: int, num_experts: int, top_k: int = 8,
                       cache_path: str | Path | None = None, use_cache: bool = True,
                       verbose: bool = False) -> ExpertIndex:
    """Scan the shard headers (reference ``index.py:145-248``); with
    ``cache_path``, a cached index is used when its pattern, sizes and
    manifest hash match, and a fresh one is written there.  Raises
    ``ValueError`` when the index does not cover every (layer, expert)."""
    model_dir = Path(model_dir)
    t0 = time.perf_counter()
    shards, tensors_total = list_shards(model_dir)
    mhash = _manifest_hash(model_dir, shards)
    cache = Path(cache_path) if cache_path else None
    if use_cache and cache is not None and cache.exists():
        try:
            d = json.loads(cache.read_text())
            if (d.get("version") == CACHE_VERSION and d.get("pattern") == pattern and
                    d.get("num_layers") == num_layers and d.get("num_experts") == num_experts and
                    d.get("manifest_hash") == mhash):
                idx = ExpertIndex.from_dict(d)
                idx.verify()
                if verbose:
                    print(f"[expert-index] cache hit {cache} ({len(idx.entries)} experts)")
                return idx
        except (json.JSONDecodeError, KeyError, ValueError):
            pass  # rebuilt below
    rx = parse_expert_pattern(pattern)
    found: dict[tuple[int, int], tuple[str, dict, dict]] = {}
    total = 0
    for shard in shards:
        _, tensors = read_header(model_dir / shard)
        total += len(tensors)
        for name, (dtype, shape, b, e) in tensors.items():
            m = rx.match(name)
            if m is None:
                continue
            key = (int(m.group("layer")), int(m.group("expert")))
            seg_key = m.group("proj") + (name[m.end():] or ".weight")
            numel = 1
            for s in shape:
                numel *= s
            _, segs, shapes = found.setdefault(key, (shard, {}, {}))
            segs[seg_key] = (b, e - b, numel, dtype)
            shapes[seg_key] = shape
    idx = ExpertIndex(str(model_dir.resolve()), pattern, num_layers, num_experts, top_k,
                      {k: ExpertEntry(*v) for k, v in found.items()}, tensors_total or total,
                      round((time.perf_counter() - t0) * 1000, 1), mhash)
    idx.verify()
    if cache is not None:
        try:
            cache.parent.mkdir(parents=True, exist_ok=True)
            cache.write_text(json.dumps(idx.to_dict()))
        except OSError:
            pass  # a cache that cannot be written is not an error
    return idx


def load_expert_index(model_dir: str | Path, pattern: str, num_layers: int, num_experts: int, top_k: int = 8,
                      cache_path: str | Path | None = None, verbose: bool = False) -> ExpertIndex:
    """The cached index when valid, else a fresh scan (reference ``index.py:257-276``)."""
    return build_expert_index(model_dir, pattern, num_layers, num_experts, top_k, cache_path, True, verbose)
